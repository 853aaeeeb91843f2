// Host-side helpers shared by the C-ABI entry points: error reporting, argument
// checks, launch wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/m3s.h"

namespace m3s {

// Thread-local message for m3s_last_error().
void set_error(const char* fmt, ...);
void clear_error();

#define M3S_REQUIRE(cond, ...)                 \
  do {                                         \
    if (!(cond)) {                             \
      ::m3s::set_error(__VA_ARGS__);           \
      return M3S_ERR_INVALID;                  \
    }                                          \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A (B,H,L,P) operand: non-null, base 16-byte aligned, strides multiples of the
// 16-byte vector width so every row segment a lane reads is aligned.
inline bool bhlp_ok(const m3s_bhlp& t, int vec) {
  return t.ptr != nullptr && aligned16(t.ptr) && t.stride_b % vec == 0 &&
         t.stride_h % vec == 0 && t.stride_t % vec == 0;
}

inline int32_t launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return M3S_ERR_LAUNCH;
  }
  return M3S_OK;
}

// Grid -> (b, h) mapping. Blocks are dispatched round-robin over the 8 XCDs of
// MI355X; re-number them so that consecutive work items (the heads of one batch
// element, which share q/k) land on the same XCD and hit the same L2.
__device__ __forceinline__ int xcd_remap(int bid, int nwg) {
  return (nwg % 8 == 0) ? (bid % 8) * (nwg / 8) + bid / 8 : bid;
}

// Staggered start for the sequential scans. Their workgroups start together and run the
// same per-chunk phase sequence at the same pace, so the memory-heavy phases of all of
// them coincide and queue on HBM while the other phases leave it idle. Delaying a share
// of each XCD's workgroups (block i runs on XCD i % 8, so i / 8 counts within one XCD)
// by a fraction of a chunk's time spreads that traffic over the chunk: group
// g = (i / 8) % groups (groups a power of two) first sleeps g * units * ~2048 cycles
// (s_sleep 32 is 32 * 64 cycles). The cost is that delay, once. Only the first round of
// a launch starts in step (one scan workgroup per CU, 256 CUs on MI355X); a workgroup of
// a later round starts when one of the first ends, already out of phase, so it does not
// sleep (cfg5's backward, 384 workgroups: 0.794 -> 0.786 ms).
constexpr int kFirstRound = 256;
__device__ __forceinline__ void stagger_start(int bid, int groups, int units) {
  if (bid >= kFirstRound) return;
  const int g = (bid >> 3) & (groups - 1);
  for (int i = 0; i < g * units; ++i) __builtin_amdgcn_s_sleep(32);
}

}  // namespace m3s

namespace m3s {
int32_t fwd_supported(int dtype, int chunk, int n, int pdim);
int32_t fwd_raw_supported_impl(int dtype, int chunk, int n, int pdim, int nr);
int32_t bwd_supported(int dtype, int chunk, int n, int pdim);
int32_t decode_supported(int dtype, int n, int pdim);
}  // namespace m3s
