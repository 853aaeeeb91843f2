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

}  // namespace m3s

namespace m3s {
int32_t fwd_supported(int dtype, int chunk, int n, int pdim);
int32_t bwd_supported(int dtype, int chunk, int n, int pdim);
int32_t decode_supported(int dtype, int n, int pdim);
}  // namespace m3s
