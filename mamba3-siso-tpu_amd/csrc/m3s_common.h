// Shared device helpers for the gfx950 Mamba-3 SISO kernels.
//
// MFMA fragment convention used by every kernel in this library
// ------------------------------------------------------------
// All matrix products run on 16x16 output tiles held in the MFMA accumulator layout:
// lane l owns column (l & 15) and rows 4*(l >> 4) + i, i < 4.
//
// Operands are fed as "sub-fragments": a sub-fragment covers a 16-wide slice of the
// contraction axis K; lane l supplies 4 consecutive K values, k = 4*(l >> 4) + i, for
// row (A) or column (B) index (l & 15). A 32-wide K block is two sub-fragments
// (one v_mfma_f32_16x16x32_bf16); a lone 16-wide block is one v_mfma_f32_16x16x16_bf16
// (or four v_mfma_f32_16x16x4_f32 for f32 operands). The MFMA sums over K slots
// (lane group, element) and A and B always use the same slot -> k map, so the
// result is the true product whatever order the hardware assigns to the slots.
//
// The payoff: an accumulator tile R[r][c] is *already* a sub-fragment with K = r
// (as a B operand with N = c, or as an A operand with M = c). A product's output can
// therefore feed the next product straight from registers -- the within-chunk score
// matrix never touches LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace m3s {

typedef __bf16 bf16;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kPi = 3.14159265358979323846f;
constexpr float kTwoPi = 6.28318530717958647692f;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// ---- scalar conversions ---------------------------------------------------------
template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f32(float x) { return (T)x; }

// ---- sub-fragment types ---------------------------------------------------------
template <typename MT> struct Sub;
template <> struct Sub<bf16> { typedef bf16x4 type; };
template <> struct Sub<float> { typedef f32x4 type; };
template <typename MT> using sub_t = typename Sub<MT>::type;

template <typename MT>
__device__ __forceinline__ sub_t<MT> sub_from_f32(f32x4 v) {
  sub_t<MT> r;
  r[0] = (MT)v[0]; r[1] = (MT)v[1]; r[2] = (MT)v[2]; r[3] = (MT)v[3];
  return r;
}
template <typename MT>
__device__ __forceinline__ f32x4 sub_to_f32(sub_t<MT> v) {
  f32x4 r;
  r[0] = (float)v[0]; r[1] = (float)v[1]; r[2] = (float)v[2]; r[3] = (float)v[3];
  return r;
}

// ---- MFMA wrappers --------------------------------------------------------------
// acc += A(16 x 16) * B(16 x 16) over one 16-wide K sub-block.
__device__ __forceinline__ void mma16(f32x4& acc, bf16x4 a, bf16x4 b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), acc, 0, 0, 0);
}
__device__ __forceinline__ void mma16(f32x4& acc, f32x4 a, f32x4 b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], acc, 0, 0, 0);
}
// acc += A * B over one 32-wide K block given as two sub-fragments each.
__device__ __forceinline__ void mma32(f32x4& acc, bf16x4 a0, bf16x4 a1, bf16x4 b0, bf16x4 b1) {
  bf16x8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
  bf16x8 b = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma32(f32x4& acc, f32x4 a0, f32x4 a1, f32x4 b0, f32x4 b1) {
  mma16(acc, a0, b0);
  mma16(acc, a1, b1);
}

// ---- sub-fragment loads from LDS ------------------------------------------------
// Row-contiguous storage: element (r, k) at buf[r * ld + k]. ld and k0 are multiples
// of 4, so each lane's 4 values are one aligned 8-byte (bf16) / 16-byte (f32) read.
template <typename MT>
__device__ __forceinline__ sub_t<MT> ld_sub(const MT* buf, int ld, int r0, int k0) {
  const int l = lane_id();
  return *reinterpret_cast<const sub_t<MT>*>(buf + (r0 + (l & 15)) * ld + k0 + 4 * (l >> 4));
}
// Same, but only the lane's row index and K offset are returned (for fused scaling).
__device__ __forceinline__ int sub_row(int r0) { return r0 + (lane_id() & 15); }
__device__ __forceinline__ int sub_k(int k0) { return k0 + 4 * (lane_id() >> 4); }

// Full product over K (multiple of 16) of two row-contiguous LDS operands:
// acc += A[rA0 .. rA0+15][0..K) * B[rB0 .. rB0+15][0..K)^T.
template <typename MT, int K>
__device__ __forceinline__ void gemm_nt(f32x4& acc, const MT* A, int lda, int rA0,
                                        const MT* B, int ldb, int rB0) {
#pragma unroll
  for (int k0 = 0; k0 + 32 <= K; k0 += 32) {
    mma32(acc, ld_sub<MT>(A, lda, rA0, k0), ld_sub<MT>(A, lda, rA0, k0 + 16),
          ld_sub<MT>(B, ldb, rB0, k0), ld_sub<MT>(B, ldb, rB0, k0 + 16));
  }
  if constexpr (K % 32 == 16) {
    mma16(acc, ld_sub<MT>(A, lda, rA0, K - 16), ld_sub<MT>(B, ldb, rB0, K - 16));
  }
}

// ---- bf16 operands for a 32-wide K block in the hardware's own slot order ----------
// v_mfma_f32_16x16x32_bf16 gives lane l the K slots 8*(l >> 4) + s, s < 8. When both
// operands come from LDS (neither is an accumulator tile) that contiguous order is
// used: one 16-byte read per lane.
__device__ __forceinline__ void mma32x(f32x4& acc, bf16x8 a, bf16x8 b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
// Row-contiguous storage, rows r0 + (l & 15), K = k0 + 8 (l >> 4) + s. The lane index
// is an argument so a kernel can pass one it re-derived inside its loop (which keeps
// the compiler from hoisting every per-lane LDS address out of the loop).
__device__ __forceinline__ bf16x8 ld_nat8(const bf16* buf, int ld, int r0, int k0, int l) {
  return *reinterpret_cast<const bf16x8*>(buf + (r0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}

// ---- transposed bf16 reads (ds_read_b64_tr_b16) ------------------------------------
// For storage T[k][m] (element (k, m) at buf[k * ld + m]), every lane of a 16-lane
// group receives 4 consecutive k of one column:
//   ld_tr4(buf, ld, kb, m0) = { T[kb + s][m0 + (l & 15)] : s < 4 }
// where kb may differ between lane groups. The instruction returns, to lane 4r + c of
// a group, element c of the 8-byte pieces addressed by lanes r, r + 4, r + 8, r + 12
// of that group; lane j therefore addresses row kb + j / 4, columns m0 + 4 (j % 4).
// ld must keep every row 8-byte aligned (ld % 4 == 0). l is the lane index.
__device__ __forceinline__ bf16x4 ld_tr4(const bf16* buf, int ld, int kb, int m0, int l) {
  const int j = l & 15;
  const bf16* p = buf + (kb + (j >> 2)) * ld + m0 + 4 * (j & 3);
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(bf16x4, r);
}

// ---- buffer (SGPR-descriptor) global memory access ---------------------------------
// A descriptor covers [base, base + bytes) of one workgroup's stream; each access adds a
// 32-bit per-lane byte offset (one VGPR, instead of a 64-bit address pair) and a
// uniform one (an SGPR, e.g. the chunk's start). Offsets past `bytes` read as zero and
// are dropped on store. 0x00020000 is the gfx9-family descriptor word 3 for raw dword
// access (as composable_kernel uses).
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
template <typename T> __device__ __forceinline__ T buf_load(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s);
template <> __device__ __forceinline__ bf16x8 buf_load<bf16x8>(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, v, s, 0));
}
template <> __device__ __forceinline__ f32x4 buf_load<f32x4>(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, v, s, 0));
}
template <> __device__ __forceinline__ float buf_load<float>(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, v, s, 0));
}
template <> __device__ __forceinline__ bf16 buf_load<bf16>(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  return __builtin_bit_cast(bf16, __builtin_amdgcn_raw_buffer_load_b16(r, v, s, 0));
}
__device__ __forceinline__ void buf_store(bf16x8 x, __amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, x), r, v, s, 0);
}
__device__ __forceinline__ void buf_store(f32x4 x, __amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, x), r, v, s, 0);
}
__device__ __forceinline__ void buf_store(bf16x4 x, __amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, x), r, v, s, 0);
}
__device__ __forceinline__ void buf_store_f32(float x, __amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, x), r, v, s, 0);
}
__device__ __forceinline__ void buf_store_bf16(float x, __amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(short, (bf16)x), r, v, s, 0);
}

// Loads and stores at a wave-uniform base pointer plus a 32-bit unsigned byte offset: the
// compiler emits the SGPR-base global form, two SGPRs per base where a buffer descriptor
// holds four. Unlike a buffer access there is no range check: the caller keeps every
// offset inside the tensor.
template <typename T>
__device__ __forceinline__ T gld(const void* base, uint32_t off) {
  return *reinterpret_cast<const T*>(static_cast<const char*>(base) + off);
}
template <typename T>
__device__ __forceinline__ void gst(void* base, uint32_t off, T v) {
  *reinterpret_cast<T*>(static_cast<char*>(base) + off) = v;
}

// Asynchronous 16-byte-per-lane load straight into LDS (no VGPR round trip): lane l's
// 16 bytes from rsrc + voffset + soffset land at lds_block + 16 l, so one instruction
// fills a contiguous 1 KiB LDS block. lds_block must be wave-uniform. Completion is
// tracked by vmcnt: wait with vm_wait_all() before a barrier that publishes the data.
__device__ __forceinline__ void buf_load_lds16(__amdgpu_buffer_rsrc_t r, void* lds_block,
                                               uint32_t v, uint32_t s) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_block,
                                           16, v, s, 0, 0);
}
// s_waitcnt vmcnt(0), leaving expcnt / lgkmcnt unconstrained (gfx9 encoding).
__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// s_waitcnt vmcnt(n), n < 16: every vector memory operation but the n most recent has
// completed (they complete in issue order for the purpose of this count).
template <int n>
__device__ __forceinline__ void vm_wait_keep() {
  static_assert(n >= 0 && n < 16, "vmcnt field of the gfx9 encoding");
  __builtin_amdgcn_s_waitcnt(0x0F70 | n);
}

// ---- wave reductions ------------------------------------------------------------
// DPP lane moves inside a 16-lane row (no LDS round trip, unlike a lane shuffle):
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror (lane i of an 8-lane half
// reads lane 7 - i), row_mirror (lane i of a row reads lane 15 - i).
constexpr int kDppQuadSwap1 = 0xB1, kDppQuadSwap2 = 0x4E, kDppHalfMirror = 0x141,
              kDppRowMirror = 0x140;
template <int ctrl>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false));
}

// row_shr:n -- lane i of a 16-lane row reads lane i - n of that row; the first n lanes
// of the row read 0 (their write is masked off and they keep the `old` operand, 0).
template <int n>
__device__ __forceinline__ float dpp_row_shr(float v) {
  static_assert(n >= 1 && n <= 15, "row_shr range");
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x110 + n, 0xF, 0xF, false));
}
// Inclusive prefix sum along each 16-lane row: lane i of a row gets the sum of lanes
// 0 .. i of that row (Hillis-Steele, four DPP adds).
__device__ __forceinline__ float row_prefix16(float v) {
  v += dpp_row_shr<1>(v);
  v += dpp_row_shr<2>(v);
  v += dpp_row_shr<4>(v);
  v += dpp_row_shr<8>(v);
  return v;
}

// Sum over aligned groups of W lanes (W a power of two <= 64), in every lane of the
// group: after the quad swaps each quad holds its sum, the half mirror pairs the two
// quads of an 8-lane half, the row mirror the two halves of a row; across rows, lane
// shuffles.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group width");
  if constexpr (W >= 2) v += dpp_mov<kDppQuadSwap1>(v);
  if constexpr (W >= 4) v += dpp_mov<kDppQuadSwap2>(v);
  if constexpr (W >= 8) v += dpp_mov<kDppHalfMirror>(v);
  if constexpr (W >= 16) v += dpp_mov<kDppRowMirror>(v);
  if constexpr (W >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (W >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Sum over the whole wave as a wave-uniform value: row sums by DPP, then the four rows'
// sums read from lanes 0, 16, 32 and 48.
__device__ __forceinline__ float wave_total(float v) {
  v = group_sum<16>(v);
  const int i = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 48)));
}

// n / d and n % d for 0 <= n < 2^20 by a divisor d known only at run time, without an
// integer division (a software routine on the GPU): a float estimate of the quotient
// (relative error below 2^-21, so off by at most one in this range), then one correction.
struct DivMod {
  int d;
  float inv;
  __device__ explicit DivMod(int d_) : d(d_), inv(__builtin_amdgcn_rcpf((float)d_)) {}
  __device__ __forceinline__ void operator()(int n, int& q, int& r) const {
    q = (int)((float)n * inv);
    r = n - q * d;
    if (r < 0) {
      --q;
      r += d;
    } else if (r >= d) {
      ++q;
      r -= d;
    }
  }
};

// ---- elementwise maths ----------------------------------------------------------
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
// The preprocess nonlinearities of reference.py:160-209, one definition for every kernel
// that applies them (the per-token pass, the scans' raw loads, the decode step, the
// preprocess kernels), so they agree bit for bit: softplus with torch's threshold 20,
// heavy_tail(x) = max(x, 0) + 1 / (1 - min(x, 0)), the logistic sigmoid.
__device__ __forceinline__ float softplus_(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float heavy_tail_(float x) {
  return fmaxf(x, 0.f) + 1.f / (1.f - fminf(x, 0.f));
}
__device__ __forceinline__ float sigmoid_(float x) { return 1.f / (1.f + expf(-x)); }
// The same three from the hardware exp2 / log2 / reciprocal (about 2e-6 relative at |x| <=
// 20, from rounding x log2(e)): for the scans' raw loads, whose results feed bf16 products.
// log1p(e) by Goldberg's correction, log(u) e / (u - 1) with u = 1 + e, which stays accurate
// where 1 + e rounds (small dt), and is e itself where u rounds to 1.
constexpr float kLn2 = 0.69314718055994531f;
__device__ __forceinline__ float softplus_fast(float x) {
  const float e = __builtin_amdgcn_exp2f(x * kLog2e);
  const float u = 1.f + e, d = u - 1.f;
  const float r = d == 0.f ? e : (__builtin_amdgcn_logf(u) * kLn2) * (e * __builtin_amdgcn_rcpf(d));
  return x > 20.f ? x : r;
}
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
}
// tanh from the hardware exp2 / reciprocal: sign(x) (1 - e) / (1 + e), e = 2^{-2 |x| log2 e}.
// Near 0 the subtraction leaves an absolute error of a few 1e-8 (a relative one of
// ~1e-7 / |x|): for angles that are summed into a phase, where the absolute error counts.
__device__ __forceinline__ float tanh_fast(float x) {
  const float e = __builtin_amdgcn_exp2f(-2.f * kLog2e * fabsf(x));
  return copysignf((1.f - e) * __builtin_amdgcn_rcpf(1.f + e), x);
}
__device__ __forceinline__ float heavy_tail_fast(float x) {
  return fmaxf(x, 0.f) + __builtin_amdgcn_rcpf(1.f - fminf(x, 0.f));
}
// The RMS norm's row scale rsqrt(ss / n + eps) (layer.py:190-198) from a row's sum of
// squares: the mean as a product with 1 / n (exact when n is a power of two, as every
// compiled d_state is) and the hardware reciprocal square root (about one ulp, as the
// two roundings of 1 / sqrt are). One definition for every norm of the B and C rows (the
// forward norms, their angle pass, the decode step), so they agree bit for bit.
__device__ __forceinline__ float bc_rstd(float ss, float inv_n, float eps) {
  return __builtin_amdgcn_rsqf(fmaf(ss, inv_n, eps));
}
__device__ __forceinline__ float silu(float x) { return x * sigmoidf_(x); }
// silu from the hardware exp2 / reciprocal (~2 ulp): for gates whose product is rounded
// to bf16 right after.
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}
__device__ __forceinline__ float wrap_2pi(float phi) {
  return phi - kTwoPi * floorf(phi / kTwoPi);
}
// wrap_2pi without the division: the quotient from a multiply by 1 / (2 pi), one fma for
// the remainder, then a step back into [0, 2 pi) where the quotient was off by one.
__device__ __forceinline__ float wrap_2pi_fast(float phi) {
  float r = fmaf(-kTwoPi, floorf(phi * 0.15915494309189535f), phi);
  r = r < 0.f ? r + kTwoPi : r;
  return r >= kTwoPi ? r - kTwoPi : r;
}

// ---- two adjacent elements as one LDS store ---------------------------------------
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <typename MT> __device__ __forceinline__ void store_pair(MT* dst, float a, float b);
template <> __device__ __forceinline__ void store_pair<bf16>(bf16* dst, float a, float b) {
  *reinterpret_cast<bf16x2*>(dst) = bf16x2{(bf16)a, (bf16)b};
}
template <> __device__ __forceinline__ void store_pair<float>(float* dst, float a, float b) {
  *reinterpret_cast<f32x2*>(dst) = f32x2{a, b};
}

}  // namespace m3s
