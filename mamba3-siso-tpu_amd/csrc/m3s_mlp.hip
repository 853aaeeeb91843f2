// The gate of the LM's gated MLP on gfx950: a = value * silu(gate), and its backward,
// each as one HBM-bound pass over the fc1 product.
//
// Replaces the elementwise middle of `gated_mlp` (model.py:125-140): `value, gate =
// split(x @ fc1, 2)`, `fc2(value * silu(gate))`. Composed from framework ops that is a
// silu and a multiply forward, and two multiplies, a silu backward and a concatenation
// of the two halves' cotangents backward -- six passes over (rows, width) tensors where
// one each way suffices. The rounding points are those of the composed ops in the
// operand dtype: silu(gate) is rounded to the dtype before the product, and each
// cotangent is rounded once:
//   s = silu(g) = g / (1 + e^-g),  a = v s
//   dv = da s,  ds = da v,  dg = ds sig (1 + g (1 - sig)),  sig = 1 / (1 + e^-g)
// computed in f32. A thread takes one 16-byte vector of the value half and the matching
// vector of the gate half; a width that is not a multiple of 16 bytes (or unaligned
// tensors) runs the same code one element per thread.
#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

constexpr int kMlpThreads = 256;

template <typename T, bool VEC> struct MlpVec { using V = T __attribute__((ext_vector_type(1))); static constexpr int n = 1; };
template <> struct MlpVec<bf16, true> { using V = bf16x8; static constexpr int n = 8; };
template <> struct MlpVec<float, true> { using V = f32x4; static constexpr int n = 4; };

// row and vector-in-row of flat vector index i: 32-bit division when the whole range
// fits (a 64-bit divide is a long instruction sequence per 16-byte vector)
__device__ __forceinline__ void row_col(int64_t i, int64_t nvec, int wv, int64_t& r, int64_t& c) {
  if (nvec <= 0x7fffffff) {
    const uint32_t q = (uint32_t)i / (uint32_t)wv;
    r = q;
    c = (int64_t)((uint32_t)i - q * (uint32_t)wv);
  } else {
    r = i / wv;
    c = i % wv;
  }
}

template <typename T>
__device__ __forceinline__ float silu_round(float g) {
  return (float)(T)(g / (1.f + expf(-g)));
}

template <typename T, bool VEC>
__global__ void __launch_bounds__(kMlpThreads) swiglu_fwd_kernel(const T* __restrict__ h,
                                                                 T* __restrict__ a,
                                                                 int64_t nvec, int wv) {
  using V = typename MlpVec<T, VEC>::V;
  constexpr int n = MlpVec<T, VEC>::n;
  for (int64_t i = (int64_t)blockIdx.x * kMlpThreads + threadIdx.x; i < nvec;
       i += (int64_t)gridDim.x * kMlpThreads) {
    int64_t r, c;   // row, vector within the width
    row_col(i, nvec, wv, r, c);
    const V v = *reinterpret_cast<const V*>(h + (r * 2 * wv + c) * n);
    const V g = *reinterpret_cast<const V*>(h + (r * 2 * wv + wv + c) * n);
    V o;
#pragma unroll
    for (int e = 0; e < n; ++e) o[e] = (T)((float)v[e] * silu_round<T>((float)g[e]));
    *reinterpret_cast<V*>(a + i * n) = o;
  }
}

template <typename T, bool VEC>
__global__ void __launch_bounds__(kMlpThreads) swiglu_bwd_kernel(const T* __restrict__ h,
                                                                 const T* __restrict__ da,
                                                                 T* __restrict__ dh,
                                                                 int64_t nvec, int wv) {
  using V = typename MlpVec<T, VEC>::V;
  constexpr int n = MlpVec<T, VEC>::n;
  for (int64_t i = (int64_t)blockIdx.x * kMlpThreads + threadIdx.x; i < nvec;
       i += (int64_t)gridDim.x * kMlpThreads) {
    const int64_t r = i / wv, c = i % wv;   // (32-bit row_col measured slower here)
    const int64_t ov = (r * 2 * wv + c) * n, og = (r * 2 * wv + wv + c) * n;
    const V v = *reinterpret_cast<const V*>(h + ov);
    const V g = *reinterpret_cast<const V*>(h + og);
    const V d = *reinterpret_cast<const V*>(da + i * n);
    V dv, dg;
#pragma unroll
    for (int e = 0; e < n; ++e) {
      const float gf = (float)g[e], df = (float)d[e];
      dv[e] = (T)(df * silu_round<T>(gf));
      const float ds = (float)(T)(df * (float)v[e]);
      const float sig = 1.f / (1.f + expf(-gf));
      dg[e] = (T)(ds * sig * (1.f + gf * (1.f - sig)));
    }
    *reinterpret_cast<V*>(dh + ov) = dv;
    *reinterpret_cast<V*>(dh + og) = dg;
  }
}

static int32_t check_swiglu(const m3s_swiglu_args* a, const char* who, bool bwd) {
  M3S_REQUIRE(a != nullptr, "%s: args is NULL", who);
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_swiglu_args),
              "%s: struct_size %d != %d (ABI mismatch)", who, a->struct_size,
              (int)sizeof(m3s_swiglu_args));
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32, "%s: bad dtype %d", who,
              a->dtype);
  M3S_REQUIRE(a->rows >= 0 && a->width > 0, "%s: need rows >= 0 and width > 0 (got %lld, %d)",
              who, (long long)a->rows, a->width);
  if (a->rows == 0) return 0;   // nothing is read or written (empty tensors may be NULL)
  M3S_REQUIRE(a->h != nullptr && (bwd ? (a->da != nullptr && a->dh != nullptr) : a->a != nullptr),
              "%s: NULL pointer", who);
  const int esz = a->dtype == M3S_DTYPE_BF16 ? 2 : 4;
  auto elem_aligned = [esz](const void* q) { return ((uintptr_t)q % esz) == 0; };
  M3S_REQUIRE(elem_aligned(a->h) && (bwd ? (elem_aligned(a->da) && elem_aligned(a->dh))
                                         : elem_aligned(a->a)),
              "%s: tensors must be aligned to their element size", who);
  return 0;
}

static dim3 swiglu_grid(int64_t nvec) {
  const int64_t blocks = (nvec + kMlpThreads - 1) / kMlpThreads;
  return dim3((unsigned)std::min<int64_t>(std::max<int64_t>(blocks, 1), 256 * 16));
}

// 16-byte vectors when every row piece a thread touches is 16-byte aligned
static bool swiglu_vec(const m3s_swiglu_args* a, bool bwd) {
  const int n = a->dtype == M3S_DTYPE_BF16 ? 8 : 4;
  return a->width % n == 0 && aligned16(a->h) &&
         (bwd ? (aligned16(a->da) && aligned16(a->dh)) : aligned16(a->a));
}

template <typename T, bool VEC>
static void launch_swiglu(const m3s_swiglu_args* a, bool bwd, hipStream_t s) {
  constexpr int n = MlpVec<T, VEC>::n;
  const int wv = a->width / n;
  const int64_t nvec = a->rows * wv;
  if (nvec == 0) return;
  if (bwd) {
    hipLaunchKernelGGL((swiglu_bwd_kernel<T, VEC>), swiglu_grid(nvec), dim3(kMlpThreads), 0, s,
                       static_cast<const T*>(a->h), static_cast<const T*>(a->da),
                       static_cast<T*>(a->dh), nvec, wv);
  } else {
    hipLaunchKernelGGL((swiglu_fwd_kernel<T, VEC>), swiglu_grid(nvec), dim3(kMlpThreads), 0, s,
                       static_cast<const T*>(a->h), static_cast<T*>(a->a), nvec, wv);
  }
}

static int32_t run_swiglu(const m3s_swiglu_args* a, bool bwd, void* stream, const char* who) {
  if (a->rows == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = swiglu_vec(a, bwd);
  if (a->dtype == M3S_DTYPE_BF16) {
    vec ? launch_swiglu<bf16, true>(a, bwd, s) : launch_swiglu<bf16, false>(a, bwd, s);
  } else {
    vec ? launch_swiglu<float, true>(a, bwd, s) : launch_swiglu<float, false>(a, bwd, s);
  }
  return launch_status(who);
}


}  // namespace m3s

using namespace m3s;

extern "C" int32_t m3s_swiglu_fwd(const m3s_swiglu_args* a, void* stream) {
  clear_error();
  if (int32_t rc = check_swiglu(a, "m3s_swiglu_fwd", false)) return rc;
  return run_swiglu(a, false, stream, "m3s_swiglu_fwd");
}

extern "C" int32_t m3s_swiglu_bwd(const m3s_swiglu_args* a, void* stream) {
  clear_error();
  if (int32_t rc = check_swiglu(a, "m3s_swiglu_bwd", true)) return rc;
  return run_swiglu(a, true, stream, "m3s_swiglu_bwd");
}
