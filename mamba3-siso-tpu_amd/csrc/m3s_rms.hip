// The LM's block norms on gfx950: RMSNorm of the residual stream, forward and backward.
//
// Replaces `rms_norm` (layer.py:190-198) as the LM applies it to the residual stream
// before each layer, each MLP and the head (model.py:194-232), and its autograd:
//
//   forward:   rstd = 1 / sqrt(mean_j x^2 + eps),   y = (x rstd w) cast to y's dtype
//   backward:  s = sum_j dy w x,   dx = rstd (dy w - x rstd^2 s / D),   dw = sum_rows dy x rstd
//
// in f32. The stream's rows are wide (d_model), so one wave owns a row and walks it in
// 16-byte vectors. The forward reads the row twice (the second read hits the cache). The
// backward takes dy in the dtype the next product consumed (no separate cast pass), keeps
// each lane's column partials of dw in registers across the rows its wave takes, adds
// the waves of a block in LDS, and leaves one partial row per block; a second launch sums
// those in a fixed order, so dw does not depend on the order in which blocks finish.
// HBM-bound.
//
// With a residual (`add`), the forward first forms the stream's next row s = x + add (in
// f32, stored in x's dtype: the residual add of model.py:222-228 before the next norm)
// and normalises s; the backward takes the cotangent the rest of the network gives s
// (`dsum`) and returns dsum + the norm's pullback, once in the stream's dtype and once in
// add's (the cotangents of x and of the block output). Each direction is then one pass
// where the residual add, its backward and the gradient cast were three more.
#include <algorithm>

#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

constexpr int kRmsThreads = 256;                     // 4 waves, one row each at a time
constexpr int kRmsWaves = kRmsThreads / 64;
constexpr int kRmsBwdBlocks = 1024;                  // fixed grid: bounded partials
constexpr int kRmsMaxChunks = 16;                    // 64-lane passes of 4 columns: D <= 4096

template <typename T>
__device__ __forceinline__ f32x4 ld4(const T* p) {
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const f32x4*>(p);
  } else {
    const bf16x4 r = *reinterpret_cast<const bf16x4*>(p);
    return f32x4{(float)r[0], (float)r[1], (float)r[2], (float)r[3]};
  }
}
template <typename T>
__device__ __forceinline__ void st4(T* p, f32x4 v) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<f32x4*>(p) = v;
  } else {
    *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
  }
}

// rows of D columns, D a multiple of 4; lane l takes columns 4 (l + 64 k), k < D / 256
template <typename TX, typename TY>
__global__ void __launch_bounds__(kRmsThreads) rms_fwd_kernel(const TX* __restrict__ x,
                                                              const float* __restrict__ w,
                                                              TY* __restrict__ y,
                                                              float* __restrict__ rstd,
                                                              const TY* __restrict__ add,
                                                              TX* __restrict__ sum,
                                                              int64_t M, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * kRmsWaves + (threadIdx.x >> 6);
  if (r >= M) return;   // whole waves leave together
  const TX* xr = x + r * D;
  const TY* ar = add ? add + r * D : nullptr;
  // the row the norm sees: x, or s = x + add rounded to the stream's dtype (both passes
  // form it from x and add; the second pass's reads hit the cache)
  auto row = [&](int c) {
    f32x4 v = ld4(xr + c);
    if (ar) {
      const f32x4 d = ld4(ar + c);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (float)(TX)(v[i] + d[i]);
    }
    return v;
  };
  TY* yr = y + r * D;
  float ss = 0.f;
  if (D <= 4 * 256) {
    // rows up to 1024 wide stay in registers between the two passes (at most four
    // 16-byte pieces per lane), and every load of the row is issued before the sum
    // (with the residual at 32768 x 768: 0.065 -> 0.053 ms; one row 3.1 -> 2.8 us)
    f32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = 4 * lane + 256 * k;
      v[k] = c < D ? row(c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = 4 * lane + 256 * k;
      if (c < D && ar) st4(sum + r * D + c, v[k]);
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += v[k][i] * v[k][i];
    }
    ss = wave_total(ss);
    const float rs = 1.f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = 4 * lane + 256 * k;
      if (c < D) {
        const f32x4 g = *reinterpret_cast<const f32x4*>(w + c);
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = v[k][i] * rs * g[i];
        st4(yr + c, o);
      }
    }
    if (lane == 0 && rstd) rstd[r] = rs;
    return;
  }
  for (int c = 4 * lane; c < D; c += 256) {
    const f32x4 v = row(c);
    if (ar) st4(sum + r * D + c, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += v[i] * v[i];
  }
  ss = wave_total(ss);
  const float rs = 1.f / sqrtf(ss / (float)D + eps);
  for (int c = 4 * lane; c < D; c += 256) {
    const f32x4 v = row(c);
    const f32x4 g = *reinterpret_cast<const f32x4*>(w + c);
    f32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = v[i] * rs * g[i];
    st4(yr + c, o);
  }
  if (lane == 0 && rstd) rstd[r] = rs;
}

// MAXK >= D / 256 column passes per lane (4, 8 or 16 by width): the column partials
// take 4 * MAXK registers, which sets the occupancy. Up to MAXK = 8 the row's x and dy
// stay in registers for the second pass; past that it reads them again.
template <typename TX, typename TY, int MAXK>
__global__ void __launch_bounds__(kRmsThreads) rms_bwd_kernel(const TX* __restrict__ x,
                                                              const float* __restrict__ w,
                                                              const float* __restrict__ rstd,
                                                              const TY* __restrict__ dy,
                                                              TX* __restrict__ dx,
                                                              float* __restrict__ part,
                                                              const TX* __restrict__ dsum,
                                                              TY* __restrict__ dadd,
                                                              int64_t M, int D) {
  extern __shared__ float sAcc[];   // [kRmsWaves][D]: sized at launch, for occupancy
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nk = D / 256 + ((4 * lane) < (D % 256) ? 1 : 0);   // this lane's column passes
  f32x4 acc[MAXK];
#pragma unroll
  for (int k = 0; k < MAXK; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int64_t nw = (int64_t)gridDim.x * kRmsWaves;
  for (int64_t r = (int64_t)blockIdx.x * kRmsWaves + wave; r < M; r += nw) {
    const TX* xr = x + r * D;
    const TY* dr = dy + r * D;
    const float rs = rstd[r];
    constexpr bool HOLD = MAXK <= 8;
    f32x4 hv[HOLD ? MAXK : 1], hd[HOLD ? MAXK : 1];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
      if (k < nk) {
        const int c = 4 * (lane + 64 * k);
        const f32x4 v = ld4(xr + c), d = ld4(dr + c);
        if constexpr (HOLD) {
          hv[k] = v;
          hd[k] = d;
        }
        const f32x4 g = *reinterpret_cast<const f32x4*>(w + c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s += d[i] * g[i] * v[i];
          acc[k][i] += d[i] * v[i] * rs;
        }
      }
    }
    s = wave_total(s);
    const float cr = rs * rs * s / (float)D;
    TX* xo = dx + r * D;
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
      if (k < nk) {
        const int c = 4 * (lane + 64 * k);
        const f32x4 v = HOLD ? hv[HOLD ? k : 0] : ld4(xr + c);
        const f32x4 d = HOLD ? hd[HOLD ? k : 0] : ld4(dr + c);
        const f32x4 g = *reinterpret_cast<const f32x4*>(w + c);
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = rs * (d[i] * g[i] - v[i] * cr);
        if (dsum) {
          const f32x4 e = ld4(dsum + r * D + c);
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = (float)(TX)o[i] + e[i];
        }
        st4(xo + c, o);
        if (dadd) st4(dadd + r * D + c, o);
      }
    }
  }
  // the block's waves in a fixed order, then one partial row per block
#pragma unroll
  for (int k = 0; k < MAXK; ++k) {
    if (k < nk) *reinterpret_cast<f32x4*>(sAcc + wave * D + 4 * (lane + 64 * k)) = acc[k];
  }
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += kRmsThreads) {
    float t = 0.f;
#pragma unroll
    for (int v = 0; v < kRmsWaves; ++v) t += sAcc[v * D + c];
    part[(int64_t)blockIdx.x * D + c] = t;
  }
}

// dw[c] = sum over blocks of part[b][c]: a block takes 64 columns; its 4 waves take every
// 4th block row (unrolled, so the loads of a run are in flight together), then the 4
// wave sums are added in wave order
__global__ void __launch_bounds__(kRmsThreads) rms_dw_kernel(const float* __restrict__ part,
                                                             float* __restrict__ dw, int nblk,
                                                             int D) {
  __shared__ float sSum[kRmsWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float t = 0.f;
  if (c < D) {
#pragma unroll 8
    for (int b = wave; b < nblk; b += kRmsWaves) t += part[(int64_t)b * D + c];
  }
  sSum[wave][lane] = t;
  __syncthreads();
  if (wave == 0 && c < D) {
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < kRmsWaves; ++v) s += sSum[v][lane];
    dw[c] = s;
  }
}

static int32_t check_rms(const m3s_rms_args* a, const char* who, bool bwd) {
  M3S_REQUIRE(a != nullptr, "%s: args is NULL", who);
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_rms_args),
              "%s: struct_size %d != %d (ABI mismatch)", who, a->struct_size,
              (int)sizeof(m3s_rms_args));
  const auto okdt = [](int d) { return d == M3S_DTYPE_BF16 || d == M3S_DTYPE_F32; };
  M3S_REQUIRE(okdt(a->x_dtype) && okdt(a->y_dtype), "%s: bad dtype", who);
  M3S_REQUIRE(a->rows >= 0 && a->width > 0 && a->width % 4 == 0 && a->width <= 4096,
              "%s: width %d must be a positive multiple of 4, at most 4096", who, a->width);
  if (a->rows == 0) return 0;
  M3S_REQUIRE(a->x && a->weight && (bwd ? (a->rstd && a->dy && a->dx && a->dweight && a->workspace)
                                        : a->y != nullptr),
              "%s: NULL pointer", who);
  const int xs = a->x_dtype == M3S_DTYPE_BF16 ? 2 : 4, ys = a->y_dtype == M3S_DTYPE_BF16 ? 2 : 4;
  M3S_REQUIRE((uintptr_t)a->x % (4 * xs) == 0 && (uintptr_t)a->weight % 16 == 0 &&
                  (bwd ? ((uintptr_t)a->dy % (4 * ys) == 0 && (uintptr_t)a->dx % (4 * xs) == 0)
                       : (uintptr_t)a->y % (4 * ys) == 0),
              "%s: rows must be aligned to 4 elements", who);
  if (bwd) {
    M3S_REQUIRE((uintptr_t)a->dsum % (4 * xs) == 0 && (uintptr_t)a->dadd % (4 * ys) == 0,
                "%s: dsum / dadd rows must be aligned to 4 elements", who);
  } else {
    M3S_REQUIRE((a->add == nullptr) == (a->sum == nullptr),
                "%s: give both add and sum, or neither", who);
    M3S_REQUIRE((uintptr_t)a->add % (4 * ys) == 0 && (uintptr_t)a->sum % (4 * xs) == 0,
                "%s: add / sum rows must be aligned to 4 elements", who);
  }
  return 0;
}

template <typename TX, typename TY>
static void launch_rms_fwd(const m3s_rms_args* a, hipStream_t s) {
  const int64_t blocks = (a->rows + kRmsWaves - 1) / kRmsWaves;
  hipLaunchKernelGGL((rms_fwd_kernel<TX, TY>), dim3((unsigned)blocks), dim3(kRmsThreads), 0, s,
                     static_cast<const TX*>(a->x), a->weight, static_cast<TY*>(a->y), a->rstd,
                     static_cast<const TY*>(a->add), static_cast<TX*>(a->sum), a->rows, a->width,
                     a->eps);
}

template <typename TX, typename TY>
static void launch_rms_bwd(const m3s_rms_args* a, hipStream_t s) {
  const int nblk = (int)std::min<int64_t>(kRmsBwdBlocks, (a->rows + kRmsWaves - 1) / kRmsWaves);
  float* part = static_cast<float*>(a->workspace);
  const size_t lds = (size_t)kRmsWaves * a->width * sizeof(float);
  const auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(nblk), dim3(kRmsThreads), lds, s, static_cast<const TX*>(a->x),
                       a->weight, a->rstd, static_cast<const TY*>(a->dy), static_cast<TX*>(a->dx),
                       part, static_cast<const TX*>(a->dsum), static_cast<TY*>(a->dadd), a->rows,
                       a->width);
  };
  if (a->width <= 1024) go(rms_bwd_kernel<TX, TY, 4>);
  else if (a->width <= 2048) go(rms_bwd_kernel<TX, TY, 8>);
  else go(rms_bwd_kernel<TX, TY, kRmsMaxChunks>);
  hipLaunchKernelGGL(rms_dw_kernel, dim3((a->width + 63) / 64), dim3(kRmsThreads), 0, s, part,
                     a->dweight, nblk, a->width);
}

template <bool BWD>
static void dispatch_rms(const m3s_rms_args* a, hipStream_t s) {
  const bool xb = a->x_dtype == M3S_DTYPE_BF16, yb = a->y_dtype == M3S_DTYPE_BF16;
  if constexpr (BWD) {
    if (xb) yb ? launch_rms_bwd<bf16, bf16>(a, s) : launch_rms_bwd<bf16, float>(a, s);
    else yb ? launch_rms_bwd<float, bf16>(a, s) : launch_rms_bwd<float, float>(a, s);
  } else {
    if (xb) yb ? launch_rms_fwd<bf16, bf16>(a, s) : launch_rms_fwd<bf16, float>(a, s);
    else yb ? launch_rms_fwd<float, bf16>(a, s) : launch_rms_fwd<float, float>(a, s);
  }
}

}  // namespace m3s

using namespace m3s;

extern "C" int64_t m3s_rms_bwd_workspace_bytes(int32_t width) {
  if (width <= 0) return -1;
  return (int64_t)kRmsBwdBlocks * width * 4;
}

extern "C" int32_t m3s_rms_fwd(const m3s_rms_args* a, void* stream) {
  clear_error();
  if (int32_t rc = check_rms(a, "m3s_rms_fwd", false)) return rc;
  if (a->rows == 0) return 0;
  dispatch_rms<false>(a, static_cast<hipStream_t>(stream));
  return launch_status("m3s_rms_fwd");
}

extern "C" int32_t m3s_rms_bwd(const m3s_rms_args* a, void* stream) {
  clear_error();
  if (int32_t rc = check_rms(a, "m3s_rms_bwd", true)) return rc;
  if (a->rows == 0) return 0;
  dispatch_rms<true>(a, static_cast<hipStream_t>(stream));
  return launch_status("m3s_rms_bwd");
}
