// The layer's BCNorm on gfx950: RMSNorm over the state axis of the projection's B and
// C slices, forward and backward, both norms in one launch.
//
// Replaces `layer.rms_norm` (layer.py:190-198) as applied to B and C at
// layer.py:235-236, and its autograd:
//
//   forward:   rstd = rsqrt(mean_n x^2 + eps),   y = (x rstd w) cast to x's dtype   (f32 math)
//   backward:  g = dy cast to x's dtype (the layer hands its q/k cotangent back in the
//              primal dtype, siso.py:140-148), then in f32
//              dx = rstd g w - (rstd^3 / N) x sum_n(g w x),   dw = sum_rows g x rstd
//
// A row of N values is owned by a group of G lanes (16 bytes each, G a power of two,
// lanes past N idle); the row statistic is a shuffle reduction inside the group. Rows
// are read in place through (b, t) strides, so the slices of the fused projection need
// no copy, and dx lands directly in the slices of the projection's gradient. The gain
// gradient is summed per block in a fixed order, then over blocks by a second launch,
// so it does not depend on the order in which blocks finish. HBM-bound.
#include <algorithm>
#include <type_traits>
#include <mutex>

#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

constexpr int kNormThreads = 256;
constexpr int kNormBwdBlocks = 1024;   // fixed grid of the backward: bounded partials

struct NormRows {
  const void* x[2];
  int64_t xsb[2], xst[2];
  const float* w[2];
};

// The rotary angles' per-token work, done in the same launch as the norms (a third
// role after the `count` norm roles), for the forward scan's raw mode (reference.py:134-157
// split between this pass and the scan): the head-shared table theta_table = tanh(angles)
// pi; for every head, theta_t = theta_table[t] softplus(dt_raw[t] + dt_bias) summed over
// each 16-token strip, and the strip sums' exclusive prefix within each chunk of `chunk`
// tokens (the angle a strip starts at, relative to its chunk's start); and each chunk's
// total. The scan carries the chunk totals across its chunks and adds the rest per row.
struct NormThetaParams {
  const void* ang;
  int64_t asb, ast;
  const void* dtr;
  int64_t dsb, dst;
  const float* dt_bias;
  float* tab;    // (B, L, Nr)
  float* pre;    // (B, H, L / 16, Nr) strip starts within their chunk
  float* ctot;   // (B, H, L / chunk, Nr) chunk totals
  int H, Nr, chunk, nblk;
};

struct NormFwdParams {
  NormRows in;
  int B, L, N, G, count;
  float eps, inv_n;   // inv_n = 1 / N
  void* y[2];
  float* rstd[2];
  NormThetaParams th;
};

struct NormBwdParams {
  NormRows in;
  int B, L, N, G;
  const float* rstd[2];
  const float* dy[2];
  void* dx[2];
  int64_t dxsb[2], dxst[2];
  float* part;   // (gridDim.x, 2, N) gain partials
};

template <typename T> struct NVec;
template <> struct NVec<bf16> { static constexpr int n = 8; typedef bf16x8 type; };
template <> struct NVec<float> { static constexpr int n = 4; typedef f32x4 type; };

template <typename T>
__device__ __forceinline__ void load_row(const T* p, float (&v)[NVec<T>::n]) {
  const auto r = *reinterpret_cast<const typename NVec<T>::type*>(p);
#pragma unroll
  for (int i = 0; i < NVec<T>::n; ++i) v[i] = (float)r[i];
}

template <typename T>
__device__ __forceinline__ void store_row(T* p, const float (&v)[NVec<T>::n]) {
  typename NVec<T>::type r;
#pragma unroll
  for (int i = 0; i < NVec<T>::n; ++i) r[i] = (T)v[i];
  *reinterpret_cast<typename NVec<T>::type*>(p) = r;
}

__device__ __forceinline__ float group_sum_dyn(float v, int G) {
  for (int m = 1; m < G; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// The norms together with the angle role: one 512-thread block per chunk of one batch
// element does the chunk's B and C rows and, in three parallel steps, its angle work: the
// chunk's table rows and every head's dt into LDS; every (strip, head, angle quad) sum of
// 16 rows in time order into LDS; a thread per (head, quad) walks the strips for their
// prefixes and the chunk total. The angle role's loads are issued first, so the norm rows
// stream while they are in flight. LDS: chunk (Nr + H) + (chunk / 16) H Nr floats.
constexpr int kThetaThreads = 512;
// The chunk's B and C rows, kRowBatch rows per group of G lanes at a time: every row's
// load of a batch is issued before the first row's statistic (one memory latency per
// batch). `norm_issue` loads batch `base`, `norm_finish` normalises and stores it.
constexpr int kRowBatch = 8;
template <typename T>
__device__ __forceinline__ void norm_issue(const NormFwdParams& p, int b, int t0, int base,
                                           typename NVec<T>::type (&xv)[kRowBatch]) {
  constexpr int VEC = NVec<T>::n;
  using VT = typename NVec<T>::type;
  const int C = p.th.chunk, G = p.G, gid = threadIdx.x / G, gl = threadIdx.x % G;
  const int rows = p.count * C, per_pass = kThetaThreads / G;
  const int n0 = gl * VEC;
  const bool act = n0 < p.N;
#pragma unroll
  for (int k = 0; k < kRowBatch; ++k) {   // uniform over each group of G lanes
    const int rr = base + gid + k * per_pass;
    const int which = rr >= C ? 1 : 0, t = t0 + rr - which * C;
    if (rr < rows && act)
      xv[k] = *reinterpret_cast<const VT*>(static_cast<const T*>(p.in.x[which]) + b * p.in.xsb[which] +
                                           t * p.in.xst[which] + n0);
  }
}
template <typename T>
__device__ __forceinline__ void norm_finish(const NormFwdParams& p, int b, int t0, int base,
                                            const typename NVec<T>::type (&xv)[kRowBatch]) {
  constexpr int VEC = NVec<T>::n;
  using VT = typename NVec<T>::type;
  const int C = p.th.chunk, G = p.G, gid = threadIdx.x / G, gl = threadIdx.x % G;
  const int rows = p.count * C, per_pass = kThetaThreads / G;
  const int n0 = gl * VEC;
  const bool act = n0 < p.N;
#pragma unroll
  for (int k = 0; k < kRowBatch; ++k) {
    const int rr = base + gid + k * per_pass;
    if (rr >= rows) break;
    const int which = rr >= C ? 1 : 0, t = t0 + rr - which * C;
    const int64_t r = (int64_t)b * p.L + t;
    float ss = 0.f;
    if (act) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) ss += (float)xv[k][i] * (float)xv[k][i];
    }
    ss = group_sum_dyn(ss, G);
    const float rstd = bc_rstd(ss, p.inv_n, p.eps);
    if (act) {
      const float* w = p.in.w[which] + n0;
      VT yv;
#pragma unroll
      for (int i = 0; i < VEC; ++i) yv[i] = (T)((float)xv[k][i] * rstd * w[i]);
      *reinterpret_cast<VT*>(static_cast<T*>(p.y[which]) + r * p.N + n0) = yv;
    }
    if (gl == 0 && p.rstd[which]) p.rstd[which][r] = rstd;
  }
}
template <typename T>
__global__ void __launch_bounds__(kThetaThreads) norm_theta_kernel(const NormFwdParams p) {
  extern __shared__ float dyn[];
  const NormThetaParams& q = p.th;
  const int L = p.L;
  const int Nr = q.Nr, H = q.H, C = q.chunk, nc = L / C, ns = L / 16, spc = C / 16;
  const int nq = Nr / 4;
  const int b = blockIdx.x / nc, c = blockIdx.x - b * nc, t0 = c * C;
  float* sTab = dyn;              // [C][Nr]
  float* sDt = dyn + C * Nr;      // [C][H]
  float* sSum = sDt + C * H;      // [spc][H][Nr]
  const T* ang = static_cast<const T*>(q.ang) + b * q.asb;
  const T* dtr = static_cast<const T*>(q.dtr) + b * q.dsb;
  // rounds of kThetaRound items per thread, every load of a round issued before any use
  // (one memory latency per round, not per item); the first round of all three kinds
  // (angles, dt_raw, B / C rows) is issued before any of them is used. Quotients by the
  // run-time Nr, H and pair counts through DivMod (a float estimate), not integer
  // division; tanh and softplus from the hardware exp2 / log2 / rcp (tanh_fast,
  // softplus_fast) for bf16 operands, the library functions for f32, as the preprocess
  // kernels use them.
  constexpr int kThetaRound = 8;
  constexpr int STEP = kThetaRound * kThetaThreads;
  const DivMod byNr(Nr), byH(H), byPairs(H * nq), byNq(nq);
  auto issue_ang = [&](int base, float (&v)[kThetaRound]) {
#pragma unroll
    for (int u = 0; u < kThetaRound; ++u) {
      const int i = base + threadIdx.x + u * kThetaThreads;
      int t, j;
      byNr(i, t, j);
      v[u] = i < C * Nr ? (float)ang[(int64_t)(t0 + t) * q.ast + j] : 0.f;
    }
  };
  auto finish_ang = [&](int base, const float (&v)[kThetaRound]) {
#pragma unroll
    for (int u = 0; u < kThetaRound; ++u) {
      const int i = base + threadIdx.x + u * kThetaThreads;
      if (i < C * Nr) {
        const float tp = (std::is_same<T, float>::value ? tanhf(v[u]) : tanh_fast(v[u])) * kPi;
        q.tab[((int64_t)b * L + t0) * Nr + i] = tp;   // the chunk's rows are contiguous
        sTab[i] = tp;
      }
    }
  };
  auto issue_dt = [&](int base, float (&v)[kThetaRound]) {
#pragma unroll
    for (int u = 0; u < kThetaRound; ++u) {
      const int i = base + threadIdx.x + u * kThetaThreads;
      int t, h;
      byH(i, t, h);
      v[u] = i < C * H ? (float)dtr[(int64_t)(t0 + t) * q.dst + h] + q.dt_bias[h] : 0.f;
    }
  };
  auto finish_dt = [&](int base, const float (&v)[kThetaRound]) {
#pragma unroll
    for (int u = 0; u < kThetaRound; ++u) {
      const int i = base + threadIdx.x + u * kThetaThreads;
      if (i < C * H) sDt[i] = std::is_same<T, float>::value ? softplus_(v[u]) : softplus_fast(v[u]);
    }
  };
  {
    float av[kThetaRound], dv[kThetaRound];
    typename NVec<T>::type xv[kRowBatch];
    issue_ang(0, av);
    issue_dt(0, dv);
    norm_issue<T>(p, b, t0, 0, xv);
    finish_ang(0, av);
    finish_dt(0, dv);
    norm_finish<T>(p, b, t0, 0, xv);
  }
  for (int base = STEP; base < C * Nr; base += STEP) {
    float v[kThetaRound];
    issue_ang(base, v);
    finish_ang(base, v);
  }
  for (int base = STEP; base < C * H; base += STEP) {
    float v[kThetaRound];
    issue_dt(base, v);
    finish_dt(base, v);
  }
  const int rows_step = kRowBatch * (kThetaThreads / p.G);
  for (int base = rows_step; base < p.count * C; base += rows_step) {
    typename NVec<T>::type xv[kRowBatch];
    norm_issue<T>(p, b, t0, base, xv);
    norm_finish<T>(p, b, t0, base, xv);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < spc * H * nq; i += kThetaThreads) {   // (strip, head, quad)
    int st, r, h, jq;
    byPairs(i, st, r);
    byNq(r, h, jq);
    const int j0 = 4 * jq;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const f32x4 tb = *reinterpret_cast<const f32x4*>(sTab + (16 * st + t) * Nr + j0);
      const float dt = sDt[(16 * st + t) * H + h];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += tb[e] * dt;
    }
    *reinterpret_cast<f32x4*>(sSum + (st * H + h) * Nr + j0) = acc;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < H * nq; i += kThetaThreads) {
    int h, jq;
    byNq(i, h, jq);
    const int j0 = 4 * jq;
    float* pre = q.pre + (((int64_t)b * H + h) * ns + t0 / 16) * Nr + j0;
    f32x4 run = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < spc; ++s) {
      *reinterpret_cast<f32x4*>(pre + s * Nr) = run;
      run += *reinterpret_cast<const f32x4*>(sSum + (s * H + h) * Nr + j0);
    }
    *reinterpret_cast<f32x4*>(q.ctot + (((int64_t)b * H + h) * nc + c) * Nr + j0) = run;
  }
}

// One (B or C) row of one token: G lanes, 16 bytes each; the row statistic is a shuffle
// reduction inside the group, so all G lanes of a group call this together.
template <typename T>
__device__ __forceinline__ void norm_row(const NormFwdParams& p, int which, int b, int t,
                                         int64_t r, int gl) {
  constexpr int VEC = NVec<T>::n;
  const int n0 = gl * VEC;
  const bool act = n0 < p.N;
  const T* xrow = static_cast<const T*>(p.in.x[which]) + b * p.in.xsb[which] + t * p.in.xst[which];
  float x[VEC];
  float ss = 0.f;
  if (act) {
    load_row<T>(xrow + n0, x);
#pragma unroll
    for (int i = 0; i < VEC; ++i) ss += x[i] * x[i];
  }
  ss = group_sum_dyn(ss, p.G);
  const float rstd = bc_rstd(ss, p.inv_n, p.eps);
  if (act) {
    const float* w = p.in.w[which] + n0;
    float y[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) y[i] = x[i] * rstd * w[i];
    store_row<T>(static_cast<T*>(p.y[which]) + r * p.N + n0, y);
  }
  if (gl == 0 && p.rstd[which]) p.rstd[which][r] = rstd;
}

template <typename T>
__global__ void __launch_bounds__(kNormThreads) norm_fwd_kernel(const NormFwdParams p) {
  const int which = blockIdx.y;
  const int G = p.G, gid = threadIdx.x / G, gl = threadIdx.x % G;
  const int rows_per_block = kNormThreads / G;
  const int64_t M = (int64_t)p.B * p.L;
  const int64_t r = (int64_t)blockIdx.x * rows_per_block + gid;
  if (r >= M) return;   // whole groups leave together: the shuffles stay in-group
  norm_row<T>(p, which, (int)(r / p.L), (int)(r % p.L), r, gl);
}

template <typename T>
__global__ void __launch_bounds__(kNormThreads) norm_bwd_kernel(const NormBwdParams p) {
  constexpr int VEC = NVec<T>::n;
  __shared__ float sAcc[kNormThreads * VEC];
  const int which = blockIdx.y;
  const int G = p.G, gid = threadIdx.x / G, gl = threadIdx.x % G;
  const int rows_per_pass = kNormThreads / G;
  const int64_t M = (int64_t)p.B * p.L;
  const int n0 = gl * VEC;
  const bool act = n0 < p.N;
  const float* w = p.in.w[which] + (act ? n0 : 0);
  float wv[VEC], acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    wv[i] = act ? w[i] : 0.f;
    acc[i] = 0.f;
  }
  const float inv_n = 1.f / (float)p.N;
  for (int64_t r = (int64_t)blockIdx.x * rows_per_pass + gid; r < M;
       r += (int64_t)gridDim.x * rows_per_pass) {
    const int b = (int)(r / p.L), t = (int)(r % p.L);
    const float rstd = p.rstd[which][r];
    float x[VEC], g[VEC];
    float s = 0.f;
    if (act) {
      load_row<T>(static_cast<const T*>(p.in.x[which]) + b * p.in.xsb[which] + t * p.in.xst[which] + n0, x);
      const float* dyr = p.dy[which] + r * p.N + n0;
#pragma unroll
      for (int i = 0; i < VEC; i += 4) {
        const f32x4 d = *reinterpret_cast<const f32x4*>(dyr + i);
#pragma unroll
        for (int k = 0; k < 4; ++k) g[i + k] = (float)(T)d[k];   // the primal-dtype cast
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        s += g[i] * wv[i] * x[i];
        acc[i] += g[i] * x[i] * rstd;
      }
    }
    s = group_sum_dyn(s, G);
    if (act) {
      const float c = rstd * rstd * rstd * inv_n * s;
      float dx[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) dx[i] = rstd * g[i] * wv[i] - c * x[i];
      store_row<T>(static_cast<T*>(p.dx[which]) + b * p.dxsb[which] + t * p.dxst[which] + n0, dx);
    }
  }
  // gain partials: sum the groups of this block in a fixed order
#pragma unroll
  for (int i = 0; i < VEC; ++i) sAcc[threadIdx.x * VEC + i] = acc[i];
  __syncthreads();
  for (int n = threadIdx.x; n < p.N; n += kNormThreads) {
    const int l = n / VEC, i = n % VEC;
    float tot = 0.f;
    for (int q = 0; q < rows_per_pass; ++q) tot += sAcc[(q * G + l) * VEC + i];
    p.part[((int64_t)blockIdx.x * 2 + which) * p.N + n] = tot;
  }
}

// dw[which][n] = sum over blocks of the partials. A block takes 64 columns; each of its four
// waves sums a quarter of the block partials (eight independent accumulators, fixed order),
// and the four quarters are added in wave order.
__global__ void __launch_bounds__(kNormThreads) norm_gain_kernel(const float* __restrict__ part,
                                                                 float* dw0, float* dw1,
                                                                 int nblk, int N) {
  __shared__ float sq[kNormThreads];
  const int which = blockIdx.y;
  const int col = threadIdx.x % 64, slice = threadIdx.x / 64;
  const int n = blockIdx.x * 64 + col;
  const int per = (nblk + 3) / 4, k0 = slice * per, k1 = min(nblk, k0 + per);
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (n < N) {
    int k = k0;
    for (; k + 8 <= k1; k += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) a[u] += part[((int64_t)(k + u) * 2 + which) * N + n];
    }
    for (; k < k1; ++k) a[0] += part[((int64_t)k * 2 + which) * N + n];
  }
  sq[threadIdx.x] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  __syncthreads();
  if (slice == 0 && n < N)
    (which ? dw1 : dw0)[n] = (sq[col] + sq[64 + col]) + (sq[128 + col] + sq[192 + col]);
}

static int norm_group(int N, int vec) {
  int lanes = N / vec, G = 1;
  while (G < lanes) G <<= 1;
  return G;
}

static bool blx_ok(const m3s_blx& t, int vec) {
  return t.ptr != nullptr && aligned16(t.ptr) && t.stride_b % vec == 0 && t.stride_t % vec == 0;
}

}  // namespace m3s

using namespace m3s;

extern "C" int64_t m3s_norm_bwd_workspace_bytes(int32_t width) {
  if (width <= 0) return -1;
  return (int64_t)kNormBwdBlocks * 2 * width * 4;
}

extern "C" int32_t m3s_norm_fwd(const m3s_norm_fwd_args* a, void* stream) {
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_norm_fwd: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_norm_fwd_args),
              "m3s_norm_fwd: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_norm_fwd_args));
  const int B = a->batch, L = a->seqlen, N = a->width, cnt = a->count;
  M3S_REQUIRE(B > 0 && L > 0 && N > 0 && (cnt == 1 || cnt == 2), "m3s_norm_fwd: bad dimension");
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32,
              "m3s_norm_fwd: bad dtype %d", a->dtype);
  const int vec = a->dtype == M3S_DTYPE_BF16 ? 8 : 4;
  M3S_REQUIRE(N % vec == 0 && N / vec <= 64,
              "m3s_norm_fwd: width %d must be a multiple of %d and at most %d", N, vec, 64 * vec);
  M3S_REQUIRE((int64_t)B * L < (1ll << 31), "m3s_norm_fwd: B*L too large");
  NormFwdParams p{};
  for (int i = 0; i < cnt; ++i) {
    M3S_REQUIRE(blx_ok(a->x[i], vec), "m3s_norm_fwd: x[%d] must be 16-byte aligned rows", i);
    M3S_REQUIRE(a->weight[i] && a->y[i] && aligned16(a->y[i]),
                "m3s_norm_fwd: weight[%d] NULL or y[%d] NULL / misaligned", i, i);
    p.in.x[i] = a->x[i].ptr; p.in.xsb[i] = a->x[i].stride_b; p.in.xst[i] = a->x[i].stride_t;
    p.in.w[i] = a->weight[i];
    p.y[i] = a->y[i];
    p.rstd[i] = a->rstd[i];
  }
  p.B = B; p.L = L; p.N = N; p.G = norm_group(N, vec); p.eps = a->eps; p.count = cnt;
  p.inv_n = 1.f / (float)N;
  const bool theta = a->theta_table || a->theta_prefix || a->theta_chunk_totals ||
                     a->angles.ptr || a->dt_raw.ptr;
  size_t dyn = 0;
  if (theta) {
    const int H = a->nheads, Nr = a->n_angles, C = a->theta_chunk;
    M3S_REQUIRE(a->theta_table && a->theta_prefix && a->theta_chunk_totals && a->angles.ptr &&
                    a->dt_raw.ptr && a->dt_bias,
                "m3s_norm_fwd: give angles, dt_raw, dt_bias, theta_table, theta_prefix and "
                "theta_chunk_totals together (or none)");
    M3S_REQUIRE(H > 0 && Nr > 0 && Nr % 4 == 0 && H <= 1024 && Nr <= 1024,
                "m3s_norm_fwd: nheads %d / n_angles %d out of range (n_angles %% 4 == 0)", H, Nr);
    M3S_REQUIRE(C >= 16 && C % 16 == 0 && L % C == 0,
                "m3s_norm_fwd: theta_chunk %d must be a multiple of 16 dividing seqlen %d", C, L);
    M3S_REQUIRE(((int64_t)C * (H + Nr) + (int64_t)(C / 16) * H * Nr) * 4 <= 65536,
                "m3s_norm_fwd: theta_chunk %d, nheads %d and n_angles %d too large for the angle "
                "kernel's LDS (chunk (H + Nr) + (chunk / 16) H Nr floats <= 64 KiB)", C, H, Nr);
    M3S_REQUIRE(aligned16(a->theta_prefix) && aligned16(a->theta_chunk_totals),
                "m3s_norm_fwd: theta_prefix / theta_chunk_totals must be 16-byte aligned");
    p.th.ang = a->angles.ptr; p.th.asb = a->angles.stride_b; p.th.ast = a->angles.stride_t;
    p.th.dtr = a->dt_raw.ptr; p.th.dsb = a->dt_raw.stride_b; p.th.dst = a->dt_raw.stride_t;
    p.th.dt_bias = a->dt_bias;
    p.th.tab = a->theta_table;
    p.th.pre = a->theta_prefix;
    p.th.ctot = a->theta_chunk_totals;
    p.th.H = H; p.th.Nr = Nr; p.th.chunk = C; p.th.nblk = B * (L / C);
    dyn = ((size_t)C * (H + Nr) + (size_t)(C / 16) * H * Nr) * sizeof(float);
  }
  const int64_t rows_per_block = kNormThreads / p.G;
  const int64_t nblk = ((int64_t)B * L + rows_per_block - 1) / rows_per_block;
  const dim3 grid((unsigned)nblk, cnt);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (theta) {   // one launch: each block does a chunk's norms and its angle work
    if (a->dtype == M3S_DTYPE_BF16)
      hipLaunchKernelGGL(norm_theta_kernel<bf16>, dim3(p.th.nblk), dim3(kThetaThreads), dyn, s, p);
    else
      hipLaunchKernelGGL(norm_theta_kernel<float>, dim3(p.th.nblk), dim3(kThetaThreads), dyn, s, p);
    return launch_status("m3s_norm_fwd");
  }
  if (a->dtype == M3S_DTYPE_BF16)
    hipLaunchKernelGGL(norm_fwd_kernel<bf16>, grid, dim3(kNormThreads), 0, s, p);
  else
    hipLaunchKernelGGL(norm_fwd_kernel<float>, grid, dim3(kNormThreads), 0, s, p);
  return launch_status("m3s_norm_fwd");
}

namespace m3s {

// Argument checks shared by m3s_norm_bwd and m3s_norm_bwd_noalloc: fills every field of
// `p` but the gain-partials buffer, and the backward's block count. `what` names the
// entry point in error messages.
static int32_t norm_bwd_prepare(const m3s_norm_bwd_args* a, const char* what,
                                bool need_workspace, NormBwdParams* p, int* nblk) {
  M3S_REQUIRE(a != nullptr, "%s: args is NULL", what);
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_norm_bwd_args),
              "%s: struct_size %d != %d (ABI mismatch)", what, a->struct_size,
              (int)sizeof(m3s_norm_bwd_args));
  const int B = a->batch, L = a->seqlen, N = a->width, cnt = a->count;
  M3S_REQUIRE(B > 0 && L > 0 && N > 0 && (cnt == 1 || cnt == 2), "%s: bad dimension", what);
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32,
              "%s: bad dtype %d", what, a->dtype);
  const int vec = a->dtype == M3S_DTYPE_BF16 ? 8 : 4;
  M3S_REQUIRE(N % vec == 0 && N / vec <= 64,
              "%s: width %d must be a multiple of %d and at most %d", what, N, vec, 64 * vec);
  M3S_REQUIRE((int64_t)B * L < (1ll << 31), "%s: B*L too large", what);
  M3S_REQUIRE(!need_workspace || (a->workspace && aligned16(a->workspace)),
              "%s: workspace NULL or misaligned", what);
  *p = NormBwdParams{};
  for (int i = 0; i < cnt; ++i) {
    M3S_REQUIRE(blx_ok(a->x[i], vec), "%s: x[%d] must be 16-byte aligned rows", what, i);
    M3S_REQUIRE(blx_ok(a->dx[i], vec), "%s: dx[%d] must be 16-byte aligned rows", what, i);
    M3S_REQUIRE(a->weight[i] && a->rstd[i] && a->dy[i] && aligned16(a->dy[i]) && a->dweight[i],
                "%s: weight/rstd/dy/dweight[%d] NULL or dy misaligned", what, i);
    p->in.x[i] = a->x[i].ptr; p->in.xsb[i] = a->x[i].stride_b; p->in.xst[i] = a->x[i].stride_t;
    p->in.w[i] = a->weight[i];
    p->rstd[i] = a->rstd[i];
    p->dy[i] = a->dy[i];
    p->dx[i] = a->dx[i].ptr; p->dxsb[i] = a->dx[i].stride_b; p->dxst[i] = a->dx[i].stride_t;
  }
  p->B = B; p->L = L; p->N = N; p->G = norm_group(N, vec);
  const int64_t rows_per_pass = kNormThreads / p->G;
  *nblk = (int)std::min<int64_t>(kNormBwdBlocks, ((int64_t)B * L + rows_per_pass - 1) / rows_per_pass);
  return M3S_OK;
}

// The two kernels, with p.part as the gain-partials buffer ((nblk, count, width) f32;
// every entry the second kernel reads is written by the first, so it needs no clearing).
static int32_t norm_bwd_run(const m3s_norm_bwd_args* a, const NormBwdParams& p, int nblk,
                            const char* what, void* stream) {
  const int cnt = a->count;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->dtype == M3S_DTYPE_BF16)
    hipLaunchKernelGGL(norm_bwd_kernel<bf16>, dim3(nblk, cnt), dim3(kNormThreads), 0, s, p);
  else
    hipLaunchKernelGGL(norm_bwd_kernel<float>, dim3(nblk, cnt), dim3(kNormThreads), 0, s, p);
  int32_t rc = launch_status(what);
  if (rc) return rc;
  hipLaunchKernelGGL(norm_gain_kernel, dim3((p.N + 63) / 64, cnt),
                     dim3(kNormThreads), 0, s, p.part, a->dweight[0], cnt > 1 ? a->dweight[1] : nullptr,
                     nblk, p.N);
  return launch_status(what);
}

// ---- scratch of m3s_norm_bwd_noalloc ------------------------------------------------
// The gain partials at the widest accepted width (64 16-byte vectors of bf16 = 512):
// (kNormBwdBlocks, 2, 512) f32 = 4 MiB. A __device__ array exists once per device and
// lives until the process ends. In host code its name is only a stand-in for the symbol,
// so the device address is looked up (hipGetSymbolAddress) once per device, with that
// device current, and only that address is handed to kernels. The kept address is valid
// until the device is reset (hipDeviceReset unloads the code object holding the array);
// the header tells callers that reset a device to reload the library.
constexpr int kNormScratchWidth = 512;
constexpr int64_t kNormScratchBytes = (int64_t)kNormBwdBlocks * 2 * kNormScratchWidth * 4;
static __device__ __align__(256) float scratch[kNormBwdBlocks * 2 * kNormScratchWidth];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[kMaxDevices];

static int32_t scratch_for_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("m3s_norm_bwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return M3S_ERR_LAUNCH;
  }
  M3S_REQUIRE(dev >= 0 && dev < kMaxDevices, "m3s_norm_bwd_noalloc: device ordinal %d past %d",
              dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("m3s_norm_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                dev, hipGetErrorString(e));
      return M3S_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return M3S_OK;
}

}  // namespace m3s

extern "C" int32_t m3s_norm_bwd(const m3s_norm_bwd_args* a, void* stream) {
  clear_error();
  NormBwdParams p;
  int nblk = 0;
  int32_t rc = norm_bwd_prepare(a, "m3s_norm_bwd", true, &p, &nblk);
  if (rc != M3S_OK) return rc;
  p.part = static_cast<float*>(a->workspace);
  return norm_bwd_run(a, p, nblk, "m3s_norm_bwd", stream);
}

extern "C" int32_t m3s_norm_bwd_noalloc(const m3s_norm_bwd_args* a, void* stream) {
  clear_error();
  NormBwdParams p;
  int nblk = 0;
  int32_t rc = norm_bwd_prepare(a, "m3s_norm_bwd_noalloc", false, &p, &nblk);
  if (rc != M3S_OK) return rc;
  const int64_t need = (int64_t)nblk * 2 * p.N * 4;
  M3S_REQUIRE(need <= kNormScratchBytes,
              "m3s_norm_bwd_noalloc: width %d needs %lld bytes of scratch, past the %lld reserved",
              p.N, (long long)need, (long long)kNormScratchBytes);
  float* part = nullptr;
  rc = scratch_for_current_device(&part);
  if (rc != M3S_OK) return rc;
  p.part = part;
  return norm_bwd_run(a, p, nblk, "m3s_norm_bwd_noalloc", stream);
}
