// Per-token preprocessing of the Mamba-3 SISO layer on gfx950: the forward and its
// backward (the reference leaves the backward to jax.grad of `preprocess`).
//
// Replaces `reference.preprocess` (reference.py:160-199) and its helpers
// `heavy_tail` (202-209), `trapezoid_coeffs` (104-131) and `cumulative_angles`
// (134-157), whose XLA lowering materialises the phi cumulative sum:
//
//   dt    = softplus(dt_raw + dt_bias)          lam = sigmoid(trap_raw)
//   a     = min(-heavy_tail(a_raw), -a_floor)   heavy_tail(x) = max(x,0) + 1/(1 - min(x,0))
//   adt   = a dt,  gamma = dt lam,  scale_t = gamma_t + dt_{t+1} (1 - lam_{t+1})  (0 past L-1)
//   theta = tanh(angles) pi dt (angles shared by the heads),  phi = wrap(phi_init + cumsum_t theta)
//
// Kernels (all HBM-bound):
//  * prep_fwd_kernel, one workgroup per (b, h): the (B, H, L) scalars with consecutive
//    threads on consecutive t, then the phi prefix sum as a two-level scan -- each
//    thread owns a column quad and a contiguous time range, the range totals are
//    scanned in LDS, and a second pass writes phi as 16-byte rows.
//  * prep_dphi_suffix_kernel, one workgroup per (b, h): dtheta_t = dphi_final +
//    sum_{s>=t} dphi_s (the adjoint of the cumulative sum), same two-level scheme.
//  * prep_bwd_kernel, one workgroup per (b, block of 64 tokens) holding every head:
//    sums the per-head angle cotangents over heads in registers (angles are shared
//    across heads), and writes the raw-slice cotangents as contiguous (t, h) rows.
//  * prep_bias_kernel: the deterministic sum of the per-block dt_bias partials.
// Gradient conventions follow torch autograd of the same ops (clamp masks inclusive,
// softplus threshold 20), which is what the oracle's autograd produces.
#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

constexpr float kPiF = 3.14159265358979323846f;
constexpr float kTwoPiF = 6.28318530717958647692f;
constexpr int kPrepThreads = 256;
constexpr int kPrepTB = 64;  // tokens per block of prep_bwd_kernel

template <typename RT>
__device__ __forceinline__ float ldr(const RT* base, int64_t i) { return (float)base[i]; }

__device__ __forceinline__ float softplus_(float x) {
  return x > 20.f ? x : log1pf(expf(x));
}
__device__ __forceinline__ float heavy_tail_(float x) {
  return fmaxf(x, 0.f) + 1.f / (1.f - fminf(x, 0.f));
}
__device__ __forceinline__ float wrap_(float x) {
  return x - kTwoPiF * floorf(x / kTwoPiF);
}

struct PrepFwdParams {
  int B, L, H, Nr;
  float a_floor;
  const void* dtr; int64_t dtr_sb, dtr_st;
  const void* ar;  int64_t ar_sb, ar_st;
  const void* tr;  int64_t tr_sb, tr_st;
  const void* ang; int64_t ang_sb, ang_st;
  const float* dt_bias;
  const float* phi_init;
  float* adt; float* gamma; float* scale; float* lam; float* dt;
  float* phi;
  float* phi_final;
};

// Column quad jg of row `row` of a (rows, Nr) f32 array, zero past Nr.
__device__ __forceinline__ f32x4 ld_quad(const float* row, int j0, int Nr) {
  if (j0 + 4 <= Nr && (Nr & 3) == 0) return *reinterpret_cast<const f32x4*>(row + j0);
  f32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (j0 + i < Nr) ? row[j0 + i] : 0.f;
  return r;
}
__device__ __forceinline__ void st_quad(float* row, int j0, int Nr, f32x4 v) {
  if (j0 + 4 <= Nr && (Nr & 3) == 0) {
    *reinterpret_cast<f32x4*>(row + j0) = v;
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (j0 + i < Nr) row[j0 + i] = v[i];
}
template <typename RT>
__device__ __forceinline__ f32x4 ld_quad_raw(const RT* row, int j0, int Nr) {
  f32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (j0 + i < Nr) ? (float)row[j0 + i] : 0.f;
  return r;
}

template <typename RT>
__global__ void __launch_bounds__(kPrepThreads) prep_fwd_kernel(const PrepFwdParams p) {
  __shared__ f32x4 sPart[kPrepThreads];
  const int tid = threadIdx.x;
  const int bh = xcd_remap(blockIdx.x, gridDim.x);
  const int b = bh / p.H, h = bh % p.H;
  const int L = p.L, Nr = p.Nr;
  const RT* dtr = static_cast<const RT*>(p.dtr) + b * p.dtr_sb + h;
  const RT* ar = static_cast<const RT*>(p.ar) + b * p.ar_sb + h;
  const RT* tr = static_cast<const RT*>(p.tr) + b * p.tr_sb + h;
  const float bias = p.dt_bias[h];
  const int64_t o = (int64_t)bh * L;

  // ---- (B, H, L) scalars -------------------------------------------------------
  for (int t = tid; t < L; t += kPrepThreads) {
    const float dt = softplus_(ldr(dtr, t * p.dtr_st) + bias);
    const float lam = 1.f / (1.f + expf(-ldr(tr, t * p.tr_st)));
    const float a = fminf(-heavy_tail_(ldr(ar, t * p.ar_st)), -p.a_floor);
    float nxt = 0.f;
    if (t + 1 < L) {
      const float dtn = softplus_(ldr(dtr, (t + 1) * p.dtr_st) + bias);
      const float lamn = 1.f / (1.f + expf(-ldr(tr, (t + 1) * p.tr_st)));
      nxt = dtn * (1.f - lamn);
    }
    const float gam = dt * lam;
    p.adt[o + t] = a * dt;
    p.gamma[o + t] = gam;
    p.scale[o + t] = gam + nxt;
    p.lam[o + t] = lam;
    p.dt[o + t] = dt;
  }
  if (Nr == 0) return;
  __syncthreads();  // dt above is read back below by other threads of this block

  // ---- phi: two-level prefix sum over t, one column quad per thread -------------
  const int J4 = (Nr + 3) / 4;
  const int G = kPrepThreads / J4;
  const int jg = tid % J4, g = tid / J4;
  const bool act = g < G;
  const int TS = (L + G - 1) / G;
  const int tb = act ? min(L, g * TS) : L, te = act ? min(L, tb + TS) : L;
  const RT* ang = static_cast<const RT*>(p.ang) + b * p.ang_sb;
  const int j0 = 4 * jg;
  auto theta = [&](int t) {
    const float dt = p.dt[o + t];
    f32x4 a = ld_quad_raw(ang + t * p.ang_st, j0, Nr);
    f32x4 th;
#pragma unroll
    for (int i = 0; i < 4; ++i) th[i] = tanhf(a[i]) * kPiF * dt;
    return th;
  };
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int t = tb; t < te; ++t) {
    const f32x4 th = theta(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] += th[i];
  }
  sPart[tid] = s;
  __syncthreads();
  if (!act) return;
  f32x4 run = {0.f, 0.f, 0.f, 0.f};
  for (int gg = 0; gg < g; ++gg) {
    const f32x4 q = sPart[gg * J4 + jg];
#pragma unroll
    for (int i = 0; i < 4; ++i) run[i] += q[i];
  }
  f32x4 init = {0.f, 0.f, 0.f, 0.f};
  if (p.phi_init) init = ld_quad(p.phi_init + (int64_t)bh * Nr, j0, Nr);
#pragma unroll 4
  for (int t = tb; t < te; ++t) {
    const f32x4 th = theta(t);
    f32x4 out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      run[i] += th[i];
      out[i] = wrap_(run[i] + init[i]);
    }
    st_quad(p.phi + (o + t) * Nr, j0, Nr, out);
    if (t == L - 1) st_quad(p.phi_final + (int64_t)bh * Nr, j0, Nr, out);
  }
}

// dtheta_t = dphi_final + sum_{s >= t} dphi_s, written to `dth` (B, H, L, Nr).
__global__ void __launch_bounds__(kPrepThreads)
prep_dphi_suffix_kernel(const float* __restrict__ dphi, const float* __restrict__ dphi_final,
                        float* __restrict__ dth, float* __restrict__ dphi_init, int L, int Nr) {
  __shared__ f32x4 sPart[kPrepThreads];
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.x;
  const int J4 = (Nr + 3) / 4;
  const int G = kPrepThreads / J4;
  const int jg = tid % J4, g = tid / J4;
  const bool act = g < G;
  const int TS = (L + G - 1) / G;
  const int tb = act ? min(L, g * TS) : L, te = act ? min(L, tb + TS) : L;
  const int j0 = 4 * jg;
  const float* src = dphi ? dphi + bh * L * Nr : nullptr;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  if (src) {
    for (int t = tb; t < te; ++t) {
      const f32x4 d = ld_quad(src + (int64_t)t * Nr, j0, Nr);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] += d[i];
    }
  }
  sPart[tid] = s;
  __syncthreads();
  if (!act) return;
  f32x4 run = {0.f, 0.f, 0.f, 0.f};
  if (dphi_final) run = ld_quad(dphi_final + bh * Nr, j0, Nr);
  for (int gg = G - 1; gg > g; --gg) {
    const f32x4 q = sPart[gg * J4 + jg];
#pragma unroll
    for (int i = 0; i < 4; ++i) run[i] += q[i];
  }
  float* dst = dth + bh * L * Nr;
  for (int t = te - 1; t >= tb; --t) {
    if (src) {
      const f32x4 d = ld_quad(src + (int64_t)t * Nr, j0, Nr);
#pragma unroll
      for (int i = 0; i < 4; ++i) run[i] += d[i];
    }
    st_quad(dst + (int64_t)t * Nr, j0, Nr, run);
  }
  if (tb == 0 && dphi_init) st_quad(dphi_init + bh * Nr, j0, Nr, run);
}

struct PrepBwdParams {
  int B, L, H, Nr, nblk;
  float a_floor;
  const void* dtr; int64_t dtr_sb, dtr_st;
  const void* ar;  int64_t ar_sb, ar_st;
  const void* tr;  int64_t tr_sb, tr_st;
  const void* ang; int64_t ang_sb, ang_st;
  const float* dt_bias;
  const float* dadt; const float* dgamma; const float* dscale;
  const float* dlam; const float* ddt;
  const float* dth;      // (B, H, L, Nr) suffix-summed dphi, or NULL
  void* ddtr; int64_t ddtr_sb, ddtr_st;
  void* dar;  int64_t dar_sb, dar_st;
  void* dtrr; int64_t dtrr_sb, dtrr_st;
  void* dang; int64_t dang_sb, dang_st;
  float* bias_part;      // (B * nblk, H)
};

// LDS layout of prep_bwd_kernel (floats): per (t, h) tables of TB x H, the TB x Nr
// tanh table, and the dscale value just before the block for each head.
__host__ __device__ inline int prep_bwd_lds_floats(int H, int Nr) {
  return 6 * kPrepTB * H + kPrepTB * Nr + H;
}

template <typename RT>
__global__ void __launch_bounds__(kPrepThreads) prep_bwd_kernel(const PrepBwdParams p) {
  extern __shared__ float lds[];
  const int H = p.H, Nr = p.Nr, L = p.L;
  float* sDt = lds;                    // [TB][H] dt
  float* sLam = sDt + kPrepTB * H;     // [TB][H] lambda
  float* sDadt = sLam + kPrepTB * H;   // [TB][H] incoming cotangents (t-major)
  float* sDgam = sDadt + kPrepTB * H;
  float* sDscl = sDgam + kPrepTB * H;
  float* sPhi = sDscl + kPrepTB * H;   // [TB][H] sum_j dtheta tanh pi
  float* sBias = sDadt;                // [TB][H] d dt_raw for the dt_bias partial; each
                                       // thread overwrites only entries it has read
  float* sT = sPhi + kPrepTB * H;      // [TB][Nr] tanh(angles)
  float* sDsPrev = sT + kPrepTB * Nr;  // [H] dscale at t0 - 1

  const int tid = threadIdx.x;
  const int blk = blockIdx.x, b = blockIdx.y;
  const int t0 = blk * kPrepTB;
  const int nt = min(kPrepTB, L - t0);
  const RT* dtr = static_cast<const RT*>(p.dtr) + b * p.dtr_sb;
  const RT* ar = static_cast<const RT*>(p.ar) + b * p.ar_sb;
  const RT* tr = static_cast<const RT*>(p.tr) + b * p.tr_sb;
  const RT* ang = static_cast<const RT*>(p.ang) + b * p.ang_sb;

  // ---- stage: recomputed dt / lambda, incoming cotangents, tanh table -------------
  for (int i = tid; i < nt * H; i += kPrepThreads) {
    const int t = i / H, h = i % H;
    sDt[i] = softplus_(ldr(dtr, (int64_t)(t0 + t) * p.dtr_st + h) + p.dt_bias[h]);
    sLam[i] = 1.f / (1.f + expf(-ldr(tr, (int64_t)(t0 + t) * p.tr_st + h)));
    sPhi[i] = 0.f;
  }
  for (int i = tid; i < nt * H; i += kPrepThreads) {  // (h, t) order: coalesced reads
    const int h = i / nt, t = i % nt;
    const int64_t g = ((int64_t)b * H + h) * L + t0 + t;
    sDadt[t * H + h] = p.dadt ? p.dadt[g] : 0.f;
    sDgam[t * H + h] = p.dgamma ? p.dgamma[g] : 0.f;
    sDscl[t * H + h] = p.dscale ? p.dscale[g] : 0.f;
  }
  for (int h = tid; h < H; h += kPrepThreads)
    sDsPrev[h] = (p.dscale && t0 > 0) ? p.dscale[((int64_t)b * H + h) * L + t0 - 1] : 0.f;
  for (int i = tid; i < nt * Nr; i += kPrepThreads) {
    const int t = i / Nr, j = i % Nr;
    sT[i] = tanhf(ldr(ang, (int64_t)(t0 + t) * p.ang_st + j));
  }
  __syncthreads();

  // ---- angles: d angles = pi (1 - tanh^2) sum_h dtheta_h dt_h; and per (t, h)
  //      the dt term sum_j dtheta tanh pi --------------------------------------------
  if (Nr > 0) {
    const int J4 = (Nr + 3) / 4;
    const bool pow2 = (J4 & (J4 - 1)) == 0;
    RT* dang = static_cast<RT*>(p.dang) + b * p.dang_sb;
    const int npair = nt * J4;
    // every lane of a wave runs the same number of iterations (the shuffles need it)
    const int iters = (npair + kPrepThreads - 1) / kPrepThreads;
    for (int it = 0; it < iters; ++it) {
      const int pr = tid + it * kPrepThreads;
      const bool valid = pr < npair;
      const int tt = valid ? pr / J4 : 0, jg = valid ? pr % J4 : 0, j0 = 4 * jg;
      f32x4 tq = {0.f, 0.f, 0.f, 0.f};
      if (valid) {
#pragma unroll
        for (int i = 0; i < 4; ++i) tq[i] = (j0 + i < Nr) ? sT[tt * Nr + j0 + i] : 0.f;
      }
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int h = 0; h < H; ++h) {
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
        if (valid && p.dth) d = ld_quad(p.dth + (((int64_t)b * H + h) * L + t0 + tt) * Nr, j0, Nr);
        const float dth = valid ? sDt[tt * H + h] : 0.f;
        float ph = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i] += d[i] * dth;
          ph += d[i] * (tq[i] * kPiF);
        }
        if (pow2 && J4 <= 64) {
          for (int off = 1; off < J4; off <<= 1) ph += __shfl_xor(ph, off, 64);
          if (valid && jg == 0) sPhi[tt * H + h] = ph;
        } else if (valid) {
          atomicAdd(sPhi + tt * H + h, ph);
        }
      }
      if (valid) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = j0 + i;
          if (j < Nr)
            dang[(int64_t)(t0 + tt) * p.dang_st + j] = (RT)(acc[i] * kPiF * (1.f - tq[i] * tq[i]));
        }
      }
    }
  }
  __syncthreads();

  // ---- raw-slice cotangents, (t, h) row-major --------------------------------------
  RT* ddtr = static_cast<RT*>(p.ddtr) + b * p.ddtr_sb;
  RT* dar = static_cast<RT*>(p.dar) + b * p.dar_sb;
  RT* dtrr = static_cast<RT*>(p.dtrr) + b * p.dtrr_sb;
  for (int i = tid; i < nt * H; i += kPrepThreads) {
    const int t = i / H, h = i % H;
    const int tg = t0 + t;
    const int64_t g = ((int64_t)b * H + h) * L + tg;
    const float dt = sDt[i], lam = sLam[i];
    const float x = ldr(dtr, (int64_t)tg * p.dtr_st + h) + p.dt_bias[h];
    const float xa = ldr(ar, (int64_t)tg * p.ar_st + h);
    const float apre = -heavy_tail_(xa);
    const float a = fminf(apre, -p.a_floor);
    const float dadt = sDadt[i];
    const float dgt = sDgam[i] + sDscl[i];
    const float dsp = tg > 0 ? (t > 0 ? sDscl[i - H] : sDsPrev[h]) : 0.f;
    float ddt = dadt * a + dgt * lam + dsp * (1.f - lam) + sPhi[i];
    float dlam = dgt * dt - dsp * dt;
    if (p.ddt) ddt += p.ddt[g];
    if (p.dlam) dlam += p.dlam[g];
    // softplus'(x) = sigmoid(x), 1 above the threshold (torch: exp(x) / (exp(x) + 1))
    float dx;
    if (x > 20.f) {
      dx = ddt;
    } else {
      const float e = expf(x);
      dx = ddt * e / (e + 1.f);
    }
    // a = clamp(-heavy_tail(xa), max = -a_floor); masks inclusive as in torch
    const float da = (apre <= -p.a_floor) ? dadt * dt : 0.f;
    const float wv = 1.f - fminf(xa, 0.f);
    const float dht = (xa >= 0.f ? 1.f : 0.f) + (xa <= 0.f ? 1.f / (wv * wv) : 0.f);
    const float dxa = -da * dht;
    const float dtrap = dlam * lam * (1.f - lam);
    ddtr[(int64_t)tg * p.ddtr_st + h] = (RT)dx;
    dar[(int64_t)tg * p.dar_st + h] = (RT)dxa;
    dtrr[(int64_t)tg * p.dtrr_st + h] = (RT)dtrap;
    sBias[i] = dx;
  }
  __syncthreads();
  for (int h = tid; h < H; h += kPrepThreads) {
    float s = 0.f;
    for (int t = 0; t < nt; ++t) s += sBias[t * H + h];
    p.bias_part[((int64_t)b * p.nblk + blk) * H + h] = s;
  }
}

__global__ void __launch_bounds__(kPrepThreads)
prep_bias_kernel(const float* __restrict__ part, float* __restrict__ out, int rows, int H) {
  const int h = blockIdx.x * kPrepThreads + threadIdx.x;
  if (h >= H) return;
  float s = 0.f;
  for (int r = 0; r < rows; ++r) s += part[(int64_t)r * H + h];
  out[h] = s;
}

static bool blx_ok(const m3s_blx& t) { return t.ptr != nullptr; }

}  // namespace m3s

using namespace m3s;

extern "C" int32_t m3s_prep_fwd(const m3s_prep_fwd_args* a, void* stream) {
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_prep_fwd: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_prep_fwd_args),
              "m3s_prep_fwd: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_prep_fwd_args));
  const int B = a->batch, L = a->seqlen, H = a->nheads, Nr = a->n_angles;
  M3S_REQUIRE(B > 0 && L > 0 && H > 0 && Nr >= 0, "m3s_prep_fwd: bad dimension");
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32,
              "m3s_prep_fwd: bad dtype %d", a->dtype);
  M3S_REQUIRE(blx_ok(a->dt_raw) && blx_ok(a->a_raw) && blx_ok(a->trap_raw) &&
                  (Nr == 0 || blx_ok(a->angles)) && a->dt_bias,
              "m3s_prep_fwd: a required input pointer is NULL");
  M3S_REQUIRE(!a->has_phi_init || a->phi_init, "m3s_prep_fwd: has_phi_init but phi_init is NULL");
  M3S_REQUIRE(a->adt && a->gamma && a->scale && a->lam && a->dt && (Nr == 0 || (a->phi && a->phi_final)),
              "m3s_prep_fwd: an output pointer is NULL");
  M3S_REQUIRE(Nr % 4 != 0 || (aligned16(a->phi) && aligned16(a->phi_final) &&
                              (!a->has_phi_init || aligned16(a->phi_init))),
              "m3s_prep_fwd: phi buffers must be 16-byte aligned");
  M3S_REQUIRE((int64_t)B * H < (1ll << 31), "m3s_prep_fwd: B*H too large");
  PrepFwdParams p{};
  p.B = B; p.L = L; p.H = H; p.Nr = Nr; p.a_floor = a->a_floor;
  p.dtr = a->dt_raw.ptr; p.dtr_sb = a->dt_raw.stride_b; p.dtr_st = a->dt_raw.stride_t;
  p.ar = a->a_raw.ptr; p.ar_sb = a->a_raw.stride_b; p.ar_st = a->a_raw.stride_t;
  p.tr = a->trap_raw.ptr; p.tr_sb = a->trap_raw.stride_b; p.tr_st = a->trap_raw.stride_t;
  p.ang = a->angles.ptr; p.ang_sb = a->angles.stride_b; p.ang_st = a->angles.stride_t;
  p.dt_bias = a->dt_bias;
  p.phi_init = a->has_phi_init ? a->phi_init : nullptr;
  p.adt = a->adt; p.gamma = a->gamma; p.scale = a->scale; p.lam = a->lam; p.dt = a->dt;
  p.phi = a->phi; p.phi_final = a->phi_final;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->dtype == M3S_DTYPE_BF16)
    hipLaunchKernelGGL(prep_fwd_kernel<bf16>, dim3(B * H), dim3(kPrepThreads), 0, s, p);
  else
    hipLaunchKernelGGL(prep_fwd_kernel<float>, dim3(B * H), dim3(kPrepThreads), 0, s, p);
  return launch_status("m3s_prep_fwd");
}

extern "C" int64_t m3s_prep_bwd_workspace_bytes(int32_t batch, int32_t seqlen, int32_t nheads,
                                                 int32_t n_angles) {
  if (batch <= 0 || seqlen <= 0 || nheads <= 0 || n_angles < 0) return -1;
  const int64_t nblk = (seqlen + kPrepTB - 1) / kPrepTB;
  int64_t dth = (int64_t)batch * nheads * seqlen * n_angles * 4;
  dth = (dth + 255) / 256 * 256;
  return dth + (int64_t)batch * nblk * nheads * 4;
}

extern "C" int32_t m3s_prep_bwd(const m3s_prep_bwd_args* a, void* stream) {
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_prep_bwd: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_prep_bwd_args),
              "m3s_prep_bwd: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_prep_bwd_args));
  const int B = a->batch, L = a->seqlen, H = a->nheads, Nr = a->n_angles;
  M3S_REQUIRE(B > 0 && L > 0 && H > 0 && Nr >= 0, "m3s_prep_bwd: bad dimension");
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32,
              "m3s_prep_bwd: bad dtype %d", a->dtype);
  M3S_REQUIRE(blx_ok(a->dt_raw) && blx_ok(a->a_raw) && blx_ok(a->trap_raw) &&
                  (Nr == 0 || blx_ok(a->angles)) && a->dt_bias,
              "m3s_prep_bwd: a forward input pointer is NULL");
  M3S_REQUIRE(blx_ok(a->ddt_raw) && blx_ok(a->da_raw) && blx_ok(a->dtrap_raw) &&
                  (Nr == 0 || blx_ok(a->dangles)) && a->ddt_bias && a->workspace,
              "m3s_prep_bwd: an output pointer or the workspace is NULL");
  M3S_REQUIRE(aligned16(a->workspace), "m3s_prep_bwd: workspace must be 16-byte aligned");
  M3S_REQUIRE(Nr % 4 != 0 || ((!a->dphi || aligned16(a->dphi)) &&
                              (!a->dphi_final || aligned16(a->dphi_final)) &&
                              (!a->dphi_init || aligned16(a->dphi_init))),
              "m3s_prep_bwd: phi cotangent buffers must be 16-byte aligned");
  const size_t lds = (size_t)prep_bwd_lds_floats(H, Nr) * 4;
  M3S_REQUIRE(lds <= 160 * 1024, "m3s_prep_bwd: nheads=%d, n_angles=%d exceed the LDS budget", H, Nr);
  M3S_REQUIRE((int64_t)B * H < (1ll << 31), "m3s_prep_bwd: B*H too large");
  const int nblk = (L + kPrepTB - 1) / kPrepTB;
  int64_t dth_bytes = (int64_t)B * H * L * Nr * 4;
  dth_bytes = (dth_bytes + 255) / 256 * 256;
  float* dth = static_cast<float*>(a->workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + dth_bytes);
  const bool any_dphi = a->dphi || a->dphi_final;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (Nr > 0 && (any_dphi || a->dphi_init)) {
    hipLaunchKernelGGL(prep_dphi_suffix_kernel, dim3(B * H), dim3(kPrepThreads), 0, s,
                       a->dphi, a->dphi_final, dth, a->dphi_init, L, Nr);
    int32_t rc = launch_status("m3s_prep_bwd");
    if (rc) return rc;
  }
  PrepBwdParams p{};
  p.B = B; p.L = L; p.H = H; p.Nr = Nr; p.nblk = nblk; p.a_floor = a->a_floor;
  p.dtr = a->dt_raw.ptr; p.dtr_sb = a->dt_raw.stride_b; p.dtr_st = a->dt_raw.stride_t;
  p.ar = a->a_raw.ptr; p.ar_sb = a->a_raw.stride_b; p.ar_st = a->a_raw.stride_t;
  p.tr = a->trap_raw.ptr; p.tr_sb = a->trap_raw.stride_b; p.tr_st = a->trap_raw.stride_t;
  p.ang = a->angles.ptr; p.ang_sb = a->angles.stride_b; p.ang_st = a->angles.stride_t;
  p.dt_bias = a->dt_bias;
  p.dadt = a->dadt; p.dgamma = a->dgamma; p.dscale = a->dscale;
  p.dlam = a->dlam; p.ddt = a->ddt;
  p.dth = (Nr > 0 && any_dphi) ? dth : nullptr;
  p.ddtr = a->ddt_raw.ptr; p.ddtr_sb = a->ddt_raw.stride_b; p.ddtr_st = a->ddt_raw.stride_t;
  p.dar = a->da_raw.ptr; p.dar_sb = a->da_raw.stride_b; p.dar_st = a->da_raw.stride_t;
  p.dtrr = a->dtrap_raw.ptr; p.dtrr_sb = a->dtrap_raw.stride_b; p.dtrr_st = a->dtrap_raw.stride_t;
  p.dang = a->dangles.ptr; p.dang_sb = a->dangles.stride_b; p.dang_st = a->dangles.stride_t;
  p.bias_part = part;
  auto launch = [&](auto kern) {
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
      set_error("m3s_prep_bwd: cannot raise the dynamic LDS limit to %zu bytes", lds);
      return M3S_ERR_LAUNCH;
    }
    hipLaunchKernelGGL(kern, dim3(nblk, B), dim3(kPrepThreads), lds, s, p);
    return launch_status("m3s_prep_bwd");
  };
  int32_t rc = a->dtype == M3S_DTYPE_BF16 ? launch(prep_bwd_kernel<bf16>) : launch(prep_bwd_kernel<float>);
  if (rc) return rc;
  hipLaunchKernelGGL(prep_bias_kernel, dim3((H + kPrepThreads - 1) / kPrepThreads),
                     dim3(kPrepThreads), 0, s, part, a->ddt_bias, B * nblk, H);
  return launch_status("m3s_prep_bwd");
}
