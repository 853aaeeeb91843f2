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
// Every kernel works on one (batch element, block of 64 tokens) with all heads, so a
// launch has B * L / 64 workgroups and each reads its raw (t, h) rows once. The time
// recurrence (the phi prefix sum, and its adjoint, a suffix sum) is split in three
// HBM-bound launches: per-block totals, a carry scan over the blocks of each
// (b, h, angle), and the block pass that adds the carry to an in-block scan.
//  * forward: prep_scalars_kernel (adt, gamma, scale, lam, dt as (b, h) rows; the
//    tanh(angles) pi table, shared by the heads; theta totals), prep_carry_kernel,
//    prep_phi_kernel (phi as 16-byte rows).
//  * backward: prep_dphi_totals_kernel, prep_carry_kernel (suffix direction, seeded
//    with dphi_final; its total is dphi_init), prep_bwd_kernel (walks its block in
//    reverse: dtheta, the head sum of the angle cotangent by shuffles within a wave
//    and LDS adds across waves, the raw-slice cotangents as (t, h) rows, dt_bias
//    partials), prep_bias_kernel (a fixed-order tree sum of the partials).
// Gradient conventions follow torch autograd of the same ops (clamp masks inclusive,
// softplus threshold 20), which is what the oracle's autograd produces.
#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

constexpr float kPiF = 3.14159265358979323846f;
constexpr float kTwoPiF = 6.28318530717958647692f;
constexpr int kPrepThreads = 256;
constexpr int kPrepTB = 64;     // tokens per block of the forward kernels
// tokens per block of the backward kernels: 32 halves prep_bwd_kernel's LDS tables, so four
// blocks fit a CU instead of two (0.218 -> 0.175 ms at cfg3); the forward kernels are
// faster at 64
constexpr int kPrepBwdTB = 32;

template <typename RT>
__device__ __forceinline__ float ldr(const RT* base, int64_t i) { return (float)base[i]; }


// x mod 2 pi in [0, 2 pi): the quotient from a multiply by 1 / (2 pi), the remainder by
// one fma, then one correction step. Where x / (2 pi) lies within an ulp of an integer the
// quotient can differ by one from floor(x / (2 pi)); the correction keeps the result in
// range and it is the same angle.
__device__ __forceinline__ float wrap_(float x) {
  constexpr float kInvTwoPiF = 0.15915494309189535f;
  float r = fmaf(-kTwoPiF, floorf(x * kInvTwoPiF), x);
  r = r < 0.f ? r + kTwoPiF : r;
  return r >= kTwoPiF ? r - kTwoPiF : r;
}

// Column quad [j0, j0 + 4) of a row of Nr f32 values (j0 a multiple of 4 below Nr), zero
// past Nr. With Nr % 4 == 0 every quad is whole: the test is wave-uniform, so the loads
// of an unrolled run are not split by a per-lane choice of width (which would make the
// compiler wait for each one at the join).
__device__ __forceinline__ f32x4 ld_quad(const float* row, int j0, int Nr) {
  if ((Nr & 3) == 0) return *reinterpret_cast<const f32x4*>(row + j0);
  f32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (j0 + i < Nr) ? row[j0 + i] : 0.f;
  return r;
}
__device__ __forceinline__ void st_quad(float* row, int j0, int Nr, f32x4 v) {
  if ((Nr & 3) == 0) {
    *reinterpret_cast<f32x4*>(row + j0) = v;
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (j0 + i < Nr) row[j0 + i] = v[i];
}

struct PrepIn {
  const void* p;
  int64_t sb, st;
};
struct PrepOut {
  void* p;
  int64_t sb, st;
};

struct PrepFwdParams {
  int B, L, H, Nr, nblk;
  float a_floor;
  PrepIn dtr, ar, tr, ang;
  const float* dt_bias;
  const float* phi_init;
  float* adt; float* gamma; float* scale; float* lam; float* dt;
  float* phi;         // (B, H, L, Nr) or NULL
  float* phi_final;
  float* strips;      // (B, H, L / 16, Nr) phi entering each 16-token strip, or NULL
  float* tpi;  // (B, L, Nr) tanh(angles) * pi
  float* tot;  // (B, nblk, H, Nr) block totals of theta, then exclusive carries; with
               // strip_tot, (B, L / 16, H, Nr) totals of each 16-token strip
  int strip_tot;
};

// prep_scalars_kernel's LDS: three (TB + 1) x (H + 1) tables, then the TB x Nr tanh table
// from a 16-byte boundary (its rows are read as 16-byte quads)
__host__ __device__ inline int prep_fwd_tables_floats(int H) {
  return (3 * (kPrepTB + 1) * (H + 1) + 3) & ~3;
}
__host__ __device__ inline int prep_fwd_lds_floats(int H, int Nr) {
  return prep_fwd_tables_floats(H) + kPrepTB * Nr;
}

template <typename RT>
__global__ void __launch_bounds__(kPrepThreads) prep_scalars_kernel(const PrepFwdParams p) {
  extern __shared__ float lds[];
  const int H = p.H, Nr = p.Nr, L = p.L;
  const int tid = threadIdx.x, blk = blockIdx.x, b = blockIdx.y;
  const int t0 = blk * kPrepTB;
  const int nt = min(kPrepTB, L - t0), nt1 = min(kPrepTB + 1, L - t0);
  // [t][h] tables with a padded row stride HS = H + 1: written in (t, h) order and read in
  // (h, t) order, so that the reads of consecutive t fall in distinct LDS banks
  const int HS = H + 1;
  float* sDt = lds;                          // [TB + 1][HS]
  float* sLam = sDt + (kPrepTB + 1) * HS;    // [TB + 1][HS]
  float* sA = sLam + (kPrepTB + 1) * HS;     // [TB + 1][HS]
  float* sT = lds + prep_fwd_tables_floats(H);   // [TB][Nr]  tanh(angles) * pi
  const RT* dtr = static_cast<const RT*>(p.dtr.p) + b * p.dtr.sb;
  const RT* ar = static_cast<const RT*>(p.ar.p) + b * p.ar.sb;
  const RT* tr = static_cast<const RT*>(p.tr.p) + b * p.tr.sb;
  const RT* ang = static_cast<const RT*>(p.ang.p) + b * p.ang.sb;

  // KU items per thread per round, every load of a round issued before any use: one
  // memory latency per round instead of one per item
  constexpr int KU = 4;
  const DivMod byH(H), byNr(Nr > 0 ? Nr : 1), byNt(nt);
  const int n1 = nt1 * H;
  for (int i0 = tid; i0 < n1; i0 += KU * kPrepThreads) {
    float vd[KU], vl[KU], va[KU], vb[KU];
    int kk[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = min(i0 + u * kPrepThreads, n1 - 1);
      int t, h;
      byH(i, t, h);
      kk[u] = t * HS + h;
      const int64_t tg = t0 + t;
      vd[u] = ldr(dtr, tg * p.dtr.st + h);
      vl[u] = ldr(tr, tg * p.tr.st + h);
      va[u] = ldr(ar, tg * p.ar.st + h);
      vb[u] = p.dt_bias[h];
    }
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = i0 + u * kPrepThreads;
      if (i < n1) {
        const int k = kk[u];
        sDt[k] = softplus_(vd[u] + vb[u]);
        sLam[k] = sigmoid_(vl[u]);
        sA[k] = fminf(-heavy_tail_(va[u]), -p.a_floor);
      }
    }
  }
  const int n2 = nt * Nr;
  for (int i0 = tid; i0 < n2; i0 += KU * kPrepThreads) {
    float vg[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = min(i0 + u * kPrepThreads, n2 - 1);
      int t, j;
      byNr(i, t, j);
      vg[u] = ldr(ang, (int64_t)(t0 + t) * p.ang.st + j);
    }
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = i0 + u * kPrepThreads;
      if (i < n2) {
        const float tp = tanhf(vg[u]) * kPiF;
        sT[i] = tp;
        p.tpi[((int64_t)b * L + t0) * Nr + i] = tp;
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < H * nt; i += kPrepThreads) {  // (h, t) order: (b, h) rows
    int h, t;
    byNt(i, h, t);
    const int k = t * HS + h;
    const float dt = sDt[k], lam = sLam[k];
    const float nxt = (t0 + t + 1 < L) ? sDt[k + HS] * (1.f - sLam[k + HS]) : 0.f;
    const float gam = dt * lam;
    const int64_t o = ((int64_t)b * H + h) * L + t0 + t;
    p.adt[o] = sA[k] * dt;
    p.gamma[o] = gam;
    p.scale[o] = gam + nxt;
    p.lam[o] = lam;
    p.dt[o] = dt;
  }
  if (Nr == 0) return;
  const int J4 = (Nr + 3) / 4;
  for (int pr = tid; pr < H * J4; pr += kPrepThreads) {
    const int h = pr / J4, j0 = 4 * (pr % J4);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    // a quad per row (zeros past Nr): with Nr % 4 == 0 one 16-byte LDS read and no
    // per-lane branch; a branch per element made each read wait for the one before
    // (0.061 -> 0.056 ms for the three forward launches at B=8, L=8192, H=32, Nr=32;
    // four quarter sums side by side instead of one chain were slower, 0.084 ms)
    auto add_row = [&](f32x4& acc, int t) {
      const float dt = sDt[t * HS + h];
      const f32x4 th = ld_quad(sT + t * Nr, j0, Nr);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += th[i] * dt;
    };
    if (p.strip_tot) {   // one total per 16-token strip (L % 16 == 0)
      const int ns = L >> 4, s0 = t0 >> 4;
      for (int st = 0; st < (nt >> 4); ++st) {
        f32x4 q = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 16; ++t) add_row(q, 16 * st + t);
        st_quad(p.tot + (((int64_t)b * ns + s0 + st) * H + h) * Nr, j0, Nr, q);
      }
      continue;
    }
    if (nt == kPrepTB) {   // whole blocks: a fixed trip count the compiler can pipeline
#pragma unroll 16
      for (int t = 0; t < kPrepTB; ++t) add_row(s, t);
    } else {
      for (int t = 0; t < nt; ++t) add_row(s, t);
    }
    st_quad(p.tot + (((int64_t)b * p.nblk + blk) * H + h) * Nr, j0, Nr, s);
  }
}

// Over the blocks of one (b, h, angle): replace each block total by the exclusive
// running sum -- in time order (reverse = 0), or from the end, seeded with `init`,
// with the full sum written to `total` (reverse = 1).
// A workgroup takes kCarryR consecutive (h, angle) columns of one batch element and cuts
// the walk over the blocks into kCarrySeg segments, one thread per (column, segment):
// each thread sums its segment, the segment sums are combined in segment order through
// LDS, and each thread walks its segment again from that offset (the second reads hit
// L2). That is kCarrySeg walks of nblk / kCarrySeg blocks side by side instead of one
// of nblk; each walk issues a group's loads before its stores, one memory latency per
// group (a store could alias the next load as far as the compiler knows).
constexpr int kCarryR = 16;
constexpr int kCarrySeg = kPrepThreads / kCarryR;
__global__ void __launch_bounds__(kPrepThreads)
prep_carry_kernel(float* __restrict__ tot, const float* __restrict__ init,
                  float* __restrict__ total, int HN, int nblk, int reverse) {
  __shared__ float part[kCarrySeg][kCarryR];
  const int rl = threadIdx.x % kCarryR, seg = threadIdx.x / kCarryR;
  const int r = blockIdx.x * kCarryR + rl, b = blockIdx.y;
  const bool valid = r < HN;
  float* base = tot + (int64_t)b * nblk * HN + r;
  const int len = (nblk + kCarrySeg - 1) / kCarrySeg;
  const int s0 = min(seg * len, nblk), s1 = min(s0 + len, nblk);
  // the u-th block of the walk (from the end when reverse)
  auto at = [&](int u) -> int64_t { return (int64_t)(reverse ? nblk - 1 - u : u) * HN; };
  constexpr int G = 8;
  float sum = 0.f;
  if (valid) {
    for (int u0 = s0; u0 < s1; u0 += G) {
      float q[G];
#pragma unroll
      for (int g = 0; g < G; ++g) q[g] = (u0 + g < s1) ? base[at(u0 + g)] : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) sum += q[g];
    }
  }
  part[seg][rl] = sum;
  __syncthreads();
  float run = (reverse && init && valid) ? init[(int64_t)b * HN + r] : 0.f;
  for (int k = 0; k < seg; ++k) run += part[k][rl];
  if (reverse && total && valid && seg == kCarrySeg - 1) total[(int64_t)b * HN + r] = run + sum;
  if (!valid) return;
  for (int u0 = s0; u0 < s1; u0 += G) {
    float q[G];
#pragma unroll
    for (int g = 0; g < G; ++g) q[g] = (u0 + g < s1) ? base[at(u0 + g)] : 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (u0 + g < s1) base[at(u0 + g)] = run;
      run += q[g];
    }
  }
}

// The compact phi form straight from strip totals: over the 16-token strips of one
// (b, h, angle), the angle entering each strip, wrap(phi_init + exclusive running sum of
// the strip totals), written as strips (B, H, L / 16, Nr); the full sum gives phi_final.
// The same segmented walk as prep_carry_kernel (kCarrySeg segments per column, their
// sums combined in segment order), which makes a separate pass over the rows
// (prep_phi_kernel) unnecessary when phi itself is not wanted.
__global__ void __launch_bounds__(kPrepThreads)
prep_strip_carry_kernel(const float* __restrict__ tot, const float* __restrict__ init,
                        float* __restrict__ strips, float* __restrict__ phi_final, int H,
                        int Nr, int ns) {
  __shared__ float part[kCarrySeg][kCarryR];
  const int HN = H * Nr;
  const int rl = threadIdx.x % kCarryR, seg = threadIdx.x / kCarryR;
  const int r = blockIdx.x * kCarryR + rl, b = blockIdx.y;
  const bool valid = r < HN;
  const int h = valid ? r / Nr : 0, j = valid ? r % Nr : 0;
  const float* src = tot + (int64_t)b * ns * HN + r;
  float* dst = strips + (((int64_t)b * H + h) * ns) * Nr + j;
  const int len = (ns + kCarrySeg - 1) / kCarrySeg;
  const int s0 = min(seg * len, ns), s1 = min(s0 + len, ns);
  constexpr int G = 8;
  float sum = 0.f;
  if (valid) {
    for (int u0 = s0; u0 < s1; u0 += G) {
      float q[G];
#pragma unroll
      for (int g = 0; g < G; ++g) q[g] = (u0 + g < s1) ? src[(int64_t)(u0 + g) * HN] : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) sum += q[g];
    }
  }
  part[seg][rl] = sum;
  __syncthreads();
  if (!valid) return;
  float run = 0.f;
  for (int k = 0; k < seg; ++k) run += part[k][rl];
  const float phi0 = init ? init[((int64_t)b * H + h) * Nr + j] : 0.f;
  if (seg == kCarrySeg - 1) phi_final[((int64_t)b * H + h) * Nr + j] = wrap_(run + sum + phi0);
  for (int u0 = s0; u0 < s1; u0 += G) {
    float q[G];
#pragma unroll
    for (int g = 0; g < G; ++g) q[g] = (u0 + g < s1) ? src[(int64_t)(u0 + g) * HN] : 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (u0 + g < s1) dst[(int64_t)(u0 + g) * Nr] = wrap_(run + phi0);
      run += q[g];
    }
  }
}

// phi for one (batch element, block of 64 tokens): one thread per (head, group of 4
// angles) walks the block's rows in order with its running angle in registers, starting
// from the block's carry. The tanh(angles) pi rows (shared by the heads) are LDS
// broadcasts; every head's dt row is staged in LDS in one coalesced pass, with a padded
// stride so that lanes of different heads read distinct banks. It writes each row
// wrapped to [0, 2 pi) into phi, and/or, into strips, the angle before each row whose
// index is a multiple of 16 (the angle entering that 16-token strip).
__global__ void __launch_bounds__(kPrepThreads) prep_phi_kernel(const PrepFwdParams p) {
  extern __shared__ float sm[];
  const int H = p.H, Nr = p.Nr, L = p.L;
  const int tid = threadIdx.x, blk = blockIdx.x, b = blockIdx.y;
  const int t0 = blk * kPrepTB;
  const int nt = min(kPrepTB, L - t0);
  constexpr int DS = kPrepTB + 1;
  float* sT = sm;                   // [kPrepTB][Nr]
  float* sD = sT + kPrepTB * Nr;    // [H][DS]
  const float* trow = p.tpi + ((int64_t)b * L + t0) * Nr;
  for (int i = tid; i < nt * Nr; i += kPrepThreads) sT[i] = trow[i];
  for (int i = tid; i < H * kPrepTB; i += kPrepThreads) {
    const int h = i / kPrepTB, t = i % kPrepTB;
    sD[h * DS + t] = t < nt ? p.dt[((int64_t)b * H + h) * L + t0 + t] : 0.f;
  }
  __syncthreads();
  const int J4 = (Nr + 3) / 4;
  for (int pr = tid; pr < H * J4; pr += kPrepThreads) {
    const int h = pr / J4, j0 = 4 * (pr % J4);
    const int64_t bh = (int64_t)b * H + h;
    f32x4 run = ld_quad(p.tot + (((int64_t)b * p.nblk + blk) * H + h) * Nr, j0, Nr);
    f32x4 init = {0.f, 0.f, 0.f, 0.f};
    if (p.phi_init) init = ld_quad(p.phi_init + bh * Nr, j0, Nr);
    float* prow = p.phi ? p.phi + (bh * L + t0) * Nr : nullptr;
    float* srow = p.strips ? p.strips + (bh * (L >> 4) + (t0 >> 4)) * Nr : nullptr;
    const float* drow = sD + h * DS;
    auto row = [&](int t) {
      if (srow && (t & 15) == 0) {   // t0 is a multiple of 16
        f32x4 enter;
#pragma unroll
        for (int c = 0; c < 4; ++c) enter[c] = wrap_(run[c] + init[c]);
        st_quad(srow + (t >> 4) * Nr, j0, Nr, enter);
      }
      const f32x4 tp = ld_quad(sT + t * Nr, j0, Nr);
      const float d = drow[t];
#pragma unroll
      for (int c = 0; c < 4; ++c) run[c] += tp[c] * d;
      if (prow || t0 + t == L - 1) {
        f32x4 out;
#pragma unroll
        for (int c = 0; c < 4; ++c) out[c] = wrap_(run[c] + init[c]);
        if (prow) st_quad(prow + t * Nr, j0, Nr, out);
        if (t0 + t == L - 1) st_quad(p.phi_final + bh * Nr, j0, Nr, out);
      }
    };
    if (nt == kPrepTB) {   // whole blocks: a fixed trip count
#pragma unroll 8
      for (int t = 0; t < kPrepTB; ++t) row(t);
    } else {
      for (int t = 0; t < nt; ++t) row(t);
    }
  }
}

__global__ void __launch_bounds__(kPrepThreads)
prep_fill_zero_kernel(float* __restrict__ x, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kPrepThreads + threadIdx.x;
  if (i < n) x[i] = 0.f;
}

__global__ void __launch_bounds__(kPrepThreads)
prep_dphi_totals_kernel(const float* __restrict__ dphi, float* __restrict__ tot, int L, int H,
                        int Nr, int nblk) {
  const int tid = threadIdx.x, blk = blockIdx.x, b = blockIdx.y;
  const int t0 = blk * kPrepBwdTB;
  const int nt = min(kPrepBwdTB, L - t0);
  const int Q = Nr >> 2;   // 16-byte quads per row
  if ((Nr & 3) == 0 && Q > 0 && Q <= 64 && (Q & (Q - 1)) == 0) {
    // A wave per head: the block's rows are nt * Nr contiguous floats, read as 16-byte
    // pieces by consecutive lanes (1 KB per load), not a 128-byte row piece from each of
    // the wave's heads. Q divides 64, so lane l always holds quad l % Q of some row, and
    // the row sum is an xor-shuffle sum over the lanes of equal l % Q (a fixed order).
    const int wave = tid >> 6, lane = tid & 63;
    const int E4 = nt * Q;
    for (int h = wave; h < H; h += kPrepThreads / 64) {
      const f32x4* src =
          reinterpret_cast<const f32x4*>(dphi + (((int64_t)b * H + h) * L + t0) * Nr);
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int e = lane; e < E4; e += 64) {
        const f32x4 d = src[e];
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] += d[i];
      }
      for (int off = Q; off < 64; off <<= 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] += __shfl_xor(s[i], off, 64);
      }
      if (lane < Q)
        *reinterpret_cast<f32x4*>(tot + (((int64_t)b * nblk + blk) * H + h) * Nr + 4 * lane) = s;
    }
    return;
  }
  const int J4 = (Nr + 3) / 4;
  for (int pr = tid; pr < H * J4; pr += kPrepThreads) {
    const int h = pr / J4, j0 = 4 * (pr % J4);
    const float* src = dphi + (((int64_t)b * H + h) * L + t0) * Nr;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int t = 0; t < nt; ++t) {
      const f32x4 d = ld_quad(src + t * Nr, j0, Nr);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] += d[i];
    }
    st_quad(tot + (((int64_t)b * nblk + blk) * H + h) * Nr, j0, Nr, s);
  }
}

struct PrepBwdParams {
  int B, L, H, Nr, nblk;
  float a_floor;
  PrepIn dtr, ar, tr, ang;
  const float* dt_bias;
  const float* dadt; const float* dgamma; const float* dscale;
  const float* dlam; const float* ddt;
  const float* dphi;   // (B, H, L, Nr) or NULL
  const float* carry;  // (B, nblk, H, Nr) suffix carries of dphi incl. dphi_final, or NULL
  PrepOut ddtr, dar, dtrr, dang;
  float* bias_part;    // (B * nblk, H)
};

// Tokens per run of prep_bwd_kernel's reverse walk over dphi: a run's loads are issued
// before its first use, and the waves' angle-cotangent partials of a run are summed in
// wave order at its end.
constexpr int kPrepRun = 8;

// LDS of prep_bwd_kernel (floats): six TB x H tables, the TB x Nr tanh table and
// angle-cotangent accumulator, dscale just before the block for each head, and each
// wave's angle-cotangent partials of one run.
__host__ __device__ inline int prep_bwd_lds_floats(int H, int Nr) {
  return 3 * kPrepBwdTB * H + 3 * kPrepBwdTB * (H + 1) + 2 * kPrepBwdTB * Nr + H +
         (kPrepThreads / 64) * kPrepRun * Nr;
}

template <typename RT>
__global__ void __launch_bounds__(kPrepThreads) prep_bwd_kernel(const PrepBwdParams p) {
  extern __shared__ float lds[];
  const int H = p.H, Nr = p.Nr, L = p.L;
  // the incoming cotangents are read from HBM in (h, t) order (coalesced) and stored
  // t-major: their tables have a padded row stride HS = H + 1, so that consecutive t of
  // one head fall in distinct LDS banks
  const int HS = H + 1;
  float* sDt = lds;                    // [TB][H] dt
  float* sLam = sDt + kPrepBwdTB * H;     // [TB][H] lambda
  float* sDadt = sLam + kPrepBwdTB * H;   // [TB][HS] incoming cotangents (t-major)
  float* sDgam = sDadt + kPrepBwdTB * HS;
  float* sDscl = sDgam + kPrepBwdTB * HS;
  float* sPhi = sDscl + kPrepBwdTB * HS;  // [TB][H] sum_j dtheta tanh pi
  float* sBias = sDadt;                // [TB][HS] d dt_raw for the dt_bias partial; each
                                       // thread overwrites only entries it has read
  float* sT = sPhi + kPrepBwdTB * H;      // [TB][Nr] tanh(angles)
  float* sAng = sT + kPrepBwdTB * Nr;     // [TB][Nr] sum_h dtheta dt
  float* sDsPrev = sAng + kPrepBwdTB * Nr;  // [H] dscale at t0 - 1
  float* sStage = sDsPrev + H;           // [wave][kPrepRun][Nr] this run's partials

  const int tid = threadIdx.x, lane = tid & 63;
  const int blk = blockIdx.x, b = blockIdx.y;
  const int t0 = blk * kPrepBwdTB;
  const int nt = min(kPrepBwdTB, L - t0);
  const RT* dtr = static_cast<const RT*>(p.dtr.p) + b * p.dtr.sb;
  const RT* ar = static_cast<const RT*>(p.ar.p) + b * p.ar.sb;
  const RT* tr = static_cast<const RT*>(p.tr.p) + b * p.tr.sb;
  const RT* ang = static_cast<const RT*>(p.ang.p) + b * p.ang.sb;

  // ---- stage: recomputed dt / lambda, incoming cotangents, tanh table -------------
  // (KU items per thread per round, every load of a round issued before any use)
  constexpr int KU = 4;
  const DivMod byH(H), byNr(Nr > 0 ? Nr : 1), byNt(nt);
  const int nh = nt * H;
  for (int i0 = tid; i0 < nh; i0 += KU * kPrepThreads) {
    float vd[KU], vl[KU], vb[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = min(i0 + u * kPrepThreads, nh - 1);
      int t, h;
      byH(i, t, h);
      vd[u] = ldr(dtr, (int64_t)(t0 + t) * p.dtr.st + h);
      vl[u] = ldr(tr, (int64_t)(t0 + t) * p.tr.st + h);
      vb[u] = p.dt_bias[h];
    }
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = i0 + u * kPrepThreads;
      if (i < nh) {
        sDt[i] = softplus_(vd[u] + vb[u]);
        sLam[i] = sigmoid_(vl[u]);
        sPhi[i] = 0.f;
      }
    }
  }
  for (int i0 = tid; i0 < nh; i0 += KU * kPrepThreads) {  // (h, t) order: coalesced reads
    float va[KU], vg[KU], vs[KU];
    int kk[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = min(i0 + u * kPrepThreads, nh - 1);
      int h, t;
      byNt(i, h, t);
      kk[u] = t * HS + h;
      const int64_t g = ((int64_t)b * H + h) * L + t0 + t;
      va[u] = p.dadt ? p.dadt[g] : 0.f;
      vg[u] = p.dgamma ? p.dgamma[g] : 0.f;
      vs[u] = p.dscale ? p.dscale[g] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = i0 + u * kPrepThreads;
      if (i < nh) {
        sDadt[kk[u]] = va[u];
        sDgam[kk[u]] = vg[u];
        sDscl[kk[u]] = vs[u];
      }
    }
  }
  for (int h = tid; h < H; h += kPrepThreads)
    sDsPrev[h] = (p.dscale && t0 > 0) ? p.dscale[((int64_t)b * H + h) * L + t0 - 1] : 0.f;
  const int nj = nt * Nr;
  for (int i0 = tid; i0 < nj; i0 += KU * kPrepThreads) {
    float vg[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = min(i0 + u * kPrepThreads, nj - 1);
      int t, j;
      byNr(i, t, j);
      vg[u] = ldr(ang, (int64_t)(t0 + t) * p.ang.st + j);
    }
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int i = i0 + u * kPrepThreads;
      if (i < nj) {
        sT[i] = tanhf(vg[u]);
        sAng[i] = 0.f;
      }
    }
  }
  __syncthreads();

  // ---- dtheta_t = carry + sum_{s >= t in block} dphi_s, walked in reverse; per t:
  //      sPhi[t][h] = sum_j dtheta tanh pi and sAng[t][j] = sum_h dtheta dt -----------
  // A lane takes one (head, group of 4 angles) pair; the J4 groups of a head are
  // consecutive lanes (J4 rounded up to a power of two, the groups past Nr idle), so the
  // sum over j is a butterfly inside a wave. The sum over h: a butterfly over the wave's
  // heads, then the waves' partials summed in wave order at the end of every run of
  // tokens -- a fixed order, so the result does not depend on wave timing.
  if (Nr > 0 && p.carry) {
    int J4 = 1;
    while (4 * J4 < Nr) J4 <<= 1;   // <= 64: n_angles <= 256
    const int npair = H * J4;
    const int wave = tid >> 6;
    // every lane of a wave runs the same iterations (the shuffles and barriers need all)
    const int iters = (npair + kPrepThreads - 1) / kPrepThreads;
    for (int it = 0; it < iters; ++it) {
      const int pr = tid + it * kPrepThreads;
      const bool valid = pr < npair;
      // jg = pr % J4 even past npair: lanes 0..J4-1 then cover every angle group, so
      // each wave writes every stage entry of the run (zeros from idle lanes)
      const int h = valid ? pr / J4 : 0, jg = pr % J4, j0 = 4 * jg;
      const bool live = valid && j0 < Nr;
      const int64_t bh = (int64_t)b * H + h;
      f32x4 run = {0.f, 0.f, 0.f, 0.f};
      if (live) run = ld_quad(p.carry + (((int64_t)b * p.nblk + blk) * H + h) * Nr, j0, Nr);
      const float* src = p.dphi ? p.dphi + (bh * L + t0) * Nr : nullptr;
      for (int tr = nt - 1; tr >= 0; tr -= kPrepRun) {
        // all of a run's loads issued before its first use (idle lanes load nothing)
        f32x4 dq[kPrepRun];
#pragma unroll
        for (int u = 0; u < kPrepRun; ++u) {
          dq[u] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (src && live && tr - u >= 0) dq[u] = ld_quad(src + (tr - u) * Nr, j0, Nr);
        }
#pragma unroll
        for (int u = 0; u < kPrepRun; ++u) {
          const int t = tr - u;
          if (t < 0) break;
#pragma unroll
          for (int i = 0; i < 4; ++i) run[i] += dq[u][i];
          // LDS reads on every lane (an idle lane reads a valid entry, then zeros it): a
          // read under a per-lane branch would wait for each read at the join
          const float dt0 = sDt[t * H + h];
          const f32x4 tq0 = ld_quad(sT + t * Nr, live ? j0 : 0, Nr);
          const float dt = live ? dt0 : 0.f;
          float ph = 0.f;
          f32x4 ag;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float tq = live ? tq0[i] : 0.f;
            ph += run[i] * (tq * kPiF);
            ag[i] = run[i] * dt;
          }
          for (int off = 1; off < J4; off <<= 1) ph += __shfl_xor(ph, off, 64);
          if (valid && jg == 0) sPhi[t * H + h] = ph;
          for (int off = J4; off < 64; off <<= 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) ag[i] += __shfl_xor(ag[i], off, 64);
          }
          if (lane < J4) {   // lanes jg = lane hold this wave's sum over its heads
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (j0 + i < Nr) sStage[(wave * kPrepRun + u) * Nr + j0 + i] = ag[i];
          }
        }
        __syncthreads();
        for (int e = tid; e < kPrepRun * Nr; e += kPrepThreads) {
          int u, j;
          byNr(e, u, j);
          const int t = tr - u;
          if (t >= 0) {
            float acc = sAng[t * Nr + j];
#pragma unroll
            for (int w = 0; w < kPrepThreads / 64; ++w) acc += sStage[(w * kPrepRun + u) * Nr + j];
            sAng[t * Nr + j] = acc;
          }
        }
        __syncthreads();
      }
    }
  }
  __syncthreads();
  if (Nr > 0) {
    RT* dang = static_cast<RT*>(p.dang.p) + b * p.dang.sb;
    for (int i = tid; i < nt * Nr; i += kPrepThreads) {
      int t, j;
      byNr(i, t, j);
      const float tq = sT[i];
      dang[(int64_t)(t0 + t) * p.dang.st + j] = (RT)(sAng[i] * kPiF * (1.f - tq * tq));
    }
  }

  // ---- raw-slice cotangents, (t, h) row-major --------------------------------------
  RT* ddtr = static_cast<RT*>(p.ddtr.p) + b * p.ddtr.sb;
  RT* dar = static_cast<RT*>(p.dar.p) + b * p.dar.sb;
  RT* dtrr = static_cast<RT*>(p.dtrr.p) + b * p.dtrr.sb;
  for (int i0 = tid; i0 < nh; i0 += KU * kPrepThreads) {
   float vx[KU], vxa[KU], vdd[KU], vdl[KU];
#pragma unroll
   for (int u = 0; u < KU; ++u) {
    const int i = min(i0 + u * kPrepThreads, nh - 1);
    int t, h;
    byH(i, t, h);
    const int tg = t0 + t;
    const int64_t g = ((int64_t)b * H + h) * L + tg;
    vx[u] = ldr(dtr, (int64_t)tg * p.dtr.st + h) + p.dt_bias[h];
    vxa[u] = ldr(ar, (int64_t)tg * p.ar.st + h);
    vdd[u] = p.ddt ? p.ddt[g] : 0.f;
    vdl[u] = p.dlam ? p.dlam[g] : 0.f;
   }
#pragma unroll
   for (int u = 0; u < KU; ++u) {
    const int i = i0 + u * kPrepThreads;
    if (i >= nh) break;
    int t, h;
    byH(i, t, h);
    const int tg = t0 + t;
    const float dt = sDt[i], lam = sLam[i];
    const float x = vx[u];
    const float xa = vxa[u];
    const float apre = -heavy_tail_(xa);
    const float a = fminf(apre, -p.a_floor);
    const int ip = t * HS + h;   // in the padded tables
    const float dadt = sDadt[ip];
    const float dgt = sDgam[ip] + sDscl[ip];
    const float dsp = tg > 0 ? (t > 0 ? sDscl[ip - HS] : sDsPrev[h]) : 0.f;
    const float ddt = dadt * a + dgt * lam + dsp * (1.f - lam) + sPhi[i] + vdd[u];
    const float dlam = dgt * dt - dsp * dt + vdl[u];
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
    ddtr[(int64_t)tg * p.ddtr.st + h] = (RT)dx;
    dar[(int64_t)tg * p.dar.st + h] = (RT)dxa;
    dtrr[(int64_t)tg * p.dtrr.st + h] = (RT)dtrap;
    sBias[ip] = dx;
   }
  }
  __syncthreads();
  for (int h = tid; h < H; h += kPrepThreads) {
    float s = 0.f;
    for (int t = 0; t < nt; ++t) s += sBias[t * HS + h];
    p.bias_part[((int64_t)b * p.nblk + blk) * H + h] = s;
  }
}

// out[h] = sum_r part[r][h], one workgroup per head, fixed summation order.
__global__ void __launch_bounds__(kPrepThreads)
prep_bias_kernel(const float* __restrict__ part, float* __restrict__ out, int rows, int H) {
  __shared__ float red[kPrepThreads];
  const int h = blockIdx.x, tid = threadIdx.x;
  float s = 0.f;
  for (int r = tid; r < rows; r += kPrepThreads) s += part[(int64_t)r * H + h];
  red[tid] = s;
  __syncthreads();
  for (int w = kPrepThreads / 2; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (tid == 0) out[h] = red[0];
}

static PrepIn prep_in(const m3s_blx& t) { return PrepIn{t.ptr, t.stride_b, t.stride_t}; }
static PrepOut prep_out(const m3s_blx& t) { return PrepOut{t.ptr, t.stride_b, t.stride_t}; }

// Launch with `lds` bytes of dynamic LDS, raising the per-kernel limit when needed.
template <typename K, typename P>
static int32_t launch_lds(K kern, dim3 grid, size_t lds, hipStream_t s, const P& prm,
                          const char* what) {
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
    set_error("%s: cannot raise the dynamic LDS limit to %zu bytes", what, lds);
    return M3S_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(kern, grid, dim3(kPrepThreads), lds, s, prm);
  return launch_status(what);
}

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace m3s

using namespace m3s;

extern "C" int64_t m3s_prep_fwd_workspace_bytes(int32_t batch, int32_t seqlen, int32_t nheads,
                                                 int32_t n_angles) {
  if (batch <= 0 || seqlen <= 0 || nheads <= 0 || n_angles < 0) return -1;
  // the totals: per 64-token block, or per 16-token strip in the compact-only form
  const int64_t nst = (seqlen + 15) / 16;
  return align256((int64_t)batch * seqlen * n_angles * 4) +
         align256((int64_t)batch * nst * nheads * n_angles * 4);
}

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
  M3S_REQUIRE(a->dt_raw.ptr && a->a_raw.ptr && a->trap_raw.ptr && (Nr == 0 || a->angles.ptr) &&
                  a->dt_bias,
              "m3s_prep_fwd: a required input pointer is NULL");
  M3S_REQUIRE(!a->has_phi_init || a->phi_init, "m3s_prep_fwd: has_phi_init but phi_init is NULL");
  M3S_REQUIRE(a->adt && a->gamma && a->scale && a->lam && a->dt &&
                  (Nr == 0 || ((a->phi || a->phi_strips) && a->phi_final && a->workspace)),
              "m3s_prep_fwd: an output pointer or the workspace is NULL (phi or phi_strips "
              "is needed)");
  M3S_REQUIRE(Nr == 0 || aligned16(a->workspace), "m3s_prep_fwd: workspace must be 16-byte aligned");
  M3S_REQUIRE(Nr % 4 != 0 || ((!a->phi || aligned16(a->phi)) && aligned16(a->phi_final) &&
                              (!a->phi_strips || aligned16(a->phi_strips)) &&
                              (!a->theta_table || aligned16(a->theta_table)) &&
                              (!a->has_phi_init || aligned16(a->phi_init))),
              "m3s_prep_fwd: phi buffers must be 16-byte aligned");
  M3S_REQUIRE(!a->phi_strips || L % 16 == 0,
              "m3s_prep_fwd: phi_strips needs seqlen %% 16 == 0, got %d", L);
  const size_t lds = (size_t)prep_fwd_lds_floats(H, Nr) * 4;
  M3S_REQUIRE(lds <= 160 * 1024, "m3s_prep_fwd: nheads=%d, n_angles=%d exceed the LDS budget", H, Nr);
  M3S_REQUIRE(Nr <= 256, "m3s_prep_fwd: n_angles %d > 256 (a phi row must fit one wave)", Nr);
  M3S_REQUIRE((int64_t)B * H < (1ll << 31), "m3s_prep_fwd: B*H too large");
  const int nblk = (L + kPrepTB - 1) / kPrepTB;
  PrepFwdParams p{};
  p.B = B; p.L = L; p.H = H; p.Nr = Nr; p.nblk = nblk; p.a_floor = a->a_floor;
  p.dtr = prep_in(a->dt_raw); p.ar = prep_in(a->a_raw); p.tr = prep_in(a->trap_raw);
  p.ang = prep_in(a->angles);
  p.dt_bias = a->dt_bias;
  p.phi_init = a->has_phi_init ? a->phi_init : nullptr;
  p.adt = a->adt; p.gamma = a->gamma; p.scale = a->scale; p.lam = a->lam; p.dt = a->dt;
  p.phi = a->phi; p.phi_final = a->phi_final; p.strips = a->phi_strips;
  p.tpi = a->theta_table ? a->theta_table : static_cast<float*>(a->workspace);
  p.tot = reinterpret_cast<float*>(static_cast<char*>(a->workspace) +
                                   align256((int64_t)B * L * Nr * 4));
  // without phi itself the compact form comes from 16-token strip totals in two launches
  // (0.051 -> 0.043 ms at B=8, L=8192, H=32, Nr=32); phi needs the per-row pass
  p.strip_tot = (a->phi_strips && !a->phi) ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(nblk, B);
  int32_t rc = a->dtype == M3S_DTYPE_BF16
                   ? launch_lds(prep_scalars_kernel<bf16>, grid, lds, s, p, "m3s_prep_fwd")
                   : launch_lds(prep_scalars_kernel<float>, grid, lds, s, p, "m3s_prep_fwd");
  if (rc || Nr == 0) return rc;
  const int hn = H * Nr;
  if (p.strip_tot) {
    hipLaunchKernelGGL(prep_strip_carry_kernel, dim3((hn + kCarryR - 1) / kCarryR, B),
                       dim3(kPrepThreads), 0, s, p.tot, p.phi_init, p.strips, p.phi_final, H, Nr,
                       L / 16);
    return launch_status("m3s_prep_fwd");
  }
  hipLaunchKernelGGL(prep_carry_kernel, dim3((hn + kCarryR - 1) / kCarryR, B),
                     dim3(kPrepThreads), 0, s, p.tot, nullptr, nullptr, hn, nblk, 0);
  if ((rc = launch_status("m3s_prep_fwd"))) return rc;
  hipLaunchKernelGGL(prep_phi_kernel, grid, dim3(kPrepThreads),
                     (size_t)(kPrepTB * Nr + H * (kPrepTB + 1)) * 4, s, p);
  return launch_status("m3s_prep_fwd");
}

extern "C" int64_t m3s_prep_bwd_workspace_bytes(int32_t batch, int32_t seqlen, int32_t nheads,
                                                 int32_t n_angles) {
  if (batch <= 0 || seqlen <= 0 || nheads <= 0 || n_angles < 0) return -1;
  const int64_t nblk = (seqlen + kPrepBwdTB - 1) / kPrepBwdTB;
  return align256((int64_t)batch * nblk * nheads * n_angles * 4) +
         (int64_t)batch * nblk * nheads * 4;
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
  M3S_REQUIRE(a->dt_raw.ptr && a->a_raw.ptr && a->trap_raw.ptr && (Nr == 0 || a->angles.ptr) &&
                  a->dt_bias,
              "m3s_prep_bwd: a forward input pointer is NULL");
  M3S_REQUIRE(a->ddt_raw.ptr && a->da_raw.ptr && a->dtrap_raw.ptr && (Nr == 0 || a->dangles.ptr) &&
                  a->ddt_bias && a->workspace,
              "m3s_prep_bwd: an output pointer or the workspace is NULL");
  M3S_REQUIRE(aligned16(a->workspace), "m3s_prep_bwd: workspace must be 16-byte aligned");
  M3S_REQUIRE(Nr % 4 != 0 || ((!a->dphi || aligned16(a->dphi)) &&
                              (!a->dphi_final || aligned16(a->dphi_final)) &&
                              (!a->dphi_init || aligned16(a->dphi_init))),
              "m3s_prep_bwd: phi cotangent buffers must be 16-byte aligned");
  M3S_REQUIRE(Nr <= 256, "m3s_prep_bwd: n_angles %d > 256 (a head's angle groups must fit one wave)", Nr);
  const size_t lds = (size_t)prep_bwd_lds_floats(H, Nr) * 4;
  M3S_REQUIRE(lds <= 160 * 1024, "m3s_prep_bwd: nheads=%d, n_angles=%d exceed the LDS budget", H, Nr);
  M3S_REQUIRE((int64_t)B * H < (1ll << 31), "m3s_prep_bwd: B*H too large");
  const int nblk = (L + kPrepBwdTB - 1) / kPrepBwdTB;
  float* carry = static_cast<float*>(a->workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(a->workspace) +
                                         align256((int64_t)B * nblk * H * Nr * 4));
  const bool any_dphi = a->dphi || a->dphi_final;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(nblk, B);
  int32_t rc;
  const int hn = H * Nr;
  if (Nr > 0 && (any_dphi || a->dphi_init)) {
    if (a->dphi) {
      hipLaunchKernelGGL(prep_dphi_totals_kernel, grid, dim3(kPrepThreads), 0, s, a->dphi, carry,
                         L, H, Nr, nblk);
    } else {
      hipLaunchKernelGGL(prep_fill_zero_kernel, dim3((B * nblk * hn + kPrepThreads - 1) / kPrepThreads),
                         dim3(kPrepThreads), 0, s, carry, (int64_t)B * nblk * hn);
    }
    if ((rc = launch_status("m3s_prep_bwd"))) return rc;
    hipLaunchKernelGGL(prep_carry_kernel, dim3((hn + kCarryR - 1) / kCarryR, B),
                       dim3(kPrepThreads), 0, s, carry, a->dphi_final, a->dphi_init, hn, nblk, 1);
    if ((rc = launch_status("m3s_prep_bwd"))) return rc;
  }
  PrepBwdParams p{};
  p.B = B; p.L = L; p.H = H; p.Nr = Nr; p.nblk = nblk; p.a_floor = a->a_floor;
  p.dtr = prep_in(a->dt_raw); p.ar = prep_in(a->a_raw); p.tr = prep_in(a->trap_raw);
  p.ang = prep_in(a->angles);
  p.dt_bias = a->dt_bias;
  p.dadt = a->dadt; p.dgamma = a->dgamma; p.dscale = a->dscale;
  p.dlam = a->dlam; p.ddt = a->ddt;
  p.dphi = a->dphi;
  p.carry = (Nr > 0 && any_dphi) ? carry : nullptr;
  p.ddtr = prep_out(a->ddt_raw); p.dar = prep_out(a->da_raw); p.dtrr = prep_out(a->dtrap_raw);
  p.dang = prep_out(a->dangles);
  p.bias_part = part;
  rc = a->dtype == M3S_DTYPE_BF16
           ? launch_lds(prep_bwd_kernel<bf16>, grid, lds, s, p, "m3s_prep_bwd")
           : launch_lds(prep_bwd_kernel<float>, grid, lds, s, p, "m3s_prep_bwd");
  if (rc) return rc;
  hipLaunchKernelGGL(prep_bias_kernel, dim3(H), dim3(kPrepThreads), 0, s, part, a->ddt_bias,
                     B * nblk, H);
  return launch_status("m3s_prep_bwd");
}
