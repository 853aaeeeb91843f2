// Single-token decode of the Mamba-3 SISO layer on gfx950, in place.
//
// Replaces `_decode_kernel` / `_folded_kernel` (kernel_decode.py:56-233). Three-term
// trapezoidal update (the next token's dt/lambda are unknown, so the collapsed form of
// the chunked kernels does not apply):
//
//   phi' = wrap(phi + tanh(angles) pi dt)
//   S'   = e^{adt} S + e^{adt} dt (1 - lam) (v_prev (x) k_prev) + dt lam (v (x) R_phi'(k + kb))
//   y    = (S' R_phi'(q + qb) + D v) * silu(z)
//
// The step is HBM-bound: S is B*H*P*N f32 read once and written once. One workgroup
// owns one (b, h) state (P x N f32, 32 KiB at P=64, N=128); its 256 threads sweep the
// state as 16-byte vectors with consecutive threads on consecutive addresses, so each
// load/store instruction of the workgroup moves one contiguous 4 KiB span. All loads
// are issued before any arithmetic so every thread keeps its whole share in flight.
//
// Two entry points share the kernel. `m3s_decode` takes the step's inputs as the
// reference's decode kernel does. `m3s_decode_layer` takes the in_proj output row of
// each batch element instead and does the layer's per-token glue in the same launch
// (model.py:266-289 without the block norm): BCNorm of the B and C slices (one wave
// reduction per row; the normalised rows are rounded to the operand type as
// `rms_norm` returns them), dt = softplus(dt_raw + dt_bias), lam = sigmoid(trap_raw),
// adt = min(-heavy_tail(a_raw), -a_floor) dt, and x, z, angles read in place.
#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

struct DecParams {
  int B, H, Nr;
  int has_d, has_z;
  const void* q;
  const void* k;
  const void* v;
  const void* z;
  const float* adt;
  const float* dt;
  const float* lam;
  const float* angles;
  const float* qb;
  const float* kb;
  const float* dsk;
  float* ssm;
  float* kst;
  float* vst;
  float* phist;
  void* y;
  // layer mode: the projection rows and the layer's parameters
  const void* proj;
  int64_t proj_st;
  const float* wb;
  const float* wc;
  const float* dt_bias;
  float a_floor, eps;
};

constexpr int kDecThreads = 256;

// ---- readout arithmetic shared by the decode kernels ---------------------------------
// Both kernels compute y = S' q~ with these two helpers, in the same order, so that a step
// of decode_scan_kernel equals one decode_kernel launch bit for bit.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// The step's other shared expressions, with every fused multiply-add written out so that
// the compiler's contraction choices (which depend on the surrounding code) cannot make
// the two kernels round differently.
// phi' = wrap(phi + (tanh(angle) pi) dt), tp = tanh(angle) pi
__device__ __forceinline__ float phi_advance(float phi, float tp, float dt) {
  return wrap_2pi(fmaf(tp, dt, phi));
}
// the rotated pair: (lo cos - hi sin, hi cos + lo sin)
__device__ __forceinline__ float rot_lo(float lo, float hi, float cs, float sn) {
  return fmaf(lo, cs, -(hi * sn));
}
__device__ __forceinline__ float rot_hi(float lo, float hi, float cs, float sn) {
  return fmaf(hi, cs, lo * sn);
}
// S' = alpha S + beta v_prev k_prev + gamma v k~ for one element (bvp = beta v_prev,
// gv = gamma v)
__device__ __forceinline__ float state_step(float s, float alpha, float bvp, float kp, float gv,
                                            float kt) {
  return fmaf(gv, kt, fmaf(bvp, kp, alpha * s));
}

// One thread's share of a readout row: S'[p, n0 : n0 + 4] . q~[n0 : n0 + 4]. The bf16
// policy rounds S' to bf16 (kernel_decode.py:216-222; q~ already is) and takes the two
// two-term products on the bf16 dot instruction (exact bf16 products, f32 sums); f32
// multiplies and adds in order. q~ comes packed as the operand type (QPack).
template <typename MT> struct QPack { f32x4 v; };
template <> struct QPack<bf16> { bf16x2 lo, hi; };

template <typename MT>
__device__ __forceinline__ QPack<MT> pack_q(const f32x4& q) {
  if constexpr (std::is_same<MT, float>::value) {
    return QPack<MT>{q};
  } else {
    return QPack<MT>{bf16x2{(bf16)q[0], (bf16)q[1]}, bf16x2{(bf16)q[2], (bf16)q[3]}};
  }
}

template <typename MT>
__device__ __forceinline__ float readout4(const f32x4& s, const QPack<MT>& q) {
  if constexpr (std::is_same<MT, float>::value) {
    float acc = s[0] * q.v[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) acc = fmaf(s[i], q.v[i], acc);
    return acc;
  } else {
    const bf16x2 s01 = {(bf16)s[0], (bf16)s[1]}, s23 = {(bf16)s[2], (bf16)s[3]};
    return __builtin_amdgcn_fdot2_f32_bf16(
        s23, q.hi, __builtin_amdgcn_fdot2_f32_bf16(s01, q.lo, 0.f, false), false);
  }
}

// Exchange with the partner across bit B of the lane index: lane shuffles for B >= 4, the
// row mirror (lane i <-> 15 - i) for B = 3, the half-row mirror (i <-> 7 - i) for B = 2,
// quad swaps for B = 1, 0. The mirrors also flip the bits below B; the stages below B
// only need the partner to agree on the bits above B and differ in bit B.
template <int B>
__device__ __forceinline__ float lane_xchg(float v) {
  if constexpr (B >= 4) return __shfl_xor(v, 1 << B, 64);
  else if constexpr (B == 3) return dpp_mov<kDppRowMirror>(v);
  else if constexpr (B == 2) return dpp_mov<kDppHalfMirror>(v);
  else if constexpr (B == 1) return dpp_mov<kDppQuadSwap2>(v);
  else return dpp_mov<kDppQuadSwap1>(v);
}

constexpr int ilog2(int x) { return x <= 1 ? 0 : 1 + ilog2(x / 2); }

// Reduce-scatter of IT row partials over an aligned group of RV lanes (IT <= RV, powers
// of two): the first log2(IT) stages halve the rows a lane carries (it keeps the half its
// lane bit selects and adds the partner's partials of that half), the rest are plain
// butterfly adds. Lane l of the group ends with the full sum of row
// it = l >> (log2 RV - log2 IT), the same in each of its 2^(log2 RV - log2 IT) lanes.
// Every row is summed over the same tree of lane pairs whichever `it` slot carries it.
// log2(IT) + (log2 RV - log2 IT) exchanges instead of IT * log2(RV).
template <int RV, int IT, int S = 0>
__device__ __forceinline__ void rows_reduce_scatter(float* w, int lane) {
  constexpr int LR = ilog2(RV), LI = ilog2(IT);
  if constexpr (S < LR) {
    constexpr int B = LR - 1 - S;
    if constexpr (S < LI) {
      constexpr int HALF = IT >> (S + 1);
      const bool hi = (lane >> B) & 1;
#pragma unroll
      for (int k = 0; k < HALF; ++k) {
        const float keep = hi ? w[HALF + k] : w[k];
        const float send = hi ? w[k] : w[HALF + k];
        w[k] = keep + lane_xchg<B>(send);
      }
    } else {
      w[0] += lane_xchg<B>(w[0]);
    }
    rows_reduce_scatter<RV, IT, S + 1>(w, lane);
  }
}


template <typename MT, int N, int P, bool LAYER>
__global__ void __launch_bounds__(kDecThreads) decode_kernel(const DecParams p) {
  constexpr int NT = kDecThreads;
  constexpr int H2 = N / 2;
  constexpr int RV = N / 4;                         // float4 per state row
  constexpr int NV = P * N / 4;                     // float4 per state
  constexpr int IT = (NV + NT - 1) / NT;            // float4 per thread
  static_assert(RV <= 64 && (RV & (RV - 1)) == 0, "row must fit a wave");
  static_assert(NT % RV == 0, "rows must not straddle threads");

  __shared__ float sQt[N];      // q~ rounded to the readout operand type
  __shared__ float sKt[N];      // k~ (f32)
  __shared__ float sKp[N];      // k_prev
  __shared__ float sVp[P];      // v_prev
  __shared__ float sV[P];       // v (f32)

  const int tid = threadIdx.x;
  const int wid = xcd_remap(blockIdx.x, gridDim.x);
  const int b = wid / p.H, h = wid % p.H;
  const int64_t bh = (int64_t)b * p.H + h;

  // ---- issue the state loads first --------------------------------------------
  f32x4* sg = reinterpret_cast<f32x4*>(p.ssm + bh * P * N);
  f32x4 st[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int f = it * NT + tid;
    if (f < NV) st[it] = __builtin_nontemporal_load(sg + f);
  }

  // projection row of this batch element (layer mode): [z, x, B, C, dt, a, trap, angles]
  const int HP = p.H * P;
  const MT* prow = LAYER ? static_cast<const MT*>(p.proj) + (int64_t)b * p.proj_st : nullptr;
  float adt, dt, lam;
  if constexpr (LAYER) {
    const MT* sc = prow + 2 * HP + 2 * N;
    dt = softplus_((float)sc[h] + p.dt_bias[h]);
    lam = 1.f / (1.f + expf(-(float)sc[2 * p.H + h]));
    adt = fminf(-heavy_tail_((float)sc[p.H + h]), -p.a_floor) * dt;
  } else {
    adt = p.adt[bh];
    dt = p.dt[bh];
    lam = p.lam[bh];
  }
  // ---- angle advance + rotation (wave 0; lane l takes the pairs j = l + 64 u) ---------
  if (tid < 64) {
    constexpr int JP = (H2 + 63) / 64;   // pairs per lane
    float qlo[JP], qhi[JP], klo[JP], khi[JP];
    if constexpr (LAYER) {
      // BCNorm of the C (query) and B (key) rows, f32, output rounded to MT
      const MT* crow = prow + 2 * HP + N;
      const MT* brow = prow + 2 * HP;
      float cl[JP], ch[JP], bl[JP], bh_[JP];
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int u = 0; u < JP; ++u) {
        const int j = tid + 64 * u;
        cl[u] = ch[u] = bl[u] = bh_[u] = 0.f;
        if (j < H2) {
          cl[u] = (float)crow[j]; ch[u] = (float)crow[H2 + j];
          bl[u] = (float)brow[j]; bh_[u] = (float)brow[H2 + j];
        }
        sq += cl[u] * cl[u] + ch[u] * ch[u];
        sk += bl[u] * bl[u] + bh_[u] * bh_[u];
      }
      sq = group_sum<64>(sq);
      sk = group_sum<64>(sk);
      const float rq = bc_rstd(sq, 1.f / N, p.eps), rk = bc_rstd(sk, 1.f / N, p.eps);
#pragma unroll
      for (int u = 0; u < JP; ++u) {
        const int j = tid + 64 * u;
        qlo[u] = qhi[u] = klo[u] = khi[u] = 0.f;
        if (j < H2) {
          qlo[u] = (float)(MT)(cl[u] * rq * p.wc[j]);
          qhi[u] = (float)(MT)(ch[u] * rq * p.wc[H2 + j]);
          klo[u] = (float)(MT)(bl[u] * rk * p.wb[j]);
          khi[u] = (float)(MT)(bh_[u] * rk * p.wb[H2 + j]);
        }
      }
    } else {
      const MT* qg = static_cast<const MT*>(p.q) + (int64_t)b * N;
      const MT* kg = static_cast<const MT*>(p.k) + (int64_t)b * N;
#pragma unroll
      for (int u = 0; u < JP; ++u) {
        const int j = tid + 64 * u;
        qlo[u] = qhi[u] = klo[u] = khi[u] = 0.f;
        if (j < H2) {
          qlo[u] = (float)qg[j]; qhi[u] = (float)qg[H2 + j];
          klo[u] = (float)kg[j]; khi[u] = (float)kg[H2 + j];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < JP; ++u) {
      const int j = tid + 64 * u;
      if (j < H2) {
        const float ulo = qlo[u] + p.qb[h * N + j];
        const float uhi = qhi[u] + p.qb[h * N + H2 + j];
        const float wlo = klo[u] + p.kb[h * N + j];
        const float whi = khi[u] + p.kb[h * N + H2 + j];
        float sn = 0.f, cs = 1.f;
        if (j < p.Nr) {
          const float ang = LAYER ? (float)prow[2 * HP + 2 * N + 3 * p.H + j] : p.angles[(int64_t)b * p.Nr + j];
          const float phi = phi_advance(p.phist[bh * p.Nr + j], tanhf(ang) * kPi, dt);
          p.phist[bh * p.Nr + j] = phi;
          sincosf(phi, &sn, &cs);
        }
        sQt[j] = (float)(MT)rot_lo(ulo, uhi, cs, sn);
        sQt[H2 + j] = (float)(MT)rot_hi(ulo, uhi, cs, sn);
        sKt[j] = rot_lo(wlo, whi, cs, sn);
        sKt[H2 + j] = rot_hi(wlo, whi, cs, sn);
      }
    }
  }
  const MT* vrow = LAYER ? prow + HP + h * P : static_cast<const MT*>(p.v) + bh * P;
  for (int i = tid; i < N; i += NT) sKp[i] = p.kst[bh * N + i];
  for (int i = tid; i < P; i += NT) {
    sVp[i] = p.vst[bh * P + i];
    sV[i] = (float)vrow[i];
  }
  __syncthreads();
  // the carried (k, v) pair is now in LDS: overwrite it with this token's
  for (int i = tid; i < N; i += NT) p.kst[bh * N + i] = sKt[i];
  for (int i = tid; i < P; i += NT) p.vst[bh * P + i] = sV[i];

  const float alpha = expf(adt);
  const float beta = alpha * dt * (1.0f - lam);
  const float gamma = dt * lam;

  // ---- update + readout ----------------------------------------------------------
  const int n0 = (tid % RV) * 4;       // fixed across iterations since NT % RV == 0
  const f32x4 kp = *reinterpret_cast<const f32x4*>(sKp + n0);
  const f32x4 kt = *reinterpret_cast<const f32x4*>(sKt + n0);
  const QPack<MT> qt = pack_q<MT>(*reinterpret_cast<const f32x4*>(sQt + n0));
  MT* yg = static_cast<MT*>(p.y) + bh * P;
  const MT* zg = LAYER ? prow + h * P : (p.has_z ? static_cast<const MT*>(p.z) + bh * P : nullptr);
  const float dsk = p.has_d ? p.dsk[h] : 0.f;
  float part[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int f = it * NT + tid;
    const bool valid = f < NV;
    const int prow = valid ? f / RV : 0;
    const float bvp = beta * sVp[prow];
    const float gv = gamma * sV[prow];
    f32x4 s = st[it];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = state_step(s[i], alpha, bvp, kp[i], gv, kt[i]);
    // a plain store (the loads are non-temporal): at B=256 a non-temporal store made the
    // step 17% slower, and plain loads 10%
    if (valid) sg[f] = s;
    part[it] = readout4<MT>(s, qt);
  }
  // row sums: lane l of each RV-lane group ends with the row of slot l >> LO
  constexpr int LO = ilog2(RV) - ilog2(IT);
  const int lane = tid % RV;
  rows_reduce_scatter<RV, IT>(part, lane);
  const int itr = lane >> LO;
  const int yrow = (itr * NT + tid) / RV;
  if ((lane & ((1 << LO) - 1)) == 0 && itr * NT + tid < NV) {
    float yv = fmaf(dsk, sV[yrow], part[0]);
    if (zg) yv *= silu((float)zg[yrow]);
    yg[yrow] = (MT)yv;
  }
}

// ---- T steps in one launch ------------------------------------------------------------
// decode_scan_kernel: a known-length run of T steps (kernel_decode.py:474-533, a lax.scan of
// decode_step). One workgroup per (b, h) as in decode_kernel, but the state stays in the
// workgroup's registers for all T steps: it is read once and written once, where T
// separate steps stream it T times. The steps go in windows of W (16; 8 at N = 256):
//   1. all threads stage the window's inputs in LDS: v and z rows, the step coefficients
//      (alpha, beta, gamma) and the angle increments tanh(angles) pi dt;
//   2. one thread per angle runs phi through the window (a serial add-and-wrap chain);
//   3. all threads rotate the window's q / k rows (one pair per thread and step);
//   4. the W steps' update + readout, with no barrier between steps (each thread's state
//      rows are its own; the window's operands are already in LDS); gated y goes to LDS;
//   5. the window's y leaves as contiguous 16-byte stores.
// Every value is computed by decode_kernel's expressions in the same order and the
// readout uses the same helpers (readout4, rows_reduce_scatter; a row's sum does not
// depend on which thread slot carries it), so the results equal T decode_kernel launches
// bit for bit. k~ and v sit in rings of 2W steps so that step t - 1's pair is still
// there at a window's first step.
struct DecScanParams {
  int B, H, Nr, T;
  int has_d, has_z;
  const void* q;        // (B, T, N)
  const void* k;        // (B, T, N)
  const void* v;        // (B, H, T, P)
  const void* z;        // (B, H, T, P)
  const float* adt;     // (B, H, T)
  const float* dt;      // (B, H, T)
  const float* lam;     // (B, H, T)
  const float* angles;  // (B, T, Nr)
  const float* qb;
  const float* kb;
  const float* dsk;
  float* ssm;
  float* kst;
  float* vst;
  float* phist;
  void* y;              // (B, H, T, P)
};

// (The waves-per-EU hint only steers register allocation. Without it the N = 128 kernels
// take 189 VGPRs: two workgroups per CU. A hint of five waves makes the allocator stop at
// 127 without spilling (a hint of four spills), and LDS then allows four workgroups; the
// compiler warns that five is not met. N = 256 holds 64 state floats per thread and is
// left at two waves per SIMD.)
template <typename MT, int N, int P>
__global__ void __launch_bounds__(kDecThreads)
__attribute__((amdgpu_waves_per_eu(N >= 256 ? 2 : 5, 8)))
decode_scan_kernel(const DecScanParams p) {
  constexpr int NT = kDecThreads;
  constexpr int H2 = N / 2;
  constexpr int RV = N / 4;                   // float4 per state row = lanes per row group
  constexpr int NV = P * N / 4;               // float4 per state
  constexpr int IT = (NV + NT - 1) / NT;      // float4 (rows) per thread
  constexpr int G = NT / RV;                  // row groups; group g owns rows g*IT .. +IT
  constexpr int W = N >= 256 ? 8 : 16;        // steps per window
  constexpr int W2 = 2 * W;                   // ring slots of k~ and v
  constexpr int LO = ilog2(RV) - ilog2(IT);
  static_assert(RV <= 64 && (RV & (RV - 1)) == 0, "row must fit a wave");
  static_assert(NT % RV == 0 && NT % H2 == 0 && (P & (P - 1)) == 0, "layout");
  static_assert(IT == 1 || G * IT == P, "row groups cover the state");
  static_assert((W * P * sizeof(MT)) % 16 == 0, "y window in 16-byte vectors");

  __shared__ __align__(16) float sK[W2][N];   // k~ by step (slot t mod 2W)
  __shared__ __align__(16) float sV[W2][P];   // v by step (slot t mod 2W)
  __shared__ __align__(16) MT sQ[W][N];       // q~, by window step
  __shared__ __align__(16) float sZ[W][P];    // silu(z)
  __shared__ __align__(16) float sC[W][4];    // alpha, beta, gamma, dt
  __shared__ float sPh[W][H2];                // angle increments, then phi
  __shared__ __align__(16) MT sY[W][P];       // gated y of the window

  const int tid = threadIdx.x;
  const int wid = xcd_remap(blockIdx.x, gridDim.x);
  const int b = wid / p.H, h = wid % p.H;
  const int64_t bh = (int64_t)b * p.H + h;
  const int T = p.T, Nr = p.Nr;
  const int g = tid / RV, lane = tid % RV, n0 = lane * 4;

  // the state: thread (g, lane) holds S[g*IT + it, n0 : n0 + 4]
  f32x4* sg = reinterpret_cast<f32x4*>(p.ssm + bh * P * N);
  f32x4 st[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    st[it] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (g * IT + it < P) st[it] = __builtin_nontemporal_load(sg + (g * IT + it) * RV + lane);
  }
  // the carried (k~, v) pair is step -1's, in ring slot 2W - 1
  for (int i = tid; i < N; i += NT) sK[W2 - 1][i] = p.kst[bh * N + i];
  for (int i = tid; i < P; i += NT) sV[W2 - 1][i] = p.vst[bh * P + i];
  float ph = tid < Nr ? p.phist[bh * Nr + tid] : 0.f;   // phi of angle `tid`
  const int jr = tid % H2, wr = tid / H2;                // rotation: pair jr of steps wr + k NT/H2
  const float qbl = p.qb[h * N + jr], qbh = p.qb[h * N + H2 + jr];
  const float kbl = p.kb[h * N + jr], kbh = p.kb[h * N + H2 + jr];
  const float dsk = p.has_d ? p.dsk[h] : 0.f;
  const MT* qg = static_cast<const MT*>(p.q) + (int64_t)b * T * N;
  const MT* kg = static_cast<const MT*>(p.k) + (int64_t)b * T * N;
  const MT* vg = static_cast<const MT*>(p.v) + bh * T * P;
  const MT* zg = p.has_z ? static_cast<const MT*>(p.z) + bh * T * P : nullptr;
  const float* ag = p.angles + (int64_t)b * T * Nr;
  const float* adtg = p.adt + bh * T;
  const float* dtg = p.dt + bh * T;
  const float* lamg = p.lam + bh * T;
  char* yb = reinterpret_cast<char*>(static_cast<MT*>(p.y) + bh * T * P);
  constexpr int YV = W * P * (int)sizeof(MT) / 16;        // 16-byte vectors of a full window

  for (int t0 = 0; t0 < T; t0 += W) {
    const int wn = T - t0 < W ? T - t0 : W;
    // ---- window inputs: v, z, the step coefficients, the angle increments ----------
    for (int i = tid; i < wn * P; i += NT) {
      const int w = i / P, pp = i % P;
      sV[(t0 + w) & (W2 - 1)][pp] = (float)vg[(int64_t)(t0 + w) * P + pp];
      if (zg) sZ[w][pp] = silu((float)zg[(int64_t)(t0 + w) * P + pp]);
    }
    if (tid < wn) {
      const float adt = adtg[t0 + tid], dt = dtg[t0 + tid], lam = lamg[t0 + tid];
      const float alpha = expf(adt);
      sC[tid][0] = alpha;
      sC[tid][1] = alpha * dt * (1.0f - lam);
      sC[tid][2] = dt * lam;
      sC[tid][3] = dt;
    }
    for (int i = tid; i < wn * H2; i += NT) {
      const int w = i / H2, j = i % H2;
      if (j < Nr) sPh[w][j] = tanhf(ag[(int64_t)(t0 + w) * Nr + j]) * kPi;
    }
    __syncthreads();
    // ---- phi, one serial chain per angle ---------------------------------------------
    if (tid < Nr) {
      for (int w = 0; w < wn; ++w) {
        ph = phi_advance(ph, sPh[w][tid], sC[w][3]);
        sPh[w][tid] = ph;
      }
    }
    __syncthreads();
    // ---- rotated q~ / k~ of the window -----------------------------------------------
    for (int w = wr; w < wn; w += NT / H2) {
      const int64_t t = t0 + w;
      const float ulo = (float)qg[t * N + jr] + qbl;
      const float uhi = (float)qg[t * N + H2 + jr] + qbh;
      const float wlo = (float)kg[t * N + jr] + kbl;
      const float whi = (float)kg[t * N + H2 + jr] + kbh;
      float sn = 0.f, cs = 1.f;
      if (jr < Nr) sincosf(sPh[w][jr], &sn, &cs);
      sQ[w][jr] = (MT)rot_lo(ulo, uhi, cs, sn);
      sQ[w][H2 + jr] = (MT)rot_hi(ulo, uhi, cs, sn);
      sK[t & (W2 - 1)][jr] = rot_lo(wlo, whi, cs, sn);
      sK[t & (W2 - 1)][H2 + jr] = rot_hi(wlo, whi, cs, sn);
    }
    __syncthreads();
    // ---- the window's steps: update + readout, no barrier between them ---------------
    for (int w = 0; w < wn; ++w) {
      const int t = t0 + w;
      const int sc = t & (W2 - 1), sp = (t - 1) & (W2 - 1);
      const f32x4 cf = *reinterpret_cast<const f32x4*>(&sC[w][0]);
      const f32x4 kp = *reinterpret_cast<const f32x4*>(&sK[sp][n0]);
      const f32x4 kt = *reinterpret_cast<const f32x4*>(&sK[sc][n0]);
      const QPack<MT> qt = *reinterpret_cast<const QPack<MT>*>(&sQ[w][n0]);
      // v of the group's rows at steps t - 1 and t (IT consecutive floats)
      float vp[IT], vc[IT];
      if constexpr (IT % 4 == 0) {
#pragma unroll
        for (int u = 0; u < IT / 4; ++u) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(&sV[sp][g * IT + 4 * u]);
          const f32x4 c = *reinterpret_cast<const f32x4*>(&sV[sc][g * IT + 4 * u]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            vp[4 * u + i] = a[i];
            vc[4 * u + i] = c[i];
          }
        }
      } else {
#pragma unroll
        for (int it = 0; it < IT; ++it) {
          const int prow = g * IT + it < P ? g * IT + it : 0;
          vp[it] = sV[sp][prow];
          vc[it] = sV[sc][prow];
        }
      }
      float part[IT];
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const float bvp = cf[1] * vp[it];
        const float gv = cf[2] * vc[it];
#pragma unroll
        for (int i = 0; i < 4; ++i) st[it][i] = state_step(st[it][i], cf[0], bvp, kp[i], gv, kt[i]);
        part[it] = readout4<MT>(st[it], qt);
      }
      rows_reduce_scatter<RV, IT>(part, lane);
      const int prow = g * IT + (lane >> LO);
      if ((lane & ((1 << LO) - 1)) == 0 && prow < P) {
        float yv = fmaf(dsk, sV[sc][prow], part[0]);
        if (zg) yv *= sZ[w][prow];
        sY[w][prow] = (MT)yv;
      }
    }
    __syncthreads();
    // ---- the window's y, as contiguous 16-byte stores ---------------------------------
    const int nv = wn == W ? YV : wn * P * (int)sizeof(MT) / 16;
    for (int i = tid; i < nv; i += NT)
      reinterpret_cast<uint4*>(yb + (int64_t)t0 * P * sizeof(MT))[i] =
          reinterpret_cast<const uint4*>(&sY[0][0])[i];
  }
  // ---- write back: the state, the last step's (k~, v) pair and phi -------------------
#pragma unroll
  for (int it = 0; it < IT; ++it)
    if (g * IT + it < P) sg[(g * IT + it) * RV + lane] = st[it];
  const int sl = (T - 1) & (W2 - 1);
  for (int i = tid; i < N; i += NT) p.kst[bh * N + i] = sK[sl][i];
  for (int i = tid; i < P; i += NT) p.vst[bh * P + i] = sV[sl][i];
  if (tid < Nr) p.phist[bh * Nr + tid] = ph;
}

template <typename MT, int N, int P>
static int32_t launch_dec_scan(const DecScanParams& prm, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((decode_scan_kernel<MT, N, P>), dim3(grid), dim3(kDecThreads), 0, stream, prm);
  return launch_status("m3s_decode_scan");
}

template <typename MT, int N, int P, bool LAYER>
static int32_t launch_dec(const DecParams& prm, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((decode_kernel<MT, N, P, LAYER>), dim3(grid), dim3(kDecThreads), 0, stream, prm);
  return launch_status(LAYER ? "m3s_decode_layer" : "m3s_decode");
}

#define M3S_DEC_CONFIGS(X) \
  X(bf16, 128, 64)         \
  X(bf16, 64, 64)          \
  X(bf16, 32, 16)          \
  X(bf16, 16, 16)          \
  X(bf16, 256, 64)         \
  X(float, 128, 64)        \
  X(float, 64, 64)         \
  X(float, 32, 16)         \
  X(float, 16, 16)

template <typename MT> constexpr int dcode();
template <> constexpr int dcode<bf16>() { return M3S_DTYPE_BF16; }
template <> constexpr int dcode<float>() { return M3S_DTYPE_F32; }

int32_t decode_supported(int dtype, int n, int pdim) {
#define X(MT, N, P) if (dtype == dcode<MT>() && n == N && pdim == P) return 1;
  M3S_DEC_CONFIGS(X)
#undef X
  return 0;
}

}  // namespace m3s

extern "C" int32_t m3s_decode(const m3s_decode_args* a, void* stream) {
  using namespace m3s;
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_decode: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_decode_args),
              "m3s_decode: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_decode_args));
  const int B = a->batch, H = a->nheads, P = a->headdim, N = a->state_dim, Nr = a->n_angles;
  M3S_REQUIRE(B > 0 && H > 0 && P > 0 && N > 0, "m3s_decode: non-positive dimension");
  M3S_REQUIRE(Nr >= 0 && 2 * Nr <= N, "m3s_decode: n_angles %d exceeds state_dim/2", Nr);
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32,
              "m3s_decode: bad dtype %d", a->dtype);
  if (!decode_supported(a->dtype, N, P)) {
    set_error("m3s_decode: no kernel for dtype=%s state_dim=%d headdim=%d",
              a->dtype == M3S_DTYPE_BF16 ? "bf16" : "f32", N, P);
    return M3S_ERR_UNSUPPORTED;
  }
  M3S_REQUIRE(a->q && a->k && a->v && a->adt && a->dt && a->lam && a->q_bias && a->k_bias,
              "m3s_decode: a required input pointer is NULL");
  M3S_REQUIRE(Nr == 0 || a->angles, "m3s_decode: angles is NULL");
  M3S_REQUIRE(!a->has_d || a->d_skip, "m3s_decode: has_d but d_skip is NULL");
  M3S_REQUIRE(!a->has_z || a->z, "m3s_decode: has_z but z is NULL");
  M3S_REQUIRE(a->ssm && aligned16(a->ssm) && a->k_state && a->v_state &&
              (Nr == 0 || a->phi_state) && a->y,
              "m3s_decode: state/output pointers NULL or ssm misaligned");
  M3S_REQUIRE((int64_t)B * H < (1ll << 31), "m3s_decode: B*H too large");
  DecParams prm{};
  prm.B = B; prm.H = H; prm.Nr = Nr; prm.has_d = a->has_d; prm.has_z = a->has_z;
  prm.q = a->q; prm.k = a->k; prm.v = a->v; prm.z = a->z;
  prm.adt = a->adt; prm.dt = a->dt; prm.lam = a->lam; prm.angles = a->angles;
  prm.qb = a->q_bias; prm.kb = a->k_bias; prm.dsk = a->d_skip;
  prm.ssm = a->ssm; prm.kst = a->k_state; prm.vst = a->v_state; prm.phist = a->phi_state;
  prm.y = a->y;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define X(MT, NN, PP) \
  if (a->dtype == dcode<MT>() && N == NN && P == PP) return launch_dec<MT, NN, PP, false>(prm, B * H, s);
  M3S_DEC_CONFIGS(X)
#undef X
  set_error("m3s_decode: unreachable dispatch");
  return M3S_ERR_UNSUPPORTED;
}

extern "C" int32_t m3s_decode_layer(const m3s_decode_layer_args* a, void* stream) {
  using namespace m3s;
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_decode_layer: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_decode_layer_args),
              "m3s_decode_layer: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_decode_layer_args));
  const int B = a->batch, H = a->nheads, P = a->headdim, N = a->state_dim, Nr = a->n_angles;
  M3S_REQUIRE(B > 0 && H > 0 && P > 0 && N > 0, "m3s_decode_layer: non-positive dimension");
  M3S_REQUIRE(Nr >= 0 && 2 * Nr <= N, "m3s_decode_layer: n_angles %d exceeds state_dim/2", Nr);
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32,
              "m3s_decode_layer: bad dtype %d", a->dtype);
  if (!decode_supported(a->dtype, N, P)) {
    set_error("m3s_decode_layer: no kernel for dtype=%s state_dim=%d headdim=%d",
              a->dtype == M3S_DTYPE_BF16 ? "bf16" : "f32", N, P);
    return M3S_ERR_UNSUPPORTED;
  }
  const int64_t width = 2LL * H * P + 2LL * N + 3LL * H + Nr;
  M3S_REQUIRE(a->proj && a->proj_stride >= width, "m3s_decode_layer: proj NULL or row stride %lld < %lld",
              (long long)a->proj_stride, (long long)width);
  M3S_REQUIRE(a->b_norm_weight && a->c_norm_weight && a->dt_bias && a->q_bias && a->k_bias,
              "m3s_decode_layer: a parameter pointer is NULL");
  M3S_REQUIRE(a->ssm && aligned16(a->ssm) && a->k_state && a->v_state &&
              (Nr == 0 || a->phi_state) && a->y,
              "m3s_decode_layer: state/output pointers NULL or ssm misaligned");
  M3S_REQUIRE((int64_t)B * H < (1ll << 31), "m3s_decode_layer: B*H too large");
  DecParams prm{};
  prm.B = B; prm.H = H; prm.Nr = Nr; prm.has_d = a->d_skip != nullptr; prm.has_z = 1;
  prm.qb = a->q_bias; prm.kb = a->k_bias; prm.dsk = a->d_skip;
  prm.ssm = a->ssm; prm.kst = a->k_state; prm.vst = a->v_state; prm.phist = a->phi_state;
  prm.y = a->y;
  prm.proj = a->proj; prm.proj_st = a->proj_stride;
  prm.wb = a->b_norm_weight; prm.wc = a->c_norm_weight; prm.dt_bias = a->dt_bias;
  prm.a_floor = a->a_floor; prm.eps = a->norm_eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define X(MT, NN, PP) \
  if (a->dtype == dcode<MT>() && N == NN && P == PP) return launch_dec<MT, NN, PP, true>(prm, B * H, s);
  M3S_DEC_CONFIGS(X)
#undef X
  set_error("m3s_decode_layer: unreachable dispatch");
  return M3S_ERR_UNSUPPORTED;
}

extern "C" int32_t m3s_decode_scan(const m3s_decode_scan_args* a, void* stream) {
  using namespace m3s;
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_decode_scan: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_decode_scan_args),
              "m3s_decode_scan: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_decode_scan_args));
  const int B = a->batch, T = a->steps, H = a->nheads, P = a->headdim, N = a->state_dim,
            Nr = a->n_angles;
  M3S_REQUIRE(B > 0 && T > 0 && H > 0 && P > 0 && N > 0, "m3s_decode_scan: non-positive dimension");
  M3S_REQUIRE(Nr >= 0 && 2 * Nr <= N, "m3s_decode_scan: n_angles %d exceeds state_dim/2", Nr);
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32,
              "m3s_decode_scan: bad dtype %d", a->dtype);
  if (!decode_supported(a->dtype, N, P)) {
    set_error("m3s_decode_scan: no kernel for dtype=%s state_dim=%d headdim=%d",
              a->dtype == M3S_DTYPE_BF16 ? "bf16" : "f32", N, P);
    return M3S_ERR_UNSUPPORTED;
  }
  M3S_REQUIRE(a->q && a->k && a->v && a->adt && a->dt && a->lam && a->q_bias && a->k_bias,
              "m3s_decode_scan: a required input pointer is NULL");
  M3S_REQUIRE(Nr == 0 || a->angles, "m3s_decode_scan: angles is NULL");
  M3S_REQUIRE(!a->has_d || a->d_skip, "m3s_decode_scan: has_d but d_skip is NULL");
  M3S_REQUIRE(!a->has_z || a->z, "m3s_decode_scan: has_z but z is NULL");
  M3S_REQUIRE(a->ssm && aligned16(a->ssm) && a->k_state && a->v_state &&
              (Nr == 0 || a->phi_state) && a->y && aligned16(a->y),
              "m3s_decode_scan: state/output pointers NULL, or ssm / y not 16-byte aligned");
  M3S_REQUIRE((int64_t)B * H < (1ll << 31) && (int64_t)B * H * T * (P > N ? P : N) < (1ll << 40),
              "m3s_decode_scan: B*H or B*H*T too large");
  DecScanParams prm{};
  prm.B = B; prm.H = H; prm.Nr = Nr; prm.T = T; prm.has_d = a->has_d; prm.has_z = a->has_z;
  prm.q = a->q; prm.k = a->k; prm.v = a->v; prm.z = a->z;
  prm.adt = a->adt; prm.dt = a->dt; prm.lam = a->lam; prm.angles = a->angles;
  prm.qb = a->q_bias; prm.kb = a->k_bias; prm.dsk = a->d_skip;
  prm.ssm = a->ssm; prm.kst = a->k_state; prm.vst = a->v_state; prm.phist = a->phi_state;
  prm.y = a->y;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define X(MT, NN, PP) \
  if (a->dtype == dcode<MT>() && N == NN && P == PP) return launch_dec_scan<MT, NN, PP>(prm, B * H, s);
  M3S_DEC_CONFIGS(X)
#undef X
  set_error("m3s_decode_scan: unreachable dispatch");
  return M3S_ERR_UNSUPPORTED;
}
