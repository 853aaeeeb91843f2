// Reverse-scan backward of the Mamba-3 SISO chunked scan on gfx950 (MI355X).
//
// Replaces `_bwd_kernel` / `siso_backward_kernel` (kernel_bwd.py:103-511) and the
// dfinal_v injection of `siso_backward` (kernel_bwd.py:632-637). Per chunk, walked in
// reverse with the adjoint G of the chunk-end state (f32, MFMA registers):
//
//   g      = dy * silu(z);  dz = dy * ybar * sig(z) (1 + z (1 - sig(z)))
//   W      = tril_strict(q~ khat^T * dec),   dM = tril_strict(g v^T * dec),  dec = 2^{min(A_i - A_j, 0)}
//   dq~    = dM khat + 2^A (g S)
//   dkhat  = dM^T q~ + 2^{A_last - A} (v G)
//   dv     = W^T g + 2^{A_last - A} (khat G^T) + (D + gamma u.w) g
//   dadt   = suffix_sum(q~.dq~ - khat.dkhat) + [2^{A_last} <G, S> + <khat, 2^{A_last-A}(v G)>]
//   dscale = dkhat . k~,  du = R_{-phi}(dq~) + dqk gamma w,  dw = R_{-phi}(dkhat scale) + dqk gamma u
//   dphi   = rope_dphi(q~, dq~) + rope_dphi(k~, dk~)
//   dq += sum_h du, dk += sum_h dw;  G <- 2^{A_last} G + (2^A g)^T q~
//
// One workgroup per (b, h). Wave w owns position strip [16w, 16w+16) both as queries
// (dq~) and as keys (dkhat, dv), which balances the causal triangle across waves.
// Score-like tiles (W, dM, dM^T) never leave registers: an MFMA accumulator tile is
// already an operand fragment with its row index as K (see m3s_common.h). Operands
// whose K is their row index (q~, khat, g over time) are served from transposed LDS
// copies, built in place by one transpose pass between the two product phases. The
// elementwise pullback runs row-major on f32 dq~/dkhat staged through LDS and writes
// each head's du/dw rows to the workspace with coalesced 16-byte stores; a second,
// HBM-bound launch (headsum_kernel) sums them over heads into dq/dk, so the result
// does not depend on the order in which workgroups finish.
#include <type_traits>

#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

struct BwdParams {
  int B, L, H, Nr, nc;
  int has_d, has_z;
  const void* dy;
  int64_t dy_sb, dy_sh, dy_st;
  const void* ybar;   // (B, H, L, P) in the matmul dtype
  const void* z;
  int64_t z_sb, z_sh, z_st;
  const void* q;
  const void* k;
  const void* v;
  int64_t v_sb, v_sh, v_st;
  const float* adt;
  const float* gamma;
  const float* scale;
  const float* phi;
  const float* tht;    // phi_strips mode (see FwdParams); else NULL
  const float* pdt;
  const float* pstr;
  const float* qb;
  const float* kb;
  const float* dsk;
  const void* cstates;
  const float* dfs;
  const float* dfv;
  float* dq;
  float* dk;
  void* dv;
  int64_t dv_sb, dv_sh, dv_st;
  void* dz;
  int64_t dz_sb, dz_sh, dz_st;
  float* dadt;
  float* dqk;
  float* dscale;
  float* uw;
  float* dphi;
  float* dqb;
  float* dkb;
  float* kfin;
  float* dseed;
  void* part;   // (2, B, H, L, N) per-head du / dw rows, MT
};

template <typename MT> struct BV16;
template <> struct BV16<bf16> { typedef bf16x8 type; static constexpr int n = 8; };
template <> struct BV16<float> { typedef f32x4 type; static constexpr int n = 4; };

constexpr int cmax(int a, int b) { return a > b ? a : b; }

template <typename MT, int C, int N, int P, int NW>
struct BwdCfg {
  static constexpr int NT = NW * 64;
  static constexpr int VEC = BV16<MT>::n;
  static constexpr int H2 = N / 2;
  static constexpr int PAD = 16 / (int)sizeof(MT);
  static constexpr int LDQ = N + PAD;   // sQ, sK rows (positions)
  static constexpr int LDP = P + PAD;   // sG, sV rows (positions), sST / sGT rows (n)
  static constexpr int LDT = C + PAD;   // sQT, sKT, sGT rows
  static constexpr int LDF = N + 4;     // f32 staging rows of dq~ / dkhat
  static constexpr int PB = P / 16, NB = N / 16, CB = C / 16;
  static constexpr int T4 = PB * NB;
  static constexpr int SPW = (T4 + NW - 1) / NW;
  static constexpr int E = C >= 64 ? C / 64 : 1;
  static constexpr int QKG = H2 / VEC;
  static constexpr int QKT = (C / 2) * QKG;
  static constexpr int QKR = (QKT + NT - 1) / NT;
  static constexpr int VG = P / VEC;
  static constexpr int VT = (C / 2) * VG;
  static constexpr int VR = (VT + NT - 1) / NT;
  static constexpr int SV = N * P / VEC;           // 16-byte pieces of a chunk state
  static constexpr int SR = (SV + NT - 1) / NT;
  // transpose-pass tasks: (row pair, column group) over sQ, sK (C x N) and sG (C x P)
  static constexpr int TQ = (C / 2) * (N / VEC);
  static constexpr int TG = (C / 2) * (P / VEC);
  static constexpr int TQR = (TQ + NT - 1) / NT;
  static constexpr int TGR = (TG + NT - 1) / NT;
  // ---- LDS layout -----------------------------------------------------------------
  static constexpr int SZ_QQ = cmax(C * LDQ, N * LDT) * (int)sizeof(MT);  // sQ | sQT
  static constexpr int SZ_GG = cmax(C * LDP, P * LDT) * (int)sizeof(MT);  // sG | sGT
  static constexpr int SZ_V = C * LDP * (int)sizeof(MT);
  static constexpr int SZ_ST = N * LDP * (int)sizeof(MT);                  // S^T [n][p]
  static constexpr int SZ_X = 2 * SZ_QQ + SZ_GG + SZ_V + SZ_ST;
  static constexpr int SZ_STAGE = 2 * C * LDF * 4;                         // dq~, dkhat f32
  static constexpr int SZ_R = cmax(SZ_X, SZ_STAGE);
  static constexpr int SZ_GAT = N * LDP * (int)sizeof(MT);                 // G^T [n][p]
  static constexpr int SZ_SC = (8 * C + 4 * N + 16) * 4;
  static constexpr int LDS_BYTES = SZ_R + SZ_GAT + SZ_SC;
  static_assert(NW >= CB, "one position strip per wave");
  static_assert(QKG <= 64 && (QKG & (QKG - 1)) == 0, "row groups must fit a wave");
  static_assert(VG <= 64 && (VG & (VG - 1)) == 0, "row groups must fit a wave");
  static_assert(C % 32 == 0 && N % 16 == 0 && P % 16 == 0, "tile shape");
  static_assert(LDS_BYTES <= 163840, "LDS budget of one gfx950 CU");
};

template <typename MT>
__device__ __forceinline__ sub_t<MT> zero_sub() {
  return sub_from_f32<MT>(f32x4{0.f, 0.f, 0.f, 0.f});
}

template <typename MT, int C, int N, int P, int NW, bool STRIPS>
__global__ void __launch_bounds__(NW * 64) bwd_kernel(const BwdParams p) {
  using F = BwdCfg<MT, C, N, P, NW>;
  using vec = typename BV16<MT>::type;
  constexpr int NT = F::NT, VEC = F::VEC, H2 = F::H2;
  constexpr int LDQ = F::LDQ, LDP = F::LDP, LDT = F::LDT, LDF = F::LDF;
  constexpr int PB = F::PB, NB = F::NB, CB = F::CB;

  __shared__ __align__(16) unsigned char smem[F::LDS_BYTES];
  // Buffer offsets go through an opaque SGPR. Otherwise every access above 64 KiB (the
  // reach of a ds_read immediate) gets its own address VGPR, and LICM keeps all of them
  // live across the chunk loop -- enough to spill.
  auto opq = [](int x) { asm volatile("" : "+s"(x)); return x; };
  MT* sQ = reinterpret_cast<MT*>(smem);                       // q~ [t][n]  -> sQT [n][t]
  MT* sK = reinterpret_cast<MT*>(smem + opq(F::SZ_QQ));            // khat [j][n] -> sKT [n][j]
  MT* sG = reinterpret_cast<MT*>(smem + opq(2 * F::SZ_QQ));        // g [t][p]  -> sGT [p][t]
  MT* sV = reinterpret_cast<MT*>(smem + opq(2 * F::SZ_QQ + F::SZ_GG));
  MT* sST = reinterpret_cast<MT*>(smem + opq(2 * F::SZ_QQ + F::SZ_GG + F::SZ_V));
  MT* sQT = sQ;
  MT* sKT = sK;
  MT* sGT = sG;
  float* sDQ = reinterpret_cast<float*>(smem);                // staging, after the products
  float* sDK = reinterpret_cast<float*>(smem + opq(C * LDF * 4));
  MT* sGaT = reinterpret_cast<MT*>(smem + opq(F::SZ_R));           // adjoint G^T [n][p]
  float* sA = reinterpret_cast<float*>(smem + opq(F::SZ_R + F::SZ_GAT));
  float* sExpA = sA + C;
  float* sFac = sExpA + C;
  float* sGam = sFac + C;
  float* sScl = sGam + C;
  float* sDqk = sScl + C;
  float* sCoef = sDqk + C;
  float* sDA = sCoef + C;
  float* sQb = sDA + C;
  float* sKb = sQb + N;
  // [w]: wave w's share of 2^{A_last}<G,S> + <v, dv_inter> for the current chunk, summed
  // in wave order (no float atomics: the result does not depend on wave timing)
  float* sRed = sKb + 3 * N;
  static_assert(NW <= 16, "one sRed slot per wave");

  const int tid = threadIdx.x, lane = tid & 63, g4 = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wid = xcd_remap(blockIdx.x, gridDim.x);
  const int b = wid / p.H, h = wid % p.H;
  const int64_t bh = (int64_t)b * p.H + h;
  const int L = p.L, Nr = p.Nr, nc = p.nc;

  for (int i = tid; i < N; i += NT) {
    sQb[i] = p.qb[h * N + i];
    sKb[i] = p.kb[h * N + i];
  }
  const float dsk = p.has_d ? p.dsk[h] : 0.f;
  // this lane's running bias-gradient partials over its row pairs of every chunk: a lane
  // keeps the same columns j0.. in every chunk (NT is a multiple of QKG), so the sums
  // stay in registers and are reduced once, in a fixed order, after the last chunk
  float bqa[2][F::VEC], bka[2][F::VEC];
#pragma unroll
  for (int i = 0; i < F::VEC; ++i) bqa[0][i] = bqa[1][i] = bka[0][i] = bka[1][i] = 0.f;

  const MT* qg = static_cast<const MT*>(p.q) + (int64_t)b * L * N;
  const MT* kg = static_cast<const MT*>(p.k) + (int64_t)b * L * N;
  const MT* vg = static_cast<const MT*>(p.v) + b * p.v_sb + h * p.v_sh;
  const MT* dyg = static_cast<const MT*>(p.dy) + b * p.dy_sb + h * p.dy_sh;
  const MT* zg = p.has_z ? static_cast<const MT*>(p.z) + b * p.z_sb + h * p.z_sh : nullptr;
  MT* dzg = p.has_z ? static_cast<MT*>(p.dz) + b * p.dz_sb + h * p.dz_sh : nullptr;
  MT* dvg = static_cast<MT*>(p.dv) + b * p.dv_sb + h * p.dv_sh;
  const MT* ybg = static_cast<const MT*>(p.ybar) + bh * (int64_t)L * P;
  const float* adtg = p.adt + bh * L;
  const float* gamg = p.gamma + bh * L;
  const float* sclg = p.scale + bh * L;
  const float* phig = STRIPS ? nullptr : p.phi + bh * (int64_t)L * Nr;
  const MT* csg = static_cast<const MT*>(p.cstates) + bh * (int64_t)nc * N * P;
  MT* dug = static_cast<MT*>(p.part) + bh * (int64_t)L * N;                 // du rows of (b, h)
  MT* dwg = static_cast<MT*>(p.part) + ((int64_t)p.B * p.H + bh) * L * N;   // dw rows of (b, h)
  const bool phi_vec = (Nr % 4) == 0;
  // phi of row t (global index) at angles j0 .. j0 + VEC - 1, 0 past Nr: read, or
  // (phi_strips mode) the strip's entering angle plus theta = tanh(angles) pi dt over the
  // strip's rows up to t (at most 16)
  auto phi_row = [&](int64_t t, int j0, float (&out)[VEC]) {
    if constexpr (STRIPS) {
      const int64_t s16 = t >> 4;
      const float* ps = p.pstr + (bh * (L / 16) + s16) * Nr;
#pragma unroll
      for (int i = 0; i < VEC; ++i) out[i] = (j0 + i < Nr) ? ps[j0 + i] : 0.f;
      for (int64_t u = 16 * s16; u <= t; ++u) {
        const float du = p.pdt[bh * L + u];
        const float* tr = p.tht + ((int64_t)b * L + u) * Nr;
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          if (j0 + i < Nr) out[i] += tr[j0 + i] * du;
      }
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) out[i] = (j0 + i < Nr) ? phig[t * Nr + j0 + i] : 0.f;
    }
  };

  // ---- adjoint G (registers, MFMA layout [p][n]) -----------------------------------
  f32x4 Gacc[F::SPW];
#pragma unroll
  for (int m = 0; m < F::SPW; ++m) {
    const int s = wave + NW * m;
    Gacc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (s < F::T4 && p.dfs) {
      const int pb = s % PB, nb = s / PB;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        Gacc[m][i] = p.dfs[(bh * P + pb * 16 + 4 * g4 + i) * N + nb * 16 + l16];
    }
  }
  auto publish_adjoint = [&]() {
#pragma unroll
    for (int m = 0; m < F::SPW; ++m) {
      const int s = wave + NW * m;
      if (s < F::T4) {
        const int pb = s % PB, nb = s / PB;
        *reinterpret_cast<sub_t<MT>*>(sGaT + (nb * 16 + l16) * LDP + pb * 16 + 4 * g4) =
            sub_from_f32<MT>(Gacc[m]);
      }
    }
  };
  publish_adjoint();

  // ---- register prefetch of one chunk's raw inputs ----------------------------------
  vec rq[F::QKR][2][2], rk[F::QKR][2][2];
  f32x4 rphi[F::QKR][2][VEC / 4];
  float rscale[F::QKR][2];
  vec rv[F::VR][2], rdy[F::VR][2], rz[F::VR][2], ryb[F::VR][2];
  vec rs[F::SR];
  float radt[F::E], rgam_s, rscl_s;

  auto load_qk = [&](int c, vec (&q_)[F::QKR][2][2], vec (&k_)[F::QKR][2][2],
                     f32x4 (&ph_)[F::QKR][2][VEC / 4], float (&sc_)[F::QKR][2]) {
    const int t0 = c * C;
#pragma unroll
    for (int r = 0; r < F::QKR; ++r) {
      const int task = tid + r * NT;
      if (task < F::QKT) {
        const int tp = task / F::QKG, j0 = (task % F::QKG) * VEC;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int64_t t = t0 + 2 * tp + e;
          q_[r][e][0] = *reinterpret_cast<const vec*>(qg + t * N + j0);
          q_[r][e][1] = *reinterpret_cast<const vec*>(qg + t * N + H2 + j0);
          k_[r][e][0] = *reinterpret_cast<const vec*>(kg + t * N + j0);
          k_[r][e][1] = *reinterpret_cast<const vec*>(kg + t * N + H2 + j0);
          if constexpr (STRIPS) {
            float pv[VEC];
            phi_row(t, j0, pv);
#pragma unroll
            for (int i = 0; i < VEC; ++i) ph_[r][e][i / 4][i % 4] = pv[i];
          } else {
            const float* pr = phig + t * Nr;
#pragma unroll
            for (int qd = 0; qd < VEC / 4; ++qd) {
              const int j = j0 + 4 * qd;
              if (phi_vec && j + 4 <= Nr) {
                ph_[r][e][qd] = *reinterpret_cast<const f32x4*>(pr + j);
              } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) ph_[r][e][qd][i] = (j + i < Nr) ? pr[j + i] : 0.f;
              }
            }
          }
          sc_[r][e] = sclg[t];
        }
      }
    }
  };
  auto prefetch = [&](int c) {
    const int t0 = c * C;
    load_qk(c, rq, rk, rphi, rscale);
#pragma unroll
    for (int r = 0; r < F::VR; ++r) {
      const int task = tid + r * NT;
      if (task < F::VT) {
        const int tp = task / F::VG, p0 = (task % F::VG) * VEC;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int64_t t = t0 + 2 * tp + e;
          rv[r][e] = *reinterpret_cast<const vec*>(vg + t * p.v_st + p0);
          rdy[r][e] = *reinterpret_cast<const vec*>(dyg + t * p.dy_st + p0);
          if (zg) {
            rz[r][e] = *reinterpret_cast<const vec*>(zg + t * p.z_st + p0);
            ryb[r][e] = *reinterpret_cast<const vec*>(ybg + t * P + p0);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < F::SR; ++r) {
      const int f = tid + r * NT;
      if (f < F::SV) rs[r] = *reinterpret_cast<const vec*>(csg + (int64_t)c * N * P + f * VEC);
    }
    if (wave == 0) {
#pragma unroll
      for (int e = 0; e < F::E; ++e) {
        const int tt = lane * F::E + e;
        radt[e] = tt < C ? adtg[t0 + tt] : 0.f;
      }
    }
    if (tid < C) {
      rgam_s = gamg[t0 + tid];
      rscl_s = sclg[t0 + tid];
    }
  };

  prefetch(nc - 1);
  __syncthreads();

  for (int c = nc - 1; c >= 0; --c) {
    const int t0 = c * C;
    // Lane/wave indices re-derived opaquely each chunk, so the per-lane LDS address
    // arithmetic is recomputed near its uses instead of being hoisted out of the loop.
    int lane_v = threadIdx.x;
    asm volatile("" : "+v"(lane_v));
    const int tid = lane_v, lane = tid & 63, g4 = lane >> 4, l16 = lane & 15;
    int wave_s = __builtin_amdgcn_readfirstlane(tid >> 6);
    asm volatile("" : "+s"(wave_s));
    const int wave = wave_s;

    // ============ phase L: raw -> LDS (q~, khat, g, v, S^T), dz, dqk, uw ==============
    if (wave == 0) {
      float a[F::E];
      float run = 0.f;
#pragma unroll
      for (int e = 0; e < F::E; ++e) {
        run += radt[e] * kLog2e;
        a[e] = run;
      }
      float incl = run;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
      }
      const float excl = incl - run;
      const float a_last = __shfl(incl, (C - 1) / F::E, 64);
#pragma unroll
      for (int e = 0; e < F::E; ++e) {
        const int tt = lane * F::E + e;
        if (tt < C) {
          const float A = excl + a[e];
          sA[tt] = A;
          sExpA[tt] = exp2f(A);
          sFac[tt] = exp2f(a_last - A);
        }
      }
    }
    if (tid < C) {
      sGam[tid] = rgam_s;
      sScl[tid] = rscl_s;
    }
#pragma unroll
    for (int r = 0; r < F::QKR; ++r) {
      const int task = tid + r * NT;
      const bool valid = task < F::QKT;
      const int tp = valid ? task / F::QKG : 0, j0 = valid ? (task % F::QKG) * VEC : 0;
      float uw[2] = {0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        if (valid) {
          const int t = 2 * tp + e;
          vec oq0, oq1, ok0, ok1;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const int j = j0 + i;
            const float ulo = (float)rq[r][e][0][i] + sQb[j];
            const float uhi = (float)rq[r][e][1][i] + sQb[H2 + j];
            const float wlo = (float)rk[r][e][0][i] + sKb[j];
            const float whi = (float)rk[r][e][1][i] + sKb[H2 + j];
            uw[e] += ulo * wlo + uhi * whi;
            float sn = 0.f, cs = 1.f;
            if (j < Nr) sincosf(rphi[r][e][i / 4][i % 4], &sn, &cs);
            const float sc = rscale[r][e];
            oq0[i] = (MT)(ulo * cs - uhi * sn);
            oq1[i] = (MT)(uhi * cs + ulo * sn);
            ok0[i] = (MT)((wlo * cs - whi * sn) * sc);
            ok1[i] = (MT)((whi * cs + wlo * sn) * sc);
          }
          *reinterpret_cast<vec*>(sQ + t * LDQ + j0) = oq0;
          *reinterpret_cast<vec*>(sQ + t * LDQ + H2 + j0) = oq1;
          *reinterpret_cast<vec*>(sK + t * LDQ + j0) = ok0;
          *reinterpret_cast<vec*>(sK + t * LDQ + H2 + j0) = ok1;
        }
      }
      uw[0] = group_sum<F::QKG>(uw[0]);
      uw[1] = group_sum<F::QKG>(uw[1]);
      if (valid && j0 == 0) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int t = 2 * tp + e;
          p.uw[bh * L + t0 + t] = uw[e];
          sCoef[t] = p.gamma[bh * L + t0 + t] * uw[e] + dsk;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < F::VR; ++r) {
      const int task = tid + r * NT;
      const bool valid = task < F::VT;
      const int tp = valid ? task / F::VG : 0, p0 = valid ? (task % F::VG) * VEC : 0;
      float dqk[2] = {0.f, 0.f};
      if (valid) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int t = 2 * tp + e;
          vec og, odz;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const float dy = (float)rdy[r][e][i];
            float gv = dy;
            if (zg) {
              const float zf = (float)rz[r][e][i];
              const float sg = sigmoidf_(zf);
              gv = dy * (zf * sg);
              odz[i] = (MT)(dy * (float)ryb[r][e][i] * sg * (1.f + zf * (1.f - sg)));
            }
            dqk[e] += gv * (float)rv[r][e][i];
            og[i] = (MT)gv;
          }
          *reinterpret_cast<vec*>(sG + t * LDP + p0) = og;
          *reinterpret_cast<vec*>(sV + t * LDP + p0) = rv[r][e];
          if (dzg) *reinterpret_cast<vec*>(dzg + (int64_t)(t0 + t) * p.dz_st + p0) = odz;
        }
      }
      dqk[0] = group_sum<F::VG>(dqk[0]);
      dqk[1] = group_sum<F::VG>(dqk[1]);
      if (valid && p0 == 0) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int t = 2 * tp + e;
          sDqk[t] = dqk[e];
          p.dqk[bh * L + t0 + t] = dqk[e];
        }
      }
    }
#pragma unroll
    for (int r = 0; r < F::SR; ++r) {
      const int f = tid + r * NT;
      if (f < F::SV) {
        const int n = (f * VEC) / P, pp = (f * VEC) % P;
        *reinterpret_cast<vec*>(sST + n * LDP + pp) = rs[r];
      }
    }
    __syncthreads();

    if (c > 0) prefetch(c - 1);   // in flight during the products of this chunk
    // ============ phase P1: register score tiles, inter-chunk terms ===================
    const int w = wave;
    const bool strip = w < CB;
    sub_t<MT> Wt[CB], dMt[CB], dMT[CB];
    f32x4 dQ[NB], dKh[NB], dV[PB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      dQ[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      dKh[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) dV[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float red = 0.f;
    if (strip) {
      const int jcol = w * 16 + l16;     // this lane's key position (cols of W, dM)
      const float Aj = sA[jcol];
#pragma unroll
      for (int tb = 0; tb < CB; ++tb) {
        if (tb >= w) {
          f32x4 aw = {0.f, 0.f, 0.f, 0.f}, am = {0.f, 0.f, 0.f, 0.f};
          gemm_nt<MT, N>(aw, sQ, LDQ, tb * 16, sK, LDQ, w * 16);   // W[t][j]
          gemm_nt<MT, P>(am, sG, LDP, tb * 16, sV, LDP, w * 16);   // dM[t][j]
          f32x4 vw, vm;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = tb * 16 + 4 * g4 + i;
            const float dec = (t > jcol) ? exp2f(fminf(sA[t] - Aj, 0.f)) : 0.f;
            vw[i] = aw[i] * dec;
            vm[i] = am[i] * dec;
          }
          Wt[tb] = sub_from_f32<MT>(vw);
          dMt[tb] = sub_from_f32<MT>(vm);
        } else {
          Wt[tb] = zero_sub<MT>();
          dMt[tb] = zero_sub<MT>();
        }
      }
      const int tcol = w * 16 + l16;     // this lane's query position (cols of dM^T)
      const float At = sA[tcol];
#pragma unroll
      for (int jb = 0; jb < CB; ++jb) {
        if (jb <= w) {
          f32x4 am = {0.f, 0.f, 0.f, 0.f};
          gemm_nt<MT, P>(am, sV, LDP, jb * 16, sG, LDP, w * 16);   // dM^T[j][t]
          f32x4 vm;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = jb * 16 + 4 * g4 + i;
            vm[i] = (tcol > j) ? am[i] * exp2f(fminf(At - sA[j], 0.f)) : 0.f;
          }
          dMT[jb] = sub_from_f32<MT>(vm);
        } else {
          dMT[jb] = zero_sub<MT>();
        }
      }
      // dq~ inter: 2^{A_t} sum_p g[t][p] S[p][n]   (rows t, cols n)
      // dkhat inter: 2^{A_last-A_j} sum_p v[j][p] G[p][n]   (rows j, cols n)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        gemm_nt<MT, P>(dQ[nb], sG, LDP, w * 16, sST, LDP, nb * 16);
        gemm_nt<MT, P>(dKh[nb], sV, LDP, w * 16, sGaT, LDP, nb * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = w * 16 + 4 * g4 + i;
          dQ[nb][i] *= sExpA[r];
          dKh[nb][i] *= sFac[r];
        }
      }
      // dv inter: 2^{A_last-A_j} sum_n khat[j][n] G[p][n]   (rows j, cols p)
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
#pragma unroll
        for (int k0 = 0; k0 < N; k0 += 16) {
          sub_t<MT> bsub;
          const int kk = sub_k(k0);
#pragma unroll
          for (int i = 0; i < 4; ++i) bsub[i] = sGaT[(kk + i) * LDP + pb * 16 + l16];
          mma16(dV[pb], ld_sub<MT>(sK, LDQ, w * 16, k0), bsub);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = w * 16 + 4 * g4 + i;
          dV[pb][i] *= sFac[j];
          // <v, dv_inter> == <khat, dk_inter>: the A_last share of the state update
          red += (float)sV[j * LDP + pb * 16 + l16] * dV[pb][i];
        }
      }
    }
    // 2^{A_last} <G, S>: this wave's adjoint tiles against the chunk-start state
    {
      float gs = 0.f;
#pragma unroll
      for (int m = 0; m < F::SPW; ++m) {
        const int s = wave + NW * m;
        if (s < F::T4) {
          const int pb = s % PB, nb = s / PB;
          const f32x4 sv =
              sub_to_f32<MT>(*reinterpret_cast<const sub_t<MT>*>(sST + (nb * 16 + l16) * LDP + pb * 16 + 4 * g4));
#pragma unroll
          for (int i = 0; i < 4; ++i) gs += Gacc[m][i] * sv[i];
        }
      }
      red += sExpA[C - 1] * gs;
    }
    red = group_sum<64>(red);
    if (lane == 0) sRed[wave] = red;
    __syncthreads();

    // ============ transpose pass: q~, khat, g to [x][position], one tile at a time =====
    auto transpose_tile = [&](MT* buf, int ldr, int cols) {
      // in place: every thread reads its share, barrier, writes it transposed
      constexpr int MAXR = (C / 2) * (N / VEC) / NT + 1;
      vec tv[MAXR][2];
      const int groups = cols / VEC, tasks = (C / 2) * groups;
#pragma unroll
      for (int r = 0; r < MAXR; ++r) {
        const int task = tid + r * NT;
        if (task < tasks) {
          const int tp = task / groups, c0 = (task % groups) * VEC;
          tv[r][0] = *reinterpret_cast<const vec*>(buf + (2 * tp) * ldr + c0);
          tv[r][1] = *reinterpret_cast<const vec*>(buf + (2 * tp + 1) * ldr + c0);
        }
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < MAXR; ++r) {
        const int task = tid + r * NT;
        if (task < tasks) {
          const int tp = task / groups, c0 = (task % groups) * VEC;
#pragma unroll
          for (int i = 0; i < VEC; ++i)
            store_pair<MT>(buf + (c0 + i) * LDT + 2 * tp, (float)tv[r][0][i], (float)tv[r][1][i]);
        }
      }
    };
    transpose_tile(sQ, LDQ, N);
    transpose_tile(sK, LDQ, N);
    transpose_tile(sG, LDP, P);
    __syncthreads();

    // ============ phase P2: intra-chunk products, adjoint update ======================
    if (strip) {
      // dv[j][p] += sum_t W[t][j] g[t][p];  dkhat[j][n] += sum_t dM[t][j] q~[t][n]
#pragma unroll
      for (int tb = 0; tb < CB; tb += 2) {
        if (tb + 1 >= w) {
#pragma unroll
          for (int pb = 0; pb < PB; ++pb)
            mma32(dV[pb], Wt[tb], Wt[tb + 1], ld_sub<MT>(sGT, LDT, pb * 16, tb * 16),
                  ld_sub<MT>(sGT, LDT, pb * 16, tb * 16 + 16));
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            mma32(dKh[nb], dMt[tb], dMt[tb + 1], ld_sub<MT>(sQT, LDT, nb * 16, tb * 16),
                  ld_sub<MT>(sQT, LDT, nb * 16, tb * 16 + 16));
        }
      }
      // dq~[t][n] += sum_j dM^T[j][t] khat[j][n]
#pragma unroll
      for (int jb = 0; jb < CB; jb += 2) {
        if (jb <= w) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            mma32(dQ[nb], dMT[jb], dMT[jb + 1], ld_sub<MT>(sKT, LDT, nb * 16, jb * 16),
                  ld_sub<MT>(sKT, LDT, nb * 16, jb * 16 + 16));
        }
      }
    }
    // G <- 2^{A_last} G + sum_t (2^{A_t} g[t][p]) q~[t][n]
    {
      const float eAl = sExpA[C - 1];
#pragma unroll
      for (int m = 0; m < F::SPW; ++m) {
        const int s = wave + NW * m;
        if (s < F::T4) {
          const int pb = s % PB, nb = s / PB;
#pragma unroll
          for (int i = 0; i < 4; ++i) Gacc[m][i] *= eAl;
#pragma unroll
          for (int k0 = 0; k0 < C; k0 += 32) {
            f32x4 a0 = sub_to_f32<MT>(ld_sub<MT>(sGT, LDT, pb * 16, k0));
            f32x4 a1 = sub_to_f32<MT>(ld_sub<MT>(sGT, LDT, pb * 16, k0 + 16));
            const int kk = sub_k(k0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              a0[i] *= sExpA[kk + i];
              a1[i] *= sExpA[kk + 16 + i];
            }
            mma32(Gacc[m], sub_from_f32<MT>(a0), sub_from_f32<MT>(a1),
                  ld_sub<MT>(sQT, LDT, nb * 16, k0), ld_sub<MT>(sQT, LDT, nb * 16, k0 + 16));
          }
        }
      }
    }
    // dv epilogue: + (D + gamma u.w) g, + dfinal_v on the sequence's last row; store
    if (strip) {
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        const int pcol = pb * 16 + l16;
        const f32x4 gv = sub_to_f32<MT>(
            *reinterpret_cast<const sub_t<MT>*>(sGT + pcol * LDT + w * 16 + 4 * g4));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = w * 16 + 4 * g4 + i;
          float d = dV[pb][i] + sCoef[j] * gv[i];
          if (p.dfv && t0 + j == L - 1) d += p.dfv[bh * P + pcol];
          dvg[(int64_t)(t0 + j) * p.dv_st + pcol] = (MT)d;
        }
      }
    }
    __syncthreads();

    // ============ stage dq~ [t][n] and dkhat [j][n] as f32 rows =======================
    if (strip) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = w * 16 + 4 * g4 + i;
          sDQ[r * LDF + nb * 16 + l16] = dQ[nb][i];
          sDK[r * LDF + nb * 16 + l16] = dKh[nb][i];
        }
      }
    }
    __syncthreads();

    // ============ phase R: rotation pullback, per-row reductions, head sum ============
#pragma unroll
    for (int r = 0; r < F::QKR; ++r) {
      const int task = tid + r * NT;
      const bool valid = task < F::QKT;
      const int tp = valid ? task / F::QKG : 0, j0 = valid ? (task % F::QKG) * VEC : 0;
      float dA[2] = {0.f, 0.f}, dsc[2] = {0.f, 0.f};
      float bq[2][VEC], bk[2][VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) bq[0][i] = bq[1][i] = bk[0][i] = bk[1][i] = 0.f;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        if (valid) {
          const int t = 2 * tp + e;
          const int64_t tg = t0 + t;
          const vec q0 = *reinterpret_cast<const vec*>(qg + tg * N + j0);
          const vec q1 = *reinterpret_cast<const vec*>(qg + tg * N + H2 + j0);
          const vec k0 = *reinterpret_cast<const vec*>(kg + tg * N + j0);
          const vec k1 = *reinterpret_cast<const vec*>(kg + tg * N + H2 + j0);
          const float sc = sScl[t];
          const float cd = sDqk[t] * sGam[t];
          float pr[VEC];
          phi_row(tg, j0, pr);
          vec du0, du1, dw0, dw1;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const int j = j0 + i;
            const float ulo = (float)q0[i] + sQb[j];
            const float uhi = (float)q1[i] + sQb[H2 + j];
            const float wlo = (float)k0[i] + sKb[j];
            const float whi = (float)k1[i] + sKb[H2 + j];
            float sn = 0.f, cs = 1.f;
            if (j < Nr) sincosf(pr[i], &sn, &cs);
            const float qlo = ulo * cs - uhi * sn, qhi = uhi * cs + ulo * sn;
            const float klo = wlo * cs - whi * sn, khi = whi * cs + wlo * sn;
            const float dqlo = sDQ[t * LDF + j], dqhi = sDQ[t * LDF + H2 + j];
            const float dklo = sDK[t * LDF + j], dkhi = sDK[t * LDF + H2 + j];
            dA[e] += qlo * dqlo + qhi * dqhi - (klo * sc) * dklo - (khi * sc) * dkhi;
            dsc[e] += dklo * klo + dkhi * khi;
            const float dtlo = dklo * sc, dthi = dkhi * sc;   // d k~
            // R^T = R(-phi): lo' = lo cos + hi sin, hi' = hi cos - lo sin
            const float dulo = dqlo * cs + dqhi * sn + cd * wlo;
            const float duhi = dqhi * cs - dqlo * sn + cd * whi;
            const float dwlo = dtlo * cs + dthi * sn + cd * ulo;
            const float dwhi = dthi * cs - dtlo * sn + cd * uhi;
            if (j < Nr)
              p.dphi[(bh * L + tg) * Nr + j] = (dqhi * qlo - dqlo * qhi) + (dthi * klo - dtlo * khi);
            if (c == nc - 1 && t == C - 1) {
              p.kfin[bh * N + j] = klo;
              p.kfin[bh * N + H2 + j] = khi;
            }
            du0[i] = dulo;
            du1[i] = duhi;
            dw0[i] = dwlo;
            dw1[i] = dwhi;
            bq[0][i] += dulo;
            bq[1][i] += duhi;
            bk[0][i] += dwlo;
            bk[1][i] += dwhi;
          }
          // this head's du / dw row pieces; the head sum happens in headsum_kernel
          *reinterpret_cast<vec*>(dug + tg * N + j0) = du0;
          *reinterpret_cast<vec*>(dug + tg * N + H2 + j0) = du1;
          *reinterpret_cast<vec*>(dwg + tg * N + j0) = dw0;
          *reinterpret_cast<vec*>(dwg + tg * N + H2 + j0) = dw1;
        }
      }
      dA[0] = group_sum<F::QKG>(dA[0]);
      dA[1] = group_sum<F::QKG>(dA[1]);
      dsc[0] = group_sum<F::QKG>(dsc[0]);
      dsc[1] = group_sum<F::QKG>(dsc[1]);
      if (valid && j0 == 0) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          sDA[2 * tp + e] = dA[e];
          p.dscale[bh * L + t0 + 2 * tp + e] = dsc[e];
        }
      }
      // bias partials: into this lane's running sums (zero for an idle task)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          bqa[hh][i] += bq[hh][i];
          bka[hh][i] += bk[hh][i];
        }
      }
    }
    __syncthreads();

    // ============ phase S: dadt = suffix_sum(dA) + A_last share; publish G ============
    if (wave == 0) {
      float extra = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) extra += sRed[w];
      float a[F::E];
      float run = 0.f;
#pragma unroll
      for (int e = F::E - 1; e >= 0; --e) {
        const int tt = lane * F::E + e;
        run += (tt < C) ? sDA[tt] : 0.f;
        a[e] = run;
      }
      // suffix scan across lanes: inclusive sum over lanes >= this one
      float incl = run;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_down(incl, off, 64);
        if (lane + off < 64) incl += o;
      }
      const float excl = incl - run;
#pragma unroll
      for (int e = 0; e < F::E; ++e) {
        const int tt = lane * F::E + e;
        if (tt < C) p.dadt[bh * L + t0 + tt] = excl + a[e] + extra;
      }
    }
    publish_adjoint();
    __syncthreads();
  }

  // ---- per-(b, h) outputs ------------------------------------------------------------
#pragma unroll
  for (int m = 0; m < F::SPW; ++m) {
    const int s = wave + NW * m;
    if (s < F::T4) {
      const int pb = s % PB, nb = s / PB;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        p.dseed[(bh * P + pb * 16 + 4 * g4 + i) * N + nb * 16 + l16] = Gacc[m][i];
    }
  }
  // bias gradients: the lanes sharing columns j0.. (lane bits log2(QKG)..5) summed by a
  // butterfly, each wave's totals into its own LDS slot (the staging area is free now),
  // then the slots summed in wave order
  __syncthreads();
  {
    float* sBias = sDQ;   // [NW][2N]: q's N entries, then k's
    const int j0 = (tid % F::QKG) * VEC;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float vq = bqa[hh][i], vk = bka[hh][i];
#pragma unroll
        for (int m = F::QKG; m < 64; m <<= 1) {
          vq += __shfl_xor(vq, m, 64);
          vk += __shfl_xor(vk, m, 64);
        }
        if (lane < F::QKG) {
          sBias[wave * 2 * N + hh * H2 + j0 + i] = vq;
          sBias[wave * 2 * N + N + hh * H2 + j0 + i] = vk;
        }
      }
    }
    __syncthreads();
    for (int i = tid; i < 2 * N; i += NT) {
      float acc = 0.f;
      for (int w = 0; w < NW; ++w) acc += sBias[w * 2 * N + i];
      if (i < N) p.dqb[bh * N + i] = acc;
      else p.dkb[bh * N + i - N] = acc;
    }
  }
}

// ===================================================================================
// bwd_bf16_kernel: the bf16 backward for state_dim % 64 == 0 (the configs[2] shape).
//
// Same maths and rounding points as bwd_kernel. Rebuilt like fwd_bf16_kernel:
//  * No transpose pass. Operands whose contraction axis is time or the state index
//    (g^T, q~^T, khat^T, G^T read by columns) come from ds_read_b64_tr_b16 on the
//    row-major tiles, so the three in-place transposes and their barriers are gone.
//  * Each score-like tile pair (W, dM for the wave's key strip; dM^T for its query
//    strip) is consumed by its products as soon as it is built: only two tiles live.
//  * Global traffic through per-(b, h) buffer descriptors (32-bit offsets), and the
//    lane index re-derived per phase, so nothing spills.
//  * The previous chunk's raw rows are prefetched during the pullback, into registers
//    it frees as it goes: v, dy, z after its first row, ybar and the chunk state after
//    the bias butterfly, q, k, phi before the pullback's closing barrier. None of them coexists with the
//    product accumulators. Phase R reloads q, k, phi before the staging barrier.
// ===================================================================================

template <int C, int N, int P>
struct Bwd2Cfg {
  static constexpr int NW = C / 16;
  static constexpr int NT = NW * 64;
  static constexpr int VEC = 8;
  static constexpr int H2 = N / 2;
  static constexpr int LDQ = N + 8;     // sQ, sK rows (positions)
  static constexpr int LDP = P + 8;     // sG, sV rows (positions); sST, sGaT rows (n)
  static constexpr int LDF = N + 4;     // f32 staging rows of dq~ / dkhat
  static constexpr int PB = P / 16, NB = N / 16, CB = C / 16;
  static constexpr int T4 = PB * NB;
  static constexpr int SPW = T4 / NW;
  static constexpr int E = C / 64;
  static constexpr int QKG = H2 / VEC;
  static constexpr int QKT = (C / 2) * QKG;
  static constexpr int QKR = (QKT + NT - 1) / NT;
  static constexpr int VG = P / VEC;
  static constexpr int VT = (C / 2) * VG;
  static constexpr int VR = (VT + NT - 1) / NT;
  static constexpr int SV = N * P / VEC;           // 16-byte pieces of a chunk state
  static constexpr int SR = (SV + NT - 1) / NT;
  static constexpr int SZ_Q = C * LDQ * 2;
  static constexpr int SZ_G = C * LDP * 2;
  static constexpr int SZ_ST = N * LDP * 2;
  static constexpr int SZ_X = 2 * SZ_Q + 2 * SZ_G + SZ_ST;     // sQ sK sG sV sST
  static constexpr int SZ_STAGE = 2 * C * LDF * 4;            // dq~, dkhat f32
  static constexpr int SZ_R = cmax(SZ_X, SZ_STAGE);
  static constexpr int SZ_GAT = N * LDP * 2;                  // G^T [n][p]
  static constexpr int SZ_SC = (8 * C + 4 * N + 16) * 4;
  static constexpr int LDS_BYTES = SZ_R + SZ_GAT + SZ_SC;
  static_assert(N % 64 == 0 && P % 16 == 0 && C % 64 == 0, "tile shape");
  static_assert(T4 % NW == 0 && NW % PB == 0, "adjoint tiles split evenly, one pb per wave");
  static_assert(QKG <= 64 && VG <= 64, "row groups must fit a wave");
  static_assert(LDS_BYTES <= 163840, "LDS budget of one gfx950 CU");
  static_assert(C <= N, "the dv rows are staged in the adjoint's N-row slot");
};

template <int C, int N, int P, bool STRIPS>
__global__ void __launch_bounds__(C / 16 * 64) bwd_bf16_kernel(const BwdParams p) {
  using F = Bwd2Cfg<C, N, P>;
  // the in-strip angle prefix (angles_to_turns) shuffles over the 8 row pairs of a strip,
  // which must be lanes QKG apart in one wave
  static_assert(!STRIPS || 8 * F::QKG <= 64, "a strip's row pairs span more than one wave");
  using vec = bf16x8;
  constexpr int NW = F::NW, NT = F::NT, VEC = F::VEC, H2 = F::H2;
  constexpr int LDQ = F::LDQ, LDP = F::LDP, LDF = F::LDF;
  constexpr int PB = F::PB, NB = F::NB, CB = F::CB, SPW = F::SPW;

  // half of each XCD's workgroups start ~28 K cycles (about half of phase R plus the
  // staging) late: at B=8 L=8192 H=32 that took the backward from 1.667 to 1.614 ms
  if (p.nc >= 16) stagger_start(blockIdx.x, 2, 14);
  __shared__ __align__(16) unsigned char smem[F::LDS_BYTES];
  auto opq = [](int x) { asm volatile("" : "+s"(x)); return x; };
  bf16* sQ = reinterpret_cast<bf16*>(smem);                                        // q~ [t][n]
  bf16* sK = reinterpret_cast<bf16*>(smem + opq(F::SZ_Q));                         // khat [j][n]
  bf16* sG = reinterpret_cast<bf16*>(smem + opq(2 * F::SZ_Q));                     // g [t][p]
  bf16* sV = reinterpret_cast<bf16*>(smem + opq(2 * F::SZ_Q + F::SZ_G));           // v [t][p]
  bf16* sST = reinterpret_cast<bf16*>(smem + opq(2 * F::SZ_Q + 2 * F::SZ_G));      // S^T [n][p]
  float* sDQ = reinterpret_cast<float*>(smem);                 // staging, after the products
  float* sDK = reinterpret_cast<float*>(smem + opq(C * LDF * 4));
  bf16* sGaT = reinterpret_cast<bf16*>(smem + opq(F::SZ_R));                       // G^T [n][p]
  float* sA = reinterpret_cast<float*>(smem + opq(F::SZ_R + F::SZ_GAT));
  float* sExpA = sA + C;
  float* sFac = sExpA + C;
  float* sGam = sFac + C;
  float* sScl = sGam + C;
  float* sDqk = sScl + C;
  float* sCoef = sDqk + C;
  float* sDA = sCoef + C;
  float* sQb = sDA + C;
  float* sKb = sQb + N;
  // [w]: wave w's share of 2^{A_last}<G,S> + <v, dv_inter> for the current chunk, summed
  // in wave order (no float atomics: the result does not depend on wave timing)
  float* sRed = sKb + 3 * N;
  static_assert(NW <= 16, "one sRed slot per wave");
  // bias butterfly: BROUNDS rounds leave each lane the group sums of BFIN entries (below)
  constexpr int BFIN = VEC * 4 * F::QKG / 64;
  constexpr int BROUNDS = (F::QKG == 4) ? 4 : (F::QKG == 8) ? 3 : (F::QKG == 16) ? 2 : 1;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wid = xcd_remap(blockIdx.x, gridDim.x);
  const int b = wid / p.H, h = wid % p.H;
  const int64_t bh = (int64_t)b * p.H + h;
  const int L = p.L, Nr = p.Nr, nc = p.nc;

  for (int i = tid; i < N; i += NT) {
    sQb[i] = p.qb[h * N + i];
    sKb[i] = p.kb[h * N + i];
  }
  // this lane's running bias-gradient sums: the butterfly leaves a lane the same BFIN
  // entries in every row and chunk (its columns j0.. and `base` depend on lane bits only),
  // so they are summed in registers and reduced once, in a fixed order, at the end
  float bsum[BFIN];
#pragma unroll
  for (int k = 0; k < BFIN; ++k) bsum[k] = 0.f;
  const float dsk = p.has_d ? p.dsk[h] : 0.f;

  const bf16* qg = static_cast<const bf16*>(p.q) + (int64_t)b * L * N;
  const bf16* kg = static_cast<const bf16*>(p.k) + (int64_t)b * L * N;
  const bf16* vg = static_cast<const bf16*>(p.v) + b * p.v_sb + h * p.v_sh;
  const bf16* dyg = static_cast<const bf16*>(p.dy) + b * p.dy_sb + h * p.dy_sh;
  const bf16* zg = p.has_z ? static_cast<const bf16*>(p.z) + b * p.z_sb + h * p.z_sh : nullptr;
  bf16* dzg = p.has_z ? static_cast<bf16*>(p.dz) + b * p.dz_sb + h * p.dz_sh : nullptr;
  bf16* dvg = static_cast<bf16*>(p.dv) + b * p.dv_sb + h * p.dv_sh;
  const bf16* ybg = static_cast<const bf16*>(p.ybar) + bh * (int64_t)L * P;
  // phi rows of this (b, h), or (phi_strips mode) the head-shared tanh(angles) pi rows of
  // batch element b with the same addressing, plus dt and the strips' entering angles
  const float* phig = STRIPS ? p.tht + (int64_t)b * L * Nr : p.phi + bh * (int64_t)L * Nr;
  const float* pdtg = STRIPS ? p.pdt + bh * L : nullptr;
  const float* pstrg = STRIPS ? p.pstr + bh * (int64_t)(L / 16) * Nr : nullptr;
  const bf16* csg = static_cast<const bf16*>(p.cstates) + bh * (int64_t)nc * N * P;
  bf16* dug = static_cast<bf16*>(p.part) + bh * (int64_t)L * N;                 // du rows of (b, h)
  bf16* dwg = static_cast<bf16*>(p.part) + ((int64_t)p.B * p.H + bh) * L * N;   // dw rows of (b, h)
  const bool phi_vec = (Nr % 4) == 0;
  auto span = [&](int64_t st) { return (uint32_t)(((int64_t)(L - 1) * st + P) * 2); };
  // q, k, v, dy, phi, states and every output go through SGPR-base global accesses
  // (offsets stay below 2^32 bytes: the ABI's span checks); z and ybar keep buffer
  // descriptors so that a zero-size descriptor turns their loads into zeros without z.
  const auto rZ = make_rsrc(zg, zg ? span(p.z_st) : 0u);
  // without z, ybar is not read: a zero-size descriptor makes its (unconditional) loads
  // return zeros, as it does for z
  const auto rYb = make_rsrc(zg ? ybg : nullptr, zg ? (uint32_t)L * P * 2 : 0u);
  // phi[t][j .. j+3] for j < Nr. With Nr % 4 == 0 (wave-uniform) every lane issues one
  // 16-byte load: a per-lane choice of load width would make the compiler drain the load
  // queue at the join.
  auto phi_quad = [&](int t, int j, uint32_t sphi) {
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (phi_vec) {
      // quads past Nr load the chunk's first quad instead and are never read (every use
      // is under j < Nr): no select here, so the load need not complete in this block
      const bool ok = j + 4 <= Nr;
      v = gld<f32x4>(phig, sphi + (ok ? (uint32_t)(t * Nr + j) * 4 : 0u));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = (j + i < Nr) ? gld<float>(phig, sphi + (uint32_t)(t * Nr + j + i) * 4) : 0.f;
    }
    return v;
  };
  // the (B, H, L) scalar streams: a uniform row base plus a 32-bit offset (SGPR-base
  // global access), which keeps them out of the descriptor set
  const float* adt_r = p.adt + bh * L;
  const float* gam_r = p.gamma + bh * L;
  const float* scl_r = p.scale + bh * L;
  float* uw_r = p.uw + bh * L;
  float* dqk_r = p.dqk + bh * L;
  float* dsc_r = p.dscale + bh * L;
  float* dadt_r = p.dadt + bh * L;
  float* dphig = p.dphi ? p.dphi + bh * (int64_t)L * Nr : nullptr;

  // ---- adjoint G (registers, MFMA layout [p][n]); wave owns (pb_w, nb0 + NSTEP m) --
  constexpr int NSTEP = NW / PB;
  const int pb_w = wave % PB, nb0 = wave / PB;
  f32x4 Gacc[SPW];
#pragma unroll
  for (int m = 0; m < SPW; ++m) {
    Gacc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (p.dfs) {
      const int nb = nb0 + NSTEP * m;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        Gacc[m][i] = p.dfs[(bh * P + pb_w * 16 + 4 * (lane >> 4) + i) * N + nb * 16 + (lane & 15)];
    }
  }
  auto publish_adjoint = [&]() {
#pragma unroll
    for (int m = 0; m < SPW; ++m) {
      const int nb = nb0 + NSTEP * m;
      *reinterpret_cast<bf16x4*>(sGaT + (nb * 16 + (lane & 15)) * LDP + pb_w * 16 + 4 * (lane >> 4)) =
          sub_from_f32<bf16>(Gacc[m]);
    }
  };
  publish_adjoint();

  // ---- register prefetch of one chunk's raw inputs, in two parts -------------------
  vec rq[F::QKR][2][2], rk[F::QKR][2][2];
  f32x4 rphi[F::QKR][2][VEC / 4];   // phi (or the tanh(angles) pi rows), then turns
  float rpdt[F::QKR][2];             // phi_strips mode: dt of the two rows
  f32x4 rstr[STRIPS ? F::QKR : 1][VEC / 4];   // phi_strips mode: the strip's entering angles
  float rscale[F::QKR][2];
  vec rv[F::VR][2], rdy[F::VR][2], rz[F::VR][2], ryb[F::VR][2];
  vec rs[F::SR];
  float radt[F::E], rgam_s, rscl_s;

  auto prefetch_qk = [&](int c) {
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
    const int tid = ln;
    const uint32_t sqk = (uint32_t)c * C * N * 2, sphi = (uint32_t)c * C * Nr * 4;
#pragma unroll
    for (int r = 0; r < F::QKR; ++r) {
      const int task = tid + r * NT;
      if ((F::QKT % NT == 0 || task < F::QKT)) {
        const int tp = task / F::QKG, j0 = (task % F::QKG) * VEC;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int t = 2 * tp + e;
          const uint32_t o = (uint32_t)(t * N + j0) * 2;
          rq[r][e][0] = gld<vec>(qg, sqk + o);
          rq[r][e][1] = gld<vec>(qg, sqk + o + 2 * H2);
          rk[r][e][0] = gld<vec>(kg, sqk + o);
          rk[r][e][1] = gld<vec>(kg, sqk + o + 2 * H2);
#pragma unroll
          for (int qd = 0; qd < VEC / 4; ++qd)
            rphi[r][e][qd] = phi_quad(t, j0 + 4 * qd, sphi);
          rscale[r][e] = scl_r[(uint32_t)(c * C + t)];
          if constexpr (STRIPS) rpdt[r][e] = pdtg[(uint32_t)(c * C + t)];
        }
        if constexpr (STRIPS) {
          // both rows of the pair lie in strip (c C + 2 tp) / 16
          const uint32_t so = (uint32_t)((c * C + 2 * tp) >> 4) * Nr;
#pragma unroll
          for (int qd = 0; qd < VEC / 4; ++qd) {
            const int j = j0 + 4 * qd;
            if (phi_vec) {
              rstr[r][qd] = gld<f32x4>(pstrg, (so + (j + 4 <= Nr ? (uint32_t)j : 0u)) * 4);
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i)
                rstr[r][qd][i] = (j + i < Nr) ? gld<float>(pstrg, (so + j + i) * 4) : 0.f;
            }
          }
        }
      }
    }
  };
  // rphi -> the rows' angles in turns, in place, once the loads have landed. phi mode:
  // phi / (2 pi) (phi is wrapped). phi_strips mode: the strip's entering angle plus the
  // inclusive prefix of theta = table * dt over the strip's rows; a lane holds two rows
  // (a row pair), and the strip's eight row pairs are the lanes QKG apart that share
  // j0, so the exclusive part is a shuffle scan over those lanes. Quads past Nr (never
  // used) hold junk.
  auto angles_to_turns = [&]() {
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
    const int lane = ln & 63;
    const int pos = (lane / F::QKG) & 7;   // row pair within the strip
#pragma unroll
    for (int r = 0; r < F::QKR; ++r) {
#pragma unroll
      for (int qd = 0; qd < VEC / 4; ++qd) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (STRIPS) {
            const float t0v = rphi[r][0][qd][i] * rpdt[r][0];
            const float t1v = rphi[r][1][qd][i] * rpdt[r][1];
            float incl = t0v + t1v;
#pragma unroll
            for (int k = 1; k < 8; k <<= 1) {
              const float o = __shfl_up(incl, k * F::QKG, 64);
              incl += (pos >= k) ? o : 0.f;
            }
            const float before = rstr[r][qd][i] + (incl - (t0v + t1v));
            rphi[r][0][qd][i] = __builtin_amdgcn_fractf((before + t0v) * 0.15915494309189535f);
            rphi[r][1][qd][i] = __builtin_amdgcn_fractf((before + t0v + t1v) * 0.15915494309189535f);
          } else {
            rphi[r][0][qd][i] *= 0.15915494309189535f;
            rphi[r][1][qd][i] *= 0.15915494309189535f;
          }
        }
      }
    }
  };
  // part 1: v, dy, z rows; part 2: ybar rows, the state and the row scalars
  auto prefetch_rest = [&](int c, int part) {
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
    const int tid = ln, lane = ln & 63;
#pragma unroll
    for (int r = 0; r < F::VR; ++r) {
      const int task = tid + r * NT;
      if ((F::VT % NT == 0 || task < F::VT)) {
        const int tp = task / F::VG, p0 = (task % F::VG) * VEC;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int t = 2 * tp + e;
          if (part & 1) {
            rv[r][e] = gld<vec>(vg, (uint32_t)(c * C * p.v_st * 2) + (uint32_t)(t * p.v_st + p0) * 2);
            rdy[r][e] = gld<vec>(dyg, (uint32_t)(c * C * p.dy_st * 2) + (uint32_t)(t * p.dy_st + p0) * 2);
            rz[r][e] = buf_load<vec>(rZ, (uint32_t)(t * p.z_st + p0) * 2, (uint32_t)(c * C * p.z_st * 2));
          }
          if (part & 2)
            ryb[r][e] = buf_load<vec>(rYb, (uint32_t)(t * P + p0) * 2, (uint32_t)c * C * P * 2);
        }
      }
    }
    if (!(part & 2)) return;
#pragma unroll
    for (int r = 0; r < F::SR; ++r) {
      const int f = tid + r * NT;
      if ((F::SV % NT == 0 || f < F::SV)) rs[r] = gld<vec>(csg, (uint32_t)c * N * P * 2 + (uint32_t)f * VEC * 2);
    }
    if (wave == 0) {
#pragma unroll
      for (int e = 0; e < F::E; ++e)
        radt[e] = adt_r[(uint32_t)(c * C + lane * F::E + e)];
    }
    if (tid < C) {
      rgam_s = gam_r[(uint32_t)(c * C + tid)];
      rscl_s = scl_r[(uint32_t)(c * C + tid)];
    }
  };

  prefetch_qk(nc - 1);
  prefetch_rest(nc - 1, 3);
  __syncthreads();

  for (int c = nc - 1; c >= 0; --c) {
    const int t0 = c * C;
    // ============ phase L: raw -> LDS (q~, khat, g, v, S^T), dz, dqk, uw ==============
    // This chunk's raw rows were prefetched during the previous iteration's pullback and
    // tail, v/dy/z first and q/k/phi/scale last; they are consumed in that order.
    {
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int tid = ln, lane = ln & 63;
      if (wave == 0) {
        float a[F::E];
        float run = 0.f;
#pragma unroll
        for (int e = 0; e < F::E; ++e) {
          run += radt[e] * kLog2e;
          a[e] = run;
        }
        float incl = run;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const float o = __shfl_up(incl, off, 64);
          if (lane >= off) incl += o;
        }
        const float excl = incl - run;
        const float a_last = __shfl(incl, 63, 64);
#pragma unroll
        for (int e = 0; e < F::E; ++e) {
          const int tt = lane * F::E + e;
          const float A = excl + a[e];
          sA[tt] = A;
          sExpA[tt] = exp2f(A);
          sFac[tt] = exp2f(a_last - A);
        }
      }
      if (tid < C) {
        sGam[tid] = rgam_s;
        sScl[tid] = rscl_s;
      }
#pragma unroll
      for (int r = 0; r < F::VR; ++r) {
        const int task = tid + r * NT;
        const bool valid = (F::VT % NT == 0 || task < F::VT);
        const int tp = valid ? task / F::VG : 0, p0 = valid ? (task % F::VG) * VEC : 0;
        float dqk[2] = {0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int t = 2 * tp + e;
          __builtin_amdgcn_sched_barrier(0);
          if (valid) {
            vec og, odz;
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
              const float dy = (float)rdy[r][e][i];
              float gv = dy;
              if (zg) {
                const float zf = (float)rz[r][e][i];
                const float sg = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-zf * kLog2e));
                gv = dy * (zf * sg);
                odz[i] = (bf16)(dy * (float)ryb[r][e][i] * sg * (1.f + zf * (1.f - sg)));
              }
              dqk[e] += gv * (float)rv[r][e][i];
              og[i] = (bf16)gv;
            }
            *reinterpret_cast<vec*>(sG + t * LDP + p0) = og;
            *reinterpret_cast<vec*>(sV + t * LDP + p0) = rv[r][e];
            if (dzg) gst<vec>(dzg, (uint32_t)(t0 * p.dz_st * 2) + (uint32_t)(t * p.dz_st + p0) * 2, odz);
          }
        }
        dqk[0] = group_sum<F::VG>(dqk[0]);
        dqk[1] = group_sum<F::VG>(dqk[1]);
        if (valid && p0 == 0) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int t = 2 * tp + e;
            sDqk[t] = dqk[e];
            dqk_r[(uint32_t)(t0 + t)] = dqk[e];
          }
        }
      }
#pragma unroll
      for (int r = 0; r < F::SR; ++r) {
        const int f = tid + r * NT;
        if ((F::SV % NT == 0 || f < F::SV)) {
          const int n = (f * VEC) / P, pp = (f * VEC) % P;
          *reinterpret_cast<vec*>(sST + n * LDP + pp) = rs[r];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      angles_to_turns();
#pragma unroll
      for (int r = 0; r < F::QKR; ++r) {
        const int task = tid + r * NT;
        const bool valid = (F::QKT % NT == 0 || task < F::QKT);
        const int tp = valid ? task / F::QKG : 0, j0 = valid ? (task % F::QKG) * VEC : 0;
        float uw[2] = {0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int t = 2 * tp + e;
          __builtin_amdgcn_sched_barrier(0);   // rows one after the other: fewer live values
          if (valid) {
            vec oq0, oq1, ok0, ok1;
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
              const int j = j0 + i;
              const float ulo = (float)rq[r][e][0][i] + sQb[j];
              const float uhi = (float)rq[r][e][1][i] + sQb[H2 + j];
              const float wlo = (float)rk[r][e][0][i] + sKb[j];
              const float whi = (float)rk[r][e][1][i] + sKb[H2 + j];
              uw[e] += ulo * wlo + uhi * whi;
              // phi in [0, 2 pi): hardware sin / cos, argument in turns; the identity past
              // Nr by select (no divergent branch: half of every wave's lanes rotate)
              const float turns = rphi[r][e][i / 4][i % 4];
              const float sn = (j < Nr) ? __builtin_amdgcn_sinf(turns) : 0.f;
              const float cs = (j < Nr) ? __builtin_amdgcn_cosf(turns) : 1.f;
              const float sc = rscale[r][e];
              oq0[i] = (bf16)(ulo * cs - uhi * sn);
              oq1[i] = (bf16)(uhi * cs + ulo * sn);
              ok0[i] = (bf16)((wlo * cs - whi * sn) * sc);
              ok1[i] = (bf16)((whi * cs + wlo * sn) * sc);
            }
            *reinterpret_cast<vec*>(sQ + t * LDQ + j0) = oq0;
            *reinterpret_cast<vec*>(sQ + t * LDQ + H2 + j0) = oq1;
            *reinterpret_cast<vec*>(sK + t * LDQ + j0) = ok0;
            *reinterpret_cast<vec*>(sK + t * LDQ + H2 + j0) = ok1;
          }
        }
        uw[0] = group_sum<F::QKG>(uw[0]);
        uw[1] = group_sum<F::QKG>(uw[1]);
        if (valid && j0 == 0) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int t = 2 * tp + e;
            uw_r[(uint32_t)(t0 + t)] = uw[e];
            sCoef[t] = gam_r[(uint32_t)(t0 + t)] * uw[e] + dsk;
          }
        }
      }
    }
    __syncthreads();

    // ============ products: score tiles consumed as they are built ===================
    f32x4 dQ[NB], dKh[NB], dV[PB];
    bf16x4 dvo[PB];   // this wave's dv rows (MFMA layout), stored through LDS after the barrier
    {
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int lane = ln & 63, g4 = lane >> 4, l16 = lane & 15;
      const int w = wave;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        dQ[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        dKh[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int i = 0; i < PB; ++i) dV[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      float red = 0.f;
      const int jcol = w * 16 + l16;     // this lane's key position (cols of W, dM)
      const float Aj = sA[jcol];
      // W[t][j] and dM[t][j] for query strip tb (rows t) and key strip w (cols j)
      auto wdm = [&](int tb, bf16x4& wt, bf16x4& mt) {
        if (tb < w) {
          wt = sub_from_f32<bf16>(f32x4{0.f, 0.f, 0.f, 0.f});
          mt = wt;
          return;
        }
        f32x4 aw = {0.f, 0.f, 0.f, 0.f}, am = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = 0; k0 < N; k0 += 32)
          mma32x(aw, ld_nat8(sQ, LDQ, tb * 16, k0, lane), ld_nat8(sK, LDQ, w * 16, k0, lane));
#pragma unroll
        for (int k0 = 0; k0 < P; k0 += 32)
          mma32x(am, ld_nat8(sG, LDP, tb * 16, k0, lane), ld_nat8(sV, LDP, w * 16, k0, lane));
        // branch-free mask: 2^{min(A_t - A_j, 0)} is finite for every entry
        const f32x4 at = *reinterpret_cast<const f32x4*>(sA + tb * 16 + 4 * g4);
        f32x4 vw, vm;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = tb * 16 + 4 * g4 + i;
          const float e = __builtin_amdgcn_exp2f(fminf(at[i] - Aj, 0.f));
          const float dec = (t > jcol) ? e : 0.f;
          vw[i] = aw[i] * dec;
          vm[i] = am[i] * dec;
        }
        wt = sub_from_f32<bf16>(vw);
        mt = sub_from_f32<bf16>(vm);
      };
      // dv[j][p] += sum_t W[t][j] g[t][p];  dkhat[j][n] += sum_t dM[t][j] q~[t][n]
      for (int tb = w & ~1; tb < CB; tb += 2) {
        __builtin_amdgcn_sched_barrier(0);
        bf16x4 w0, m0, w1, m1;
        wdm(tb, w0, m0);
        wdm(tb + 1, w1, m1);
        const int kb = tb * 16 + 4 * g4;
#pragma unroll
        for (int pb = 0; pb < PB; ++pb)
          mma32(dV[pb], w0, w1, ld_tr4(sG, LDP, kb, pb * 16, lane), ld_tr4(sG, LDP, kb + 16, pb * 16, lane));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          mma32(dKh[nb], m0, m1, ld_tr4(sQ, LDQ, kb, nb * 16, lane), ld_tr4(sQ, LDQ, kb + 16, nb * 16, lane));
      }
      // dq~[t][n] += sum_j dM^T[j][t] khat[j][n]   (query strip w, key strips jb <= w)
      const int tcol = w * 16 + l16;
      const float At = sA[tcol];
      auto dmt = [&](int jb) {
        if (jb > w) return sub_from_f32<bf16>(f32x4{0.f, 0.f, 0.f, 0.f});
        f32x4 am = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = 0; k0 < P; k0 += 32)
          mma32x(am, ld_nat8(sV, LDP, jb * 16, k0, lane), ld_nat8(sG, LDP, w * 16, k0, lane));
        const f32x4 aj = *reinterpret_cast<const f32x4*>(sA + jb * 16 + 4 * g4);
        f32x4 vm;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = jb * 16 + 4 * g4 + i;
          const float e = __builtin_amdgcn_exp2f(fminf(At - aj[i], 0.f));
          vm[i] = (tcol > j) ? am[i] * e : 0.f;
        }
        return sub_from_f32<bf16>(vm);
      };
      for (int jb = 0; jb <= w; jb += 2) {
        __builtin_amdgcn_sched_barrier(0);
        const bf16x4 d0 = dmt(jb), d1 = dmt(jb + 1);
        const int kb = jb * 16 + 4 * g4;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          mma32(dQ[nb], d0, d1, ld_tr4(sK, LDQ, kb, nb * 16, lane), ld_tr4(sK, LDQ, kb + 16, nb * 16, lane));
      }
      // dq~ inter: 2^{A_t} sum_p g[t][p] S[p][n];  dkhat inter: 2^{A_last-A_j} sum_p v[j][p] G[p][n]
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        f32x4 iq = {0.f, 0.f, 0.f, 0.f}, ik = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = 0; k0 < P; k0 += 32) {
          mma32x(iq, ld_nat8(sG, LDP, w * 16, k0, lane), ld_nat8(sST, LDP, nb * 16, k0, lane));
          mma32x(ik, ld_nat8(sV, LDP, w * 16, k0, lane), ld_nat8(sGaT, LDP, nb * 16, k0, lane));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = w * 16 + 4 * g4 + i;
          dQ[nb][i] += iq[i] * sExpA[r];
          dKh[nb][i] += ik[i] * sFac[r];
        }
      }
      // dv inter: 2^{A_last-A_j} sum_n khat[j][n] G[p][n]   (G^T read by columns)
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        f32x4 iv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = 0; k0 < N; k0 += 32) {
          const int kb = k0 + 4 * g4;
          mma32(iv, ld_sub<bf16>(sK, LDQ, w * 16, k0), ld_sub<bf16>(sK, LDQ, w * 16, k0 + 16),
                ld_tr4(sGaT, LDP, kb, pb * 16, lane), ld_tr4(sGaT, LDP, kb + 16, pb * 16, lane));
        }
        const bf16x4 vj = ld_tr4(sV, LDP, w * 16 + 4 * g4, pb * 16, lane);   // v[j][p]
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = w * 16 + 4 * g4 + i;
          iv[i] *= sFac[j];
          dV[pb][i] += iv[i];
          // <v, dv_inter> == <khat, dk_inter>: the A_last share of the state update
          red += (float)vj[i] * iv[i];
        }
      }
      // 2^{A_last} <G, S> from this wave's adjoint tiles (before the G update)
      {
        float gs = 0.f;
#pragma unroll
        for (int m = 0; m < SPW; ++m) {
          const int nb = nb0 + NSTEP * m;
          const f32x4 sv = sub_to_f32<bf16>(
              *reinterpret_cast<const bf16x4*>(sST + (nb * 16 + l16) * LDP + pb_w * 16 + 4 * g4));
#pragma unroll
          for (int i = 0; i < 4; ++i) gs += Gacc[m][i] * sv[i];
        }
        red += sExpA[C - 1] * gs;
      }
      red = wave_total(red);
      if (lane == 0) sRed[wave] = red;
      // G <- 2^{A_last} G + sum_t (2^{A_t} g[t][p]) q~[t][n]   (K = time, both by columns)
      const float eAl = sExpA[C - 1];
#pragma unroll
      for (int m = 0; m < SPW; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) Gacc[m][i] *= eAl;
      }
#pragma unroll 1
      for (int k0 = 0; k0 < C; k0 += 32) {
        const int kb = k0 + 4 * g4;
        bf16x4 a0 = ld_tr4(sG, LDP, kb, pb_w * 16, lane);
        bf16x4 a1 = ld_tr4(sG, LDP, kb + 16, pb_w * 16, lane);
        const f32x4 e0 = *reinterpret_cast<const f32x4*>(sExpA + kb);
        const f32x4 e1 = *reinterpret_cast<const f32x4*>(sExpA + kb + 16);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          a0[s] = (bf16)((float)a0[s] * e0[s]);
          a1[s] = (bf16)((float)a1[s] * e1[s]);
        }
#pragma unroll
        for (int m = 0; m < SPW; ++m) {
          const int nb = nb0 + NSTEP * m;
          mma32(Gacc[m], a0, a1, ld_tr4(sQ, LDQ, kb, nb * 16, lane), ld_tr4(sQ, LDQ, kb + 16, nb * 16, lane));
        }
      }
      // dv epilogue: + (D + gamma u.w) g, + dfinal_v on the sequence's last row
      const bool last_chunk = p.dfv && c == nc - 1;
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        const int pcol = pb * 16 + l16;
        const f32x4 gv = sub_to_f32<bf16>(ld_tr4(sG, LDP, w * 16 + 4 * g4, pb * 16, lane));
        const f32x4 cf = *reinterpret_cast<const f32x4*>(sCoef + w * 16 + 4 * g4);
        f32x4 d;
#pragma unroll
        for (int i = 0; i < 4; ++i) d[i] = dV[pb][i] + cf[i] * gv[i];
        if (last_chunk && w * 16 + 4 * g4 + 3 == C - 1) d[3] += p.dfv[bh * P + pcol];
        dvo[pb] = sub_from_f32<bf16>(d);
      }
    }
    __syncthreads();

    // ============ stage dq~ [t][n] and dkhat [j][n] as f32 rows =======================
    {
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int lane = ln & 63, g4 = lane >> 4, l16 = lane & 15;
      const int w = wave;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = w * 16 + 4 * g4 + i;
          sDQ[r * LDF + nb * 16 + l16] = dQ[nb][i];
          sDK[r * LDF + nb * 16 + l16] = dKh[nb][i];
        }
      }
      // dv rows into the adjoint's LDS slot (free until the tail republishes G), [j][p]
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sGaT[(w * 16 + 4 * g4 + i) * LDP + pb * 16 + l16] = dvo[pb][i];
      }
    }
    prefetch_qk(c);   // phase R's raw q, k, phi rows: their latency overlaps the barrier
    __syncthreads();

    // dv: whole 16-byte row pieces from LDS, coalesced stores
    {
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int tid = ln;
      constexpr int VGP = P / VEC, DVR = (C * VGP + NT - 1) / NT;
#pragma unroll
      for (int r = 0; r < DVR; ++r) {
        const int f = tid + r * NT;
        if ((C * VGP) % NT == 0 || f < C * VGP) {
          const int j = f / VGP, p0 = (f % VGP) * VEC;
          gst<vec>(dvg, (uint32_t)(t0 * p.dv_st * 2) + (uint32_t)(j * p.dv_st + p0) * 2,
                   *reinterpret_cast<const vec*>(sGaT + j * LDP + p0));
        }
      }
    }

    // ============ phase R: rotation pullback, per-row reductions, head sum ============
    {
      angles_to_turns();
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int tid = ln, lane = ln & 63;
      const uint32_t sqk = (uint32_t)t0 * N * 2, sphi = (uint32_t)t0 * Nr * 4;
#pragma unroll
      for (int r = 0; r < F::QKR; ++r) {
        const int task = tid + r * NT;
        const bool valid = (F::QKT % NT == 0 || task < F::QKT);
        // j0 depends on the lane alone (NT % QKG == 0), also for idle lanes: the bias
        // reduction below pairs lanes that share it
        const int tp = valid ? task / F::QKG : 0, j0 = (task % F::QKG) * VEC;
        // bias partials of this lane's two rows: [element][du lo, du hi, dw lo, dw hi]
        float bacc[VEC * 4];
#pragma unroll
        for (int k = 0; k < VEC * 4; ++k) bacc[k] = 0.f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          __builtin_amdgcn_sched_barrier(0);   // rows one after the other: fewer live values
          // dA = sum(q~ . dq~) - sc * sum(k~ . dk^) over the row; dsc is the second sum
          float dqq = 0.f, dsc = 0.f;
          if (valid) {
            const int t = 2 * tp + e;
            const uint32_t o = (uint32_t)(t * N + j0) * 2;
            const vec q0 = rq[r][e][0], q1 = rq[r][e][1];
            const vec k0 = rk[r][e][0], k1 = rk[r][e][1];
            float ph[VEC];
#pragma unroll
            for (int qd = 0; qd < VEC / 4; ++qd) {
#pragma unroll
              for (int i = 0; i < 4; ++i) ph[4 * qd + i] = rphi[r][e][qd][i];
            }
            const float sc = sScl[t];
            const float cd = sDqk[t] * sGam[t];
            vec du0, du1, dw0, dw1;
            float dphv[VEC], kfl[VEC], kfh[VEC];
            f32x4 dql[VEC / 4], dqh[VEC / 4], dkl[VEC / 4], dkh[VEC / 4];   // 16-byte LDS reads
#pragma unroll
            for (int h4 = 0; h4 < VEC / 4; ++h4) {
              dql[h4] = *reinterpret_cast<const f32x4*>(sDQ + t * LDF + j0 + 4 * h4);
              dqh[h4] = *reinterpret_cast<const f32x4*>(sDQ + t * LDF + H2 + j0 + 4 * h4);
              dkl[h4] = *reinterpret_cast<const f32x4*>(sDK + t * LDF + j0 + 4 * h4);
              dkh[h4] = *reinterpret_cast<const f32x4*>(sDK + t * LDF + H2 + j0 + 4 * h4);
            }
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
              const int j = j0 + i;
              const float ulo = (float)q0[i] + sQb[j];
              const float uhi = (float)q1[i] + sQb[H2 + j];
              const float wlo = (float)k0[i] + sKb[j];
              const float whi = (float)k1[i] + sKb[H2 + j];
              const float turns = ph[i];
              const float sn = (j < Nr) ? __builtin_amdgcn_sinf(turns) : 0.f;
              const float cs = (j < Nr) ? __builtin_amdgcn_cosf(turns) : 1.f;
              const float qlo = ulo * cs - uhi * sn, qhi = uhi * cs + ulo * sn;
              const float klo = wlo * cs - whi * sn, khi = whi * cs + wlo * sn;
              const float dqlo = dql[i / 4][i % 4], dqhi = dqh[i / 4][i % 4];
              const float dklo = dkl[i / 4][i % 4], dkhi = dkh[i / 4][i % 4];
              dqq += qlo * dqlo + qhi * dqhi;
              dsc += dklo * klo + dkhi * khi;
              const float dtlo = dklo * sc, dthi = dkhi * sc;   // d k~
              // R^T = R(-phi): lo' = lo cos + hi sin, hi' = hi cos - lo sin
              const float dulo = dqlo * cs + dqhi * sn + cd * wlo;
              const float duhi = dqhi * cs - dqlo * sn + cd * whi;
              const float dwlo = dtlo * cs + dthi * sn + cd * ulo;
              const float dwhi = dthi * cs - dtlo * sn + cd * uhi;
              dphv[i] = (dqhi * qlo - dqlo * qhi) + (dthi * klo - dtlo * khi);
              kfl[i] = klo;
              kfh[i] = khi;
              du0[i] = dulo;
              du1[i] = duhi;
              dw0[i] = dwlo;
              dw1[i] = dwhi;
              bacc[4 * i + 0] += dulo;
              bacc[4 * i + 1] += duhi;
              bacc[4 * i + 2] += dwlo;
              bacc[4 * i + 3] += dwhi;
            }
            if (c == nc - 1 && t == C - 1) {   // the sequence's last k~ row (f32)
#pragma unroll
              for (int h4 = 0; h4 < VEC / 4; ++h4) {
                gst<f32x4>(p.kfin + bh * N, (uint32_t)(j0 + 4 * h4) * 4,
                           f32x4{kfl[4 * h4], kfl[4 * h4 + 1], kfl[4 * h4 + 2], kfl[4 * h4 + 3]});
                gst<f32x4>(p.kfin + bh * N, (uint32_t)(H2 + j0 + 4 * h4) * 4,
                           f32x4{kfh[4 * h4], kfh[4 * h4 + 1], kfh[4 * h4 + 2], kfh[4 * h4 + 3]});
              }
            }
            if (p.dphi) {
#pragma unroll
              for (int qd = 0; qd < VEC / 4; ++qd) {
                const int j = j0 + 4 * qd;
                const uint32_t op = (uint32_t)(t * Nr + j) * 4;
                if (phi_vec && j + 4 <= Nr) {
                  gst<f32x4>(dphig, sphi + op,
                             f32x4{dphv[4 * qd], dphv[4 * qd + 1], dphv[4 * qd + 2], dphv[4 * qd + 3]});
                } else {
#pragma unroll
                  for (int i = 0; i < 4; ++i)
                    if (j + i < Nr) gst<float>(dphig, sphi + op + 4 * i, dphv[4 * qd + i]);
                }
              }
            }
            // this head's du / dw row pieces; the head sum happens in headsum_kernel. Stored
            // non-temporally: 1.07 GB at cfg3 that only the head sum reads back, streamed past
            // the caches the scan's own operands use (0.5-1% faster than plain stores)
            auto nts = [&](bf16* base, uint32_t off, vec x) {
              __builtin_nontemporal_store(x, reinterpret_cast<vec*>(reinterpret_cast<char*>(base) + off));
            };
            nts(dug, sqk + o, du0);
            nts(dug, sqk + o + 2 * H2, du1);
            nts(dwg, sqk + o, dw0);
            nts(dwg, sqk + o + 2 * H2, dw1);
          }
          dqq = group_sum<F::QKG>(dqq);
          dsc = group_sum<F::QKG>(dsc);
          if (valid && j0 == 0) {
            sDA[2 * tp + e] = dqq - sScl[2 * tp + e] * dsc;
            dsc_r[(uint32_t)(t0 + 2 * tp + e)] = dsc;
          }
          // The previous chunk's v, dy and z rows, for its phase L, into registers this
          // row has freed: the loads overlap the second row's arithmetic. Issued on every
          // iteration (chunk 0 reloads itself on the last one): a conditional prefetch
          // would keep the consumed registers alive through the whole loop body for the
          // skipped path. The rest follows the bias butterfly.
          if (r == F::QKR - 1 && e == 0) prefetch_rest(c > 0 ? c - 1 : 0, 1);
        }
        // The lanes that share j0 differ in lane bits log2(QKG)..5. A transposing
        // butterfly over those bits halves the entries a lane keeps each round (it sends
        // the half its partner keeps), so each lane ends with the group sums of
        // BFIN consecutive entries (which ones: the epilogue recomputes it from the lane
        // bits), added to its running sums.
        static_assert((VEC * 4) >> BROUNDS == BFIN && BFIN >= 1, "bias butterfly shape");
#pragma unroll
        for (int rd = 0; rd < BROUNDS; ++rd) {
          const int m = 32 >> rd, half = (VEC * 2) >> rd;
          const bool up = (lane & m) != 0;
#pragma unroll
          for (int k = 0; k < half; ++k) {
            const float lo = bacc[k], hi = bacc[half + k];   // values, not addresses, selected
            const float send = up ? lo : hi;
            const float keep = up ? hi : lo;
            bacc[k] = keep + __shfl_xor(send, m, 64);
          }
        }
        // the previous chunk's ybar rows, state and row scalars, into registers the
        // butterfly has freed
        if (r == F::QKR - 1) prefetch_rest(c > 0 ? c - 1 : 0, 2);
#pragma unroll
        for (int k = 0; k < BFIN; ++k) bsum[k] += bacc[k];
      }
    }
    // the previous chunk's q, k, phi rows for its phase L, into the registers phase R
    // has just consumed: in flight during the barrier wait
    prefetch_qk(c > 0 ? c - 1 : 0);
    __syncthreads();

    // ============ phase S: dadt = suffix_sum(dA) + A_last share; publish G ============
    if (wave == 0) {
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int lane = ln & 63;
      float extra = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) extra += sRed[w];
      float a[F::E];
      float run = 0.f;
#pragma unroll
      for (int e = F::E - 1; e >= 0; --e) {
        run += sDA[lane * F::E + e];
        a[e] = run;
      }
      float incl = run;   // suffix scan across lanes: inclusive sum over lanes >= this one
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_down(incl, off, 64);
        if (lane + off < 64) incl += o;
      }
      const float excl = incl - run;
#pragma unroll
      for (int e = 0; e < F::E; ++e)
        dadt_r[(uint32_t)(t0 + lane * F::E + e)] = excl + a[e] + extra;
    }
    publish_adjoint();
    __syncthreads();
  }

  // ---- per-(b, h) outputs ------------------------------------------------------------
#pragma unroll
  for (int m = 0; m < SPW; ++m) {
    const int nb = nb0 + NSTEP * m;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      p.dseed[(bh * P + pb_w * 16 + 4 * (lane >> 4) + i) * N + nb * 16 + (lane & 15)] = Gacc[m][i];
  }
  // bias gradients: each wave's sums into its own LDS slot (the staging area is free
  // now; every entry is held by exactly one lane of each wave), then the slots summed in
  // wave order
  __syncthreads();
  {
    float* sBias = sDQ;   // [NW][2N]: q's N entries, then k's
    static_assert(NW * 2 * N * 4 <= F::SZ_STAGE, "bias slots fit the staging area");
    const int j0 = (tid % F::QKG) * VEC;
    int base = 0;
#pragma unroll
    for (int rd = 0; rd < BROUNDS; ++rd)   // the butterfly keeps the upper half on a set bit
      base += (lane & (32 >> rd)) ? ((VEC * 2) >> rd) : 0;
#pragma unroll
    for (int k = 0; k < BFIN; ++k) {
      const int idx = base + k, u = idx & 3;
      sBias[wave * 2 * N + (u >> 1) * N + (u & 1) * H2 + j0 + (idx >> 2)] = bsum[k];
    }
    __syncthreads();
    for (int i = tid; i < 2 * N; i += NT) {
      float acc = 0.f;
      for (int w = 0; w < NW; ++w) acc += sBias[w * 2 * N + i];
      if (i < N) p.dqb[bh * N + i] = acc;
      else p.dkb[bh * N + i - N] = acc;
    }
  }
}

// dq[b, t, :] = sum_h du[b, h, t, :] (and dk from dw): one thread per 8 consecutive
// elements of a (b, t) row (LN is a multiple of 8), summing over heads in f32, heads in
// order. Bandwidth-bound; the rows are read once, so the loads are non-temporal.
template <typename MT>
__global__ void __launch_bounds__(256) headsum_kernel(const MT* __restrict__ part,
                                                      float* __restrict__ dq,
                                                      float* __restrict__ dk, int B, int H,
                                                      int64_t LN) {
  const int64_t i8 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  const int which = blockIdx.y;           // 0: dq from du, 1: dk from dw
  const int b = blockIdx.z;
  if (i8 >= LN) return;
  const MT* src = part + ((int64_t)which * B + b) * H * LN + i8;
  f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
  for (int h = 0; h < H; ++h) {
    const sub_t<MT>* row = reinterpret_cast<const sub_t<MT>*>(src + h * LN);
    lo += sub_to_f32<MT>(__builtin_nontemporal_load(row));
    hi += sub_to_f32<MT>(__builtin_nontemporal_load(row + 1));
  }
  float* dst = (which ? dk : dq) + (int64_t)b * LN + i8;
  *reinterpret_cast<f32x4*>(dst) = lo;
  *reinterpret_cast<f32x4*>(dst + 4) = hi;
}

// Every per-(b, h) stream of bwd_bf16_kernel must be addressable with 31-bit byte
// offsets from its buffer descriptor.
static bool bwd_fits_rsrc(const BwdParams& p, int N, int P) {
  const int64_t lim = (int64_t(1) << 31) - 1;
  const int64_t L = p.L;
  auto span = [&](int64_t st) { return ((L - 1) * st + P) * 2; };
  return L * N * 2 <= lim && L * p.Nr * 4 <= lim && L * P * 4 <= lim && span(p.v_st) <= lim &&
         span(p.dy_st) <= lim && span(p.dv_st) <= lim &&
         (!p.has_z || (span(p.z_st) <= lim && span(p.dz_st) <= lim)) &&
         (int64_t)p.nc * N * P * 2 <= lim;
}

template <typename MT, int C, int N, int P>
static int32_t launch_bwd(const BwdParams& prm, int grid, hipStream_t stream) {
  bool done = false;
  const bool strips = prm.pstr != nullptr;
  if constexpr (std::is_same<MT, bf16>::value && N % 64 == 0 && C % 64 == 0 && C <= N &&
                N / 16 <= 8) {   // N <= 128: a strip's row pairs in one wave (phi strips)
    if (bwd_fits_rsrc(prm, N, P)) {
      if (strips)
        hipLaunchKernelGGL((bwd_bf16_kernel<C, N, P, true>), dim3(grid), dim3(C / 16 * 64), 0, stream, prm);
      else
        hipLaunchKernelGGL((bwd_bf16_kernel<C, N, P, false>), dim3(grid), dim3(C / 16 * 64), 0, stream, prm);
      done = true;
    }
  }
  if (!done) {
    constexpr int NW = (C / 16) > 4 ? (C / 16) : 4;
    if (strips)
      hipLaunchKernelGGL((bwd_kernel<MT, C, N, P, NW, true>), dim3(grid), dim3(NW * 64), 0, stream, prm);
    else
      hipLaunchKernelGGL((bwd_kernel<MT, C, N, P, NW, false>), dim3(grid), dim3(NW * 64), 0, stream, prm);
  }
  int32_t rc = launch_status("m3s_bwd");
  if (rc != M3S_OK) return rc;
  const int64_t LN = (int64_t)prm.L * N;
  static_assert(N % 8 == 0, "head sum threads take 8 elements");
  const dim3 hgrid((unsigned)((LN / 8 + 255) / 256), 2, prm.B);
  hipLaunchKernelGGL((headsum_kernel<MT>), hgrid, dim3(256), 0, stream,
                     static_cast<const MT*>(prm.part), prm.dq, prm.dk, prm.B, prm.H, LN);
  return launch_status("m3s_bwd (head sum)");
}

#define M3S_BWD_CONFIGS(X) \
  X(bf16, 128, 128, 64)    \
  X(bf16, 64, 128, 64)     \
  X(bf16, 32, 128, 64)     \
  X(bf16, 128, 64, 64)     \
  X(bf16, 64, 64, 64)      \
  X(bf16, 32, 64, 64)      \
  X(bf16, 128, 32, 16)     \
  X(bf16, 64, 32, 16)      \
  X(bf16, 32, 32, 16)      \
  X(bf16, 128, 16, 16)     \
  X(bf16, 64, 16, 16)      \
  X(bf16, 32, 16, 16)      \
  X(bf16, 32, 256, 64)     \
  X(float, 32, 128, 64)    \
  X(float, 64, 64, 64)     \
  X(float, 32, 64, 64)     \
  X(float, 128, 32, 16)    \
  X(float, 64, 32, 16)     \
  X(float, 32, 32, 16)     \
  X(float, 128, 16, 16)    \
  X(float, 64, 16, 16)     \
  X(float, 32, 16, 16)

template <typename MT> constexpr int bcode();
template <> constexpr int bcode<bf16>() { return M3S_DTYPE_BF16; }
template <> constexpr int bcode<float>() { return M3S_DTYPE_F32; }

int32_t bwd_supported(int dtype, int chunk, int n, int pdim) {
#define X(MT, C, N, P) \
  if (dtype == bcode<MT>() && chunk == C && n == N && pdim == P) return 1;
  M3S_BWD_CONFIGS(X)
#undef X
  return 0;
}

}  // namespace m3s

extern "C" int64_t m3s_bwd_workspace_bytes(int32_t dtype, int32_t batch, int32_t seqlen,
                                           int32_t nheads, int32_t state_dim) {
  const int64_t el = dtype == M3S_DTYPE_BF16 ? 2 : 4;
  return 2 * (int64_t)batch * nheads * seqlen * state_dim * el;
}

extern "C" int32_t m3s_bwd(const m3s_bwd_args* a, void* stream) {
  using namespace m3s;
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_bwd: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_bwd_args),
              "m3s_bwd: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_bwd_args));
  const int B = a->batch, L = a->seqlen, H = a->nheads, P = a->headdim, N = a->state_dim,
            Nr = a->n_angles, C = a->chunk;
  M3S_REQUIRE(B > 0 && L > 0 && H > 0 && P > 0 && N > 0 && C > 0,
              "m3s_bwd: non-positive dimension");
  M3S_REQUIRE(L % C == 0, "m3s_bwd: seqlen %d is not a multiple of chunk %d", L, C);
  M3S_REQUIRE(Nr >= 0 && 2 * Nr <= N, "m3s_bwd: n_angles %d exceeds state_dim/2", Nr);
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32, "m3s_bwd: bad dtype %d",
              a->dtype);
  if (!bwd_supported(a->dtype, C, N, P)) {
    set_error("m3s_bwd: no kernel for dtype=%s chunk=%d state_dim=%d headdim=%d",
              a->dtype == M3S_DTYPE_BF16 ? "bf16" : "f32", C, N, P);
    return M3S_ERR_UNSUPPORTED;
  }
  const int vec = a->dtype == M3S_DTYPE_BF16 ? 8 : 4;
  M3S_REQUIRE(bhlp_ok(a->dy, vec) && bhlp_ok(a->v, vec) && bhlp_ok(a->dv, vec),
              "m3s_bwd: dy/v/dv null, misaligned or strides not multiples of %d", vec);
  M3S_REQUIRE(!a->has_z || (bhlp_ok(a->z, vec) && bhlp_ok(a->dz, vec) && a->ybar &&
                            aligned16(a->ybar)),
              "m3s_bwd: has_z needs z, dz and an aligned ybar");
  M3S_REQUIRE(a->q && a->k && aligned16(a->q) && aligned16(a->k), "m3s_bwd: q/k null or misaligned");
  const bool strips = a->theta_table || a->phi_dt || a->phi_strips;
  M3S_REQUIRE(!strips || (a->theta_table && a->phi_dt && a->phi_strips && !a->phi),
              "m3s_bwd: give phi, or theta_table, phi_dt and phi_strips (not both)");
  M3S_REQUIRE(!strips || L % 16 == 0, "m3s_bwd: phi_strips needs seqlen %% 16 == 0");
  M3S_REQUIRE(a->adt && a->gamma && a->scale && (a->phi || strips) && a->q_bias && a->k_bias,
              "m3s_bwd: a required input pointer is NULL");
  M3S_REQUIRE(Nr == 0 || Nr % 4 != 0 ||
                  (strips ? aligned16(a->theta_table) && aligned16(a->phi_strips) : aligned16(a->phi)),
              "m3s_bwd: phi (or theta_table / phi_strips) misaligned");
  M3S_REQUIRE(a->chunk_states && aligned16(a->chunk_states), "m3s_bwd: chunk_states null or misaligned");
  M3S_REQUIRE(!a->has_d || a->d_skip, "m3s_bwd: has_d but d_skip is NULL");
  M3S_REQUIRE(a->dq && a->dk && aligned16(a->dq) && aligned16(a->dk) && a->dadt && a->dqk_diag &&
                  a->dscale && a->uw && a->dq_bias && a->dk_bias && a->k_final && a->dseed_ssm &&
                  (Nr == 0 || a->dphi) && a->workspace && aligned16(a->workspace),
              "m3s_bwd: an output or workspace pointer is NULL or misaligned");
  M3S_REQUIRE((int64_t)B * H < (1ll << 31), "m3s_bwd: B*H too large");

  BwdParams prm{};
  prm.B = B; prm.L = L; prm.H = H; prm.Nr = Nr; prm.nc = L / C;
  prm.has_d = a->has_d; prm.has_z = a->has_z;
  prm.dy = a->dy.ptr; prm.dy_sb = a->dy.stride_b; prm.dy_sh = a->dy.stride_h; prm.dy_st = a->dy.stride_t;
  prm.ybar = a->ybar;
  prm.z = a->has_z ? a->z.ptr : nullptr;
  prm.z_sb = a->z.stride_b; prm.z_sh = a->z.stride_h; prm.z_st = a->z.stride_t;
  prm.q = a->q; prm.k = a->k;
  prm.v = a->v.ptr; prm.v_sb = a->v.stride_b; prm.v_sh = a->v.stride_h; prm.v_st = a->v.stride_t;
  prm.adt = a->adt; prm.gamma = a->gamma; prm.scale = a->scale; prm.phi = a->phi;
  prm.tht = strips ? a->theta_table : nullptr;
  prm.pdt = strips ? a->phi_dt : nullptr;
  prm.pstr = strips ? a->phi_strips : nullptr;
  prm.qb = a->q_bias; prm.kb = a->k_bias; prm.dsk = a->d_skip;
  prm.cstates = a->chunk_states; prm.dfs = a->dfinal_ssm; prm.dfv = a->dfinal_v;
  prm.dq = a->dq; prm.dk = a->dk;
  prm.dv = a->dv.ptr; prm.dv_sb = a->dv.stride_b; prm.dv_sh = a->dv.stride_h; prm.dv_st = a->dv.stride_t;
  prm.dz = a->has_z ? a->dz.ptr : nullptr;
  prm.dz_sb = a->dz.stride_b; prm.dz_sh = a->dz.stride_h; prm.dz_st = a->dz.stride_t;
  prm.dadt = a->dadt; prm.dqk = a->dqk_diag; prm.dscale = a->dscale; prm.uw = a->uw;
  prm.dphi = a->dphi; prm.dqb = a->dq_bias; prm.dkb = a->dk_bias; prm.kfin = a->k_final;
  prm.dseed = a->dseed_ssm;
  prm.part = a->workspace;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid = B * H;
#define X(MT, CC, NN, PP)                                              \
  if (a->dtype == bcode<MT>() && C == CC && N == NN && P == PP)        \
    return launch_bwd<MT, CC, NN, PP>(prm, grid, s);
  M3S_BWD_CONFIGS(X)
#undef X
  set_error("m3s_bwd: unreachable dispatch");
  return M3S_ERR_UNSUPPORTED;
}
