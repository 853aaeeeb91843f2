// Chunked forward of the Mamba-3 SISO scan on gfx950 (MI355X).
//
// Replaces the reference's `_fwd_kernel` / `siso_forward` (kernel_fwd.py:55-388).
// Maths per chunk of C tokens, local log2-decay A_t = sum_{s<=t} adt_s * log2(e):
//
//   ybar = 2^A (q~ S^T) + tril_strict(q~ khat^T 2^{min(A_i - A_j, 0)}) v + (D + gamma u.w) v
//   y    = ybar * silu(z)
//   S   <- 2^{A_last} S + (v 2^{A_last - A})^T khat
//
// Design (one workgroup per (b, h), walking the chunks of that sequence in order):
//  * The carried state S (P x N, f32) lives in MFMA accumulator registers for the
//    whole sequence; it is never re-read from HBM. Each wave owns a fixed set of its
//    16x16 tiles.
//  * Per chunk the raw tiles (q, k, v, z, phi, scalars) are prefetched into registers
//    one chunk ahead, then bias + rotary + scale are applied on the way into LDS, so
//    q~/khat exist only as bf16 LDS tiles (no HBM round trip).
//  * Wave w owns query strip t in [16w, 16w+16): it builds the transposed, masked,
//    decay-weighted score strip s^T[j][t] with MFMA, keeps it in registers and feeds it
//    straight into the s.v product (an accumulator tile is already an operand
//    fragment with its row index as K -- see m3s_common.h), adds the inter-chunk term
//    2^A (q~ S^T), and stages the result through LDS so the epilogue (diagonal, skip,
//    gate, stores) runs on contiguous rows with 16-byte global accesses.
//  * XCD-aware block numbering keeps the H heads of one batch element (which share
//    q/k) on one XCD's L2.
#include <algorithm>
#include <type_traits>

#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

struct FwdParams {
  int B, L, H, Nr, nc;
  int has_d, has_z, has_seed, save;
  const void* q;
  const void* k;
  const void* v;
  int64_t v_sb, v_sh, v_st;
  const void* z;
  int64_t z_sb, z_sh, z_st;
  const float* adt;
  const float* gamma;
  const float* scale;
  const float* phi;
  const float* tht;    // phi_strips mode: tanh(angles) pi (B, L, Nr), dt (B, H, L),
  const float* pdt;    // phi entering each 16-token strip (B, H, L / 16, Nr); else NULL
  const float* pstr;
  const float* qb;
  const float* kb;
  const float* dsk;
  const float* seed_ssm;
  const float* seed_k;
  const float* seed_v;
  const float* seed_coef;
  void* y;
  int64_t y_sb, y_sh, y_st;
  void* ybar;     // (B, H, L, P) in the matmul dtype
  void* cstates;
  float* fssm;
  float* fk;
  float* fv;
  // raw mode: the dt slice of the projection (the a and trap slices a_off / t_off
  // elements after it in each row; sc_span = max(a_off, t_off) + 1), its b / t strides,
  // the head biases, each strip's theta prefix within its chunk (B, H, L / 16, Nr) and
  // the chunk totals (B, H, nc, Nr), phi_init (or NULL) and the phi_final output
  const void* sc;
  int64_t sc_sb, sc_st;
  int a_off, t_off, sc_span;
  float a_floor;
  const float* dt_bias;
  const float* tpre;
  const float* ctot;
  const float* phi_init;
  float* phi_final;
};

template <typename MT> struct V16;
template <> struct V16<bf16> { typedef bf16x8 type; static constexpr int n = 8; };
template <> struct V16<float> { typedef f32x4 type; static constexpr int n = 4; };

template <typename MT, int C, int N, int P, int NW>
struct FwdCfg {
  static constexpr int NT = NW * 64;
  static constexpr int VEC = V16<MT>::n;          // elements per 16-byte access
  static constexpr int H2 = N / 2;
  static constexpr int PAD = 16 / (int)sizeof(MT);
  static constexpr int LDQ = N + PAD;             // sQ, sK, sS row stride
  static constexpr int LDT = C + PAD;             // sVT, sKT row stride
  static constexpr int LDO = P + 4;               // sOut row stride (f32)
  static constexpr int QKG = H2 / VEC;            // rotary pair groups per row
  static constexpr int QKT = (C / 2) * QKG;       // q/k tasks: (row pair, pair group)
  static constexpr int QKR = (QKT + NT - 1) / NT;
  static constexpr int VG = P / VEC;
  static constexpr int VT = (C / 2) * VG;         // v / epilogue tasks: (row pair, col group)
  static constexpr int VR = (VT + NT - 1) / NT;
  static constexpr int PB = P / 16, NB = N / 16, CB = C / 16;
  static constexpr int T4 = PB * NB;              // state tiles
  static constexpr int SPW = (T4 + NW - 1) / NW;  // state tiles per wave
  static constexpr int E = C >= 64 ? C / 64 : 1;  // scan values per lane of wave 0
  static constexpr int SZ_Q = C * LDQ * (int)sizeof(MT);
  static constexpr int SZ_VT = P * LDT * (int)sizeof(MT);
  static constexpr int SZ_S = P * LDQ * (int)sizeof(MT);
  static constexpr int SZ_KT = N * LDT * (int)sizeof(MT);
  static constexpr int SZ_OUT = C * LDO * 4;
  static constexpr int SZ_U = SZ_KT > SZ_OUT ? SZ_KT : SZ_OUT;
  static constexpr int SZ_SC = (4 * C + 2 * N) * 4;
  static constexpr int LDS_BYTES = 2 * SZ_Q + SZ_VT + SZ_S + SZ_U + SZ_SC;
  static_assert(NW >= CB, "one query strip per wave");
  static_assert(QKG <= 64 && (QKG & (QKG - 1)) == 0, "row groups must fit a wave");
  static_assert(C % 32 == 0 && N % 16 == 0 && P % 16 == 0, "tile shape");
  static_assert(LDS_BYTES <= 163840, "LDS budget of one gfx950 CU");
};

// STRIPS: phi built from the compact form (phi_strips mode). RAW (raw mode, with STRIPS):
// the row scalars from the raw dt / a / trap slices (the library functions the preprocess
// kernels use, so the same values), and each row's angle from a carry across chunks that
// every thread keeps for its angle group, the strip's prefix within its chunk and the
// strip's table rows times their dt.
template <typename MT, int C, int N, int P, int NW, bool STRIPS, bool RAW = false>
__global__ void __launch_bounds__(NW * 64) fwd_kernel(const FwdParams p) {
  using F = FwdCfg<MT, C, N, P, NW>;
  static_assert(!RAW || STRIPS, "raw mode builds phi");
  using vec = typename V16<MT>::type;
  constexpr int NT = F::NT, VEC = F::VEC, H2 = F::H2;
  constexpr int LDQ = F::LDQ, LDT = F::LDT, LDO = F::LDO;

  __shared__ __align__(16) unsigned char smem[F::LDS_BYTES];
  // Buffer offsets go through an opaque SGPR. Otherwise every access above 64 KiB (the
  // reach of a ds_read immediate) gets its own address VGPR, and LICM keeps all of them
  // live across the chunk loop -- enough to spill.
  auto opq = [](int x) { asm volatile("" : "+s"(x)); return x; };
  MT* sQ = reinterpret_cast<MT*>(smem);
  MT* sK = reinterpret_cast<MT*>(smem + opq(F::SZ_Q));
  MT* sVT = reinterpret_cast<MT*>(smem + opq(2 * F::SZ_Q));
  MT* sS = reinterpret_cast<MT*>(smem + opq(2 * F::SZ_Q + F::SZ_VT));
  unsigned char* uni = smem + opq(2 * F::SZ_Q + F::SZ_VT + F::SZ_S);
  MT* sKT = reinterpret_cast<MT*>(uni);        // live during the products
  float* sOut = reinterpret_cast<float*>(uni);  // live during the epilogue
  float* sA = reinterpret_cast<float*>(smem + opq(2 * F::SZ_Q + F::SZ_VT + F::SZ_S + F::SZ_U));
  float* sExpA = sA + C;   // 2^{A_t}
  float* sFac = sExpA + C; // 2^{A_last - A_t}
  float* sCoef = sFac + C; // D + gamma_t (u_t . w_t)
  float* sQb = sCoef + C;
  float* sKb = sQb + N;

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
  const float dsk = p.has_d ? p.dsk[h] : 0.f;

  const MT* qg = static_cast<const MT*>(p.q) + (int64_t)b * L * N;
  const MT* kg = static_cast<const MT*>(p.k) + (int64_t)b * L * N;
  const MT* vg = static_cast<const MT*>(p.v) + b * p.v_sb + h * p.v_sh;
  const MT* zg = p.has_z ? static_cast<const MT*>(p.z) + b * p.z_sb + h * p.z_sh : nullptr;
  MT* yg = static_cast<MT*>(p.y) + b * p.y_sb + h * p.y_sh;
  const float* adtg = p.adt + bh * L;
  const float* gamg = p.gamma + bh * L;
  const float* sclg = p.scale + bh * L;
  const float* phig = STRIPS ? nullptr : p.phi + bh * (int64_t)L * Nr;
  MT* csg = p.save ? static_cast<MT*>(p.cstates) + bh * (int64_t)nc * N * P : nullptr;
  // raw mode: this (b, h)'s raw scalars (dt at element t sc_st, a and trap a_off / t_off
  // further) and dt bias
  const MT* scg = RAW ? static_cast<const MT*>(p.sc) + b * p.sc_sb + h : nullptr;
  const int64_t sc_st = RAW ? p.sc_st : 0;
  const float dtb = RAW ? p.dt_bias[h] : 0.f;
  auto raw_dt = [&](int64_t t) { return softplus_((float)scg[t * sc_st] + dtb); };
  auto raw_lam = [&](int64_t t) { return sigmoid_((float)scg[t * sc_st + p.t_off]); };

  // ---- carried state: registers, MFMA layout ------------------------------------
  f32x4 Sacc[F::SPW];
#pragma unroll
  for (int m = 0; m < F::SPW; ++m) {
    const int s = wave + NW * m;
    Sacc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (s < F::T4 && p.has_seed) {
      const int pb = s % F::PB, nb = s / F::PB;
      const int ncol = nb * 16 + (lane & 15);
      const float coef = p.seed_coef[bh];
      const float kp = p.seed_k[bh * N + ncol];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int prow = pb * 16 + 4 * (lane >> 4) + i;
        Sacc[m][i] = p.seed_ssm[(bh * P + prow) * N + ncol] + coef * p.seed_v[bh * P + prow] * kp;
      }
    }
  }
  auto publish_state = [&](int cidx) {
    // S (registers) -> sS as the MFMA operand type, and the chunk_states residual.
#pragma unroll
    for (int m = 0; m < F::SPW; ++m) {
      const int s = wave + NW * m;
      if (s < F::T4) {
        const int pb = s % F::PB, nb = s / F::PB;
        const int ncol = nb * 16 + (lane & 15);
        const int prow0 = pb * 16 + 4 * (lane >> 4);
        sub_t<MT> sv = sub_from_f32<MT>(Sacc[m]);
#pragma unroll
        for (int i = 0; i < 4; ++i) sS[(prow0 + i) * LDQ + ncol] = sv[i];
        if (csg && cidx < nc)
          *reinterpret_cast<sub_t<MT>*>(csg + ((int64_t)cidx * N + ncol) * P + prow0) = sv;
      }
    }
  };
  publish_state(0);

  // ---- register prefetch of one chunk's raw inputs --------------------------------
  vec rq[F::QKR][2][2], rk[F::QKR][2][2];
  f32x4 rphi[F::QKR][2][VEC / 4];
  float rscale[F::QKR][2], rgam[F::QKR][2];
  vec rv[F::VR][2], rz[F::VR][2];
  float radt[F::E];
  // raw mode: the angle entering the chunk being prefetched, for this thread's angle groups
  float pin[RAW ? F::QKR : 1][VEC];
  if constexpr (RAW) {
#pragma unroll
    for (int r = 0; r < F::QKR; ++r) {
      const int j0 = ((tid + r * NT) % F::QKG) * VEC;
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        pin[r][i] = (p.phi_init && j0 + i < Nr) ? p.phi_init[bh * Nr + j0 + i] : 0.f;
    }
  }

  const bool phi_vec = (Nr % 4) == 0;
  auto prefetch = [&](int c) {
    const int t0 = c * C;
#pragma unroll
    for (int r = 0; r < F::QKR; ++r) {
      const int task = tid + r * NT;
      if (task < F::QKT) {
        const int tp = task / F::QKG, j0 = (task % F::QKG) * VEC;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int64_t t = t0 + 2 * tp + e;
          rq[r][e][0] = *reinterpret_cast<const vec*>(qg + t * N + j0);
          rq[r][e][1] = *reinterpret_cast<const vec*>(qg + t * N + H2 + j0);
          rk[r][e][0] = *reinterpret_cast<const vec*>(kg + t * N + j0);
          rk[r][e][1] = *reinterpret_cast<const vec*>(kg + t * N + H2 + j0);
          if constexpr (STRIPS) {
            // the strip's entering angle plus theta = tanh(angles) pi dt over the strip's
            // rows up to t (at most 16); raw mode: the entering angle is the chunk's carry
            // plus the strip's prefix within the chunk, and dt comes from the raw slice
            const int64_t s16 = t >> 4;
            const float* ps = (RAW ? p.tpre : p.pstr) + (bh * (L / 16) + s16) * Nr;
            const float* tb = p.tht + (int64_t)b * L * Nr;
            const float* db = RAW ? nullptr : p.pdt + bh * L;
#pragma unroll
            for (int qd = 0; qd < VEC / 4; ++qd) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int j = j0 + 4 * qd + i;
                float e0 = j < Nr ? ps[j] : 0.f;
                if constexpr (RAW) e0 += pin[r][4 * qd + i];
                rphi[r][e][qd][i] = e0;
              }
            }
            for (int64_t u = s16 * 16; u <= t; ++u) {
              const float du = RAW ? raw_dt(u) : db[u];
#pragma unroll
              for (int qd = 0; qd < VEC / 4; ++qd) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  const int j = j0 + 4 * qd + i;
                  if (j < Nr) rphi[r][e][qd][i] += tb[u * Nr + j] * du;
                }
              }
            }
          } else {
            const float* pr = phig + t * Nr;
#pragma unroll
            for (int qd = 0; qd < VEC / 4; ++qd) {
              const int j = j0 + 4 * qd;
              if (phi_vec && j + 4 <= Nr) {
                rphi[r][e][qd] = *reinterpret_cast<const f32x4*>(pr + j);
              } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) rphi[r][e][qd][i] = (j + i < Nr) ? pr[j + i] : 0.f;
              }
            }
          }
          if constexpr (RAW) {   // reference.py:104-131: gamma, and the t+1 scale shift
            const float dtt = raw_dt(t), lamt = raw_lam(t);
            const float nxt = t + 1 < L ? raw_dt(t + 1) * (1.f - raw_lam(t + 1)) : 0.f;
            rgam[r][e] = dtt * lamt;
            rscale[r][e] = rgam[r][e] + nxt;
          } else {
            rscale[r][e] = sclg[t];
            rgam[r][e] = gamg[t];
          }
        }
      }
    }
    if constexpr (RAW) {   // the carry moves past this chunk
#pragma unroll
      for (int r = 0; r < F::QKR; ++r) {
        const int j0 = ((tid + r * NT) % F::QKG) * VEC;
        const float* ct = p.ctot + (bh * nc + c) * Nr;
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          if (j0 + i < Nr) pin[r][i] = wrap_2pi(pin[r][i] + ct[j0 + i]);
      }
    }
#pragma unroll
    for (int r = 0; r < F::VR; ++r) {
      const int task = tid + r * NT;
      if (task < F::VT) {
        const int tp = task / F::VG, p0 = (task % F::VG) * VEC;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int64_t t = t0 + 2 * tp + e;
          rv[r][e] = *reinterpret_cast<const vec*>(vg + t * p.v_st + p0);
          if (zg) rz[r][e] = *reinterpret_cast<const vec*>(zg + t * p.z_st + p0);
        }
      }
    }
    if (wave == 0) {
#pragma unroll
      for (int e = 0; e < F::E; ++e) {
        const int tt = lane * F::E + e;
        if constexpr (RAW) {   // a = min(-heavy_tail(a_raw), -a_floor)
          radt[e] = tt < C ? fminf(-heavy_tail_((float)scg[(t0 + tt) * sc_st + p.a_off]), -p.a_floor) *
                                 raw_dt(t0 + tt)
                           : 0.f;
        } else {
          radt[e] = tt < C ? adtg[t0 + tt] : 0.f;
        }
      }
    }
  };

  prefetch(0);
  __syncthreads();  // sQb/sKb, sS

  vec cv[F::VR][2], cz[F::VR][2];

  for (int c = 0; c < nc; ++c) {
    const int t0 = c * C;
    const bool last_chunk = (c == nc - 1);
    // Lane/wave indices re-derived opaquely each chunk, so the per-lane LDS address
    // arithmetic is recomputed near its uses instead of being hoisted out of the loop.
    int lane_v = threadIdx.x;
    asm volatile("" : "+v"(lane_v));
    const int tid = lane_v, lane = tid & 63;
    int wave_s = __builtin_amdgcn_readfirstlane(tid >> 6);
    asm volatile("" : "+s"(wave_s));
    const int wave = wave_s;

    // ================= phase L: raw registers -> LDS tiles ==========================
    if (wave == 0) {
      // inclusive prefix sum of adt*log2(e) over the chunk
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
#pragma unroll
    for (int r = 0; r < F::QKR; ++r) {
      const int task = tid + r * NT;
      const bool valid = task < F::QKT;
      const int tp = valid ? task / F::QKG : 0, j0 = valid ? (task % F::QKG) * VEC : 0;
      float khat[2][2][VEC];
      float uw[2] = {0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        float qt[2][VEC], kt[2][VEC];
        if (valid) {
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
            qt[0][i] = ulo * cs - uhi * sn;
            qt[1][i] = uhi * cs + ulo * sn;
            kt[0][i] = wlo * cs - whi * sn;
            kt[1][i] = whi * cs + wlo * sn;
          }
          const int t = 2 * tp + e;
          vec oq0, oq1, ok0, ok1;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            khat[e][0][i] = kt[0][i] * rscale[r][e];
            khat[e][1][i] = kt[1][i] * rscale[r][e];
            oq0[i] = (MT)qt[0][i];
            oq1[i] = (MT)qt[1][i];
            ok0[i] = (MT)khat[e][0][i];
            ok1[i] = (MT)khat[e][1][i];
          }
          *reinterpret_cast<vec*>(sQ + t * LDQ + j0) = oq0;
          *reinterpret_cast<vec*>(sQ + t * LDQ + H2 + j0) = oq1;
          *reinterpret_cast<vec*>(sK + t * LDQ + j0) = ok0;
          *reinterpret_cast<vec*>(sK + t * LDQ + H2 + j0) = ok1;
          if (last_chunk && t == C - 1) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
              p.fk[bh * N + j0 + i] = kt[0][i];
              p.fk[bh * N + H2 + j0 + i] = kt[1][i];
            }
          }
        }
      }
      // u.w per row: reduce over the QKG lanes that share the row pair
      uw[0] = group_sum<F::QKG>(uw[0]);
      uw[1] = group_sum<F::QKG>(uw[1]);
      if (valid) {
        if (j0 == 0) {
          sCoef[2 * tp] = rgam[r][0] * uw[0] + dsk;
          sCoef[2 * tp + 1] = rgam[r][1] * uw[1] + dsk;
        }
        // khat^T for the state update: pack rows (2tp, 2tp+1) into one store
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const int n = hh * H2 + j0 + i;
            store_pair<MT>(sKT + n * LDT + 2 * tp, khat[0][hh][i], khat[1][hh][i]);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < F::VR; ++r) {
      const int task = tid + r * NT;
      if (task < F::VT) {
        const int tp = task / F::VG, p0 = (task % F::VG) * VEC;
        cv[r][0] = rv[r][0];
        cv[r][1] = rv[r][1];
        if (zg) {
          cz[r][0] = rz[r][0];
          cz[r][1] = rz[r][1];
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          store_pair<MT>(sVT + (p0 + i) * LDT + 2 * tp, (float)rv[r][0][i], (float)rv[r][1][i]);
        }
        if (last_chunk && 2 * tp + 1 == C - 1) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) p.fv[bh * P + p0 + i] = (float)rv[r][1][i];
        }
      }
    }
    __syncthreads();

    if (c + 1 < nc) prefetch(c + 1);

    // ================= phase G: products ============================================
    f32x4 out[F::PB];
#pragma unroll
    for (int pb = 0; pb < F::PB; ++pb) out[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int tb = wave;
    const int tcol = tb * 16 + (lane & 15);
    if (tb < F::CB) {
      const float At = sA[tcol];
      sub_t<MT> sT[F::CB];
#pragma unroll
      for (int jb = 0; jb < F::CB; ++jb) {
        if (jb <= tb) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          gemm_nt<MT, N>(acc, sK, LDQ, jb * 16, sQ, LDQ, tb * 16);
          f32x4 sv;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = jb * 16 + 4 * (lane >> 4) + i;
            sv[i] = (tcol > j) ? acc[i] * exp2f(fminf(At - sA[j], 0.f)) : 0.f;
          }
          sT[jb] = sub_from_f32<MT>(sv);
        } else {
          sT[jb] = sub_from_f32<MT>(f32x4{0.f, 0.f, 0.f, 0.f});
        }
      }
      // intra-chunk: out^T[p][t] += sum_j v^T[p][j] s^T[j][t]
#pragma unroll
      for (int jb = 0; jb < F::CB; jb += 2) {
        if (jb <= tb) {
#pragma unroll
          for (int pb = 0; pb < F::PB; ++pb) {
            if (jb + 1 <= tb) {
              mma32(out[pb], ld_sub<MT>(sVT, LDT, pb * 16, jb * 16),
                    ld_sub<MT>(sVT, LDT, pb * 16, jb * 16 + 16), sT[jb], sT[jb + 1]);
            } else {
              mma16(out[pb], ld_sub<MT>(sVT, LDT, pb * 16, jb * 16), sT[jb]);
            }
          }
        }
      }
      // inter-chunk: out^T[p][t] += 2^{A_t} sum_n S[p][n] q~[t][n]
      const float eA = sExpA[tcol];
#pragma unroll
      for (int pb = 0; pb < F::PB; ++pb) {
        f32x4 it = {0.f, 0.f, 0.f, 0.f};
        gemm_nt<MT, N>(it, sS, LDQ, pb * 16, sQ, LDQ, tb * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) out[pb][i] += eA * it[i];
      }
    }
    // state: S <- 2^{A_last} S + sum_t (v_t 2^{A_last - A_t}) khat_t^T
    {
      const float eAl = sExpA[C - 1];
#pragma unroll
      for (int m = 0; m < F::SPW; ++m) {
        const int s = wave + NW * m;
        if (s < F::T4) {
          const int pb = s % F::PB, nb = s / F::PB;
#pragma unroll
          for (int i = 0; i < 4; ++i) Sacc[m][i] *= eAl;
#pragma unroll
          for (int k0 = 0; k0 < C; k0 += 32) {
            sub_t<MT> a0, a1;
            {
              f32x4 v0 = sub_to_f32<MT>(ld_sub<MT>(sVT, LDT, pb * 16, k0));
              f32x4 v1 = sub_to_f32<MT>(ld_sub<MT>(sVT, LDT, pb * 16, k0 + 16));
              const int kk = sub_k(k0);
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                v0[i] *= sFac[kk + i];
                v1[i] *= sFac[kk + 16 + i];
              }
              a0 = sub_from_f32<MT>(v0);
              a1 = sub_from_f32<MT>(v1);
            }
            mma32(Sacc[m], a0, a1, ld_sub<MT>(sKT, LDT, nb * 16, k0),
                  ld_sub<MT>(sKT, LDT, nb * 16, k0 + 16));
          }
        }
      }
    }
    __syncthreads();

    // ================= phase W: out^T -> sOut, new S -> sS ===========================
    if (tb < F::CB) {
#pragma unroll
      for (int pb = 0; pb < F::PB; ++pb)
        *reinterpret_cast<f32x4*>(sOut + tcol * LDO + pb * 16 + 4 * (lane >> 4)) = out[pb];
    }
    publish_state(c + 1);
    __syncthreads();

    // ================= phase E: diagonal + skip + gate, stores ======================
#pragma unroll
    for (int r = 0; r < F::VR; ++r) {
      const int task = tid + r * NT;
      if (task < F::VT) {
        const int tp = task / F::VG, p0 = (task % F::VG) * VEC;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int t = 2 * tp + e;
          const float coef = sCoef[t];
          float yb[VEC];
#pragma unroll
          for (int i = 0; i < VEC; i += 4) {
            const f32x4 o = *reinterpret_cast<const f32x4*>(sOut + t * LDO + p0 + i);
#pragma unroll
            for (int u = 0; u < 4; ++u) yb[i + u] = o[u] + coef * (float)cv[r][e][i + u];
          }
          if (p.save) {
            vec ybv;
#pragma unroll
            for (int i = 0; i < VEC; ++i) ybv[i] = (MT)yb[i];
            *reinterpret_cast<vec*>(static_cast<MT*>(p.ybar) + (bh * L + t0 + t) * (int64_t)P + p0) = ybv;
          }
          vec yo;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const float g = zg ? silu((float)cz[r][e][i]) : 1.f;
            yo[i] = (MT)(yb[i] * g);
          }
          *reinterpret_cast<vec*>(yg + (int64_t)(t0 + t) * p.y_st + p0) = yo;
        }
      }
    }
    __syncthreads();
  }

  // final state
#pragma unroll
  for (int m = 0; m < F::SPW; ++m) {
    const int s = wave + NW * m;
    if (s < F::T4) {
      const int pb = s % F::PB, nb = s / F::PB;
      const int ncol = nb * 16 + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int prow = pb * 16 + 4 * (lane >> 4) + i;
        p.fssm[(bh * P + prow) * N + ncol] = Sacc[m][i];
      }
    }
  }
  if constexpr (RAW) {   // the carry past the last chunk: phi at L-1
#pragma unroll
    for (int r = 0; r < F::QKR; ++r) {
      const int task = tid + r * NT;
      const int j0 = (task % F::QKG) * VEC;
      if (task < F::QKG) {
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          if (j0 + i < Nr) p.phi_final[bh * Nr + j0 + i] = pin[r][i];
      }
    }
  }
}

// ===================================================================================
// fwd_bf16_kernel: the bf16 forward for state_dim % 64 == 0 (the configs[1] shape).
//
// Same maths and rounding points as fwd_kernel; the data flow is rebuilt around three
// gfx950 facts measured on fwd_kernel (LDS bandwidth and bank conflicts, not MFMA or
// HBM, bounded it, and four barriers per chunk serialised its phases):
//  * The wave that owns query strip w loads, biases and rotates the q/k rows of that
//    strip itself, in the MFMA operand order (lane: row l & 15, K slots 8 (l >> 4) + s).
//    q~ never goes to LDS: it stays in registers as the B operand of the score and
//    inter-chunk products. khat goes to LDS once, row-major.
//  * Operands whose contraction axis is time (v^T for P = W^T-weighted sums, v^T and
//    khat^T for the state update) are read with ds_read_b64_tr_b16 from the same
//    row-major tiles, so no transposed copy is ever written.
//  * The chunk loop is software-pipelined with two barriers per chunk: phase A stages
//    chunk c-1's output and chunk c's state into LDS and builds chunk c's tiles; phase
//    B runs chunk c-1's epilogue (gate, stores) alongside chunk c's products, so the
//    store-heavy epilogue of one wave overlaps the MFMA work of another.
// ===================================================================================

template <int C, int N, int P>
struct Fwd2Cfg {
  static constexpr int NW = C / 16;        // one query strip per wave
  static constexpr int NT = NW * 64;
  static constexpr int NBK = N / 32;       // 32-wide K blocks over N
  static constexpr int LOB = N / 64;       // blocks in the rotated half; partner = +LOB
  static constexpr int LDK = N + 8;        // sK, sS row stride (bf16)
  static constexpr int LDO = P + 4;        // sOut row stride (f32)
  static constexpr int PB = P / 16, NB = N / 16, CB = C / 16;
  static constexpr int SPW = PB * NB / NW; // state tiles per wave
  static constexpr int NSTEP = NW / PB;    // nb stride between a wave's state tiles
  // v / z tiles: C rows of P bf16 (128 bytes), unpadded, the 16-byte pieces of row r
  // stored at slot piece ^ (r & 7) so transposed and row reads hit distinct banks.
  // Every wave prefetches VPL 16-byte pieces of each into registers one phase ahead
  // and writes them in phase A, so one LDS tile of each suffices.
  static constexpr int VPL = C * P * 2 / (NT * 16);  // 16-byte pieces per lane per tile
  static constexpr int NWL = NW / 2;              // light waves: run the epilogue
  static constexpr int VG = P / 8;                // epilogue column groups (16 bytes)
  static constexpr int VT = (C / 2) * VG;         // epilogue tasks: (row pair, group)
  static constexpr int VTH = NWL * 64;            // epilogue threads
  static constexpr int VR = (VT + VTH - 1) / VTH;
  static constexpr int E = C / 64;                // A-scan values per lane of wave 0
  static constexpr int SZ_K = C * LDK * 2;
  static constexpr int SZ_V = C * P * 2;          // one v or z tile
  static constexpr int SZ_S = P * LDK * 2;
  static constexpr int SZ_O = C * LDO * 4;
  // sQb, sKb, then two buffers of the row scalars [A, 2^A, 2^(A_last - A), coef, dk]
  static constexpr int SZ_SC = (10 * C + 2 * N) * 4;
  // k-hat tiles and row scalars are double-buffered: chunk c+1's are written at the end
  // of chunk c's phase B, while the products of chunk c read the other buffer
  static constexpr int LDS_BYTES = 2 * SZ_K + 2 * SZ_V + SZ_S + SZ_O + SZ_SC;
  static_assert(N % 64 == 0 && P == 64 && C % 64 == 0, "tile shape");
  static_assert(NW % PB == 0 && (PB * NB) % NW == 0, "state tiles split evenly over waves");
  static_assert(VPL * NT * 16 == C * P * 2, "v / z pieces split evenly over the lanes");
  static_assert(LDS_BYTES <= 163840, "LDS budget of one gfx950 CU");
};

// Compile-time case selector for generic lambdas (`decltype(tag)::value`).
template <int V> struct IntTag { static constexpr int value = V; };

// Element offset of (row r, column col) in a swizzled 64-column bf16 tile.
__device__ __forceinline__ int vz_off(int r, int col) {
  return r * 64 + ((((col >> 3) ^ r) & 7) << 3) + (col & 7);
}
// ld_tr4 on a swizzled 64-column tile: { T[kb + s][m0 + (l & 15)] : s < 4 }.
__device__ __forceinline__ bf16x4 ld_tr4_vz(const bf16* buf, int kb, int m0, int l) {
  const int j = l & 15;
  const bf16* ptr = buf + vz_off(kb + (j >> 2), m0 + 4 * (j & 3));
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(ptr));
  return __builtin_bit_cast(bf16x4, r);
}
// The swizzle of a row depends only on row & 7: a lane's ld_tr4_vz offset at rows
// kb + 16 i (kb + 8 i) is 1024 i (512 i) elements past its offset at row kb, so
// loops over row bands compute the offset once (vz_tr_off) and step a pointer.
__device__ __forceinline__ int vz_tr_off(int kb, int m0, int l) {
  const int j = l & 15;
  return vz_off(kb + (j >> 2), m0 + 4 * (j & 3));
}
__device__ __forceinline__ bf16x4 ld_tr4_at(const bf16* ptr) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(ptr));
  return __builtin_bit_cast(bf16x4, r);
}

// LDS of raw mode's strip angles: the angle entering each 16-token strip of a chunk, for
// the NRB 32-column blocks of rotary pairs, double-buffered by chunk parity.
template <int C, int NRB>
constexpr int raw_strip_floats() { return 2 * (C / 16) * 32 * NRB; }
template <int C, int N, int P, int NRB>
constexpr bool raw_fits() {
  return NRB > 0 && Fwd2Cfg<C, N, P>::LDS_BYTES + 4 * raw_strip_floats<C, NRB>() <= 163840;
}

// NRB = 0: phi is read. NRB > 0 (phi_strips mode): phi is built from the compact form,
// and NRB is the number of 32-column blocks that hold rotary pairs (Nr <= 32 NRB).
// RAW (raw mode, NRB > 0): the row scalars come from the projection's raw dt / a / trap
// slices, and the angle entering each strip from a carry across chunks this kernel keeps
// itself plus the strip's prefix within its chunk (see `carry` below), instead of phi_dt /
// phi_strips.
template <int C, int N, int P, int NRB, bool RAW = false>
__global__ void __launch_bounds__(C / 16 * 64) fwd_bf16_kernel(const FwdParams p) {
  using F = Fwd2Cfg<C, N, P>;
  constexpr bool STRIPS = NRB > 0;
  static_assert(NRB <= F::LOB, "rotary blocks lie in the rotated half");
  static_assert(!RAW || raw_fits<C, N, P, NRB>(), "raw mode needs phi built and its LDS");
  constexpr int SPC = C / 16;                  // 16-token strips per chunk
  constexpr int ELD = 32 * NRB;                // row stride of the strip-angle table
  constexpr int TQ = 64 / SPC;                 // angle quads per lane load of the carry
  constexpr int TL = RAW ? (ELD + 4 * TQ - 1) / (4 * TQ) : 1;   // such loads
  constexpr int NT = F::NT, LDK = F::LDK, LDO = F::LDO;
  constexpr int H2 = N / 2, PB = F::PB, SPW = F::SPW, NSTEP = F::NSTEP;

  // four groups of each XCD's workgroups start 0, 4, 8 and 12 K cycles late (a chunk takes
  // about 16 K): at B=8 L=8192 H=32 the scan took 2% less
  if (p.nc >= 16) stagger_start(blockIdx.x, 4, 2);
  __shared__ __align__(16) unsigned char smem[F::LDS_BYTES + 4 * (RAW ? raw_strip_floats<C, NRB>() : 0)];
  auto opq = [](int x) { asm volatile("" : "+s"(x)); return x; };
  bf16* sK2 = reinterpret_cast<bf16*>(smem);                                // [2] k-hat tiles
  bf16* sV = reinterpret_cast<bf16*>(smem + opq(2 * F::SZ_K));              // v tile
  bf16* sZ = reinterpret_cast<bf16*>(smem + opq(2 * F::SZ_K + F::SZ_V));    // z tile
  bf16* sS = reinterpret_cast<bf16*>(smem + opq(2 * F::SZ_K + 2 * F::SZ_V));
  float* sOut = reinterpret_cast<float*>(smem + opq(2 * F::SZ_K + 2 * F::SZ_V + F::SZ_S));
  float* sQb = reinterpret_cast<float*>(smem + opq(2 * F::SZ_K + 2 * F::SZ_V + F::SZ_S + F::SZ_O));
  float* sKb = sQb + N;
  float* sSc2 = sKb + N;   // [2] row scalar blocks, laid out as in `scalars` below
  float* sE = sSc2 + 10 * C;   // raw mode: [2][SPC][ELD] angle entering each strip
  // buffer b's k-hat tile, and its row scalars: A_t, 2^{A_t}, 2^{A_last - A_t},
  // D + gamma_t (u_t . w_t), and 2^{A_{16 s + 15} - A_j} (s = j's strip: a key row's
  // decay to its strip end)
  auto khat = [&](int b) { return sK2 + b * (F::SZ_K / 2); };
  struct Scalars { float *A, *ExpA, *Fac, *Coef, *Dk; };
  auto scalars = [&](int b) {
    float* base = sSc2 + b * 5 * C;
    return Scalars{base, base + C, base + 2 * C, base + 3 * C, base + 4 * C};
  };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool light = wave < F::NWL;
  // query strip of this wave: the light waves take the short end of the causal triangle
  // (strips 0 .. NW/2-1), the others the long end in reverse, so that waves w and
  // w + NW/2 -- which share a SIMD -- hold strips w and NW-1-w: every SIMD gets the same
  // number of score tiles (NW + 1) and one wave's share of the epilogue
  const int strip = light ? wave : 3 * F::NWL - 1 - wave;
  const int wid = xcd_remap(blockIdx.x, gridDim.x);
  const int b = wid / p.H, h = wid % p.H;
  const int64_t bh = (int64_t)b * p.H + h;
  const int L = p.L, Nr = p.Nr, nc = p.nc;

  for (int i = tid; i < N; i += NT) {
    sQb[i] = p.qb[h * N + i];
    sKb[i] = p.kb[h * N + i];
  }
  const float dsk = p.has_d ? p.dsk[h] : 0.f;

  const bf16* qg = static_cast<const bf16*>(p.q) + (int64_t)b * L * N;
  const bf16* kg = static_cast<const bf16*>(p.k) + (int64_t)b * L * N;
  const bf16* vg = static_cast<const bf16*>(p.v) + b * p.v_sb + h * p.v_sh;
  const bf16* zg = p.has_z ? static_cast<const bf16*>(p.z) + b * p.z_sb + h * p.z_sh : nullptr;
  bf16* yg = static_cast<bf16*>(p.y) + b * p.y_sb + h * p.y_sh;
  const float* adtg = p.adt + bh * L;
  const float* gamg = p.gamma + bh * L;
  const float* sclg = p.scale + bh * L;
  // phi rows of this (b, h), or (phi_strips mode) the head-shared tanh(angles) pi rows of
  // batch element b, read with the same row addressing; then dt and the strip values
  const float* phig = STRIPS ? p.tht + (int64_t)b * L * Nr : p.phi + bh * (int64_t)L * Nr;
  bf16* csg = p.save ? static_cast<bf16*>(p.cstates) + bh * (int64_t)nc * N * P : nullptr;
  // buffer descriptors of this (b, h)'s streams (the host checked every extent < 2^31)
  const auto rQ = make_rsrc(qg, (uint32_t)L * N * 2);
  const auto rK = make_rsrc(kg, (uint32_t)L * N * 2);
  const auto rPhi = make_rsrc(phig, (uint32_t)L * Nr * 4);
  // dt and the strip angles through SGPR-base global loads (two SGPRs per base where a
  // buffer descriptor takes four): past the last chunk they read chunk 0 again, unused
  const float* pdtg = STRIPS ? p.pdt + bh * L : nullptr;
  const float* pstrg = (STRIPS && !RAW) ? p.pstr + bh * (int64_t)(L / 16) * Nr : nullptr;
  const auto rScl = make_rsrc(sclg, (uint32_t)L * 4);
  const auto rGam = make_rsrc(gamg, (uint32_t)L * 4);
  const auto rAdt = make_rsrc(adtg, (uint32_t)L * 4);
  const auto rV = make_rsrc(vg, (uint32_t)(((int64_t)(L - 1) * p.v_st + P) * 2));
  const auto rZ = make_rsrc(zg, zg ? (uint32_t)(((int64_t)(L - 1) * p.z_st + P) * 2) : 0u);
  const auto rY = make_rsrc(yg, (uint32_t)(((int64_t)(L - 1) * p.y_st + P) * 2));
  const auto rYb = make_rsrc(p.save ? static_cast<bf16*>(p.ybar) + bh * L * (int64_t)P : nullptr,
                             p.save ? (uint32_t)L * P * 2 : 0u);
  const auto rCs = make_rsrc(csg, p.save ? (uint32_t)nc * N * P * 2 : 0u);
  // raw mode: this (b, h)'s raw scalars through one descriptor (dt at element t sc_st,
  // a and trap a_off / t_off further; past the sequence it reads zeros), its chunk theta
  // totals, and its dt bias
  const int64_t sc_st = RAW ? p.sc_st : 0;
  const bf16* scg = RAW ? static_cast<const bf16*>(p.sc) + b * p.sc_sb + h : nullptr;
  const auto rSc = make_rsrc(scg, RAW ? (uint32_t)(((int64_t)(L - 1) * sc_st + p.sc_span) * 2) : 0u);
  const auto rCt = make_rsrc(RAW ? p.ctot + bh * (int64_t)nc * Nr : nullptr,
                             RAW ? (uint32_t)nc * Nr * 4 : 0u);
  const auto rPre = make_rsrc(RAW ? p.tpre + bh * (int64_t)(L / 16) * Nr : nullptr,
                              RAW ? (uint32_t)(L / 16) * Nr * 4 : 0u);
  const float dtb = RAW ? p.dt_bias[h] : 0.f;

  // ---- carried state: registers; wave owns tiles (pb_w, nb0 + NSTEP m) ------------
  const int pb_w = wave % PB, nb0 = wave / PB;
  f32x4 Sacc[SPW];
#pragma unroll
  for (int m = 0; m < SPW; ++m) {
    Sacc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (p.has_seed) {
      const int ncol = (nb0 + NSTEP * m) * 16 + (lane & 15);
      const float coef = p.seed_coef[bh];
      const float kp = p.seed_k[bh * N + ncol];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int prow = pb_w * 16 + 4 * (lane >> 4) + i;
        Sacc[m][i] = p.seed_ssm[(bh * P + prow) * N + ncol] + coef * p.seed_v[bh * P + prow] * kp;
      }
    }
  }
  // chunk c's state in bf16, stored as the chunk_states residual right after chunk c's
  // products rather than in phase A: there every workgroup's 8-byte state stores joined the
  // same synchronised burst (training forward 0.475-0.483 -> 0.442-0.448 ms at cfg2)
  bf16x4 csv[SPW];
  auto publish_state = [&](int cidx) {
    // S (registers) -> sS in bf16 (and kept for the chunk_states residual)
#pragma unroll
    for (int m = 0; m < SPW; ++m) {
      const int ncol = (nb0 + NSTEP * m) * 16 + (lane & 15);
      const int prow0 = pb_w * 16 + 4 * (lane >> 4);
      const bf16x4 sv = sub_from_f32<bf16>(Sacc[m]);
      csv[m] = sv;
#pragma unroll
      for (int i = 0; i < 4; ++i) sS[(prow0 + i) * LDK + ncol] = sv[i];
    }
  };
  auto store_state = [&](int cidx) {
    if (csg && cidx < nc) {
#pragma unroll
      for (int m = 0; m < SPW; ++m) {
        const int ncol = (nb0 + NSTEP * m) * 16 + (lane & 15);
        const int prow0 = pb_w * 16 + 4 * (lane >> 4);
        buf_store(csv[m], rCs, (uint32_t)(ncol * P + prow0) * 2, (uint32_t)cidx * N * P * 2);
      }
    }
  };

  // ---- v / z tiles: 16-byte row pieces prefetched into registers, written in phase A
  // (plain loads keep every dependency visible to the compiler; a direct global->LDS
  // load makes it wait for all outstanding loads before any later LDS read)
  bf16x8 rv[F::VPL], rz[F::VPL];
  // Loads and writes are unconditional: a chunk that does not exist (v after the last
  // chunk, z before the first, z of a layer without gate) is read through a zero-size
  // descriptor, which returns zeros and touches no memory, so every iteration issues
  // the same loads and the compiler's wait counts stay exact.
  const auto rNul = make_rsrc(nullptr, 0u);
  auto prefetch_vz = [&](const __amdgpu_buffer_rsrc_t& srv, int cv,
                         const __amdgpu_buffer_rsrc_t& srz, int cz) {
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < F::VPL; ++i) {
      const int id = ln + i * NT, row = id >> 3, col = 8 * (id & 7);
      rv[i] = buf_load<bf16x8>(srv, (uint32_t)(row * p.v_st + col) * 2, (uint32_t)(cv * C * p.v_st * 2));
      rz[i] = buf_load<bf16x8>(srz, (uint32_t)(row * p.z_st + col) * 2, (uint32_t)(cz * C * p.z_st * 2));
    }
  };
  auto write_vz = [&](bool last) {
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < F::VPL; ++i) {
      const int id = ln + i * NT, row = id >> 3, col = 8 * (id & 7);
      *reinterpret_cast<bf16x8*>(sV + vz_off(row, col)) = rv[i];
      *reinterpret_cast<bf16x8*>(sZ + vz_off(row, col)) = rz[i];
      if (last && row == C - 1) {   // final_v: the sequence's last v row
#pragma unroll
        for (int e = 0; e < 8; ++e) p.fv[bh * P + col + e] = (float)rv[i][e];
      }
    }
  };

  // ---- raw q, k, phi, scale, gamma of one chunk, prefetched into registers ---------
  // Strip layout: lane row 16 strip + (lane & 15), K group 8 (lane >> 4).
  bf16x8 rq[F::NBK], rk[F::NBK];
  f32x4 rphi[STRIPS ? 1 : F::LOB][2];   // phi of the row (phi read)
  // phi_strips mode: tanh(angles) pi of the row, the angle entering its strip, its dt, and
  // the turns built from them (for the next chunk, from the middle of the products on)
  f32x4 rtab[STRIPS ? NRB : 1][2], rstr[STRIPS ? NRB : 1][2];
  float rpdt = 0.f;
  float trn_pre[STRIPS ? NRB : 1][8];
  float rscale, rgam;
  float radt[F::E];
  const bool phi_vec = (Nr % 4) == 0;
  // raw mode: this lane's raw scalar of the next chunk (lane group g = lane >> 4 holds
  // dt_raw (g = 0) or trap_raw (g = 1) of its row t, the same of row t + 1 (g = 2, 3)),
  // the A-scan rows' dt_raw and a_raw, and, used by the carry wave only (lane: strip
  // lane % SPC, angle quads lane / SPC + TQ i), the strip prefixes and the total of the
  // chunk after next and the angle entering it
  float rraw = 0.f;
  float rdr[RAW ? F::E : 1], rar[RAW ? F::E : 1];
  f32x4 rX[TL], rC[TL], Pc[TL];

  auto prefetch_qk = [&](int c) {   // c >= nc: a chunk that does not exist, read as zeros
    const bool live = c < nc;
    const auto dQ = live ? rQ : rNul, dK = live ? rK : rNul;
    if (!live) c = 0;
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
    const int lane = ln & 63;
    const int trow = 16 * strip + (lane & 15);   // row within the chunk
    const int g8 = 8 * (lane >> 4);
    const uint32_t oqk = (uint32_t)(trow * N + g8) * 2;
#pragma unroll
    for (int blk = 0; blk < F::NBK; ++blk) {
      rq[blk] = buf_load<bf16x8>(dQ, oqk + 64 * blk, (uint32_t)c * C * N * 2);
      rk[blk] = buf_load<bf16x8>(dK, oqk + 64 * blk, (uint32_t)c * C * N * 2);
    }
  };
  // the rest of chunk c's inputs; issued from the middle of the products, so that the
  // wait for free memory-request slots overlaps MFMA work instead of stalling a phase
  auto prefetch_rest = [&](int c) {   // c >= nc: read as zeros, as in prefetch_qk
    const bool live = c < nc;
    const auto dPhi = live ? rPhi : rNul, dScl = live ? rScl : rNul;
    const auto dGam = live ? rGam : rNul, dAdt = live ? rAdt : rNul;
    if (!live) c = 0;
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
    const int lane = ln & 63;
    const int trow = 16 * strip + (lane & 15);
    const int g8 = 8 * (lane >> 4);
    const uint32_t sphi = (uint32_t)c * C * Nr * 4;

#pragma unroll
    for (int lb = 0; lb < (STRIPS ? 0 : F::LOB); ++lb) {
      // wave-uniform cases first: a block of 32 columns wholly past Nr needs no load, one
      // wholly inside takes 16-byte loads; only a block that Nr cuts tests per lane (a
      // per-lane choice between load widths makes the compiler drain the load queue)
      if (32 * lb >= Nr) {
#pragma unroll
        for (int qd = 0; qd < 2; ++qd) rphi[lb][qd] = f32x4{0.f, 0.f, 0.f, 0.f};
      } else if (phi_vec && 32 * lb + 32 <= Nr) {
#pragma unroll
        for (int qd = 0; qd < 2; ++qd)
          rphi[lb][qd] = buf_load<f32x4>(dPhi, (uint32_t)(trow * Nr + 32 * lb + g8 + 4 * qd) * 4, sphi);
      } else {
#pragma unroll
        for (int qd = 0; qd < 2; ++qd) {
          const int j = 32 * lb + g8 + 4 * qd;
          const uint32_t o = (uint32_t)(trow * Nr + j) * 4;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            rphi[lb][qd][i] = (j + i < Nr) ? buf_load<float>(dPhi, o + 4 * i, sphi) : 0.f;
        }
      }
    }
    // every wave loads the A-scan inputs (only wave 0 uses them): no wave-dependent
    // branch around loads (it would cost exact wait counts)
    if constexpr (RAW) {   // the raw dt and a of the A-scan rows (gamma, scale: build_turns)
      // wave 0 alone reads them: 128 rows of the projection are 128 cache lines, so the
      // other waves' copies of the same loads go through the zero-size descriptor (a
      // wave-uniform choice of descriptor, not a branch around the loads)
      const auto dSc = (live && wave == 0) ? rSc : rNul;
      const uint32_t sc0 = (uint32_t)(c * C * sc_st * 2);
#pragma unroll
      for (int e = 0; e < F::E; ++e) {
        const uint32_t o = (uint32_t)((lane * F::E + e) * sc_st) * 2;
        rdr[e] = (float)buf_load<bf16>(dSc, o, sc0);
        rar[e] = (float)buf_load<bf16>(dSc, o + 2 * p.a_off, sc0);
      }
    } else {
      rscale = buf_load<float>(dScl, (uint32_t)trow * 4, (uint32_t)c * C * 4);
      rgam = buf_load<float>(dGam, (uint32_t)trow * 4, (uint32_t)c * C * 4);
#pragma unroll
      for (int e = 0; e < F::E; ++e)
        radt[e] = buf_load<float>(dAdt, (uint32_t)(lane * F::E + e) * 4, (uint32_t)c * C * 4);
    }
  };

  // raw mode: chunk cc's strip prefixes and total (zeros past the last chunk: the carry
  // adds the total); the other waves issue the same loads through the zero-size descriptor
  auto load_ctot = [&](int cc) {
    if constexpr (RAW) {
      const bool live = cc < nc && wave == 1;
      const auto dX = live ? rPre : rNul, dT = live ? rCt : rNul;
      if (cc >= nc) cc = 0;
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int lane = ln & 63;
      const int st = lane % SPC, q = lane / SPC;
#pragma unroll
      for (int i = 0; i < TL; ++i) {
        const uint32_t j0 = 4 * (q + i * TQ);
        rX[i] = buf_load<f32x4>(dX, (uint32_t)(st * Nr + j0) * 4, (uint32_t)cc * SPC * Nr * 4);
        rC[i] = buf_load<f32x4>(dT, j0 * 4, (uint32_t)cc * Nr * 4);
      }
    }
  };
  // raw mode, the carry wave: the angle entering each strip of chunk cc, P + the strip's
  // prefix, into sE[cc & 1]; then P (Pc, the angle entering chunk cc) moves past the chunk.
  // The other waves read their strip's entry when they build the chunk's turns, two
  // barriers later.
  auto carry = [&](int cc) {
    if constexpr (RAW) {
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int lane = ln & 63;
      const int st = lane % SPC, q = lane / SPC;
#pragma unroll
      for (int i = 0; i < TL; ++i) {
        const int j0 = 4 * (q + i * TQ);
        f32x4 ent;
#pragma unroll
        for (int e = 0; e < 4; ++e) ent[e] = Pc[i][e] + rX[i][e];
        if (j0 < ELD) *reinterpret_cast<f32x4*>(sE + ((cc & 1) * SPC + st) * ELD + j0) = ent;
#pragma unroll
        for (int e = 0; e < 4; ++e) Pc[i][e] = wrap_2pi_fast(Pc[i][e] + rC[i][e]);
      }
    }
  };

  // phi_strips mode: chunk c's table rows, strip angles and dt (issued at the start of the
  // previous chunk's products), and the turns built from them in the middle of those
  // products, where the DPP prefix interleaves with the inter-chunk and state MFMAs
  // instead of lengthening the end of the long strips' phase
  auto prefetch_angles = [&](int c) {
    if constexpr (STRIPS) {
      load_ctot(c + 1);     // raw mode: the carry's inputs for the chunk after this one
      if (c >= nc) c = 0;   // past the end: chunk 0 again, never used
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int lane = ln & 63;
      const int trow = 16 * strip + (lane & 15);
      const int g8 = 8 * (lane >> 4);
      const uint32_t sphi = (uint32_t)c * C * Nr * 4;
      const uint32_t sstr = (uint32_t)(c * (C / 16) + strip) * Nr * 4;
#pragma unroll
      for (int lb = 0; lb < NRB; ++lb) {
        if (phi_vec && 32 * lb + 32 <= Nr) {
#pragma unroll
          for (int qd = 0; qd < 2; ++qd) {
            rtab[lb][qd] = buf_load<f32x4>(rPhi, (uint32_t)(trow * Nr + 32 * lb + g8 + 4 * qd) * 4, sphi);
            if constexpr (!RAW) rstr[lb][qd] = gld<f32x4>(pstrg, sstr + (uint32_t)(32 * lb + g8 + 4 * qd) * 4);
          }
        } else {
#pragma unroll
          for (int qd = 0; qd < 2; ++qd) {
            const int j = 32 * lb + g8 + 4 * qd;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const bool in = j + i < Nr;
              rtab[lb][qd][i] = in ? buf_load<float>(rPhi, (uint32_t)(trow * Nr + j + i) * 4, sphi) : 0.f;
              if constexpr (!RAW) rstr[lb][qd][i] = in ? gld<float>(pstrg, sstr + (uint32_t)(j + i) * 4) : 0.f;
            }
          }
        }
      }
      if constexpr (RAW) {   // one raw scalar per lane: dt or trap of row trow or trow + 1
        const int g = lane >> 4;
        const uint32_t o = (uint32_t)((trow + (g >> 1)) * sc_st + ((g & 1) ? p.t_off : 0)) * 2;
        rraw = (float)buf_load<bf16>(rSc, o, (uint32_t)(c * C * sc_st * 2));
      } else {
        rpdt = gld<float>(pdtg, (uint32_t)(c * C + trow) * 4);
      }
    }
  };
  auto build_turns = [&](int c) {   // chunk c's rows
    if constexpr (RAW) {
      // the row scalars (reference.py:160-199) from the raw slices, the four per row
      // spread over the four lane groups so one softplus-or-sigmoid sequence makes them
      // all: dt_t (g = 0), lam_t (g = 1), dt_{t+1} (g = 2), lam_{t+1} (g = 3), zero past
      // the sequence (the trapezoid's dt_L = lam_L = 0). Hardware exp2 / log2 / rcp on
      // u = 1 + e^{+-x}: softplus = log(u), sigmoid = 1 / u, three transcendentals for both.
      // log(u) loses the bits of e that 1 + e rounds off: 6e-5 relative at dt = 1e-3,
      // far below the bf16 operands dt feeds here (gamma, scale, this strip's angle
      // offsets; the carry across strips comes from the BCNorm pass's exact totals).
      int ln = threadIdx.x;
      asm volatile("" : "+v"(ln));
      const int lane = ln & 63, g = lane >> 4, r = lane & 15;
      const bool isdt = (g & 1) == 0;
      const float x = rraw + (isdt ? dtb : 0.f);
      const float u = 1.f + __builtin_amdgcn_exp2f((isdt ? x : -x) * kLog2e);
      float v = isdt ? (x > 20.f ? x : __builtin_amdgcn_logf(u) * kLn2) : __builtin_amdgcn_rcpf(u);
      if (g >= 2 && c * C + 16 * strip + r + 1 >= L) v = 0.f;
      const float dtt = __shfl(v, r, 64), lamt = __shfl(v, 16 + r, 64);
      const float dtn = __shfl(v, 32 + r, 64), lamn = __shfl(v, 48 + r, 64);
      rgam = dtt * lamt;
      rscale = rgam + dtn * (1.f - lamn);
      rpdt = dtt;
      // the angle entering this wave's strip, from the carry wave
      const float* er = sE + ((c & 1) * SPC + strip) * ELD + 8 * g;
#pragma unroll
      for (int lb = 0; lb < NRB; ++lb) {
#pragma unroll
        for (int qd = 0; qd < 2; ++qd) rstr[lb][qd] = *reinterpret_cast<const f32x4*>(er + 32 * lb + 4 * qd);
      }
    }
    if constexpr (STRIPS) {
#pragma unroll
      for (int lb = 0; lb < NRB; ++lb) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const float th = row_prefix16(rtab[lb][s >> 2][s & 3] * rpdt);
          trn_pre[lb][s] = __builtin_amdgcn_fractf((rstr[lb][s >> 2][s & 3] + th) * 0.15915494309189535f);
        }
      }
    }
  };

  bf16x8 qf[F::NBK];                        // q~ of this wave's strip (MFMA B operand)
  f32x4 out[PB];                            // out^T tiles of this wave's strip

  // ---- phase L: chunk c's raw registers -> q~ (registers), khat (LDS), scalars -----
  // Chunk c's q~ fragments (qf), k-hat rows and row coefficients are computed into
  // registers at the end of chunk c-1's product phase (stage_regs), while other waves
  // still run their products, and written to LDS after the barrier (stage_write).
  bf16x8 kst[2 * F::LOB];        // this lane's k-hat row pieces of the next chunk
  float coefv = 0.f;             // D + gamma_t (u_t . w_t) of this lane's row
  float sAv[F::E], sEv[F::E], sFv[F::E], sDv[F::E];   // wave 0: A_t, 2^{A_t}, 2^{A_last - A_t},
                                                     // 2^{A_strip_end - A_t}
  auto stage_write = [&](int buf) {
    bf16* sK = khat(buf);
    const Scalars sc = scalars(buf);
    float *sA = sc.A, *sExpA = sc.ExpA, *sFac = sc.Fac, *sCoef = sc.Coef, *sDk = sc.Dk;
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
    const int lane = ln & 63;
    const int trow = 16 * strip + (lane & 15);
    const int g8 = 8 * (lane >> 4);
    if (wave == 0) {
#pragma unroll
      for (int e = 0; e < F::E; ++e) {
        const int tt = lane * F::E + e;
        sA[tt] = sAv[e];
        sExpA[tt] = sEv[e];
        sFac[tt] = sFv[e];
        sDk[tt] = sDv[e];
      }
    }
#pragma unroll
    for (int lb = 0; lb < F::LOB; ++lb) {
      *reinterpret_cast<bf16x8*>(sK + trow * LDK + 32 * lb + g8) = kst[lb];
      *reinterpret_cast<bf16x8*>(sK + trow * LDK + 32 * (lb + F::LOB) + g8) = kst[lb + F::LOB];
    }
    if ((lane >> 4) == 0) sCoef[trow] = coefv;
  };
  auto stage_regs = [&]() {
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
    const int lane = ln & 63;
    if (wave == 0) {  // inclusive prefix sum of adt * log2(e)
      float a[F::E];
      float run = 0.f;
#pragma unroll
      for (int e = 0; e < F::E; ++e) {
        float adt;
        if constexpr (RAW) {   // reference.py:160-199: a = min(-heavy_tail(a_raw), -a_floor)
          adt = fminf(-heavy_tail_fast(rar[e]), -p.a_floor) * softplus_fast(rdr[e] + dtb);
        } else {
          adt = radt[e];
        }
        run += adt * kLog2e;
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
      // A at the last row of this lane's 16-row strip (rows lane E .. lane E + E - 1)
      const float a_strip = __shfl(incl, lane | (16 / F::E - 1), 64);
#pragma unroll
      for (int e = 0; e < F::E; ++e) {
        const float A = excl + a[e];
        sAv[e] = A;
        sEv[e] = exp2f(A);
        sFv[e] = exp2f(a_last - A);
        sDv[e] = exp2f(a_strip - A);
      }
    }
    const int g8 = 8 * (lane >> 4);
    float uw = 0.f;
    // u = q + qb, w = k + kb for one pair (n, n + N/2) of this lane's block lb, s < 8
    auto pair = [&](int lb, int s, const f32x4 (&bql)[2], const f32x4 (&bqh)[2],
                    const f32x4 (&bkl)[2], const f32x4 (&bkh)[2], float& ql, float& qh,
                    float& kl, float& kh) {
      const int hb = lb + F::LOB;
      ql = (float)rq[lb][s] + bql[s >> 2][s & 3];
      qh = (float)rq[hb][s] + bqh[s >> 2][s & 3];
      kl = (float)rk[lb][s] + bkl[s >> 2][s & 3];
      kh = (float)rk[hb][s] + bkh[s >> 2][s & 3];
    };
    // angle s of this lane's block lb, in turns: phi is read wrapped to [0, 2 pi); in
    // phi_strips mode build_turns made it during the previous products (the strip's
    // entering angle plus the inclusive prefix of theta = tanh(angles) pi dt over the
    // strip's rows -- the 16 lanes of a DPP row are the strip's 16 rows -- keeping the
    // fraction of a turn); blocks at or past NRB hold no rotary pair.
    auto turns_of = [&](int lb, int s) {
      if constexpr (STRIPS) {
        return lb < NRB ? trn_pre[lb < NRB ? lb : 0][s] : 0.f;
      } else {
        return rphi[lb][s >> 2][s & 3] * 0.15915494309189535f;
      }
    };
    // rotate (lo, hi) by an angle given in turns, with the hardware sin / cos; accurate
    // far below the bf16 rounding of what they feed
    auto rotate = [](float turns, float& ql, float& qh, float& kl, float& kh) {
      const float sn = __builtin_amdgcn_sinf(turns), cs = __builtin_amdgcn_cosf(turns);
      const float q0 = ql * cs - qh * sn, q1 = qh * cs + ql * sn;
      const float k0 = kl * cs - kh * sn, k1 = kh * cs + kl * sn;
      ql = q0; qh = q1; kl = k0; kh = k1;
    };
    auto load_bias = [&](int lb, f32x4 (&bql)[2], f32x4 (&bqh)[2], f32x4 (&bkl)[2],
                         f32x4 (&bkh)[2]) {
      const int nb8 = 32 * lb + g8;   // this lane's 8 bias columns, as 16-byte LDS reads
#pragma unroll
      for (int h4 = 0; h4 < 2; ++h4) {
        bql[h4] = *reinterpret_cast<const f32x4*>(sQb + nb8 + 4 * h4);
        bqh[h4] = *reinterpret_cast<const f32x4*>(sQb + nb8 + H2 + 4 * h4);
        bkl[h4] = *reinterpret_cast<const f32x4*>(sKb + nb8 + 4 * h4);
        bkh[h4] = *reinterpret_cast<const f32x4*>(sKb + nb8 + H2 + 4 * h4);
      }
    };
#pragma unroll
    for (int lb = 0; lb < F::LOB; ++lb) {
      const int hb = lb + F::LOB;
      f32x4 bql[2], bqh[2], bkl[2], bkh[2];
      load_bias(lb, bql, bqh, bkl, bkh);
      // which of the block's 32 pairs are rotary (n < Nr) is uniform over the wave except
      // for a block that Nr cuts: one code path per case, chosen by a scalar branch, so
      // only that block tests per pair (a per-pair test costs an exec-mask branch and
      // register copies on every pair)
      auto run = [&](auto mode) {
        constexpr int M = decltype(mode)::value;   // 0: none rotary, 1: all, 2: n < Nr
        float trn[8];
        if constexpr (M != 0) {
#pragma unroll
          for (int s = 0; s < 8; ++s) trn[s] = turns_of(lb, s);
        }
        bf16x8 kl8, kh8;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          float ql, qh, kl, kh;
          pair(lb, s, bql, bqh, bkl, bkh, ql, qh, kl, kh);
          uw += ql * kl + qh * kh;
          if constexpr (M == 1) {
            rotate(trn[s], ql, qh, kl, kh);
          } else if constexpr (M == 2) {
            if (32 * lb + g8 + s < Nr) rotate(trn[s], ql, qh, kl, kh);
          }
          qf[lb][s] = (bf16)ql;
          qf[hb][s] = (bf16)qh;
          kl8[s] = (bf16)(kl * rscale);
          kh8[s] = (bf16)(kh * rscale);
        }
        kst[lb] = kl8;
        kst[hb] = kh8;
      };
      if (32 * lb + 32 <= Nr) {
        run(IntTag<1>{});
      } else if (32 * lb >= Nr) {
        run(IntTag<0>{});
      } else {
        run(IntTag<2>{});
      }
    }
    uw += __shfl_xor(uw, 16, 64);
    uw += __shfl_xor(uw, 32, 64);
    coefv = rgam * uw + dsk;
  };

  // ---- phase G: scores, intra + inter + diagonal output, state update -------------
  auto products = [&](int c) {
    const bf16* sK = khat(c & 1);
    const Scalars sc = scalars(c & 1);
    const float *sA = sc.A, *sExpA = sc.ExpA, *sFac = sc.Fac, *sCoef = sc.Coef, *sDk = sc.Dk;
    // lane index re-derived opaquely: the per-lane LDS addresses below are recomputed
    // each chunk instead of being hoisted out of the chunk loop (and spilled)
    prefetch_angles(c + 1);
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
    const int lane = ln & 63;
    const int tb = strip;
    const int tcol = tb * 16 + (lane & 15);
    const int g4 = 4 * (lane >> 4);
    const float At = sA[tcol];
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) out[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // masked, decayed score tile s^T[j][t] for key strip jb (rows j) and this wave's
    // query strip (columns t), as a sub-fragment with K = j.
    // Below the diagonal (jb < tb) every entry is causal and the decay factors through
    // the key strip's last row m: 2^{A_t - A_j} = 2^{A_t - A_m} 2^{A_m - A_j}, both
    // factors in (0, 1] since A falls along the chunk (t > m >= j); one exp per lane
    // and tile instead of one per entry. The diagonal tile keeps the exact per-entry
    // decay and the mask as a select (its decay 2^{min(A_t - A_j, 0)} is finite for
    // every entry, masked or not).
    // Each step reads all its fragments (k-hat rows of both key strips, v^T of both, the
    // decay factors) before the first MFMA: one LDS round trip per pair of key strips
    // instead of one per fragment group.
    struct PairFrags {
      bf16x8 ka[F::NBK], kb[F::NBK];   // k-hat rows of key strips jb, jb + 1
      bf16x4 va[PB], vb[PB];           // v^T of the same rows
      f32x4 da, db;                    // sDk (off-diagonal) or sA (diagonal) of the rows
      float ma, mb;                    // A at each strip's last row
    };
    int vo[PB];   // this lane's v^T read offsets in the first 16-row band
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) vo[pb] = vz_tr_off(g4, pb * 16, lane);
    // second strip: 0 none, 1 below the diagonal, 2 the diagonal strip (its decay rows
    // are A itself)
    auto load_pair = [&](int jb, int second, PairFrags& f) {
#pragma unroll
      for (int blk = 0; blk < F::NBK; ++blk) f.ka[blk] = ld_nat8(sK, LDK, jb * 16, 32 * blk, lane);
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) f.va[pb] = ld_tr4_at(sV + jb * 16 * 64 + vo[pb]);
      f.da = *reinterpret_cast<const f32x4*>(sDk + jb * 16 + g4);
      f.ma = sA[jb * 16 + 15];
      if (second) {
#pragma unroll
        for (int blk = 0; blk < F::NBK; ++blk) f.kb[blk] = ld_nat8(sK, LDK, jb * 16 + 16, 32 * blk, lane);
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) f.vb[pb] = ld_tr4_at(sV + (jb + 1) * 16 * 64 + vo[pb]);
        f.db = *reinterpret_cast<const f32x4*>((second == 2 ? sA : sDk) + jb * 16 + 16 + g4);
        f.mb = sA[jb * 16 + 31];
      }
    };
    auto qk_acc = [&](const bf16x8 (&kf)[F::NBK]) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int blk = 0; blk < F::NBK; ++blk) mma32x(acc, kf[blk], qf[blk]);
      return acc;
    };
    // below the diagonal: the factored decay
    auto decay_off = [&](const f32x4& acc, const f32x4& dk, float m) {
      const float et = __builtin_amdgcn_exp2f(At - m);
      f32x4 sv;
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = acc[i] * (et * dk[i]);
      return sub_from_f32<bf16>(sv);
    };
    // the diagonal strip: exact decay, causal mask as a select
    auto decay_diag = [&](const f32x4& acc, const f32x4& aj) {
      f32x4 sv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = tb * 16 + g4 + i;
        const float dec = __builtin_amdgcn_exp2f(fminf(At - aj[i], 0.f));
        sv[i] = (tcol > j) ? acc[i] * dec : 0.f;
      }
      return sub_from_f32<bf16>(sv);
    };
    // intra-chunk: out^T[p][t] += sum_j v^T[p][j] s^T[j][t]   (v^T by transposed reads),
    // one pair of key strips per step (K = 32): the pairs wholly below the diagonal, then
    // the diagonal strip, alone (tb even) or with the strip before it (tb odd)
    const int npair = tb >> 1;
    PairFrags fr;
#pragma unroll 1
    for (int ip = 0; ip < npair; ++ip) {
      load_pair(2 * ip, 1, fr);
      const f32x4 a0 = qk_acc(fr.ka), a1 = qk_acc(fr.kb);
      const bf16x4 s0 = decay_off(a0, fr.da, fr.ma), s1 = decay_off(a1, fr.db, fr.mb);
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) mma32(out[pb], fr.va[pb], fr.vb[pb], s0, s1);
    }
    if (tb & 1) {
      load_pair(tb - 1, 2, fr);
      const f32x4 a0 = qk_acc(fr.ka), a1 = qk_acc(fr.kb);
      const bf16x4 s0 = decay_off(a0, fr.da, fr.ma), s1 = decay_diag(a1, fr.db);
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) mma32(out[pb], fr.va[pb], fr.vb[pb], s0, s1);
    } else {
      load_pair(tb, 0, fr);
      fr.da = *reinterpret_cast<const f32x4*>(sA + tb * 16 + g4);
      const bf16x4 s0 = decay_diag(qk_acc(fr.ka), fr.da);
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) mma16(out[pb], fr.va[pb], s0);
    }
    // next chunk's inputs: issued here so the memory-issue waits overlap MFMA work
    // (the next chunk's v and this chunk's gate z, written in the next phase A)
    __builtin_amdgcn_sched_barrier(0);
    prefetch_rest(c + 1);
    prefetch_vz(c + 1 < nc ? rV : rNul, c + 1 < nc ? c + 1 : 0, rZ, c);
    __builtin_amdgcn_sched_barrier(0);
    build_turns(c + 1);   // chunk c+1's angles (phi_strips mode)
    // inter-chunk: out^T[p][t] += 2^{A_t} sum_n S[p][n] q~[t][n]
    // (every fragment of S, the diagonal v values and the scalars are read first, then
    // PB independent MFMA chains: one LDS round trip)
    const float eA = sExpA[tcol];
    const float coef = sCoef[tcol];
    bf16x8 sfr[PB][F::NBK];
    bf16x4 vd[PB];
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
#pragma unroll
      for (int blk = 0; blk < F::NBK; ++blk) sfr[pb][blk] = ld_nat8(sS, LDK, pb * 16, 32 * blk, lane);
      vd[pb] = *reinterpret_cast<const bf16x4*>(sV + vz_off(tcol, pb * 16 + g4));
    }
    f32x4 it[PB];
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) it[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int blk = 0; blk < F::NBK; ++blk) {
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) mma32x(it[pb], sfr[pb][blk], qf[blk]);
    }
    // diagonal and skip: (D + gamma_t u_t . w_t) v_t
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) out[pb][i] = (out[pb][i] + eA * it[pb][i]) + coef * (float)vd[pb][i];
    }
    // state: S <- 2^{A_last} S + sum_t (v_t 2^{A_last - A_t}) khat_t^T   (K = time)
    const float eAl = sExpA[C - 1];
#pragma unroll
    for (int m = 0; m < SPW; ++m) {
#pragma unroll
      for (int i = 0; i < 4; ++i) Sacc[m][i] *= eAl;
    }
    const int g8 = 8 * (lane >> 4);
    const int vs0 = vz_tr_off(0, pb_w * 16, lane), vs1 = vz_tr_off(4, pb_w * 16, lane);
    // software-pipelined over the C/32 K steps: step i+1's fragments are read into the
    // other register set before step i's scaling and MFMAs, so LDS latency overlaps them
    struct StepFrags {
      bf16x4 a0, a1;
      f32x4 f0, f1;
      bf16x4 kb0[SPW], kb1[SPW];
    };
    auto load_step = [&](int k0, StepFrags& fr) {
      const int kb = k0 + g8;                          // a multiple of 8
      fr.a0 = ld_tr4_at(sV + kb * 64 + vs0);
      fr.a1 = ld_tr4_at(sV + kb * 64 + vs1);
      fr.f0 = *reinterpret_cast<const f32x4*>(sFac + kb);
      fr.f1 = *reinterpret_cast<const f32x4*>(sFac + kb + 4);
#pragma unroll
      for (int m = 0; m < SPW; ++m) {
        const int nb = nb0 + NSTEP * m;
        fr.kb0[m] = ld_tr4(sK, LDK, kb, nb * 16, lane);
        fr.kb1[m] = ld_tr4(sK, LDK, kb + 4, nb * 16, lane);
      }
    };
    auto run_step = [&](StepFrags& fr) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        fr.a0[s] = (bf16)((float)fr.a0[s] * fr.f0[s]);
        fr.a1[s] = (bf16)((float)fr.a1[s] * fr.f1[s]);
      }
#pragma unroll
      for (int m = 0; m < SPW; ++m) mma32(Sacc[m], fr.a0, fr.a1, fr.kb0[m], fr.kb1[m]);
    };
    StepFrags fa, fb;
    load_step(0, fa);
#pragma unroll
    for (int k0 = 0; k0 < C; k0 += 64) {
      if (k0 + 32 < C) load_step(k0 + 32, fb);
      run_step(fa);
      if (k0 + 64 < C) load_step(k0 + 64, fa);
      if (k0 + 32 < C) run_step(fb);
    }
  };

  // ---- phase E (light waves): gate, 16-byte row stores -----------------------------
  auto epilogue = [&](int c) {
    int ln = threadIdx.x;
    asm volatile("" : "+v"(ln));
    const int tid = ln;
    const int t0 = c * C;
#pragma unroll
    for (int r = 0; r < F::VR; ++r) {
      const int task = tid + r * F::VTH;
      if (task < F::VT) {
        const int tp = task / F::VG, p0 = (task % F::VG) * 8;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int t = 2 * tp + e;
          float yb[8];
#pragma unroll
          for (int i = 0; i < 8; i += 4) {
            const f32x4 o = *reinterpret_cast<const f32x4*>(sOut + t * LDO + p0 + i);
#pragma unroll
            for (int u = 0; u < 4; ++u) yb[i + u] = o[u];
          }
          if (p.save) {
            bf16x8 ybv;
#pragma unroll
            for (int i = 0; i < 8; ++i) ybv[i] = (bf16)yb[i];
            buf_store(ybv, rYb, (uint32_t)(t * P + p0) * 2, (uint32_t)t0 * P * 2);
          }
          bf16x8 zz;
          if (zg) zz = *reinterpret_cast<const bf16x8*>(sZ + vz_off(t, p0));
          bf16x8 yo;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float g = zg ? silu_fast((float)zz[i]) : 1.f;
            yo[i] = (bf16)(yb[i] * g);
          }
          buf_store(yo, rY, (uint32_t)(t * p.y_st + p0) * 2, (uint32_t)(t0 * p.y_st * 2));
        }
      }
    }
  };

  if constexpr (RAW) {   // the carry starts from phi_init; the strip entries of chunk 0 first
    const int q = lane / SPC;
#pragma unroll
    for (int i = 0; i < TL; ++i) {
      const int j0 = 4 * (q + i * TQ);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        Pc[i][e] = (p.phi_init && j0 + e < Nr) ? p.phi_init[bh * Nr + j0 + e] : 0.f;
    }
    load_ctot(0);
    vm_wait_all();
    if (wave == 1) carry(0);
  }
  prefetch_vz(rV, 0, rNul, 0);
  prefetch_qk(0);
  prefetch_rest(0);
  prefetch_angles(0);   // (raw mode: the carry's inputs for chunk 1)
  vm_wait_all();
  if constexpr (RAW) {
    if (wave == 1) carry(1);
  }
  __syncthreads();  // sQb / sKb (raw mode: the strip entries of chunks 0 and 1)
  build_turns(0);
  stage_regs();     // chunk 0
  stage_write(0);
  prefetch_qk(1);
  // phase A of chunk c (and of the tail): out(c-1) to sOut, S(c) to sS
  auto phase_a = [&](int c) {
    if (c > 0) {
      const int tcol = strip * 16 + (lane & 15);
#pragma unroll
      for (int pb = 0; pb < PB; ++pb)
        *reinterpret_cast<f32x4*>(sOut + tcol * LDO + pb * 16 + 4 * (lane >> 4)) = out[pb];
    }
    publish_state(c);
  };
  for (int c = 0; c < nc; ++c) {
    // ---------------- phase A: also chunk c's k-hat and scalars, v of c, z of c-1 --------
    phase_a(c);
    write_vz(c == nc - 1);   // (zeros where there is no such chunk)
    __syncthreads();
    // ---------------- phase B: epilogue of c-1, products of c, then chunk c+1's rotation
    // into registers (a wave whose products end early rotates while others still run
    // theirs: the VALU work overlaps the partner wave's MFMA work on the same SIMD).
    // Every load is issued on every chunk (past the end through a zero-size
    // descriptor), so the compiler's wait counts stay exact across iterations.
    if (c > 0 && light) epilogue(c - 1);
    products(c);
    store_state(c);
    if constexpr (RAW) {   // the strip entries of chunk c+2 (its inputs came with c+1's angles)
      if (wave == 1) carry(c + 2);
    }
    stage_regs();
    stage_write((c + 1) & 1);   // chunk c+1's k-hat rows and scalars, into the other buffer
    __builtin_amdgcn_sched_barrier(0);
    prefetch_qk(c + 2);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
  }
  // tail: out and z of the last chunk, its epilogue
  phase_a(nc);
  write_vz(false);
  if constexpr (RAW) {   // the carry past the last chunk is phi at L-1: phi_final, and LDS
    if (wave == 1) {     // row 0 of the strip table (no longer read) for final_k
      const int st = lane % SPC, q = lane / SPC;
#pragma unroll
      for (int i = 0; i < TL; ++i) {
        const int j0 = 4 * (q + i * TQ);
        if (st == 0 && j0 < ELD) {
          *reinterpret_cast<f32x4*>(sE + j0) = Pc[i];
          if (j0 < Nr) *reinterpret_cast<f32x4*>(p.phi_final + bh * Nr + j0) = Pc[i];
        }
      }
    }
  }
  __syncthreads();
  if (light) epilogue(nc - 1);

  // final state
#pragma unroll
  for (int m = 0; m < SPW; ++m) {
    const int ncol = (nb0 + NSTEP * m) * 16 + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int prow = pb_w * 16 + 4 * (lane >> 4) + i;
      p.fssm[(bh * P + prow) * N + ncol] = Sacc[m][i];
    }
  }
  // final_k: the sequence's last key row, rotated and unscaled (the same arithmetic as
  // the stage), one rotary pair per lane of wave 0
  if (wave == 0 && lane < H2) {
    const int j = lane;
    const int64_t row = (int64_t)(L - 1) * N;
    float kl = (float)kg[row + j] + sKb[j], kh = (float)kg[row + H2 + j] + sKb[H2 + j];
    if (j < Nr) {
      float turns;
      if constexpr (RAW) {
        turns = __builtin_amdgcn_fractf(sE[j] * 0.15915494309189535f);
      } else if constexpr (STRIPS) {   // the last strip's entering angle plus its 16 thetas
        float ph = p.pstr[(bh * (L / 16) + L / 16 - 1) * Nr + j];
        for (int t = L - 16; t < L; ++t) ph += phig[(int64_t)t * Nr + j] * p.pdt[bh * L + t];
        turns = __builtin_amdgcn_fractf(ph * 0.15915494309189535f);
      } else {
        turns = phig[(int64_t)(L - 1) * Nr + j] * 0.15915494309189535f;
      }
      const float sn = __builtin_amdgcn_sinf(turns), cs = __builtin_amdgcn_cosf(turns);
      const float k0 = kl * cs - kh * sn, k1 = kh * cs + kl * sn;
      kl = k0;
      kh = k1;
    }
    p.fk[bh * N + j] = kl;
    p.fk[bh * N + H2 + j] = kh;
  }
}

// Every per-(b, h) stream of fwd_bf16_kernel must be addressable with 31-bit byte
// offsets from its buffer descriptor.
static bool fits_rsrc(const FwdParams& p, int N, int P) {
  const int64_t lim = (int64_t(1) << 31) - 1;
  const int64_t L = p.L;
  auto span = [&](int64_t st) { return ((L - 1) * st + P) * 2; };
  return L * N * 2 <= lim && L * p.Nr * 4 <= lim && span(p.v_st) <= lim &&
         (!p.has_z || span(p.z_st) <= lim) && span(p.y_st) <= lim && L * P * 4 <= lim &&
         (int64_t)p.nc * N * P * 2 <= lim;
}

// Raw mode's kernel for this (dtype, C, N, P, Nr): the bf16 kernel with phi built, where
// its strip-angle table fits the LDS. -1 where there is none.
template <typename MT, int C, int N, int P>
constexpr int raw_nrb_max() {
  if constexpr (std::is_same<MT, bf16>::value && N % 64 == 0 && C % 64 == 0) {
    if constexpr (N / 64 >= 2 && raw_fits<C, N, P, 2>()) return 2;
    if constexpr (raw_fits<C, N, P, 1>()) return 1;
  }
  return 0;
}

template <typename MT, int C, int N, int P>
static int32_t launch_fwd(const FwdParams& prm, int grid, hipStream_t stream) {
  const bool strips = prm.pstr != nullptr;
  if (prm.sc != nullptr) {   // raw mode: the bf16 kernel where it applies, else the generic one
    // the bf16 kernel addresses the raw slices and every stream through buffer descriptors
    const bool fast = fits_rsrc(prm, N, P) &&
                      ((int64_t)(prm.L - 1) * prm.sc_st + prm.sc_span) * (int64_t)sizeof(MT) < (1ll << 31);
    if constexpr (raw_nrb_max<MT, C, N, P>() >= 1) {
      if (fast && prm.Nr <= 32) {
        hipLaunchKernelGGL((fwd_bf16_kernel<C, N, P, 1, true>), dim3(grid), dim3(C / 16 * 64), 0, stream, prm);
        return launch_status("m3s_fwd");
      }
    }
    if constexpr (raw_nrb_max<MT, C, N, P>() >= 2) {
      if (fast && prm.Nr <= 64) {
        hipLaunchKernelGGL((fwd_bf16_kernel<C, N, P, 2, true>), dim3(grid), dim3(C / 16 * 64), 0, stream, prm);
        return launch_status("m3s_fwd");
      }
    }
    constexpr int NWr = (C / 16) > 4 ? (C / 16) : 4;
    hipLaunchKernelGGL((fwd_kernel<MT, C, N, P, NWr, true, true>), dim3(grid), dim3(NWr * 64), 0, stream, prm);
    return launch_status("m3s_fwd");
  }
  if constexpr (std::is_same<MT, bf16>::value && N % 64 == 0 && C % 64 == 0) {
    if (fits_rsrc(prm, N, P)) {
      // phi strips: NRB 32-column blocks hold the rotary pairs (Nr <= 32 NRB); only
      // NRB = 1 and 2 are compiled, so Nr > 64 takes the generic kernel below
      if (strips && prm.Nr <= 32) {
        hipLaunchKernelGGL((fwd_bf16_kernel<C, N, P, 1>), dim3(grid), dim3(C / 16 * 64), 0, stream, prm);
        return launch_status("m3s_fwd");
      }
      if constexpr (N / 64 >= 2) {
        if (strips && prm.Nr <= 64) {
          hipLaunchKernelGGL((fwd_bf16_kernel<C, N, P, 2>), dim3(grid), dim3(C / 16 * 64), 0, stream, prm);
          return launch_status("m3s_fwd");
        }
      }
      if (!strips) {
        hipLaunchKernelGGL((fwd_bf16_kernel<C, N, P, 0>), dim3(grid), dim3(C / 16 * 64), 0, stream, prm);
        return launch_status("m3s_fwd");
      }
    }
  }
  {
    constexpr int NW = (C / 16) > 4 ? (C / 16) : 4;
    if (strips)
      hipLaunchKernelGGL((fwd_kernel<MT, C, N, P, NW, true>), dim3(grid), dim3(NW * 64), 0, stream, prm);
    else
      hipLaunchKernelGGL((fwd_kernel<MT, C, N, P, NW, false>), dim3(grid), dim3(NW * 64), 0, stream, prm);
  }
  return launch_status("m3s_fwd");
}

// The (dtype, chunk, N, P) instantiations compiled into the library. Every backward
// configuration (m3s_bwd.hip) is also a forward one.
#define M3S_FWD_CONFIGS(X)  \
  X(bf16, 128, 128, 64)     \
  X(bf16, 64, 128, 64)      \
  X(bf16, 32, 128, 64)      \
  X(bf16, 128, 64, 64)      \
  X(bf16, 64, 64, 64)       \
  X(bf16, 32, 64, 64)       \
  X(bf16, 128, 32, 16)      \
  X(bf16, 64, 32, 16)       \
  X(bf16, 32, 32, 16)       \
  X(bf16, 128, 16, 16)      \
  X(bf16, 64, 16, 16)       \
  X(bf16, 32, 16, 16)       \
  X(bf16, 32, 256, 64)     \
  X(float, 64, 128, 64)     \
  X(float, 32, 128, 64)     \
  X(float, 64, 64, 64)      \
  X(float, 32, 64, 64)      \
  X(float, 128, 32, 16)     \
  X(float, 64, 32, 16)      \
  X(float, 32, 32, 16)      \
  X(float, 128, 16, 16)     \
  X(float, 64, 16, 16)      \
  X(float, 32, 16, 16)

template <typename MT> constexpr int dtype_code();
template <> constexpr int dtype_code<bf16>() { return M3S_DTYPE_BF16; }
template <> constexpr int dtype_code<float>() { return M3S_DTYPE_F32; }

int32_t fwd_supported(int dtype, int chunk, int n, int pdim) {
#define X(MT, C, N, P) \
  if (dtype == dtype_code<MT>() && chunk == C && n == N && pdim == P) return 1;
  M3S_FWD_CONFIGS(X)
#undef X
  return 0;
}

// Every compiled configuration takes raw mode: the bf16 kernel where raw_nrb_max allows,
// the generic kernel otherwise.
int32_t fwd_raw_supported_impl(int dtype, int chunk, int n, int pdim, int nr) {
  if (nr <= 0 || nr % 4 != 0) return 0;
  return fwd_supported(dtype, chunk, n, pdim);
}

}  // namespace m3s

extern "C" int32_t m3s_fwd(const m3s_fwd_args* a, void* stream) {
  using namespace m3s;
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_fwd: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_fwd_args),
              "m3s_fwd: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_fwd_args));
  const int B = a->batch, L = a->seqlen, H = a->nheads, P = a->headdim, N = a->state_dim,
            Nr = a->n_angles, C = a->chunk;
  M3S_REQUIRE(B > 0 && L > 0 && H > 0 && P > 0 && N > 0 && C > 0,
              "m3s_fwd: non-positive dimension");
  M3S_REQUIRE(L % C == 0, "m3s_fwd: seqlen %d is not a multiple of chunk %d", L, C);
  M3S_REQUIRE(Nr >= 0 && 2 * Nr <= N, "m3s_fwd: n_angles %d exceeds state_dim/2", Nr);
  M3S_REQUIRE(a->dtype == M3S_DTYPE_BF16 || a->dtype == M3S_DTYPE_F32, "m3s_fwd: bad dtype %d",
              a->dtype);
  if (!fwd_supported(a->dtype, C, N, P)) {
    set_error("m3s_fwd: no kernel for dtype=%s chunk=%d state_dim=%d headdim=%d",
              a->dtype == M3S_DTYPE_BF16 ? "bf16" : "f32", C, N, P);
    return M3S_ERR_UNSUPPORTED;
  }
  const int vec = a->dtype == M3S_DTYPE_BF16 ? 8 : 4;
  M3S_REQUIRE(a->q && a->k && aligned16(a->q) && aligned16(a->k), "m3s_fwd: q/k null or misaligned");
  M3S_REQUIRE(bhlp_ok(a->v, vec), "m3s_fwd: v null, misaligned or strides not multiples of %d", vec);
  M3S_REQUIRE(!a->has_z || bhlp_ok(a->z, vec), "m3s_fwd: z null, misaligned or bad strides");
  M3S_REQUIRE(bhlp_ok(a->y, vec), "m3s_fwd: y null, misaligned or bad strides");
  const bool raw = a->raw != 0;
  const bool strips = !raw && (a->theta_table || a->phi_dt || a->phi_strips);
  int a_off = 0, t_off = 0;
  if (raw) {
    M3S_REQUIRE(!a->adt && !a->gamma && !a->scale && !a->phi && !a->phi_dt && !a->phi_strips,
                "m3s_fwd: raw mode takes the raw slices, not adt / gamma / scale / phi");
    M3S_REQUIRE(a->theta_table && a->theta_prefix && a->theta_chunk_totals &&
                    aligned16(a->theta_table) && aligned16(a->theta_prefix) &&
                    aligned16(a->theta_chunk_totals),
                "m3s_fwd: raw mode needs theta_table, theta_prefix and theta_chunk_totals, "
                "16-byte aligned");
    M3S_REQUIRE(!a->save_residuals, "m3s_fwd: raw mode does not save residuals (the backward "
                "reads the materialised scalars)");
    M3S_REQUIRE(Nr > 0 && Nr % 4 == 0 && L % 16 == 0,
                "m3s_fwd: raw mode needs n_angles %% 4 == 0 (got %d) and seqlen %% 16 == 0", Nr);
    M3S_REQUIRE(a->dt_raw.ptr && a->a_raw.ptr && a->trap_raw.ptr && a->dt_bias && a->phi_final &&
                    aligned16(a->phi_final),
                "m3s_fwd: raw mode needs dt_raw, a_raw, trap_raw, dt_bias and phi_final");
    M3S_REQUIRE(a->a_raw.stride_b == a->dt_raw.stride_b && a->trap_raw.stride_b == a->dt_raw.stride_b &&
                    a->a_raw.stride_t == a->dt_raw.stride_t && a->trap_raw.stride_t == a->dt_raw.stride_t,
                "m3s_fwd: the raw slices must share their strides");
    const int esz = a->dtype == M3S_DTYPE_BF16 ? 2 : 4;
    const int64_t da = (const char*)a->a_raw.ptr - (const char*)a->dt_raw.ptr;
    const int64_t dtr = (const char*)a->trap_raw.ptr - (const char*)a->dt_raw.ptr;
    M3S_REQUIRE(da >= 0 && dtr >= 0 && da % esz == 0 && dtr % esz == 0 &&
                    da / esz + H <= a->dt_raw.stride_t && dtr / esz + H <= a->dt_raw.stride_t,
                "m3s_fwd: a_raw / trap_raw must start a fixed number of elements after dt_raw "
                "within each row");
    a_off = (int)(da / esz);
    t_off = (int)(dtr / esz);
    if (!fwd_raw_supported_impl(a->dtype, C, N, P, Nr)) {
      set_error("m3s_fwd: no raw-mode kernel for dtype=%s chunk=%d state_dim=%d headdim=%d "
                "n_angles=%d", a->dtype == M3S_DTYPE_BF16 ? "bf16" : "f32", C, N, P, Nr);
      return M3S_ERR_UNSUPPORTED;
    }
  }
  M3S_REQUIRE(!strips || (a->theta_table && a->phi_dt && a->phi_strips && !a->phi),
              "m3s_fwd: give phi, or theta_table, phi_dt and phi_strips (not both)");
  M3S_REQUIRE(!strips || L % 16 == 0, "m3s_fwd: phi_strips needs seqlen %% 16 == 0");
  M3S_REQUIRE((raw || (a->adt && a->gamma && a->scale && (a->phi || strips))) && a->q_bias &&
                  a->k_bias,
              "m3s_fwd: a required input pointer is NULL");
  M3S_REQUIRE(raw || Nr == 0 || Nr % 4 != 0 ||
                  (strips ? aligned16(a->theta_table) && aligned16(a->phi_strips) : aligned16(a->phi)),
              "m3s_fwd: phi (or theta_table / phi_strips) misaligned");
  M3S_REQUIRE(!a->has_d || a->d_skip, "m3s_fwd: has_d but d_skip is NULL");
  M3S_REQUIRE(!a->has_seed || (a->seed_ssm && a->seed_k && a->seed_v && a->seed_coef),
              "m3s_fwd: seed_ssm, seed_k, seed_v and seed_coef must be given together");
  M3S_REQUIRE(!a->save_residuals || (a->ybar && a->chunk_states && aligned16(a->ybar) &&
                                     aligned16(a->chunk_states)),
              "m3s_fwd: residual outputs NULL or misaligned");
  M3S_REQUIRE(a->final_ssm && a->final_k && a->final_v, "m3s_fwd: final state outputs NULL");
  M3S_REQUIRE((int64_t)B * H < (1ll << 31), "m3s_fwd: B*H too large");

  FwdParams prm{};
  prm.B = B; prm.L = L; prm.H = H; prm.Nr = Nr; prm.nc = L / C;
  prm.has_d = a->has_d; prm.has_z = a->has_z; prm.has_seed = a->has_seed;
  prm.save = a->save_residuals;
  prm.q = a->q; prm.k = a->k;
  prm.v = a->v.ptr; prm.v_sb = a->v.stride_b; prm.v_sh = a->v.stride_h; prm.v_st = a->v.stride_t;
  prm.z = a->has_z ? a->z.ptr : nullptr;
  prm.z_sb = a->z.stride_b; prm.z_sh = a->z.stride_h; prm.z_st = a->z.stride_t;
  prm.adt = a->adt; prm.gamma = a->gamma; prm.scale = a->scale; prm.phi = a->phi;
  prm.tht = (strips || raw) ? a->theta_table : nullptr;
  prm.pdt = strips ? a->phi_dt : nullptr;
  prm.pstr = strips ? a->phi_strips : nullptr;
  prm.qb = a->q_bias; prm.kb = a->k_bias; prm.dsk = a->d_skip;
  prm.seed_ssm = a->seed_ssm; prm.seed_k = a->seed_k; prm.seed_v = a->seed_v;
  prm.seed_coef = a->seed_coef;
  prm.y = a->y.ptr; prm.y_sb = a->y.stride_b; prm.y_sh = a->y.stride_h; prm.y_st = a->y.stride_t;
  prm.ybar = a->ybar; prm.cstates = a->chunk_states;
  prm.fssm = a->final_ssm; prm.fk = a->final_k; prm.fv = a->final_v;
  if (raw) {
    prm.sc = a->dt_raw.ptr; prm.sc_sb = a->dt_raw.stride_b; prm.sc_st = a->dt_raw.stride_t;
    prm.a_off = a_off; prm.t_off = t_off; prm.sc_span = std::max(a_off, t_off) + 1;
    prm.a_floor = a->a_floor;
    prm.dt_bias = a->dt_bias;
    prm.tpre = a->theta_prefix;
    prm.ctot = a->theta_chunk_totals;
    prm.phi_init = a->phi_init;
    prm.phi_final = a->phi_final;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid = B * H;
#define X(MT, CC, NN, PP)                                                     \
  if (a->dtype == dtype_code<MT>() && C == CC && N == NN && P == PP)          \
    return launch_fwd<MT, CC, NN, PP>(prm, grid, s);
  M3S_FWD_CONFIGS(X)
#undef X
  set_error("m3s_fwd: unreachable dispatch");
  return M3S_ERR_UNSUPPORTED;
}
