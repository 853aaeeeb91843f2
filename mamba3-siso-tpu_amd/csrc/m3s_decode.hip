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
      const float rq = 1.f / sqrtf(sq / (float)N + p.eps), rk = 1.f / sqrtf(sk / (float)N + p.eps);
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
          const float th = tanhf(ang) * kPi * dt;
          const float phi = wrap_2pi(p.phist[bh * p.Nr + j] + th);
          p.phist[bh * p.Nr + j] = phi;
          sincosf(phi, &sn, &cs);
        }
        sQt[j] = (float)(MT)(ulo * cs - uhi * sn);
        sQt[H2 + j] = (float)(MT)(uhi * cs + ulo * sn);
        sKt[j] = wlo * cs - whi * sn;
        sKt[H2 + j] = whi * cs + wlo * sn;
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
  const f32x4 qt = *reinterpret_cast<const f32x4*>(sQt + n0);
  MT* yg = static_cast<MT*>(p.y) + bh * P;
  const MT* zg = LAYER ? prow + h * P : (p.has_z ? static_cast<const MT*>(p.z) + bh * P : nullptr);
  const float dsk = p.has_d ? p.dsk[h] : 0.f;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int f = it * NT + tid;
    const bool valid = f < NV;
    const int prow = valid ? f / RV : 0;
    const float bvp = beta * sVp[prow];
    const float gv = gamma * sV[prow];
    f32x4 s = st[it];
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = alpha * s[i] + bvp * kp[i] + gv * kt[i];
      acc += (float)(MT)s[i] * qt[i];
    }
    // a plain store (the loads are non-temporal): at B=256 a non-temporal store made the
    // step 17% slower, and plain loads 10%
    if (valid) sg[f] = s;
    acc = group_sum<RV>(acc);
    if (valid && (tid % RV) == 0) {
      float yv = acc + dsk * sV[prow];
      if (zg) yv *= silu((float)zg[prow]);
      yg[prow] = (MT)yv;
    }
  }
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
  M3S_REQUIRE(a->ssm && aligned16(a->ssm) && a->k_state && a->v_state && a->phi_state && a->y,
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
  M3S_REQUIRE(a->ssm && aligned16(a->ssm) && a->k_state && a->v_state && a->phi_state && a->y,
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
