// The LM training step's optimizer update on gfx950: clip-then-AdamW over every float32
// parameter tensor, one HBM pass.
//
// Replaces the optimizer of the reference's training step (train.py:799-805, optax
// chain(clip_by_global_norm(1.0), adamw(...))) once the global gradient norm is known.
// Composed from framework list ops the update is eight passes over the parameters'
// bytes (clip multiply, two moment updates, square root, two divisions and adds, decay,
// parameter step); here each element's p, g, m, v are read once and p, m, v written
// once. Per element, in f32, with s the clip factor (1 without clipping):
//   g = grad s
//   m = m + (1 - b1) (g - m)                      (torch lerp for a weight below 1/2)
//   v = b2 v + (1 - b2) g^2
//   p = p (1 - lr wd) - (lr / bc1) m / (sqrt(v) / sqrt(bc2) + eps)
// with bc1 = 1 - b1^t and bc2 = 1 - b2^t for update t: optax adamw's update with the
// weight decay taken from the parameter before the step. The scalars 1 - b1, 1 - b2,
// 1 - lr wd, lr / bc1 and sqrt(bc2) come from the caller, formed in double precision
// (1 - b2 from a float32 b2 would be off by 1e-5 relative).
//
// Tensors go in groups of kAdamMaxT per launch. Each tensor is cut into blocks of
// kAdamPerBlock elements; a workgroup finds its tensor from the group's cumulative block
// counts (a scalar loop over at most kAdamMaxT entries) and takes one block, as 16-byte
// vectors when all four of the tensor's buffers are 16-byte aligned.
#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

constexpr int kAdamMaxT = 24;
constexpr int kAdamThreads = 256;
constexpr int kAdamVecPerThread = 4;
constexpr int kAdamPerBlock = kAdamThreads * kAdamVecPerThread * 4;   // elements

struct AdamGroup {
  float* p[kAdamMaxT];
  const float* g[kAdamMaxT];
  float* m[kAdamMaxT];
  float* v[kAdamMaxT];
  int64_t n[kAdamMaxT];
  int blk0[kAdamMaxT + 1];   // first block of each tensor; blk0[count] = blocks in all
  int vec[kAdamMaxT];        // 1 if p, g, m, v are all 16-byte aligned
  int count;
};

struct AdamHyper {
  const float* scale;   // clip factor (device scalar) or NULL
  float omb1, b2, omb2, eps, decay, step, bc2s;
};

__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v, float s,
                                          const AdamHyper& h) {
  g *= s;
  m = m + h.omb1 * (g - m);
  v = h.b2 * v + h.omb2 * (g * g);
  const float den = sqrtf(v) / h.bc2s + h.eps;
  p = p * h.decay - h.step * (m / den);
}

__global__ void __launch_bounds__(kAdamThreads) adamw_kernel(const AdamGroup grp,
                                                             const AdamHyper hp) {
  const int bid = blockIdx.x, tid = threadIdx.x;
  int i = 0;
  while (i + 1 < grp.count && bid >= grp.blk0[i + 1]) ++i;
  const int64_t n = grp.n[i];
  const int64_t e0 = (int64_t)(bid - grp.blk0[i]) * kAdamPerBlock;
  const int64_t e1 = e0 + kAdamPerBlock < n ? e0 + kAdamPerBlock : n;
  float* __restrict__ P = grp.p[i];
  const float* __restrict__ G = grp.g[i];
  float* __restrict__ M = grp.m[i];
  float* __restrict__ V = grp.v[i];
  const float s = hp.scale ? *hp.scale : 1.f;
  if (grp.vec[i] && e1 - e0 == kAdamPerBlock) {
    // a whole aligned block: every load of the thread issued before any arithmetic
    f32x4 rp[kAdamVecPerThread], rg[kAdamVecPerThread], rm[kAdamVecPerThread],
        rv[kAdamVecPerThread];
#pragma unroll
    for (int k = 0; k < kAdamVecPerThread; ++k) {
      const int64_t e = e0 + 4 * (tid + kAdamThreads * k);
      rp[k] = *reinterpret_cast<const f32x4*>(P + e);
      rg[k] = *reinterpret_cast<const f32x4*>(G + e);
      rm[k] = *reinterpret_cast<const f32x4*>(M + e);
      rv[k] = *reinterpret_cast<const f32x4*>(V + e);
    }
#pragma unroll
    for (int k = 0; k < kAdamVecPerThread; ++k) {
      const int64_t e = e0 + 4 * (tid + kAdamThreads * k);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float pe = rp[k][j], me = rm[k][j], ve = rv[k][j];
        adam_elem(pe, rg[k][j], me, ve, s, hp);
        rp[k][j] = pe;
        rm[k][j] = me;
        rv[k][j] = ve;
      }
      *reinterpret_cast<f32x4*>(P + e) = rp[k];
      *reinterpret_cast<f32x4*>(M + e) = rm[k];
      *reinterpret_cast<f32x4*>(V + e) = rv[k];
    }
    return;
  }
  for (int64_t e = e0 + tid; e < e1; e += kAdamThreads) {
    float p = P[e], m = M[e], v = V[e];
    adam_elem(p, G[e], m, v, s, hp);
    P[e] = p;
    M[e] = m;
    V[e] = v;
  }
}

}  // namespace m3s

extern "C" int32_t m3s_adamw(const m3s_adamw_args* a, void* stream) {
  using namespace m3s;
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_adamw: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_adamw_args),
              "m3s_adamw: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_adamw_args));
  M3S_REQUIRE(a->count >= 0, "m3s_adamw: negative tensor count %d", a->count);
  if (a->count == 0) return M3S_OK;
  M3S_REQUIRE(a->params && a->grads && a->exp_avg && a->exp_avg_sq && a->numel,
              "m3s_adamw: a tensor array is NULL");
  M3S_REQUIRE(a->bias_correction2_sqrt > 0.f,
              "m3s_adamw: bias_correction2_sqrt must be positive (update count >= 1)");
  for (int t = 0; t < a->count; ++t) {
    M3S_REQUIRE(a->numel[t] >= 0, "m3s_adamw: tensor %d has negative numel", t);
    if (a->numel[t] == 0) continue;
    M3S_REQUIRE(a->params[t] && a->grads[t] && a->exp_avg[t] && a->exp_avg_sq[t],
                "m3s_adamw: tensor %d has a NULL buffer", t);
    M3S_REQUIRE((a->numel[t] + kAdamPerBlock - 1) / kAdamPerBlock < (1ll << 30),
                "m3s_adamw: tensor %d too large", t);
  }
  AdamHyper hp{a->grad_scale, a->one_minus_beta1, a->beta2, a->one_minus_beta2, a->eps,
               a->param_decay, a->step_size, a->bias_correction2_sqrt};
  hipStream_t s = static_cast<hipStream_t>(stream);
  AdamGroup grp{};
  int64_t blocks = 0;
  auto flush = [&]() -> int32_t {
    if (grp.count == 0) return M3S_OK;
    grp.blk0[grp.count] = (int)blocks;
    hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)blocks), dim3(kAdamThreads), 0, s, grp, hp);
    grp.count = 0;
    blocks = 0;
    return launch_status("m3s_adamw");
  };
  for (int t = 0; t < a->count; ++t) {
    const int64_t n = a->numel[t];
    if (n == 0) continue;
    const int64_t nb = (n + kAdamPerBlock - 1) / kAdamPerBlock;
    if (grp.count == kAdamMaxT || blocks + nb > 0x7fffffff) {
      const int32_t rc = flush();
      if (rc != M3S_OK) return rc;
    }
    const int c = grp.count;
    grp.p[c] = a->params[t];
    grp.g[c] = a->grads[t];
    grp.m[c] = a->exp_avg[t];
    grp.v[c] = a->exp_avg_sq[t];
    grp.n[c] = n;
    grp.blk0[c] = (int)blocks;
    grp.vec[c] = aligned16(a->params[t]) && aligned16(a->grads[t]) && aligned16(a->exp_avg[t]) &&
                 aligned16(a->exp_avg_sq[t]);
    grp.count = c + 1;
    blocks += nb;
  }
  return flush();
}
