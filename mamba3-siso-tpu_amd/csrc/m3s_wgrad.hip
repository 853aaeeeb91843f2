// Weight gradient of a projection on gfx950: C = A^T B in float32 for bf16 token-major
// operands A (M x P) and B (M x Q), reduced over the M tokens.
//
// Replaces the weight-gradient half of the transposed projection products that jax.grad
// forms for the layer's and the LM's einsums (layer.py:233, 256; model.py:231, 268, 288):
// d in_proj = u^T d proj, d out_proj = y^T d out, and the MLP and head alike. Their output
// is small (P x Q, a few million entries) and their reduction long (M = B L tokens), so a
// library GEMM has too few output tiles for 256 CUs; split over the tokens, each split is
// another batched product and a sum.
//
// Here one launch covers tiles x splits workgroups, with the split count chosen so that
// they fill the CUs in whole rounds; each workgroup reduces its token range of one
// 256 x 256 output tile with v_mfma_f32_16x16x32_bf16 and writes a float32 partial, and a
// second launch adds the partials in split order (a fixed order: the result does not
// depend on timing). With a single split the tile goes straight to C.
//
// Both operands are token-major, so both MFMA operands need K = tokens along a lane's
// values: each 32-token step is staged in LDS as it lies in memory (rows = tokens, 16-byte
// pieces), and the fragments are read with ds_read_b64_tr_b16, which hands each lane four
// consecutive tokens of one column. Staging: registers one step ahead, two LDS stages,
// one barrier per step.
#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

constexpr int kWgT = 256;              // output tile edge (rows of P, columns of Q)
constexpr int kWgK = 32;               // tokens per step (a multiple of 32)
// waves over rows x columns: 4 x 2 waves of 64 x 128 (four waves of 128 x 128, with 256
// accumulator registers each, were no faster)
constexpr int kWgWP = 4, kWgWQ = 2;
constexpr int kWgThreads = 64 * kWgWP * kWgWQ;
constexpr int kWgRT = kWgT / kWgWP / 16, kWgCT = kWgT / kWgWQ / 16;   // 16 x 16 tiles per wave
constexpr int kWgPieces = kWgK * kWgT / 8 / kWgThreads;   // 16-byte pieces per thread per operand
constexpr int kWgLd = kWgT + 16;       // LDS row stride (bf16): 32 bytes of pad per row
constexpr int kWgStage = 2 * kWgK * kWgLd;   // A then B, bf16 elements per stage
constexpr int kWgMaxSplit = 16;

struct WgParams {
  const void* a;
  const void* b;
  uint32_t ea, eb;                 // the operands' extents in bytes
  float* c;
  float* part;                     // (S, P, Q) partials, S > 1
  int P, Q, ldc, tiles_q, tiles, S, nks;
  uint32_t lda2, ldb2;             // row strides in bytes
};

// Tokens steps [k0, k1) of split s: the nks steps cut as evenly as whole steps allow.
__device__ __forceinline__ void split_range(int nks, int S, int s, int& k0, int& k1) {
  k0 = (int)((int64_t)nks * s / S);
  k1 = (int)((int64_t)nks * (s + 1) / S);
}

__global__ void __launch_bounds__(kWgThreads) wgrad_kernel(const WgParams p) {
  __shared__ __attribute__((aligned(16))) bf16 lds[2 * kWgStage];
  // block -> (split, tile): consecutive blocks go to different XCDs (block i runs on XCD
  // i mod 8), so the tile index runs fastest over a block's XCD-local order
  const int nb = p.tiles * p.S;
  const int per = (nb + 7) >> 3;
  const int bid = blockIdx.x;
  const int lin = (bid & 7) * per + (bid >> 3);
  if (lin >= nb) return;   // the XCD groups are padded to equal size
  const int s = lin / p.tiles, tile = lin % p.tiles;
  const int tp = tile / p.tiles_q, tq = tile % p.tiles_q;
  const int p0 = tp * kWgT, q0 = tq * kWgT;
  int k0, k1;
  split_range(p.nks, p.S, s, k0, k1);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wp = wave % kWgWP, wq = wave / kWgWP;   // this wave's block of the tile
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.ea), rb = make_rsrc(p.b, p.eb);

  // staging: 32 rows x 256 columns per operand per step = 1024 16-byte pieces, two per
  // thread; piece i is row i / 32, columns 8 (i % 32) ..
  uint32_t va[kWgPieces], vb[kWgPieces];
  int lo[kWgPieces];
#pragma unroll
  for (int r = 0; r < kWgPieces; ++r) {
    const int i = tid + r * kWgThreads;
    const int row = i >> 5, col = (i & 31) * 8;
    va[r] = row * p.lda2 + (uint32_t)(p0 + col) * 2;
    vb[r] = row * p.ldb2 + (uint32_t)(q0 + col) * 2;
    lo[r] = row * kWgLd + col;
  }
  bf16x8 ga[kWgPieces], gb[kWgPieces];
  auto gload = [&](int ks) {
    const uint32_t sa = (uint32_t)ks * kWgK * p.lda2, sb = (uint32_t)ks * kWgK * p.ldb2;
#pragma unroll
    for (int r = 0; r < kWgPieces; ++r) {
      ga[r] = buf_load<bf16x8>(ra, va[r], sa);
      gb[r] = buf_load<bf16x8>(rb, vb[r], sb);
    }
  };
  auto swrite = [&](int st) {
    bf16* sa = lds + st * kWgStage;
    bf16* sb = sa + kWgK * kWgLd;
#pragma unroll
    for (int r = 0; r < kWgPieces; ++r) {
      *reinterpret_cast<bf16x8*>(sa + lo[r]) = ga[r];
      *reinterpret_cast<bf16x8*>(sb + lo[r]) = gb[r];
    }
  };

  f32x4 acc[kWgRT][kWgCT];
#pragma unroll
  for (int i = 0; i < kWgRT; ++i) {
#pragma unroll
    for (int j = 0; j < kWgCT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // K slots of lane group g = lane >> 4: tokens 4g .. 4g + 3 (first half of the MFMA's
  // eight) and 16 + 4g .. 16 + 4g + 3 (second half), the same for both operands. One
  // transposed read then covers 16 consecutive token rows across the four groups.
  const int kh0 = 4 * (lane >> 4), kh1 = 16 + kh0;
  auto compute = [&](int st) {
    const bf16* sa = lds + st * kWgStage;
    const bf16* sb = sa + kWgK * kWgLd;
#pragma unroll
    for (int k = 0; k < kWgK; k += 32) {
      bf16x4 a0[kWgRT], a1[kWgRT], b0[kWgCT], b1[kWgCT];
#pragma unroll
      for (int i = 0; i < kWgRT; ++i) {
        a0[i] = ld_tr4(sa, kWgLd, k + kh0, wp * 16 * kWgRT + 16 * i, lane);
        a1[i] = ld_tr4(sa, kWgLd, k + kh1, wp * 16 * kWgRT + 16 * i, lane);
      }
#pragma unroll
      for (int j = 0; j < kWgCT; ++j) {
        b0[j] = ld_tr4(sb, kWgLd, k + kh0, wq * 16 * kWgCT + 16 * j, lane);
        b1[j] = ld_tr4(sb, kWgLd, k + kh1, wq * 16 * kWgCT + 16 * j, lane);
      }
#pragma unroll
      for (int i = 0; i < kWgRT; ++i) {
#pragma unroll
        for (int j = 0; j < kWgCT; ++j) mma32(acc[i][j], a0[i], a1[i], b0[j], b1[j]);
      }
    }
  };

  // Step k is read from LDS stage k & 1; step k + 1 waits in registers (loaded during
  // step k - 1) and goes to the other stage after step k's products, then step k + 2's
  // loads are issued into the same registers.
  const int n = k1 - k0;
  if (n > 0) {
    gload(k0);
    swrite(0);
    if (n > 1) gload(k0 + 1);
    for (int it = 0; it < n; ++it) {
      // after this barrier stage it & 1 holds step it, and every wave is done reading
      // stage (it + 1) & 1 (step it - 1), which is refilled after this step's products:
      // the fragment reads start right after the barrier, not behind a burst of writes
      __syncthreads();
      compute(it & 1);
      if (it + 1 < n) swrite((it + 1) & 1);
      if (it + 2 < n) gload(k0 + it + 2);
    }
  }

  // acc[i][j][e] = C[p0 + 16 (RT wp + i) + 4 (lane >> 4) + e][q0 + 16 (CT wq + j) + (lane & 15)]
  float* out = p.S > 1 ? p.part + (int64_t)s * p.P * p.Q : p.c;
  const int ld = p.S > 1 ? p.Q : p.ldc;
  const int col0 = q0 + wq * 16 * kWgCT + (lane & 15);
  const int row0 = p0 + wp * 16 * kWgRT + 4 * (lane >> 4);
#pragma unroll
  for (int i = 0; i < kWgRT; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = row0 + 16 * i + e;
      if (row >= p.P) continue;
      float* orow = out + (int64_t)row * ld;
#pragma unroll
      for (int j = 0; j < kWgCT; ++j) {
        const int col = col0 + 16 * j;
        if (col < p.Q) orow[col] = acc[i][j][e];
      }
    }
  }
}

// C[r][c] = sum over s of part[s][r][c], s in order.
__global__ void __launch_bounds__(256) wgrad_sum_kernel(const float* __restrict__ part,
                                                        float* __restrict__ c, int P, int Q,
                                                        int ldc, int S) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t PQ = (int64_t)P * Q;
  if ((Q & 3) == 0 && (ldc & 3) == 0) {
    const int64_t e = 4 * i;
    if (e >= PQ) return;
    f32x4 v = *reinterpret_cast<const f32x4*>(part + e);
    for (int s = 1; s < S; ++s) v += *reinterpret_cast<const f32x4*>(part + s * PQ + e);
    const int64_t r = e / Q, col = e % Q;
    *reinterpret_cast<f32x4*>(c + r * ldc + col) = v;
    return;
  }
  if (i >= PQ) return;
  float v = part[i];
  for (int s = 1; s < S; ++s) v += part[s * PQ + i];
  c[(i / Q) * ldc + i % Q] = v;
}

// Split count: the smallest S <= kWgMaxSplit (and <= steps / 8) whose tiles x S fill whole
// rounds of the CUs best.
inline int wgrad_splits(int M, int P, int Q) {
  const int tiles = ((P + kWgT - 1) / kWgT) * ((Q + kWgT - 1) / kWgT);
  const int nks = M / kWgK;
  const int cus = 256;
  int best = 1;
  double best_eff = 0.0;
  for (int S = 1; S <= kWgMaxSplit && (S == 1 || nks / S >= 8); ++S) {
    const int64_t nb = (int64_t)tiles * S;
    const double eff = (double)nb / (double)(cus * ((nb + cus - 1) / cus));
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best = S;
    }
  }
  return best;
}

}  // namespace m3s

extern "C" int64_t m3s_wgrad_workspace_bytes(int32_t tokens, int32_t rows, int32_t cols) {
  if (tokens <= 0 || rows <= 0 || cols <= 0 || tokens % m3s::kWgK) return -1;
  const int S = m3s::wgrad_splits(tokens, rows, cols);
  return S > 1 ? (int64_t)S * rows * cols * 4 : 0;
}

extern "C" int32_t m3s_wgrad(const m3s_wgrad_args* a, void* stream) {
  using namespace m3s;
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_wgrad: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_wgrad_args),
              "m3s_wgrad: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_wgrad_args));
  const int M = a->tokens, P = a->rows, Q = a->cols;
  M3S_REQUIRE(M > 0 && P > 0 && Q > 0, "m3s_wgrad: non-positive dimension");
  M3S_REQUIRE(M % kWgK == 0, "m3s_wgrad: tokens %d is not a multiple of %d", M, kWgK);
  M3S_REQUIRE(a->a && a->b && a->c, "m3s_wgrad: a NULL operand");
  M3S_REQUIRE(aligned16(a->a) && aligned16(a->b) && a->lda % 8 == 0 && a->ldb % 8 == 0,
              "m3s_wgrad: operands must be 16-byte aligned with row strides a multiple of 8");
  M3S_REQUIRE(a->lda >= P && a->ldb >= Q && a->ldc >= Q, "m3s_wgrad: a row stride is too short");
  const int64_t ea = ((int64_t)(M - 1) * a->lda + P) * 2, eb = ((int64_t)(M - 1) * a->ldb + Q) * 2;
  M3S_REQUIRE(ea < (1ll << 31) && eb < (1ll << 31), "m3s_wgrad: an operand spans 2 GiB or more");
  M3S_REQUIRE(a->ldc < (1ll << 31), "m3s_wgrad: output row stride too large");
  const int S = wgrad_splits(M, P, Q);
  M3S_REQUIRE(S == 1 || (a->workspace && aligned16(a->workspace)),
              "m3s_wgrad: a 16-byte aligned workspace of m3s_wgrad_workspace_bytes() is needed");
  M3S_REQUIRE(S == 1 || (a->ldc % 4 != 0 || aligned16(a->c)), "m3s_wgrad: c must be 16-byte aligned");
  WgParams p{};
  p.a = a->a;
  p.b = a->b;
  p.ea = (uint32_t)ea;
  p.eb = (uint32_t)eb;
  p.c = a->c;
  p.part = static_cast<float*>(a->workspace);
  p.P = P; p.Q = Q; p.ldc = (int)a->ldc;
  p.tiles_q = (Q + kWgT - 1) / kWgT;
  p.tiles = ((P + kWgT - 1) / kWgT) * p.tiles_q;
  p.S = S;
  p.nks = M / kWgK;
  p.lda2 = (uint32_t)(a->lda * 2);
  p.ldb2 = (uint32_t)(a->ldb * 2);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nb = p.tiles * S;
  hipLaunchKernelGGL(wgrad_kernel, dim3(8 * ((nb + 7) / 8)), dim3(kWgThreads), 0, st, p);
  int32_t rc = launch_status("m3s_wgrad");
  if (rc || S == 1) return rc;
  const int64_t PQ = (int64_t)P * Q;
  const int64_t work = (Q % 4 == 0 && a->ldc % 4 == 0) ? (PQ + 3) / 4 : PQ;
  hipLaunchKernelGGL(wgrad_sum_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st,
                     p.part, a->c, P, Q, (int)a->ldc, S);
  return launch_status("m3s_wgrad");
}
