// Small-batch projection on gfx950: y (M x N) = x (M x K) w (K x N) for M <= 4 rows, bf16
// operands and output, float32 accumulation. The products of a one-token decode step.
//
// Replaces, for the decode step, the projections of the reference's per-token layer and
// LM step (model.py:266-296: in_proj, out_proj, the MLP's fc1 and fc2), which the
// reference leaves to XLA. At one row a library GEMM reads the weight at 0.35-0.7 TB/s
// (7-13 us for 2.4-5.3 MB); the weight is the whole cost, so the kernel is a single
// streaming pass over it with every load of a thread issued before the first use.
//
// Layout: a workgroup takes TN = 8 * CL consecutive columns (CL column lanes of 16-byte
// pieces) and all K rows; its 256 threads are CL column lanes x 256 / CL row lanes, and row
// lane r reads rows r, r + RL, ... . TN is chosen on the host so that the launch has at
// least 128 workgroups. Sums over the row lanes: xor shuffles inside a wave (a fixed
// tree), then the four waves' partials added in wave order through LDS. Deterministic.
#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

constexpr int kGvThreads = 256;
constexpr int kGvMaxRows = 4;
constexpr int kGvMaxLoads = 16;   // weight pieces per thread (K / RL), all in flight

struct GvParams {
  const bf16* x;
  const bf16* w;
  bf16* y;
  int M, K, N;
  int64_t ldx, ldw, ldy;
};

template <int CL, int NL>
__global__ void __launch_bounds__(kGvThreads) gemv_kernel(const GvParams p) {
  constexpr int RL = kGvThreads / CL;   // row lanes
  constexpr int TN = 8 * CL;
  __shared__ float part[kGvThreads / 64][kGvMaxRows][TN];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cl = tid % CL, rl = tid / CL;
  const int n = blockIdx.x * TN + 8 * cl;
  const bool col_ok = n < p.N;   // N % 8 == 0: a piece is wholly in or out
  // every weight piece of this thread first (NL = ceil(K / RL) loads)
  bf16x8 wv[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int k = rl + i * RL;
    wv[i] = (col_ok && k < p.K) ? *reinterpret_cast<const bf16x8*>(p.w + (int64_t)k * p.ldw + n)
                                : bf16x8{};
  }
  float acc[kGvMaxRows][8];
#pragma unroll
  for (int m = 0; m < kGvMaxRows; ++m) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[m][j] = 0.f;
  }
#pragma unroll
  for (int m = 0; m < kGvMaxRows; ++m) {
    if (m >= p.M) break;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int k = rl + i * RL;
      const float xv = k < p.K ? (float)p.x[m * p.ldx + k] : 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[m][j] = fmaf(xv, (float)wv[i][j], acc[m][j]);
    }
  }
  // row lanes of one column lane are the lanes cl + CL j of the wave: an xor tree over the
  // lane bits above log2(CL)
#pragma unroll
  for (int m = 0; m < kGvMaxRows; ++m) {
    if (m >= p.M) break;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = acc[m][j];
#pragma unroll
      for (int off = CL; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
      acc[m][j] = v;
    }
  }
  if (lane < CL) {
#pragma unroll
    for (int m = 0; m < kGvMaxRows; ++m) {
      if (m >= p.M) break;
#pragma unroll
      for (int j = 0; j < 8; ++j) part[wave][m][8 * lane + j] = acc[m][j];
    }
  }
  __syncthreads();
  if (tid < p.M * TN) {
    const int m = tid / TN, c = tid % TN;
    const int col = blockIdx.x * TN + c;
    if (col < p.N) {
      float s = part[0][m][c];
#pragma unroll
      for (int w = 1; w < kGvThreads / 64; ++w) s += part[w][m][c];
      p.y[m * p.ldy + col] = (bf16)s;
    }
  }
}

// Column lanes per workgroup: the widest tile (16-byte pieces per row, up to 8) that still
// gives at least 128 workgroups and at most kGvMaxLoads weight pieces per thread.
inline int gemv_col_lanes(int K, int N) {
  int cl = 8;
  auto loads = [&](int c) { return (K + kGvThreads / c - 1) / (kGvThreads / c); };
  while (cl > 1 && ((N + 8 * cl - 1) / (8 * cl) < 128 || loads(cl) > kGvMaxLoads)) cl >>= 1;
  return cl;
}

template <int CL>
int32_t gemv_launch(const GvParams& p, hipStream_t s) {
  constexpr int RL = kGvThreads / CL;
  const int nl = (p.K + RL - 1) / RL;
  const dim3 grid((unsigned)((p.N + 8 * CL - 1) / (8 * CL)));
#define M3S_GV(NL)                                                                \
  if (nl <= NL) {                                                                 \
    hipLaunchKernelGGL((gemv_kernel<CL, NL>), grid, dim3(kGvThreads), 0, s, p);   \
    return launch_status("m3s_gemv");                                             \
  }
  M3S_GV(2) M3S_GV(4) M3S_GV(8) M3S_GV(16)
#undef M3S_GV
  set_error("m3s_gemv: K = %d needs more than %d loads per thread", p.K, kGvMaxLoads);
  return M3S_ERR_UNSUPPORTED;
}

}  // namespace m3s

extern "C" int32_t m3s_gemv(const m3s_gemv_args* a, void* stream) {
  using namespace m3s;
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_gemv: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_gemv_args),
              "m3s_gemv: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_gemv_args));
  M3S_REQUIRE(a->rows >= 1 && a->rows <= kGvMaxRows, "m3s_gemv: rows %d not in [1, %d]",
              a->rows, kGvMaxRows);
  M3S_REQUIRE(a->k > 0 && a->n > 0, "m3s_gemv: non-positive k or n");
  M3S_REQUIRE(a->n % 8 == 0, "m3s_gemv: n %d is not a multiple of 8", a->n);
  M3S_REQUIRE(a->x && a->w && a->y, "m3s_gemv: a NULL operand");
  M3S_REQUIRE(aligned16(a->w) && a->ldw % 8 == 0 && a->ldw >= a->n,
              "m3s_gemv: w must be 16-byte aligned with a row stride >= n and a multiple of 8");
  M3S_REQUIRE(a->ldx >= a->k && a->ldy >= a->n, "m3s_gemv: a row stride is too short");
  GvParams p{static_cast<const bf16*>(a->x), static_cast<const bf16*>(a->w),
             static_cast<bf16*>(a->y), a->rows, a->k, a->n, a->ldx, a->ldw, a->ldy};
  hipStream_t s = static_cast<hipStream_t>(stream);
  M3S_REQUIRE(a->k <= kGvThreads * kGvMaxLoads, "m3s_gemv: k %d > %d", a->k,
              kGvThreads * kGvMaxLoads);
  switch (gemv_col_lanes(a->k, a->n)) {
    case 8: return gemv_launch<8>(p, s);
    case 4: return gemv_launch<4>(p, s);
    case 2: return gemv_launch<2>(p, s);
    default: return gemv_launch<1>(p, s);
  }
}
