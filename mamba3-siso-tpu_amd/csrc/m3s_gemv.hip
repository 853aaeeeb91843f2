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

// ---- more rows: MFMA tiles ----------------------------------------------------------
// From kGvMaxRows + 1 rows (a batch of decode tokens: 256 at the decode config) the
// products run on v_mfma_f32_16x16x32_bf16. A workgroup of RW waves (four or eight) takes
// a 16 RW x NC output tile, wave w its rows 16 w .. 16 w + 15 and all NC columns, and walks
// K in steps of kGmK = 64 (two MFMA K-blocks per step):
//  * the x rows are each wave's own A operand: per step and K-block one 16-byte piece per
//    lane (row lane & 15, K slots 8 (lane >> 4) ..), read straight into registers;
//  * the weight's kGmK x NC block of a step is shared by the RW waves: staged in LDS as
//    it lies in memory (K rows, 16-byte pieces) and read as the B operand with
//    ds_read_b64_tr_b16, which hands a lane four consecutive K of one column;
//  * both are loaded kGmD steps ahead into a ring of registers (slot = step mod kGmD, so no
//    register is copied: a copy of a register still being loaded would wait for it), and
//    a step's weight block goes to the LDS stage it is read from one step early; two
//    stages (stage = step mod 2; kGmD is even), one barrier per step.
// The step count is padded to a multiple of kGmD: a step past the last reads zeros (its
// loads go through an out-of-range offset), so every load and stage is unconditional and
// the compiler's wait counts stay exact (a conditional load made it wait for every
// outstanding load once per kGmD steps). Rows past M and columns past N read as zero
// through the buffer descriptors' range and are not stored. The row tiles of one column
// tile are consecutive blocks of one XCD, so the weight block is fetched from HBM once and
// from L2 after that. Fixed summation order: deterministic.
constexpr int kGmK = 64;     // K per step (kGmKB MFMA K-blocks of 32)
constexpr int kGmKB = kGmK / 32;
constexpr int kGmD = 4;      // steps loaded ahead (even: the LDS stage of step s0 + d is d & 1)

struct GmParams {
  const bf16* x;
  const bf16* w;
  bf16* y;
  int M, K, N, tiles_m, tiles_n;
  int64_t ldx, ldw, ldy;
  uint32_t ex, ew;   // the operands' extents in bytes
};

template <int NC, int RW>
__global__ void __launch_bounds__(64 * RW) gemm_rows_kernel(const GmParams p) {
  constexpr int TH = 64 * RW, MT = 16 * RW;   // threads; rows per workgroup
  constexpr int CT = NC / 16;                  // 16-column tiles per wave
  constexpr int LD = NC + 8;                   // LDS row stride (bf16), 16 bytes of pad
  constexpr int WPR = NC / 8;                  // 16-byte weight pieces per K row
  constexpr int WP = kGmK * WPR / TH;          // weight pieces per thread and step
  static_assert(WP >= 1 && kGmK * WPR % TH == 0, "whole weight pieces per thread");
  __shared__ __attribute__((aligned(16))) bf16 sw[2][kGmK * LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // block -> (row tile, column tile): the row tiles of one column tile on one XCD
  const int nb = p.tiles_m * p.tiles_n, per = (nb + 7) >> 3, bid = blockIdx.x;
  const int lin = (bid & 7) * per + (bid >> 3);
  if (lin >= nb) return;   // the XCD groups are padded to equal size
  const int tn = lin / p.tiles_m, tm = lin % p.tiles_m;
  const int row = tm * MT + 16 * wave + (lane & 15), n0 = tn * NC;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, p.ex), rw = make_rsrc(p.w, p.ew);
  // this lane's x pieces: row `row`, K slots 8 (lane >> 4) .. of each K-block; past M: out
  // of range
  const uint32_t ox = row < p.M ? (uint32_t)(row * p.ldx + 8 * (lane >> 4)) * 2 : p.ex;
  // this thread's weight pieces: row (tid + TH r) / WPR of the step, columns
  // 8 ((tid + TH r) % WPR) ..
  uint32_t ow[WP];
  int lo[WP];
#pragma unroll
  for (int r = 0; r < WP; ++r) {
    const int i = tid + r * TH, wr = i / WPR, wc = 8 * (i % WPR);
    ow[r] = n0 + wc < p.N ? (uint32_t)(wr * p.ldw + n0 + wc) * 2 : p.ew;
    lo[r] = wr * LD + wc;
  }
  const int ns = p.K / kGmK, nsp = (ns + kGmD - 1) / kGmD * kGmD;

  bf16x8 ra[kGmD][kGmKB], rb[kGmD][WP];
  auto load = [&](int st, int slot) {
    const bool in = st < ns;
#pragma unroll
    for (int kb = 0; kb < kGmKB; ++kb)
      ra[slot][kb] = buf_load<bf16x8>(rx, in ? ox : p.ex, in ? (uint32_t)(st * kGmK + 32 * kb) * 2 : 0u);
#pragma unroll
    for (int r = 0; r < WP; ++r)
      rb[slot][r] = buf_load<bf16x8>(rw, in ? ow[r] : p.ew, in ? (uint32_t)(st * kGmK * p.ldw) * 2 : 0u);
  };
  auto stage = [&](int buf, int slot) {
#pragma unroll
    for (int r = 0; r < WP; ++r) *reinterpret_cast<bf16x8*>(&sw[buf][lo[r]]) = rb[slot][r];
  };
  f32x4 acc[CT];
#pragma unroll
  for (int j = 0; j < CT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int g = lane >> 4;
  auto compute = [&](int buf, int slot) {
    const bf16* sb = sw[buf];
#pragma unroll
    for (int kb = 0; kb < kGmKB; ++kb) {
#pragma unroll
      for (int j = 0; j < CT; ++j) {
        const bf16x4 lo4 = ld_tr4(sb, LD, 32 * kb + 8 * g, 16 * j, lane);
        const bf16x4 hi4 = ld_tr4(sb, LD, 32 * kb + 8 * g + 4, 16 * j, lane);
        const bf16x8 b = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
        mma32x(acc[j], ra[slot][kb], b);
      }
    }
  };

#pragma unroll
  for (int d = 0; d < kGmD; ++d) load(d, d);
  stage(0, 0);
  for (int s0 = 0; s0 < nsp; s0 += kGmD) {
#pragma unroll
    for (int d = 0; d < kGmD; ++d) {
      __syncthreads();   // stage d & 1 holds step s0 + d; the other stage is free
      compute(d & 1, d);
      stage((d + 1) & 1, (d + 1) % kGmD);
      load(s0 + d + kGmD, d);
    }
  }
  // acc[j][e] = y[row0 + e][n0 + 16 j + (lane & 15)], row0 = the wave's row of 4 g
  const int row0 = tm * MT + 16 * wave + 4 * g;
#pragma unroll
  for (int j = 0; j < CT; ++j) {
    const int col = n0 + 16 * j + (lane & 15);
    if (col >= p.N) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (row0 + e < p.M) p.y[(int64_t)(row0 + e) * p.ldy + col] = (bf16)acc[j][e];
  }
}

// Tile shapes: 64 rows x 64 columns when that gives 128 to 256 workgroups; 64 x 32 below;
// above, 128 rows (eight waves sharing each weight block) x 64 columns, so that one wave
// of workgroups covers the CUs without a partly filled second one.
template <int NC, int RW>
int32_t gemm_rows_launch(GmParams p, hipStream_t s) {
  p.tiles_m = (p.M + 16 * RW - 1) / (16 * RW);
  p.tiles_n = (p.N + NC - 1) / NC;
  const int nb = p.tiles_m * p.tiles_n;
  const unsigned grid = (unsigned)(((nb + 7) >> 3) * 8);
  hipLaunchKernelGGL((gemm_rows_kernel<NC, RW>), dim3(grid), dim3(64 * RW), 0, s, p);
  return launch_status("m3s_gemv");
}

}  // namespace m3s

extern "C" int32_t m3s_gemv(const m3s_gemv_args* a, void* stream) {
  using namespace m3s;
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_gemv: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_gemv_args),
              "m3s_gemv: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_gemv_args));
  M3S_REQUIRE(a->rows >= 1, "m3s_gemv: rows %d < 1", a->rows);
  M3S_REQUIRE(a->k > 0 && a->n > 0, "m3s_gemv: non-positive k or n");
  M3S_REQUIRE(a->n % 8 == 0, "m3s_gemv: n %d is not a multiple of 8", a->n);
  M3S_REQUIRE(a->x && a->w && a->y, "m3s_gemv: a NULL operand");
  M3S_REQUIRE(aligned16(a->w) && a->ldw % 8 == 0 && a->ldw >= a->n,
              "m3s_gemv: w must be 16-byte aligned with a row stride >= n and a multiple of 8");
  M3S_REQUIRE(a->ldx >= a->k && a->ldy >= a->n, "m3s_gemv: a row stride is too short");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->rows > kGvMaxRows) {
    M3S_REQUIRE(a->k % kGmK == 0, "m3s_gemv: k %d is not a multiple of %d (rows > %d)", a->k,
                kGmK, kGvMaxRows);
    M3S_REQUIRE(aligned16(a->x) && a->ldx % 8 == 0,
                "m3s_gemv: x must be 16-byte aligned with a row stride a multiple of 8 (rows > %d)",
                kGvMaxRows);
    const int64_t ex = ((int64_t)(a->rows - 1) * a->ldx + a->k) * 2;
    const int64_t ew = ((int64_t)(a->k - 1) * a->ldw + a->n) * 2;
    M3S_REQUIRE(ex < (1ll << 31) && ew < (1ll << 31), "m3s_gemv: an operand spans 2 GiB or more");
    GmParams g{static_cast<const bf16*>(a->x), static_cast<const bf16*>(a->w),
               static_cast<bf16*>(a->y), a->rows, a->k, a->n, 0, 0, a->ldx, a->ldw, a->ldy,
               (uint32_t)ex, (uint32_t)ew};
    const int64_t t64 = (int64_t)((a->rows + 63) / 64) * ((a->n + 63) / 64);
    if (t64 > 256) return gemm_rows_launch<64, 8>(g, s);
    if (t64 >= 128) return gemm_rows_launch<64, 4>(g, s);
    return gemm_rows_launch<32, 4>(g, s);
  }
  GvParams p{static_cast<const bf16*>(a->x), static_cast<const bf16*>(a->w),
             static_cast<bf16*>(a->y), a->rows, a->k, a->n, a->ldx, a->ldw, a->ldy};
  M3S_REQUIRE(a->k <= kGvThreads * kGvMaxLoads, "m3s_gemv: k %d > %d", a->k,
              kGvThreads * kGvMaxLoads);
  switch (gemv_col_lanes(a->k, a->n)) {
    case 8: return gemv_launch<8>(p, s);
    case 4: return gemv_launch<4>(p, s);
    case 2: return gemv_launch<2>(p, s);
    default: return gemv_launch<1>(p, s);
  }
}
