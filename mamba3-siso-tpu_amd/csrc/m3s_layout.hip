// Weight layout for the layer's projection GEMMs on gfx950: a tiled transpose with a
// dtype cast and appended zero rows.
//
// The reference casts its projection weights per call (`params.in_proj.astype(u.dtype)`,
// layer.py:233, 256). The layer here computes its GEMMs against a transposed copy of each
// weight -- in_proj zero-padded to a multiple of 256 rows -- which is the operand layout
// hipBLASLt runs fastest at these shapes, and makes that copy in the same pass as the cast.
// 64 x 64 tiles through LDS (odd row pitch: no bank conflicts on the transposed read);
// reads and writes are row-contiguous across a wave. HBM-bound. When rows, cols and the
// input stride are multiples of 8 and both buffers 16-byte aligned, each thread moves
// runs of 8 elements (16-byte bf16 accesses) instead of single elements: at in_proj's
// 1024 x 4480 bf16 that is 3x faster.
#include "m3s_common.h"
#include "m3s_internal.h"

namespace m3s {

constexpr int kTrTile = 64;
constexpr int kTrThreads = 256;

template <typename TI, typename TO>
__global__ void __launch_bounds__(kTrThreads) transpose_kernel(const TI* __restrict__ in,
                                                               int64_t in_st,
                                                               TO* __restrict__ out, int rows,
                                                               int cols, int out_rows) {
  __shared__ float tile[kTrTile][kTrTile + 1];
  const int c0 = blockIdx.x * kTrTile;   // input column block = output row block
  const int r0 = blockIdx.y * kTrTile;   // input row block = output column block
  const int tx = threadIdx.x % kTrTile, ty = threadIdx.x / kTrTile;
  constexpr int RSTEP = kTrThreads / kTrTile;
  for (int i = ty; i < kTrTile; i += RSTEP) {
    const int r = r0 + i, c = c0 + tx;
    tile[i][tx] = (r < rows && c < cols) ? (float)in[(int64_t)r * in_st + c] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < kTrTile; i += RSTEP) {
    const int orow = c0 + i, ocol = r0 + tx;   // rows >= cols of the output are zeros
    if (orow < out_rows && ocol < rows) out[(int64_t)orow * rows + ocol] = (TO)tile[tx][i];
  }
}

template <typename T> struct Run8;
template <> struct Run8<bf16> {
  __device__ static void load(const bf16* p, float (&v)[8]) {
    const bf16x8 r = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = (float)r[u];
  }
  __device__ static void store(bf16* p, const float (&v)[8]) {
    bf16x8 r;
#pragma unroll
    for (int u = 0; u < 8; ++u) r[u] = (bf16)v[u];
    *reinterpret_cast<bf16x8*>(p) = r;
  }
};
template <> struct Run8<float> {
  __device__ static void load(const float* p, float (&v)[8]) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[u] = a[u];
      v[u + 4] = b[u];
    }
  }
  __device__ static void store(float* p, const float (&v)[8]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
};

// rows, cols, in_st multiples of 8: a thread takes the 8-element run (i, 8 g .. 8 g + 7)
// of the tile, i = t / 8 + 32 pass, g = t % 8, both ways
template <typename TI, typename TO>
__global__ void __launch_bounds__(kTrThreads) transpose8_kernel(const TI* __restrict__ in,
                                                                int64_t in_st,
                                                                TO* __restrict__ out, int rows,
                                                                int cols, int out_rows) {
  __shared__ float tile[kTrTile][kTrTile + 1];
  const int c0 = blockIdx.x * kTrTile, r0 = blockIdx.y * kTrTile;
  const int g8 = 8 * (threadIdx.x % 8), i0 = threadIdx.x / 8;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int i = i0 + 32 * pass, r = r0 + i, c = c0 + g8;
    float v[8];
    if (r < rows && c < cols) {
      Run8<TI>::load(in + (int64_t)r * in_st + c, v);
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) tile[i][g8 + u] = v[u];
  }
  __syncthreads();
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int j = i0 + 32 * pass, orow = c0 + j, ocol = r0 + g8;
    if (orow < out_rows && ocol < rows) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = tile[g8 + u][j];
      Run8<TO>::store(out + (int64_t)orow * rows + ocol, v);
    }
  }
}

template <typename TI, typename TO>
static int32_t launch_tr(const m3s_transpose_args* a, hipStream_t s) {
  const dim3 grid((a->out_rows + kTrTile - 1) / kTrTile, (a->rows + kTrTile - 1) / kTrTile);
  const bool runs = a->rows % 8 == 0 && a->cols % 8 == 0 && a->in_stride % 8 == 0 &&
                    aligned16(a->in) && aligned16(a->out);
  if (runs)
    hipLaunchKernelGGL((transpose8_kernel<TI, TO>), grid, dim3(kTrThreads), 0, s,
                       static_cast<const TI*>(a->in), a->in_stride, static_cast<TO*>(a->out),
                       a->rows, a->cols, a->out_rows);
  else
    hipLaunchKernelGGL((transpose_kernel<TI, TO>), grid, dim3(kTrThreads), 0, s,
                       static_cast<const TI*>(a->in), a->in_stride, static_cast<TO*>(a->out),
                       a->rows, a->cols, a->out_rows);
  return launch_status("m3s_transpose");
}

}  // namespace m3s

using namespace m3s;

extern "C" int32_t m3s_transpose(const m3s_transpose_args* a, void* stream) {
  clear_error();
  M3S_REQUIRE(a != nullptr, "m3s_transpose: args is NULL");
  M3S_REQUIRE(a->struct_size == (int32_t)sizeof(m3s_transpose_args),
              "m3s_transpose: struct_size %d != %d (ABI mismatch)", a->struct_size,
              (int)sizeof(m3s_transpose_args));
  M3S_REQUIRE(a->rows > 0 && a->cols > 0 && a->out_rows >= a->cols,
              "m3s_transpose: need rows > 0, cols > 0 and out_rows >= cols");
  M3S_REQUIRE(a->in_stride >= a->cols, "m3s_transpose: in_stride %lld < cols %d",
              (long long)a->in_stride, a->cols);
  M3S_REQUIRE(a->in && a->out, "m3s_transpose: NULL pointer");
  const bool ib = a->in_dtype == M3S_DTYPE_BF16, ob = a->out_dtype == M3S_DTYPE_BF16;
  M3S_REQUIRE((ib || a->in_dtype == M3S_DTYPE_F32) && (ob || a->out_dtype == M3S_DTYPE_F32),
              "m3s_transpose: bad dtype");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ib) return ob ? launch_tr<bf16, bf16>(a, s) : launch_tr<bf16, float>(a, s);
  return ob ? launch_tr<float, bf16>(a, s) : launch_tr<float, float>(a, s);
}
