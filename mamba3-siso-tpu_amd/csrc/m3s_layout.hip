// Weight layout for the layer's projection GEMMs on gfx950: a tiled transpose with a
// dtype cast and appended zero rows.
//
// The reference casts its projection weights per call (`params.in_proj.astype(u.dtype)`,
// layer.py:233, 256). The layer here computes its GEMMs against a transposed copy of each
// weight -- in_proj zero-padded to a multiple of 256 rows -- which is the operand layout
// hipBLASLt runs fastest at these shapes, and makes that copy in the same pass as the cast.
// 64 x 64 tiles through LDS (odd row pitch: no bank conflicts on the transposed read);
// reads and writes are row-contiguous across a wave. HBM-bound.
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

template <typename TI, typename TO>
static int32_t launch_tr(const m3s_transpose_args* a, hipStream_t s) {
  const dim3 grid((a->out_rows + kTrTile - 1) / kTrTile, (a->rows + kTrTile - 1) / kTrTile);
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
