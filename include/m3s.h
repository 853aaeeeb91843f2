/*
 * m3s.h -- C ABI of the MI355X (gfx950) Mamba-3 SISO kernels.
 *
 * The reference has no FFI for this path: its kernels are Pallas `pallas_call`s
 * invoked from Python (`mamba3_pallas/kernel_fwd.py`, `kernel_bwd.py`,
 * `kernel_decode.py`). This header is the boundary that replaces those calls; the
 * Python layer (`mamba3-siso-tpu_amd/kernels.py`) binds it with ctypes and keeps the
 * reference's Python signatures above it.
 *
 * Conventions
 *  - Every pointer is a device pointer (hipMalloc / torch CUDA memory), except the
 *    args structs themselves, which live in host memory.
 *  - "(B, H, L, P)" tensors are passed as `m3s_bhlp`: a base pointer plus element
 *    strides for the b, h and t axes; the P axis is contiguous. This lets callers hand
 *    in views of the fused in_proj output (B, L, H*P) without a transpose.
 *  - All other tensors are dense row-major in the shape given in the comment.
 *  - Calls are stream-ordered on `stream` (a hipStream_t, NULL = default stream). No
 *    call allocates or synchronises. Every call but m3s_norm_bwd_noalloc keeps no state
 *    between calls, and concurrent calls on different streams are safe; that one shares
 *    a library-owned scratch array per GPU (see its declaration).
 *  - Return value: M3S_OK (0) or a negative M3S_ERR_*; `m3s_last_error()` then holds
 *    a message (thread-local).
 */
#ifndef M3S_H_
#define M3S_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M3S_ABI_VERSION 10

#define M3S_DTYPE_F32 0  /* f32 operands, v_mfma_f32_16x16x4_f32 ("f32" policy)  */
#define M3S_DTYPE_BF16 1 /* bf16 operands, v_mfma_f32_16x16x32_bf16 ("bf16" policy) */

#define M3S_OK 0
#define M3S_ERR_INVALID (-1)     /* null pointer, bad shape or stride, misalignment */
#define M3S_ERR_UNSUPPORTED (-2) /* (dtype, chunk, N, P) has no compiled kernel     */
#define M3S_ERR_LAUNCH (-3)      /* the HIP launch itself failed                    */

typedef struct m3s_bhlp {
  void* ptr;
  int64_t stride_b, stride_h, stride_t; /* elements */
} m3s_bhlp;

/* A (B, L, X) operand: base pointer plus b and t element strides; X is contiguous.
 * The layer passes the raw slices of its fused projection (B, L, d_in_proj) this way. */
typedef struct m3s_blx {
  void* ptr;
  int64_t stride_b, stride_t; /* elements */
} m3s_blx;

/* Chunked forward. Replaces `kernel_fwd.siso_forward` (kernel_fwd.py:204-388),
 * i.e. the `pl.pallas_call(_fwd_kernel, grid=(B, nc, H))` at kernel_fwd.py:367-380. */
typedef struct m3s_fwd_args {
  int32_t struct_size; /* sizeof(m3s_fwd_args) */
  int32_t batch, seqlen, nheads, headdim, state_dim, n_angles, chunk;
  int32_t dtype; /* M3S_DTYPE_*: dtype of q, k, v, z, y, chunk_states and MFMA operands */
  int32_t has_d, has_z, has_seed, save_residuals;
  const void* q;                       /* (B, L, N)                                   */
  const void* k;                       /* (B, L, N)                                   */
  m3s_bhlp v;                          /* (B, H, L, P)                                */
  m3s_bhlp z;                          /* (B, H, L, P), if has_z                      */
  const float* adt;                    /* (B, H, L)                                   */
  const float* gamma;                  /* (B, H, L)                                   */
  const float* scale;                  /* (B, H, L)                                   */
  const float* phi;                    /* (B, H, L, Nr), or NULL with phi_strips      */
  /* phi built in the kernel instead of read (reference.py:134-157 fused into the scan):
   * phi_t = phi_strips[t / 16] + sum over t' in [16 (t / 16), t] of theta_table[t'] dt[t'],
   * angles taken mod 2 pi. Give all three (and phi = NULL) or none; L % 16 == 0. */
  const float* theta_table;            /* (B, L, Nr) tanh(angles) pi, shared by heads */
  const float* phi_dt;                 /* (B, H, L) dt                                */
  const float* phi_strips;             /* (B, H, L / 16, Nr) phi entering each strip  */
  const float* q_bias;                 /* (H, N)                                      */
  const float* k_bias;                 /* (H, N)                                      */
  const float* d_skip;                 /* (H), if has_d                               */
  const float* seed_ssm;               /* (B, H, P, N), if has_seed                   */
  const float* seed_k;                 /* (B, H, N), if has_seed                      */
  const float* seed_v;                 /* (B, H, P), if has_seed                      */
  const float* seed_coef;              /* (B, H) = dt_0 (1 - lam_0), if has_seed      */
  m3s_bhlp y;                          /* out (B, H, L, P)                            */
  void* ybar;                          /* out (B, H, L, P) pre-gate in `dtype`, if
                                          save_residuals (the reference keeps it f32) */
  void* chunk_states;                  /* out (B, H, nc, N, P) state at each chunk start,
                                          stored N-major, if save_residuals           */
  float* final_ssm;                    /* out (B, H, P, N)                            */
  float* final_k;                      /* out (B, H, N) rotated, unscaled             */
  float* final_v;                      /* out (B, H, P)                               */
  /* Raw mode (raw = 1; no counterpart in the reference, whose callers run `preprocess`
   * before its kernel, reference.py:160-199, siso.py:176-181): the kernel reads the raw
   * dt / a / trap slices of the projection in place and computes dt = softplus(dt_raw +
   * dt_bias), a = min(-heavy_tail(a_raw), -a_floor), lam = sigmoid(trap_raw), adt, gamma
   * and the t+1 scale shift on the way in; it carries phi across its chunks from the
   * chunk totals and builds each row's angle from that carry, its strip's prefix and
   * theta_table times its own dt (the three written by m3s_norm_fwd at theta_chunk =
   * chunk), starting from phi_init, and writes phi at the last position to phi_final. adt, gamma, scale, phi,
   * phi_dt and phi_strips are then NULL, theta_table is given, save_residuals is 0 (the
   * backward reads the materialised scalars), n_angles % 4 == 0 and L % 16 == 0. The
   * three raw slices share their strides, and a_raw / trap_raw start a fixed number of
   * elements (>= 0, below stride_t) after dt_raw, as slices of one projection row do.
   * M3S_ERR_UNSUPPORTED where no raw-mode kernel exists (m3s_fwd_raw_supported). */
  int32_t raw;
  float a_floor;
  m3s_blx dt_raw;                      /* (B, L, H) in dtype                          */
  m3s_blx a_raw;                       /* (B, L, H) in dtype                          */
  m3s_blx trap_raw;                    /* (B, L, H) in dtype                          */
  const float* dt_bias;                /* (H)                                         */
  const float* theta_prefix;           /* (B, H, L / 16, Nr) from m3s_norm_fwd        */
  const float* theta_chunk_totals;     /* (B, H, L / chunk, Nr) from m3s_norm_fwd     */
  const float* phi_init;               /* (B, H, Nr), or NULL for zero                */
  float* phi_final;                    /* out (B, H, Nr) in [0, 2 pi)                 */
} m3s_fwd_args;

/* Reverse-scan backward. Replaces `kernel_bwd.siso_backward_kernel`
 * (kernel_bwd.py:358-511) plus the dfinal_v injection of `siso_backward`
 * (kernel_bwd.py:632-637). The per-head dq/dk rows go to `workspace` and a second
 * launch sums them over heads into dq/dk (deterministic; no atomics). */
typedef struct m3s_bwd_args {
  int32_t struct_size; /* sizeof(m3s_bwd_args) */
  int32_t batch, seqlen, nheads, headdim, state_dim, n_angles, chunk;
  int32_t dtype;       /* dtype of dy, z, q, k, v, chunk_states, dv, dz */
  int32_t has_d, has_z;
  m3s_bhlp dy;                 /* (B, H, L, P) cotangent of the gated output           */
  const void* ybar;            /* (B, H, L, P) from the forward, in `dtype`            */
  m3s_bhlp z;                  /* (B, H, L, P), if has_z                               */
  const void* q;               /* (B, L, N)                                            */
  const void* k;               /* (B, L, N)                                            */
  m3s_bhlp v;                  /* (B, H, L, P)                                         */
  const float* adt;            /* (B, H, L)                                            */
  const float* gamma;          /* (B, H, L)                                            */
  const float* scale;          /* (B, H, L)                                            */
  const float* phi;            /* (B, H, L, Nr), or NULL with phi_strips               */
  const float* theta_table;    /* phi built in the kernel, as in m3s_fwd_args          */
  const float* phi_dt;
  const float* phi_strips;
  const float* q_bias;         /* (H, N)                                               */
  const float* k_bias;         /* (H, N)                                               */
  const float* d_skip;         /* (H), if has_d                                        */
  const void* chunk_states;    /* (B, H, nc, N, P) from the forward                    */
  const float* dfinal_ssm;     /* (B, H, P, N) or NULL                                 */
  const float* dfinal_v;       /* (B, H, P) or NULL                                    */
  float* dq;                   /* out (B, L, N), head-summed                           */
  float* dk;                   /* out (B, L, N), head-summed                           */
  m3s_bhlp dv;                 /* out (B, H, L, P)                                     */
  m3s_bhlp dz;                 /* out (B, H, L, P), if has_z                           */
  float* dadt;                 /* out (B, H, L)                                        */
  float* dqk_diag;             /* out (B, H, L)                                        */
  float* dscale;               /* out (B, H, L)                                        */
  float* uw;                   /* out (B, H, L)  u . w                                 */
  float* dphi;                 /* out (B, H, L, Nr)                                    */
  float* dq_bias;              /* out (B, H, N) per-(b, h) partial sums over time      */
  float* dk_bias;              /* out (B, H, N)                                        */
  float* k_final;              /* out (B, H, N) rotated k at the last position         */
  float* dseed_ssm;            /* out (B, H, P, N) adjoint of the seeded state         */
  void* workspace;             /* scratch, m3s_bwd_workspace_bytes() bytes, 16-aligned */
} m3s_bwd_args;

/* Single-token decode, in place. Replaces `kernel_decode.siso_decode_folded` /
 * `siso_decode` (kernel_decode.py:252-464), whose state buffers are donated
 * (`input_output_aliases={9: 1, 10: 2, 11: 3}`): ssm, k_state, v_state and
 * phi_state are read and overwritten with the next state. */
typedef struct m3s_decode_args {
  int32_t struct_size; /* sizeof(m3s_decode_args) */
  int32_t batch, nheads, headdim, state_dim, n_angles;
  int32_t dtype;       /* dtype of q, k, v, z, y and of the readout operands */
  int32_t has_d, has_z;
  const void* q;          /* (B, N)                        */
  const void* k;          /* (B, N)                        */
  const void* v;          /* (B, H, P)                     */
  const void* z;          /* (B, H, P), if has_z           */
  const float* adt;       /* (B, H)                        */
  const float* dt;        /* (B, H)                        */
  const float* lam;       /* (B, H)                        */
  const float* angles;    /* (B, Nr) raw, pre-tanh         */
  const float* q_bias;    /* (H, N)                        */
  const float* k_bias;    /* (H, N)                        */
  const float* d_skip;    /* (H), if has_d                 */
  float* ssm;             /* in/out (B, H, P, N)           */
  float* k_state;         /* in/out (B, H, N)              */
  float* v_state;         /* in/out (B, H, P)              */
  float* phi_state;       /* in/out (B, H, Nr)             */
  void* y;                /* out (B, H, P)                 */
} m3s_decode_args;

/* T decode steps in one launch. Replaces `kernel_decode.decode_scan` (kernel_decode.py:
 * 474-533: one lax.scan of decode_step over a known-length run, e.g. a fixed prompt suffix
 * or teacher forcing). Each (b, h) state stays on chip for all T steps and is read and
 * written once; every step's arithmetic is m3s_decode's, so the results equal T calls of
 * m3s_decode. Inputs carry a time axis; the state is updated in place. steps must be at
 * least 1 (a run of none has nothing to launch: the Python wrapper returns the state as it
 * was). */
typedef struct m3s_decode_scan_args {
  int32_t struct_size; /* sizeof(m3s_decode_scan_args) */
  int32_t batch, steps, nheads, headdim, state_dim, n_angles;
  int32_t dtype;       /* dtype of q, k, v, z, y and of the readout operands */
  int32_t has_d, has_z;
  const void* q;          /* (B, T, N)                     */
  const void* k;          /* (B, T, N)                     */
  const void* v;          /* (B, H, T, P)                  */
  const void* z;          /* (B, H, T, P), if has_z        */
  const float* adt;       /* (B, H, T)                     */
  const float* dt;        /* (B, H, T)                     */
  const float* lam;       /* (B, H, T)                     */
  const float* angles;    /* (B, T, Nr) raw, pre-tanh      */
  const float* q_bias;    /* (H, N)                        */
  const float* k_bias;    /* (H, N)                        */
  const float* d_skip;    /* (H), if has_d                 */
  float* ssm;             /* in/out (B, H, P, N)           */
  float* k_state;         /* in/out (B, H, N)              */
  float* v_state;         /* in/out (B, H, P)              */
  float* phi_state;       /* in/out (B, H, Nr)             */
  void* y;                /* out (B, H, T, P)              */
} m3s_decode_scan_args;

/* The layer's per-token decode step (model.py:266-289 without the block norm, residual
 * and MLP; the layer step that BASELINE configs[3] times) from the in_proj output rows:
 * BCNorm of the B and C slices (layer.py:190-198), dt = softplus(dt_raw + dt_bias),
 * lam = sigmoid(trap_raw), adt = min(-heavy_tail(a_raw), -a_floor) dt, then the step of
 * m3s_decode on x, z and the raw angles, all in one launch. The state is updated in place
 * as in m3s_decode. */
typedef struct m3s_decode_layer_args {
  int32_t struct_size;  /* sizeof(m3s_decode_layer_args) */
  int32_t batch, nheads, headdim, state_dim, n_angles;
  int32_t dtype;        /* M3S_DTYPE_* of proj and y */
  float a_floor, norm_eps;
  const void* proj;     /* (B, >= d_in_proj) rows: [z, x, B, C, dt_raw, a_raw, trap_raw, angles] */
  int64_t proj_stride;  /* elements between rows */
  const float* b_norm_weight; /* (N)    */
  const float* c_norm_weight; /* (N)    */
  const float* dt_bias; /* (H)          */
  const float* q_bias;  /* (H, N): the layer's c_bias */
  const float* k_bias;  /* (H, N): the layer's b_bias */
  const float* d_skip;  /* (H) or NULL  */
  float* ssm;           /* in/out (B, H, P, N) */
  float* k_state;       /* in/out (B, H, N)    */
  float* v_state;       /* in/out (B, H, P)    */
  float* phi_state;     /* in/out (B, H, Nr)   */
  void* y;              /* out (B, H, P) = (B, d_inner), gated */
} m3s_decode_layer_args;

/* Per-token preprocessing. Replaces `reference.preprocess` (reference.py:160-199) with
 * `heavy_tail` (202-209), `trapezoid_coeffs` (104-131) and `cumulative_angles`
 * (134-157): dt = softplus(dt_raw + dt_bias), lam = sigmoid(trap_raw),
 * a = min(-heavy_tail(a_raw), -a_floor), adt = a dt, gamma = dt lam,
 * scale_t = gamma_t + dt_{t+1}(1 - lam_{t+1}), phi = wrap(phi_init + cumsum tanh(angles) pi dt). */
typedef struct m3s_prep_fwd_args {
  int32_t struct_size; /* sizeof(m3s_prep_fwd_args) */
  int32_t batch, seqlen, nheads, n_angles;
  int32_t dtype;       /* M3S_DTYPE_* of dt_raw, a_raw, trap_raw and angles */
  int32_t has_phi_init;
  float a_floor;
  m3s_blx dt_raw;      /* (B, L, H)                       */
  m3s_blx a_raw;       /* (B, L, H)                       */
  m3s_blx trap_raw;    /* (B, L, H)                       */
  m3s_blx angles;      /* (B, L, Nr), shared by the heads */
  const float* dt_bias;  /* (H)                           */
  const float* phi_init; /* (B, H, Nr), if has_phi_init   */
  float* adt;          /* out (B, H, L)                   */
  float* gamma;        /* out (B, H, L)                   */
  float* scale;        /* out (B, H, L)                   */
  float* lam;          /* out (B, H, L)                   */
  float* dt;           /* out (B, H, L)                   */
  float* phi;          /* out (B, H, L, Nr), or NULL      */
  float* phi_final;    /* out (B, H, Nr) = phi[:, :, L-1] */
  /* The compact form m3s_fwd / m3s_bwd rebuild phi from (their phi_strips mode):
   * theta_table = tanh(angles) pi, and phi_strips[s] = wrap(phi_init + sum over t < 16 s
   * of theta_t), the angle entering token 16 s. NULL = not written; phi_strips needs
   * L % 16 == 0. At least one of phi and phi_strips is given. */
  float* theta_table;  /* out (B, L, Nr), or NULL          */
  float* phi_strips;   /* out (B, H, L / 16, Nr), or NULL  */
  void* workspace;     /* scratch, m3s_prep_fwd_workspace_bytes() bytes, 16-aligned */
} m3s_prep_fwd_args;

/* Backward of m3s_prep_fwd: the reference obtains it from jax.grad of `preprocess`
 * (siso.py:1-11). Every cotangent input may be NULL (= zero). The dangles output is
 * summed over heads (angles are shared); ddt_bias is summed over batch and time. */
typedef struct m3s_prep_bwd_args {
  int32_t struct_size; /* sizeof(m3s_prep_bwd_args) */
  int32_t batch, seqlen, nheads, n_angles;
  int32_t dtype;       /* dtype of the raw inputs and of the raw cotangents */
  float a_floor;
  m3s_blx dt_raw, a_raw, trap_raw, angles; /* the forward's inputs           */
  const float* dt_bias;                    /* (H)                            */
  const float* dadt;                       /* (B, H, L) or NULL              */
  const float* dgamma;                     /* (B, H, L) or NULL              */
  const float* dscale;                     /* (B, H, L) or NULL              */
  const float* dlam;                       /* (B, H, L) or NULL              */
  const float* ddt;                        /* (B, H, L) or NULL              */
  const float* dphi;                       /* (B, H, L, Nr) or NULL          */
  const float* dphi_final;                 /* (B, H, Nr) or NULL             */
  m3s_blx ddt_raw;                         /* out (B, L, H)                  */
  m3s_blx da_raw;                          /* out (B, L, H)                  */
  m3s_blx dtrap_raw;                       /* out (B, L, H)                  */
  m3s_blx dangles;                         /* out (B, L, Nr)                 */
  float* ddt_bias;                         /* out (H)                        */
  float* dphi_init;                        /* out (B, H, Nr) or NULL         */
  void* workspace; /* scratch, m3s_prep_bwd_workspace_bytes() bytes, 16-aligned */
} m3s_prep_bwd_args;

/* The layer's BCNorm. Replaces `layer.rms_norm` (layer.py:190-198) as applied to the B
 * and C slices of the projection (layer.py:235-236): rstd = rsqrt(mean(x^2) + eps),
 * y = (x rstd w) cast to x's dtype, computed in f32. `count` norms (1 or 2) run in one
 * launch. */
typedef struct m3s_norm_fwd_args {
  int32_t struct_size;   /* sizeof(m3s_norm_fwd_args) */
  int32_t batch, seqlen, width; /* width: the normalised axis (state_dim); a multiple of
                                   16 bytes, at most 64 * 16 bytes */
  int32_t dtype;         /* M3S_DTYPE_* of x and y */
  int32_t count;         /* 1 or 2 */
  float eps;
  m3s_blx x[2];          /* (B, L, width), 16-byte aligned rows */
  const float* weight[2];/* (width) gains */
  void* y[2];            /* out (B, L, width), dense, 16-byte aligned */
  float* rstd[2];        /* out (B, L) for the backward, or NULL */
  /* Optional, in the same launch: the rotary angles' per-token work that m3s_fwd's raw
   * mode reads (reference.py:134-157, split between this pass and the scan's carry). With
   * theta_t = theta_table[t] softplus(dt_raw[t, h] + dt_bias[h]) summed over each 16-token
   * strip in t order: theta_prefix holds, for every strip, the sum of the strips before
   * it in its chunk of theta_chunk tokens (0 for a chunk's first strip), and
   * theta_chunk_totals each chunk's sum. theta_chunk is the chunk m3s_fwd runs at (a
   * multiple of 16 dividing L); n_angles % 4 == 0. Give angles, dt_raw, dt_bias and the
   * three outputs together, or leave all NULL. */
  int32_t nheads, n_angles, theta_chunk;
  m3s_blx angles;        /* (B, L, Nr) raw angle slice, in dtype */
  m3s_blx dt_raw;        /* (B, L, H) raw dt slice, in dtype */
  const float* dt_bias;  /* (H) */
  float* theta_table;    /* out (B, L, Nr): tanh(angles) pi */
  float* theta_prefix;   /* out (B, H, L / 16, Nr), 16-byte aligned */
  float* theta_chunk_totals; /* out (B, H, L / theta_chunk, Nr), 16-byte aligned */
} m3s_norm_fwd_args;

/* Backward of m3s_norm_fwd (autograd of layer.py:190-198). dy arrives in f32 and is
 * first cast to the dtype, as the scan's q/k cotangents are cast to the primal dtype
 * (siso.py:140-148); dx is written through strides (the layer writes it into the B and
 * C slices of the projection's gradient); dweight is summed over batch and time in a
 * fixed order. */
typedef struct m3s_norm_bwd_args {
  int32_t struct_size;   /* sizeof(m3s_norm_bwd_args) */
  int32_t batch, seqlen, width;
  int32_t dtype;         /* M3S_DTYPE_* of x and dx */
  int32_t count;         /* 1 or 2 */
  m3s_blx x[2];          /* the forward's inputs */
  const float* weight[2];/* (width) */
  const float* rstd[2];  /* (B, L), from m3s_norm_fwd */
  const float* dy[2];    /* (B, L, width) f32, dense, 16-byte aligned */
  m3s_blx dx[2];         /* out (B, L, width), 16-byte aligned rows */
  float* dweight[2];     /* out (width) */
  void* workspace;       /* scratch, m3s_norm_bwd_workspace_bytes() bytes, 16-aligned */
} m3s_norm_bwd_args;

/* Weight layout for the layer's projection GEMMs: out = transpose(in), cast to
 * out_dtype, with zero rows appended up to out_rows. No counterpart in the reference,
 * which casts its weights per call (`params.in_proj.astype(u.dtype)`, layer.py:233, 256);
 * the layer computes its GEMMs against this transposed, padded copy instead. */
typedef struct m3s_transpose_args {
  int32_t struct_size;  /* sizeof(m3s_transpose_args) */
  int32_t rows, cols;   /* in is (rows, cols) */
  int32_t out_rows;     /* >= cols; out is (out_rows, rows), dense; rows >= cols are zero */
  int32_t in_dtype, out_dtype; /* M3S_DTYPE_* */
  const void* in;
  int64_t in_stride;    /* elements between rows of in */
  void* out;
} m3s_transpose_args;

/* The gate of the LM's gated MLP. Replaces the elementwise middle of `gated_mlp`
 * (model.py:125-140): with h = x @ fc1 split into value | gate halves of `width` columns,
 * forward a = value * silu(gate); backward, from da, dh = [da * silu(gate) | d gate].
 * silu(gate) is rounded to the dtype before the product, and each cotangent once, as the
 * composed framework ops round. All tensors dense, rows of 2 * width (h, dh) or width
 * (a, da) elements. 16-byte vectors when the width is a multiple of 16 bytes and every
 * tensor is 16-byte aligned, else one element per thread. */
typedef struct m3s_swiglu_args {
  int32_t struct_size;  /* sizeof(m3s_swiglu_args) */
  int32_t dtype;        /* M3S_DTYPE_* of every tensor */
  int64_t rows;
  int32_t width;
  const void* h;        /* (rows, 2 width): value | gate */
  void* a;              /* forward out (rows, width) */
  const void* da;       /* backward in (rows, width) */
  void* dh;             /* backward out (rows, 2 width) */
} m3s_swiglu_args;

/* The LM's block norms. Replaces `rms_norm` (layer.py:190-198) as the LM applies it to
 * the residual stream (model.py:194-232), and its autograd, in f32:
 * rstd = 1 / sqrt(mean(x^2) + eps), y = (x rstd w) cast to y_dtype;
 * s = sum(dy w x), dx = rstd (dy w - x rstd^2 s / width) in x_dtype,
 * dw = sum over rows of dy x rstd, summed in a fixed order. Rows are dense and aligned to
 * 4 elements; width a multiple of 4, at most 4096.
 * Residual form (the LM's residual add before each norm, model.py:222-228): with `add`
 * (y_dtype) the forward normalises s = x + add, which it writes to `sum` (x_dtype), and
 * `x` stays the stream row before the add; the backward's `x` is then that `sum`, and
 * with `dsum` (x_dtype, the cotangent of s from the rest of the network) dx becomes
 * dsum + the norm's pullback, also written to `dadd` (y_dtype) when given. */
typedef struct m3s_rms_args {
  int32_t struct_size;  /* sizeof(m3s_rms_args) */
  int32_t x_dtype;      /* M3S_DTYPE_* of x and dx (the stream) */
  int32_t y_dtype;      /* M3S_DTYPE_* of y and dy (the normalised rows) */
  int32_t width;
  int64_t rows;
  float eps;
  const void* x;        /* (rows, width) */
  const float* weight;  /* (width), 16-byte aligned */
  void* y;              /* forward out (rows, width) */
  float* rstd;          /* forward out (rows) or NULL; backward in */
  const void* dy;       /* backward in (rows, width) */
  void* dx;             /* backward out (rows, width) */
  float* dweight;       /* backward out (width) */
  void* workspace;      /* backward scratch, m3s_rms_bwd_workspace_bytes() bytes */
  const void* add;      /* forward: residual added to x first (rows, width), or NULL */
  void* sum;            /* forward out: x + add (rows, width), iff add */
  const void* dsum;     /* backward: cotangent of the sum (rows, width), or NULL */
  void* dadd;           /* backward out: dx again in y_dtype (rows, width), or NULL */
} m3s_rms_args;

/* The optimizer update of the LM training step. Replaces optax
 * chain(clip_by_global_norm, adamw) of the reference's training step (train.py:799-805)
 * once the global gradient norm is known: for each of `count` float32 tensors, in place,
 * one pass, per element (s = *grad_scale, the clip factor, or 1 when grad_scale is NULL):
 *   g = grad s;  m = m + one_minus_beta1 (g - m);  v = beta2 v + one_minus_beta2 g^2;
 *   p = p param_decay - step_size m / (sqrt(v) / bias_correction2_sqrt + eps)
 * For update t >= 1 with learning rate lr: param_decay = 1 - lr weight_decay, step_size =
 * lr / (1 - beta1^t), bias_correction2_sqrt = sqrt(1 - beta2^t); the caller forms these
 * scalars (and the complements of the betas) in double precision, as a framework's
 * scalar arguments are, so that none of them loses digits to a float32 subtraction. The
 * five arrays are host arrays of `count` entries; each tensor is dense and 4-byte
 * aligned (16-byte aligned buffers take 16-byte vectors). */
typedef struct m3s_adamw_args {
  int32_t struct_size;        /* sizeof(m3s_adamw_args) */
  int32_t count;              /* tensors */
  float* const* params;       /* [count] parameter buffers, updated */
  const float* const* grads;  /* [count] gradients */
  float* const* exp_avg;      /* [count] first moments m, updated */
  float* const* exp_avg_sq;   /* [count] second moments v, updated */
  const int64_t* numel;       /* [count] elements of each tensor */
  const float* grad_scale;    /* device scalar multiplying every gradient, or NULL */
  float one_minus_beta1, beta2, one_minus_beta2, eps;
  float param_decay, step_size, bias_correction2_sqrt;
} m3s_adamw_args;

/* The weight gradient of a projection: c (rows, cols) float32 = a^T b, reduced over the
 * tokens, for token-major bf16 operands a (tokens, rows) and b (tokens, cols) with row
 * strides lda and ldb (elements). Replaces the weight half of the transposed products
 * jax.grad forms for the projection einsums (layer.py:233, 256; model.py:231, 268, 288),
 * which the reference leaves to XLA. tokens must be a multiple of 32; a and b 16-byte
 * aligned with lda, ldb multiples of 8; each operand spans under 2 GiB. The tokens are cut
 * into a shape-dependent number of splits whose float32 partials are added in split order
 * (deterministic); with more than one split, workspace holds
 * m3s_wgrad_workspace_bytes() bytes (16-byte aligned) and c must be 16-byte aligned when
 * ldc % 4 == 0. */
typedef struct m3s_wgrad_args {
  int32_t struct_size;  /* sizeof(m3s_wgrad_args) */
  int32_t tokens, rows, cols;
  const void* a;        /* (tokens, rows) bf16 */
  int64_t lda;
  const void* b;        /* (tokens, cols) bf16 */
  int64_t ldb;
  float* c;             /* out (rows, cols) f32 */
  int64_t ldc;
  void* workspace;      /* the split partials, or NULL when one split */
} m3s_wgrad_args;

/* A projection of a decode step: y (rows, n) = x (rows, k) w (k, n), bf16 in and out,
 * float32 accumulation. Replaces, in the decode step, the per-token projections of the
 * reference's layer and LM step (model.py:266-296: in_proj, out_proj, fc1, fc2), left to
 * XLA there. n a multiple of 8; w 16-byte aligned with ldw a multiple of 8. 1 <= rows <= 4:
 * a streaming pass over w, k <= 4096. rows > 4 (a batch of tokens): MFMA tiles, k a
 * multiple of 64, x 16-byte aligned with ldx a multiple of 8, each operand under 2 GiB.
 * Row strides are in elements. Deterministic (fixed summation order). */
typedef struct m3s_gemv_args {
  int32_t struct_size;  /* sizeof(m3s_gemv_args) */
  int32_t rows, k, n;
  const void* x;        /* (rows, k) bf16 */
  int64_t ldx;
  const void* w;        /* (k, n) bf16 */
  int64_t ldw;
  void* y;              /* out (rows, n) bf16 */
  int64_t ldy;
} m3s_gemv_args;

/* Library identity; no counterpart in the reference. */
int32_t m3s_abi_version(void);
/* Message for the last non-zero return on this thread ("" if none). */
const char* m3s_last_error(void);
/* 1 if a kernel is compiled for this (dtype, chunk, N, P), else 0. For decode pass
 * chunk = 0. `which` is 0 = forward, 1 = backward, 2 = decode. */
int32_t m3s_supported(int32_t which, int32_t dtype, int32_t chunk, int32_t state_dim,
                      int32_t headdim);
/* 1 if m3s_fwd takes this (dtype, chunk, N, P, Nr) in raw mode, else 0. No counterpart in
 * the reference. */
int32_t m3s_fwd_raw_supported(int32_t dtype, int32_t chunk, int32_t state_dim, int32_t headdim,
                              int32_t n_angles);

/* Bytes of m3s_bwd_args.workspace: the per-head dq/dk rows, 2*B*H*L*N elements of
 * the dtype. No counterpart in the reference (its head sum is an in-kernel
 * accumulation over an H-innermost grid, kernel_bwd.py:324-333). */
int64_t m3s_bwd_workspace_bytes(int32_t dtype, int32_t batch, int32_t seqlen, int32_t nheads,
                                int32_t state_dim);

/* Bytes of m3s_prep_fwd_args.workspace: the tanh(angles) pi table (B, L, Nr) and the
 * theta totals per 16-token strip (B, ceil(L/16), H, Nr), f32 (per 64-token block when phi
 * itself is written). No counterpart in the reference.
 * -1 on bad dimensions. */
int64_t m3s_prep_fwd_workspace_bytes(int32_t batch, int32_t seqlen, int32_t nheads,
                                     int32_t n_angles);
/* Bytes of m3s_prep_bwd_args.workspace: the per-block dphi carries (B, ceil(L/32), H,
 * Nr) and dt_bias partials (B, ceil(L/32), H), f32. No counterpart in the reference.
 * -1 on bad dimensions. */
int64_t m3s_prep_bwd_workspace_bytes(int32_t batch, int32_t seqlen, int32_t nheads,
                                     int32_t n_angles);

/* Bytes of m3s_norm_bwd_args.workspace: per-block gain partials (1024, 2, width) f32.
 * No counterpart in the reference. -1 on a bad width. */
int64_t m3s_norm_bwd_workspace_bytes(int32_t width);
/* Bytes of m3s_rms_args.workspace: per-block gain partials (1024, width) f32. No
 * counterpart in the reference. -1 on a bad width. */
int64_t m3s_rms_bwd_workspace_bytes(int32_t width);

int32_t m3s_fwd(const m3s_fwd_args* args, void* stream);
int32_t m3s_bwd(const m3s_bwd_args* args, void* stream);
int32_t m3s_decode(const m3s_decode_args* args, void* stream);
int32_t m3s_decode_scan(const m3s_decode_scan_args* args, void* stream);
int32_t m3s_decode_layer(const m3s_decode_layer_args* args, void* stream);
int32_t m3s_prep_fwd(const m3s_prep_fwd_args* args, void* stream);
int32_t m3s_prep_bwd(const m3s_prep_bwd_args* args, void* stream);
int32_t m3s_norm_fwd(const m3s_norm_fwd_args* args, void* stream);
int32_t m3s_norm_bwd(const m3s_norm_bwd_args* args, void* stream);
/* m3s_norm_bwd without a caller workspace: no counterpart in the reference. For callers
 * that cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). The gain partials live in a library-owned device array of 4 MiB per GPU
 * (enough for every width m3s_norm_bwd accepts, at most 512), held until the process
 * ends; args->workspace is ignored and nothing is allocated or freed. Calls that overlap
 * on one GPU (different streams, or threads) share that array and race: serialise them.
 * Widths the array cannot hold are rejected with M3S_ERR_INVALID. The array's device
 * address is looked up on a device's first call and kept for the life of the process: it
 * stays valid until that device is reset (hipDeviceReset unloads the code object that
 * holds the array), so a caller that resets a device must reload the library before
 * calling this again. */
int32_t m3s_norm_bwd_noalloc(const m3s_norm_bwd_args* args, void* stream);
int32_t m3s_transpose(const m3s_transpose_args* args, void* stream);
int32_t m3s_swiglu_fwd(const m3s_swiglu_args* args, void* stream);
int32_t m3s_swiglu_bwd(const m3s_swiglu_args* args, void* stream);
int32_t m3s_rms_fwd(const m3s_rms_args* args, void* stream);
int32_t m3s_rms_bwd(const m3s_rms_args* args, void* stream);
int32_t m3s_adamw(const m3s_adamw_args* args, void* stream);
/* Bytes of m3s_wgrad_args.workspace for this shape (0 when one split suffices), -1 on bad
 * dimensions. No counterpart in the reference. */
int64_t m3s_wgrad_workspace_bytes(int32_t tokens, int32_t rows, int32_t cols);
int32_t m3s_wgrad(const m3s_wgrad_args* args, void* stream);
int32_t m3s_gemv(const m3s_gemv_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* M3S_H_ */
