"""ctypes binding of the C ABI in ``include/m3s.h`` (``csrc/libm3s.so``).

The structs below mirror the header field for field; `m3s_abi_version` and the
``struct_size`` field of each args struct guard against a stale library.
"""

from __future__ import annotations

import ctypes as C
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "csrc", "libm3s.so")
ABI_VERSION = 10

DTYPE_F32 = 0
DTYPE_BF16 = 1
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_LAUNCH = 0, -1, -2, -3

i32, i64, vp = C.c_int32, C.c_int64, C.c_void_p


class Bhlp(C.Structure):
    _fields_ = [("ptr", vp), ("stride_b", i64), ("stride_h", i64), ("stride_t", i64)]


class Blx(C.Structure):
    _fields_ = [("ptr", vp), ("stride_b", i64), ("stride_t", i64)]


class FwdArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32),
        ("batch", i32), ("seqlen", i32), ("nheads", i32), ("headdim", i32),
        ("state_dim", i32), ("n_angles", i32), ("chunk", i32),
        ("dtype", i32),
        ("has_d", i32), ("has_z", i32), ("has_seed", i32), ("save_residuals", i32),
        ("q", vp), ("k", vp), ("v", Bhlp), ("z", Bhlp),
        ("adt", vp), ("gamma", vp), ("scale", vp), ("phi", vp),
        ("theta_table", vp), ("phi_dt", vp), ("phi_strips", vp),
        ("q_bias", vp), ("k_bias", vp), ("d_skip", vp),
        ("seed_ssm", vp), ("seed_k", vp), ("seed_v", vp), ("seed_coef", vp),
        ("y", Bhlp), ("ybar", vp), ("chunk_states", vp),
        ("final_ssm", vp), ("final_k", vp), ("final_v", vp),
        ("raw", i32), ("a_floor", C.c_float),
        ("dt_raw", Blx), ("a_raw", Blx), ("trap_raw", Blx),
        ("dt_bias", vp), ("theta_prefix", vp), ("theta_chunk_totals", vp),
        ("phi_init", vp), ("phi_final", vp),
    ]


class BwdArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32),
        ("batch", i32), ("seqlen", i32), ("nheads", i32), ("headdim", i32),
        ("state_dim", i32), ("n_angles", i32), ("chunk", i32),
        ("dtype", i32),
        ("has_d", i32), ("has_z", i32),
        ("dy", Bhlp), ("ybar", vp), ("z", Bhlp), ("q", vp), ("k", vp), ("v", Bhlp),
        ("adt", vp), ("gamma", vp), ("scale", vp), ("phi", vp),
        ("theta_table", vp), ("phi_dt", vp), ("phi_strips", vp),
        ("q_bias", vp), ("k_bias", vp), ("d_skip", vp),
        ("chunk_states", vp), ("dfinal_ssm", vp), ("dfinal_v", vp),
        ("dq", vp), ("dk", vp), ("dv", Bhlp), ("dz", Bhlp),
        ("dadt", vp), ("dqk_diag", vp), ("dscale", vp), ("uw", vp), ("dphi", vp),
        ("dq_bias", vp), ("dk_bias", vp), ("k_final", vp), ("dseed_ssm", vp),
        ("workspace", vp),
    ]


class DecodeArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32),
        ("batch", i32), ("nheads", i32), ("headdim", i32), ("state_dim", i32),
        ("n_angles", i32),
        ("dtype", i32),
        ("has_d", i32), ("has_z", i32),
        ("q", vp), ("k", vp), ("v", vp), ("z", vp),
        ("adt", vp), ("dt", vp), ("lam", vp), ("angles", vp),
        ("q_bias", vp), ("k_bias", vp), ("d_skip", vp),
        ("ssm", vp), ("k_state", vp), ("v_state", vp), ("phi_state", vp),
        ("y", vp),
    ]


class DecodeScanArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32),
        ("batch", i32), ("steps", i32), ("nheads", i32), ("headdim", i32), ("state_dim", i32),
        ("n_angles", i32),
        ("dtype", i32),
        ("has_d", i32), ("has_z", i32),
        ("q", vp), ("k", vp), ("v", vp), ("z", vp),
        ("adt", vp), ("dt", vp), ("lam", vp), ("angles", vp),
        ("q_bias", vp), ("k_bias", vp), ("d_skip", vp),
        ("ssm", vp), ("k_state", vp), ("v_state", vp), ("phi_state", vp),
        ("y", vp),
    ]


class DecodeLayerArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32),
        ("batch", i32), ("nheads", i32), ("headdim", i32), ("state_dim", i32),
        ("n_angles", i32),
        ("dtype", i32), ("a_floor", C.c_float), ("norm_eps", C.c_float),
        ("proj", vp), ("proj_stride", i64),
        ("b_norm_weight", vp), ("c_norm_weight", vp), ("dt_bias", vp),
        ("q_bias", vp), ("k_bias", vp), ("d_skip", vp),
        ("ssm", vp), ("k_state", vp), ("v_state", vp), ("phi_state", vp),
        ("y", vp),
    ]


class PrepFwdArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32),
        ("batch", i32), ("seqlen", i32), ("nheads", i32), ("n_angles", i32),
        ("dtype", i32), ("has_phi_init", i32), ("a_floor", C.c_float),
        ("dt_raw", Blx), ("a_raw", Blx), ("trap_raw", Blx), ("angles", Blx),
        ("dt_bias", vp), ("phi_init", vp),
        ("adt", vp), ("gamma", vp), ("scale", vp), ("lam", vp), ("dt", vp),
        ("phi", vp), ("phi_final", vp), ("theta_table", vp), ("phi_strips", vp),
        ("workspace", vp),
    ]


class PrepBwdArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32),
        ("batch", i32), ("seqlen", i32), ("nheads", i32), ("n_angles", i32),
        ("dtype", i32), ("a_floor", C.c_float),
        ("dt_raw", Blx), ("a_raw", Blx), ("trap_raw", Blx), ("angles", Blx),
        ("dt_bias", vp),
        ("dadt", vp), ("dgamma", vp), ("dscale", vp), ("dlam", vp), ("ddt", vp),
        ("dphi", vp), ("dphi_final", vp),
        ("ddt_raw", Blx), ("da_raw", Blx), ("dtrap_raw", Blx), ("dangles", Blx),
        ("ddt_bias", vp), ("dphi_init", vp),
        ("workspace", vp),
    ]


class NormFwdArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32),
        ("batch", i32), ("seqlen", i32), ("width", i32),
        ("dtype", i32), ("count", i32), ("eps", C.c_float),
        ("x", Blx * 2), ("weight", vp * 2), ("y", vp * 2), ("rstd", vp * 2),
        ("nheads", i32), ("n_angles", i32), ("theta_chunk", i32), ("angles", Blx),
        ("dt_raw", Blx), ("dt_bias", vp), ("theta_table", vp), ("theta_prefix", vp),
        ("theta_chunk_totals", vp),
    ]


class NormBwdArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32),
        ("batch", i32), ("seqlen", i32), ("width", i32),
        ("dtype", i32), ("count", i32),
        ("x", Blx * 2), ("weight", vp * 2), ("rstd", vp * 2), ("dy", vp * 2),
        ("dx", Blx * 2), ("dweight", vp * 2),
        ("workspace", vp),
    ]


class TransposeArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32), ("rows", i32), ("cols", i32), ("out_rows", i32),
        ("in_dtype", i32), ("out_dtype", i32),
        ("inp", vp), ("in_stride", i64), ("out", vp),
    ]


class SwigluArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32), ("dtype", i32), ("rows", i64), ("width", i32),
        ("h", vp), ("a", vp), ("da", vp), ("dh", vp),
    ]


class RmsArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32), ("x_dtype", i32), ("y_dtype", i32), ("width", i32),
        ("rows", i64), ("eps", C.c_float),
        ("x", vp), ("weight", vp), ("y", vp), ("rstd", vp), ("dy", vp), ("dx", vp),
        ("dweight", vp), ("workspace", vp), ("add", vp), ("sum", vp), ("dsum", vp),
        ("dadd", vp),
    ]


class AdamwArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32), ("count", i32), ("params", vp), ("grads", vp),
        ("exp_avg", vp), ("exp_avg_sq", vp), ("numel", vp), ("grad_scale", vp),
        ("one_minus_beta1", C.c_float), ("beta2", C.c_float), ("one_minus_beta2", C.c_float),
        ("eps", C.c_float), ("param_decay", C.c_float), ("step_size", C.c_float),
        ("bias_correction2_sqrt", C.c_float),
    ]


class WgradArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32), ("tokens", i32), ("rows", i32), ("cols", i32),
        ("a", vp), ("lda", i64), ("b", vp), ("ldb", i64), ("c", vp), ("ldc", i64),
        ("workspace", vp),
    ]


class GemvArgs(C.Structure):
    _fields_ = [
        ("struct_size", i32), ("rows", i32), ("k", i32), ("n", i32),
        ("x", vp), ("ldx", i64), ("w", vp), ("ldw", i64), ("y", vp), ("ldy", i64),
    ]


#: Every symbol ``include/m3s.h`` declares.
EXPORTS = ("m3s_abi_version", "m3s_last_error", "m3s_supported", "m3s_fwd_raw_supported",
           "m3s_bwd_workspace_bytes",
           "m3s_prep_fwd_workspace_bytes", "m3s_prep_bwd_workspace_bytes", "m3s_fwd", "m3s_bwd", "m3s_decode", "m3s_decode_scan",
           "m3s_prep_fwd", "m3s_prep_bwd", "m3s_norm_bwd_workspace_bytes", "m3s_norm_fwd",
           "m3s_norm_bwd", "m3s_decode_layer", "m3s_transpose", "m3s_swiglu_fwd",
           "m3s_swiglu_bwd", "m3s_rms_fwd", "m3s_rms_bwd", "m3s_rms_bwd_workspace_bytes",
           "m3s_norm_bwd_noalloc", "m3s_adamw", "m3s_wgrad", "m3s_wgrad_workspace_bytes", "m3s_gemv")

_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load the library (torch is already imported, so the HIP runtime it loaded is
    the one the library binds to). Raises if it is missing or stale -- there is no
    fallback compute path."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python __graft_entry__.py build` "
            "(the HIP kernels are the only compute path)")
    lib = C.CDLL(path)
    lib.m3s_abi_version.restype = i32
    lib.m3s_last_error.restype = C.c_char_p
    lib.m3s_supported.restype = i32
    lib.m3s_supported.argtypes = [i32, i32, i32, i32, i32]
    lib.m3s_fwd_raw_supported.restype = i32
    lib.m3s_fwd_raw_supported.argtypes = [i32, i32, i32, i32, i32]
    lib.m3s_bwd_workspace_bytes.restype = i64
    lib.m3s_bwd_workspace_bytes.argtypes = [i32, i32, i32, i32, i32]
    lib.m3s_fwd.restype = i32
    lib.m3s_fwd.argtypes = [C.POINTER(FwdArgs), vp]
    lib.m3s_bwd.restype = i32
    lib.m3s_bwd.argtypes = [C.POINTER(BwdArgs), vp]
    lib.m3s_decode.restype = i32
    lib.m3s_decode.argtypes = [C.POINTER(DecodeArgs), vp]
    lib.m3s_decode_scan.restype = i32
    lib.m3s_decode_scan.argtypes = [C.POINTER(DecodeScanArgs), vp]
    lib.m3s_prep_fwd_workspace_bytes.restype = i64
    lib.m3s_prep_fwd_workspace_bytes.argtypes = [i32, i32, i32, i32]
    lib.m3s_prep_bwd_workspace_bytes.restype = i64
    lib.m3s_prep_bwd_workspace_bytes.argtypes = [i32, i32, i32, i32]
    lib.m3s_prep_fwd.restype = i32
    lib.m3s_prep_fwd.argtypes = [C.POINTER(PrepFwdArgs), vp]
    lib.m3s_prep_bwd.restype = i32
    lib.m3s_prep_bwd.argtypes = [C.POINTER(PrepBwdArgs), vp]
    lib.m3s_transpose.restype = i32
    lib.m3s_transpose.argtypes = [C.POINTER(TransposeArgs), vp]
    lib.m3s_decode_layer.restype = i32
    lib.m3s_decode_layer.argtypes = [C.POINTER(DecodeLayerArgs), vp]
    lib.m3s_norm_bwd_workspace_bytes.restype = i64
    lib.m3s_norm_bwd_workspace_bytes.argtypes = [i32]
    lib.m3s_norm_fwd.restype = i32
    lib.m3s_norm_fwd.argtypes = [C.POINTER(NormFwdArgs), vp]
    lib.m3s_norm_bwd.restype = i32
    lib.m3s_norm_bwd.argtypes = [C.POINTER(NormBwdArgs), vp]
    lib.m3s_norm_bwd_noalloc.restype = i32
    lib.m3s_norm_bwd_noalloc.argtypes = [C.POINTER(NormBwdArgs), vp]
    lib.m3s_rms_bwd_workspace_bytes.restype = i64
    lib.m3s_rms_bwd_workspace_bytes.argtypes = [i32]
    for fn in (lib.m3s_rms_fwd, lib.m3s_rms_bwd):
        fn.restype = i32
        fn.argtypes = [C.POINTER(RmsArgs), vp]
    for fn in (lib.m3s_swiglu_fwd, lib.m3s_swiglu_bwd):
        fn.restype = i32
        fn.argtypes = [C.POINTER(SwigluArgs), vp]
    lib.m3s_adamw.restype = i32
    lib.m3s_adamw.argtypes = [C.POINTER(AdamwArgs), vp]
    lib.m3s_wgrad.restype = i32
    lib.m3s_wgrad.argtypes = [C.POINTER(WgradArgs), vp]
    lib.m3s_wgrad_workspace_bytes.restype = i64
    lib.m3s_wgrad_workspace_bytes.argtypes = [i32, i32, i32]
    lib.m3s_gemv.restype = i32
    lib.m3s_gemv.argtypes = [C.POINTER(GemvArgs), vp]
    ver = lib.m3s_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Map a non-zero ABI return code onto the reference's exception types."""
    if rc == OK:
        return
    msg = load().m3s_last_error().decode(errors="replace")
    if rc in (ERR_INVALID, ERR_UNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def supported(which: int, dtype: int, chunk: int, state_dim: int, headdim: int) -> bool:
    return bool(load().m3s_supported(which, dtype, chunk, state_dim, headdim))


def raw_supported(dtype: int, chunk: int, state_dim: int, headdim: int, n_angles: int) -> bool:
    """Whether ``m3s_fwd`` takes this shape in raw mode (`m3s_fwd_raw_supported`)."""
    return bool(load().m3s_fwd_raw_supported(dtype, chunk, state_dim, headdim, n_angles))


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    raise ValueError(f"kernels run in bf16 or f32, got {dt}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def bhlp(t) -> Bhlp:
    """A (B, H, L, P) tensor with unit stride on P."""
    if t is None:
        return Bhlp(None, 0, 0, 0)
    if t.stride(3) != 1:
        raise ValueError("(B, H, L, P) operand must be contiguous along P")
    return Bhlp(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def blx(t) -> Blx:
    """A (B, L, X) tensor with unit stride on X."""
    if t is None:
        return Blx(None, 0, 0)
    if t.stride(2) != 1 and t.shape[2] > 1:
        raise ValueError("(B, L, X) operand must be contiguous along its last axis")
    return Blx(t.data_ptr(), t.stride(0), t.stride(1))


def stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
