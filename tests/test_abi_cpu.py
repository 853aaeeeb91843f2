"""The C-ABI library: it loads, exports every symbol include/m3s.h declares, agrees with
the header on struct layouts, and rejects bad arguments before touching the GPU.
No kernel is launched here."""

import ctypes
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "m3s.h")


@pytest.fixture(scope="module")
def lib(m3):
    from mamba3_siso_tpu_amd import _lib

    return _lib


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int32_t|int64_t|const char\*)\s+(m3s_\w+)\s*\(", text, re.M)))


def test_library_loads_and_exports_every_declared_symbol(lib):
    handle = lib.load()
    names = declared_functions()
    assert names, "no declarations parsed from include/m3s.h"
    assert set(names) == set(lib.EXPORTS)
    for name in names:
        assert hasattr(handle, name), f"{name} declared in m3s.h but not exported"
    assert handle.m3s_abi_version() == lib.ABI_VERSION == 10


def test_struct_layouts_match_the_header(lib):
    """Compile the header with gcc and compare sizeof/offsetof with the ctypes mirror."""
    src = r"""
#include <stdio.h>
#include <stddef.h>
#include "m3s.h"
int main(void) {
  printf("%zu %zu %zu %zu\n", sizeof(m3s_bhlp), sizeof(m3s_fwd_args),
         sizeof(m3s_bwd_args), sizeof(m3s_decode_args));
  printf("%zu %zu %zu\n", offsetof(m3s_fwd_args, final_v), offsetof(m3s_bwd_args, dseed_ssm),
         offsetof(m3s_decode_args, y));
  printf("%zu %zu %zu\n", sizeof(m3s_blx), sizeof(m3s_prep_fwd_args), sizeof(m3s_prep_bwd_args));
  printf("%zu %zu %zu\n", offsetof(m3s_prep_fwd_args, dt_raw), offsetof(m3s_prep_bwd_args, ddt_raw),
         offsetof(m3s_prep_bwd_args, workspace));
  printf("%zu %zu %zu %zu %zu %zu\n", sizeof(m3s_norm_fwd_args), sizeof(m3s_norm_bwd_args),
         offsetof(m3s_norm_fwd_args, x), offsetof(m3s_norm_fwd_args, rstd),
         offsetof(m3s_norm_bwd_args, dx), offsetof(m3s_norm_bwd_args, workspace));
  printf("%zu %zu %zu\n", sizeof(m3s_decode_layer_args), offsetof(m3s_decode_layer_args, proj_stride),
         offsetof(m3s_decode_layer_args, y));
  printf("%zu %zu %zu\n", sizeof(m3s_transpose_args), offsetof(m3s_transpose_args, in_stride),
         offsetof(m3s_transpose_args, out));
  printf("%zu %zu %zu\n", sizeof(m3s_swiglu_args), offsetof(m3s_swiglu_args, rows),
         offsetof(m3s_swiglu_args, dh));
  printf("%zu %zu %zu\n", sizeof(m3s_rms_args), offsetof(m3s_rms_args, x),
         offsetof(m3s_rms_args, workspace));
  printf("%zu %zu %zu\n", sizeof(m3s_adamw_args), offsetof(m3s_adamw_args, grad_scale),
         offsetof(m3s_adamw_args, bias_correction2_sqrt));
  printf("%zu %zu %zu\n", sizeof(m3s_wgrad_args), offsetof(m3s_wgrad_args, ldb),
         offsetof(m3s_wgrad_args, workspace));
  printf("%zu %zu %zu\n", sizeof(m3s_gemv_args), offsetof(m3s_gemv_args, ldw),
         offsetof(m3s_gemv_args, ldy));
  printf("%zu %zu %zu %zu\n", offsetof(m3s_fwd_args, raw), offsetof(m3s_fwd_args, phi_final),
         offsetof(m3s_norm_fwd_args, angles), offsetof(m3s_norm_fwd_args, theta_chunk_totals));
  printf("%zu %zu %zu\n", sizeof(m3s_decode_scan_args), offsetof(m3s_decode_scan_args, q),
         offsetof(m3s_decode_scan_args, y));
  return 0;
}
"""
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        exe = os.path.join(d, "t")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", os.path.dirname(HEADER), c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()
    sizes = [int(x) for x in out]
    assert sizes[:4] == [ctypes.sizeof(lib.Bhlp), ctypes.sizeof(lib.FwdArgs),
                         ctypes.sizeof(lib.BwdArgs), ctypes.sizeof(lib.DecodeArgs)]
    assert sizes[4:7] == [lib.FwdArgs.final_v.offset, lib.BwdArgs.dseed_ssm.offset,
                          lib.DecodeArgs.y.offset]
    assert sizes[7:10] == [ctypes.sizeof(lib.Blx), ctypes.sizeof(lib.PrepFwdArgs),
                           ctypes.sizeof(lib.PrepBwdArgs)]
    assert sizes[10:13] == [lib.PrepFwdArgs.dt_raw.offset, lib.PrepBwdArgs.ddt_raw.offset,
                            lib.PrepBwdArgs.workspace.offset]
    assert sizes[13:19] == [ctypes.sizeof(lib.NormFwdArgs), ctypes.sizeof(lib.NormBwdArgs),
                            lib.NormFwdArgs.x.offset, lib.NormFwdArgs.rstd.offset,
                            lib.NormBwdArgs.dx.offset, lib.NormBwdArgs.workspace.offset]
    assert sizes[19:22] == [ctypes.sizeof(lib.DecodeLayerArgs), lib.DecodeLayerArgs.proj_stride.offset,
                            lib.DecodeLayerArgs.y.offset]
    assert sizes[22:25] == [ctypes.sizeof(lib.TransposeArgs), lib.TransposeArgs.in_stride.offset,
                            lib.TransposeArgs.out.offset]
    assert sizes[25:28] == [ctypes.sizeof(lib.SwigluArgs), lib.SwigluArgs.rows.offset,
                            lib.SwigluArgs.dh.offset]
    assert sizes[28:31] == [ctypes.sizeof(lib.RmsArgs), lib.RmsArgs.x.offset,
                            lib.RmsArgs.workspace.offset]
    assert sizes[31:34] == [ctypes.sizeof(lib.AdamwArgs), lib.AdamwArgs.grad_scale.offset,
                            lib.AdamwArgs.bias_correction2_sqrt.offset]
    assert sizes[34:37] == [ctypes.sizeof(lib.WgradArgs), lib.WgradArgs.ldb.offset,
                            lib.WgradArgs.workspace.offset]
    assert sizes[40:44] == [lib.FwdArgs.raw.offset, lib.FwdArgs.phi_final.offset,
                            lib.NormFwdArgs.angles.offset, lib.NormFwdArgs.theta_chunk_totals.offset]
    assert sizes[44:] == [ctypes.sizeof(lib.DecodeScanArgs), lib.DecodeScanArgs.q.offset,
                          lib.DecodeScanArgs.y.offset]
    assert sizes[37:40] == [ctypes.sizeof(lib.GemvArgs), lib.GemvArgs.ldw.offset,
                          lib.GemvArgs.ldy.offset]


def test_null_and_stale_args_are_rejected_without_a_launch(lib):
    h = lib.load()
    assert h.m3s_fwd(None, None) == lib.ERR_INVALID
    assert b"NULL" in h.m3s_last_error()
    a = lib.FwdArgs()
    a.struct_size = 3
    assert h.m3s_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"ABI mismatch" in h.m3s_last_error()
    b = lib.BwdArgs()
    b.struct_size = ctypes.sizeof(lib.BwdArgs)
    assert h.m3s_bwd(ctypes.byref(b), None) == lib.ERR_INVALID   # zero dims
    d = lib.DecodeArgs()
    d.struct_size = ctypes.sizeof(lib.DecodeArgs)
    assert h.m3s_decode(ctypes.byref(d), None) == lib.ERR_INVALID
    e = lib.DecodeScanArgs()
    e.struct_size = ctypes.sizeof(lib.DecodeScanArgs)
    assert h.m3s_decode_scan(ctypes.byref(e), None) == lib.ERR_INVALID   # zero dims
    e.struct_size = 3
    assert h.m3s_decode_scan(ctypes.byref(e), None) == lib.ERR_INVALID
    assert b"ABI mismatch" in h.m3s_last_error()


def test_unsupported_shapes_and_bad_dims_are_reported(lib):
    h = lib.load()
    a = lib.FwdArgs()
    a.struct_size = ctypes.sizeof(lib.FwdArgs)
    a.batch, a.seqlen, a.nheads, a.headdim, a.state_dim, a.n_angles, a.chunk = 1, 128, 1, 24, 128, 32, 128
    a.dtype = lib.DTYPE_BF16
    assert h.m3s_fwd(ctypes.byref(a), None) == lib.ERR_UNSUPPORTED
    assert b"no kernel" in h.m3s_last_error()
    a.headdim, a.seqlen = 64, 100
    assert h.m3s_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"multiple of chunk" in h.m3s_last_error()
    a.seqlen, a.n_angles = 128, 65
    assert h.m3s_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    a.n_angles = 32   # now only the pointers are missing
    assert h.m3s_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"q/k" in h.m3s_last_error()


def test_workspace_size(lib):
    h = lib.load()
    assert h.m3s_bwd_workspace_bytes(lib.DTYPE_BF16, 8, 8192, 32, 128) == 2 * 8 * 32 * 8192 * 128 * 2
    assert h.m3s_bwd_workspace_bytes(lib.DTYPE_F32, 1, 64, 2, 16) == 2 * 2 * 64 * 16 * 4


def test_prep_arguments_are_checked_without_a_launch(lib):
    h = lib.load()
    assert h.m3s_prep_fwd(None, None) == lib.ERR_INVALID
    a = lib.PrepFwdArgs()
    a.struct_size = ctypes.sizeof(lib.PrepFwdArgs)
    a.batch, a.seqlen, a.nheads, a.n_angles = 1, 16, 2, 4
    a.dtype = 7
    assert h.m3s_prep_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"bad dtype" in h.m3s_last_error()
    a.dtype = lib.DTYPE_F32
    assert h.m3s_prep_fwd(ctypes.byref(a), None) == lib.ERR_INVALID   # null pointers
    b = lib.PrepBwdArgs()
    b.struct_size = ctypes.sizeof(lib.PrepBwdArgs) - 8
    assert h.m3s_prep_bwd(ctypes.byref(b), None) == lib.ERR_INVALID
    assert b"ABI mismatch" in h.m3s_last_error()
    # the backward's blocks are 32 tokens: 256 per sequence at L=8192
    assert h.m3s_prep_bwd_workspace_bytes(8, 8192, 32, 32) == 8 * 256 * 32 * 32 * 4 + 8 * 256 * 32 * 4
    assert h.m3s_prep_bwd_workspace_bytes(0, 8, 1, 1) == -1
    assert h.m3s_prep_fwd_workspace_bytes(8, 8192, 32, 32) == 8 * 8192 * 32 * 4 + 8 * 512 * 32 * 32 * 4
    assert h.m3s_prep_fwd_workspace_bytes(1, 8, 1, -1) == -1


def test_capability_table(lib):
    assert lib.supported(0, lib.DTYPE_BF16, 128, 128, 64)
    assert lib.supported(1, lib.DTYPE_BF16, 128, 128, 64)
    assert lib.supported(2, lib.DTYPE_BF16, 0, 128, 64)
    assert lib.supported(0, lib.DTYPE_F32, 64, 16, 16) and lib.supported(1, lib.DTYPE_F32, 64, 16, 16)
    # every backward configuration has a forward
    for dt in (lib.DTYPE_F32, lib.DTYPE_BF16):
        for c in (32, 64, 128, 256):
            for n in (16, 32, 64, 128):
                for p in (16, 64):
                    if lib.supported(1, dt, c, n, p):
                        assert lib.supported(0, dt, c, n, p)
    assert not lib.supported(0, lib.DTYPE_BF16, 256, 128, 64)


def test_python_kernel_table_mirrors_the_library(lib):
    """layout.KERNELS (what SISOConfig validates against without loading the library)
    equals the library's m3s_supported answer on every (role, policy, chunk, N, P) of a
    grid wider than both tables."""
    from mamba3_siso_tpu_amd import layout as LY
    codes = {"bf16": lib.DTYPE_BF16, "f32": lib.DTYPE_F32}
    roles = {"forward": 0, "backward": 1, "decode": 2}
    for role, which in roles.items():
        for pol, code in codes.items():
            for c in ((0,) if role == "decode" else (16, 32, 64, 128, 256, 512)):
                for n in (16, 32, 64, 128, 256):
                    for p in (16, 32, 64, 128):
                        want = bool(lib.supported(which, code, c, n, p))
                        assert ((pol, c, n, p) in LY.KERNELS[role]) == want, (role, pol, c, n, p)


def test_norm_arguments_are_checked_without_a_launch(lib):
    h = lib.load()
    assert h.m3s_norm_bwd_workspace_bytes(128) == 1024 * 2 * 128 * 4
    assert h.m3s_norm_bwd_workspace_bytes(0) == -1
    a = lib.NormFwdArgs()
    a.struct_size = ctypes.sizeof(lib.NormFwdArgs)
    a.batch, a.seqlen, a.width, a.dtype, a.count, a.eps = 2, 8, 128, lib.DTYPE_BF16, 3, 1e-5
    assert h.m3s_norm_fwd(ctypes.byref(a), None) == lib.ERR_INVALID      # count must be 1 or 2
    a.count = 1
    a.width = 100                                                        # not a multiple of 8
    assert h.m3s_norm_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"multiple of 8" in h.m3s_last_error()
    a.width = 128
    a.x[0] = lib.Blx(0x1008, 4480, 8 * 4480)                            # 8-byte aligned base
    assert h.m3s_norm_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"aligned" in h.m3s_last_error()
    b = lib.NormBwdArgs()
    b.struct_size = ctypes.sizeof(lib.NormBwdArgs)
    b.batch, b.seqlen, b.width, b.dtype, b.count = 2, 8, 128, lib.DTYPE_BF16, 2
    assert h.m3s_norm_bwd(ctypes.byref(b), None) == lib.ERR_INVALID      # no workspace
    assert b"workspace" in h.m3s_last_error()


def test_decode_layer_arguments_are_checked_without_a_launch(lib):
    h = lib.load()
    a = lib.DecodeLayerArgs()
    a.struct_size = ctypes.sizeof(lib.DecodeLayerArgs)
    a.batch, a.nheads, a.headdim, a.state_dim, a.n_angles = 4, 32, 64, 128, 32
    a.dtype = lib.DTYPE_BF16
    a.proj, a.proj_stride = 0x1000, 4000          # narrower than d_in_proj = 4480
    assert h.m3s_decode_layer(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"row stride" in h.m3s_last_error()
    a.state_dim = 96
    assert h.m3s_decode_layer(ctypes.byref(a), None) == lib.ERR_UNSUPPORTED


def test_transpose_arguments_are_checked_without_a_launch(lib):
    h = lib.load()
    a = lib.TransposeArgs()
    a.struct_size = ctypes.sizeof(lib.TransposeArgs)
    a.rows, a.cols, a.out_rows = 64, 100, 96                 # out_rows < cols
    a.in_dtype = a.out_dtype = lib.DTYPE_BF16
    a.inp, a.in_stride, a.out = 0x1000, 100, 0x2000
    assert h.m3s_transpose(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"out_rows" in h.m3s_last_error()
    a.out_rows, a.in_stride = 128, 50                        # row stride shorter than a row
    assert h.m3s_transpose(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"in_stride" in h.m3s_last_error()


def test_swiglu_arguments_are_checked_without_a_launch(lib):
    h = lib.load()
    assert h.m3s_swiglu_fwd(None, None) == lib.ERR_INVALID
    a = lib.SwigluArgs()
    a.struct_size = 7
    assert h.m3s_swiglu_bwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"ABI mismatch" in h.m3s_last_error()
    a.struct_size = ctypes.sizeof(lib.SwigluArgs)
    a.dtype, a.rows, a.width = lib.DTYPE_BF16, 16, 0           # empty width
    a.h, a.a = 0x1000, 0x2000
    assert h.m3s_swiglu_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"width" in h.m3s_last_error()
    a.width = 12
    a.a = 0x2001                                                # not bf16-aligned
    assert h.m3s_swiglu_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"aligned" in h.m3s_last_error()
    a.a = 0x2000                                                # backward needs da and dh
    assert h.m3s_swiglu_bwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"NULL" in h.m3s_last_error()
    a.rows = 0                                                  # nothing to do: no launch,
    assert h.m3s_swiglu_bwd(ctypes.byref(a), None) == lib.OK    # NULL tensors allowed


def test_rms_arguments_are_checked_without_a_launch(lib):
    h = lib.load()
    assert h.m3s_rms_bwd_workspace_bytes(768) == 1024 * 768 * 4
    assert h.m3s_rms_bwd_workspace_bytes(0) == -1
    a = lib.RmsArgs()
    a.struct_size = ctypes.sizeof(lib.RmsArgs)
    a.x_dtype, a.y_dtype, a.width, a.rows, a.eps = lib.DTYPE_F32, lib.DTYPE_BF16, 770, 8, 1e-5
    a.x, a.weight, a.y = 0x1000, 0x2000, 0x3000
    assert h.m3s_rms_fwd(ctypes.byref(a), None) == lib.ERR_INVALID       # width % 4
    assert b"width" in h.m3s_last_error()
    a.width = 8192
    assert h.m3s_rms_fwd(ctypes.byref(a), None) == lib.ERR_INVALID       # too wide
    a.width = 768
    assert h.m3s_rms_bwd(ctypes.byref(a), None) == lib.ERR_INVALID       # no rstd / dy / dx
    assert b"NULL" in h.m3s_last_error()
    a.x = 0x1004                                                          # f32 rows need 16 B
    assert h.m3s_rms_fwd(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"aligned" in h.m3s_last_error()
    a.rows = 0
    assert h.m3s_rms_fwd(ctypes.byref(a), None) == lib.OK


def test_wgrad_arguments_are_checked_without_a_launch(lib):
    h = lib.load()
    assert h.m3s_wgrad(None, None) == lib.ERR_INVALID
    w = lib.WgradArgs()
    w.struct_size = 8
    assert h.m3s_wgrad(ctypes.byref(w), None) == lib.ERR_INVALID
    assert b"struct_size" in h.m3s_last_error()
    w.struct_size = ctypes.sizeof(lib.WgradArgs)
    w.tokens, w.rows, w.cols = 100, 64, 64
    assert h.m3s_wgrad(ctypes.byref(w), None) == lib.ERR_INVALID   # tokens % 32
    assert b"multiple of 32" in h.m3s_last_error()
    w.tokens = 4096
    assert h.m3s_wgrad(ctypes.byref(w), None) == lib.ERR_INVALID   # NULL operands
    w.a, w.b, w.c = 0x1000, 0x2008, 0x3000
    w.lda, w.ldb, w.ldc = 64, 64, 64
    assert h.m3s_wgrad(ctypes.byref(w), None) == lib.ERR_INVALID   # b not 16-byte aligned
    assert b"aligned" in h.m3s_last_error()
    w.b = 0x2000
    w.ldb = 60
    assert h.m3s_wgrad(ctypes.byref(w), None) == lib.ERR_INVALID   # ldb too short
    w.ldb = 64
    # 4096 tokens over one 64 x 64 tile: split over the tokens, so a workspace is needed
    assert h.m3s_wgrad_workspace_bytes(4096, 64, 64) > 0
    assert h.m3s_wgrad(ctypes.byref(w), None) == lib.ERR_INVALID
    assert b"workspace" in h.m3s_last_error()
    assert h.m3s_wgrad_workspace_bytes(4096, 64, 0) == -1
    assert h.m3s_wgrad_workspace_bytes(100, 64, 64) == -1
    # one step of 32 tokens cannot be split
    assert h.m3s_wgrad_workspace_bytes(32, 64, 64) == 0


def test_gemv_arguments_are_checked_without_a_launch(lib):
    h = lib.load()
    assert h.m3s_gemv(None, None) == lib.ERR_INVALID
    a = lib.GemvArgs()
    a.struct_size = 4
    assert h.m3s_gemv(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"struct_size" in h.m3s_last_error()
    a.struct_size = ctypes.sizeof(lib.GemvArgs)
    a.rows, a.k, a.n = 0, 64, 64
    assert h.m3s_gemv(ctypes.byref(a), None) == lib.ERR_INVALID   # rows < 1
    a.rows = 1
    a.n = 60
    assert h.m3s_gemv(ctypes.byref(a), None) == lib.ERR_INVALID   # n % 8
    a.n = 64
    assert h.m3s_gemv(ctypes.byref(a), None) == lib.ERR_INVALID   # NULL operands
    a.x, a.w, a.y = 0x1000, 0x2008, 0x3000
    a.ldx, a.ldw, a.ldy = 64, 64, 64
    assert h.m3s_gemv(ctypes.byref(a), None) == lib.ERR_INVALID   # w misaligned
    assert b"aligned" in h.m3s_last_error()
    a.w = 0x2000
    a.k, a.ldx = 5000, 5000
    assert h.m3s_gemv(ctypes.byref(a), None) == lib.ERR_INVALID   # k > 4096
    a.rows, a.k, a.ldx = 64, 96, 96
    assert h.m3s_gemv(ctypes.byref(a), None) == lib.ERR_INVALID   # the tiles: k % 64
    assert b"multiple of 64" in h.m3s_last_error()
    a.k, a.ldx, a.x = 128, 132, 0x1000
    assert h.m3s_gemv(ctypes.byref(a), None) == lib.ERR_INVALID   # the tiles: x row stride


def test_adamw_arguments_are_checked_without_a_launch(lib):
    h = lib.load()
    assert h.m3s_adamw(None, None) == lib.ERR_INVALID
    a = lib.AdamwArgs()
    a.struct_size = 12
    assert h.m3s_adamw(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"struct_size" in h.m3s_last_error()
    a.struct_size = ctypes.sizeof(lib.AdamwArgs)
    a.count = -1
    assert h.m3s_adamw(ctypes.byref(a), None) == lib.ERR_INVALID
    a.count = 0
    assert h.m3s_adamw(ctypes.byref(a), None) == lib.OK   # nothing to update
    a.count = 2
    assert h.m3s_adamw(ctypes.byref(a), None) == lib.ERR_INVALID   # NULL arrays
    assert b"NULL" in h.m3s_last_error()
    ptrs = (ctypes.c_void_p * 2)(0x1000, 0x2000)
    numel = (ctypes.c_int64 * 2)(4, -1)
    for f in ("params", "grads", "exp_avg", "exp_avg_sq"):
        setattr(a, f, ctypes.cast(ptrs, ctypes.c_void_p))
    a.numel = ctypes.cast(numel, ctypes.c_void_p)
    a.bias_correction2_sqrt = 0.0
    assert h.m3s_adamw(ctypes.byref(a), None) == lib.ERR_INVALID   # update count 0
    assert b"bias" in h.m3s_last_error()
    a.bias_correction2_sqrt = 0.1
    assert h.m3s_adamw(ctypes.byref(a), None) == lib.ERR_INVALID   # negative numel
    assert b"numel" in h.m3s_last_error()
