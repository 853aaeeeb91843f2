"""m3s_norm_bwd_noalloc: the BCNorm backward with the library's own scratch array, called
through the C ABI, against m3s_norm_bwd with a caller workspace.

Both entry points run the same two kernels in the same order, so the outputs must be
bit-identical. Two calls in a row, the second on a smaller input (fewer rows, a narrower
width, one norm instead of two), check that nothing left in the shared scratch by the
first call reaches the second.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(m3, dev, b, l, n, count, dtype, seed):
    """Inputs in the layout the layer hands over: B and C as (B, L, N) slices of one
    wider buffer, rstd from the forward kernel, f32 cotangents."""
    g = torch.Generator().manual_seed(seed)
    vec = 16 // torch.empty((), dtype=dtype).element_size()
    width = 2 * n + 3 * vec
    buf = (torch.randn(b, l, width, generator=g) * 1.5).to(dtype).to(dev)
    offs = (vec, vec + n)[:count]
    xs = [buf[..., o:o + n] for o in offs]
    ws = [(torch.rand(n, generator=g) + 0.5).to(dev) for _ in range(count)]
    _, rstds = m3.kernels.bcnorm_forward(xs, ws, 1e-5)
    dys = [torch.randn(b, l, n, generator=g).to(dev) for _ in range(count)]
    return buf, offs, xs, ws, rstds, dys


def _run(m3, lib, entry, case, n, dtype):
    buf, offs, xs, ws, rstds, dys = case
    dxbuf = torch.full_like(buf, float("nan"))
    dxs = [dxbuf[..., o:o + n] for o in offs]
    dws = [torch.full((n,), float("nan"), device=buf.device) for _ in xs]
    a = lib.NormBwdArgs()
    a.struct_size = ctypes.sizeof(lib.NormBwdArgs)
    a.batch, a.seqlen, a.width = buf.shape[0], buf.shape[1], n
    a.dtype, a.count = lib.dtype_code(dtype), len(xs)
    for i, x in enumerate(xs):
        a.x[i], a.dx[i] = lib.blx(x), lib.blx(dxs[i])
        a.weight[i], a.rstd[i] = ws[i].data_ptr(), rstds[i].data_ptr()
        a.dy[i], a.dweight[i] = dys[i].data_ptr(), dws[i].data_ptr()
    work = None
    if entry == "m3s_norm_bwd":
        work = torch.empty(lib.load().m3s_norm_bwd_workspace_bytes(n), device=buf.device,
                           dtype=torch.uint8)
        a.workspace = work.data_ptr()
    rc = getattr(lib.load(), entry)(ctypes.byref(a), lib.stream_handle(buf.device))
    lib.check(rc, entry)
    torch.cuda.synchronize()
    return dxbuf, dws


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_norm_backward_equals_workspace_entry_point(m3, dev, dtype):
    from mamba3_siso_tpu_amd import _lib as lib

    big = (4, 4096, 128, 2)      # enough rows for every one of the 1024 partial blocks
    small = (1, 37, 64, 1) if dtype == torch.bfloat16 else (2, 53, 32, 1)
    for k, (b, l, n, count) in enumerate((big, small)):
        print(f"[no-alloc] call {k}: dtype={dtype} B={b} L={l} width={n} count={count}",
              flush=True)
        case = _case(m3, dev, b, l, n, count, dtype, seed=31 + k)
        want_dx, want_dw = _run(m3, lib, "m3s_norm_bwd", case, n, dtype)
        got_dx, got_dw = _run(m3, lib, "m3s_norm_bwd_noalloc", case, n, dtype)
        assert torch.equal(torch.isnan(got_dx), torch.isnan(want_dx))
        assert not bool(torch.isnan(want_dw[0]).any())
        assert torch.equal(got_dx.nan_to_num(0.0), want_dx.nan_to_num(0.0)), f"dx, call {k}"
        for i in range(count):
            assert torch.equal(got_dw[i], want_dw[i]), f"dweight[{i}], call {k}"


def test_noalloc_rejects_a_width_past_its_scratch(m3, dev):
    """Widths the entry points do not accept at all are refused before any launch."""
    from mamba3_siso_tpu_amd import _lib as lib

    a = lib.NormBwdArgs()
    a.struct_size = ctypes.sizeof(lib.NormBwdArgs)
    a.batch, a.seqlen, a.width, a.count = 1, 8, 1024, 1
    a.dtype = lib.DTYPE_BF16
    assert lib.load().m3s_norm_bwd_noalloc(ctypes.byref(a), None) == lib.ERR_INVALID
    assert b"at most 512" in lib.load().m3s_last_error()
