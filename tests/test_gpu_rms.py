"""GPU parity of the LM block-norm kernels (`m3s_rms_fwd` / `m3s_rms_bwd`) against
``F.rms_norm`` (the composed form they replace) and float64 maths.

Tolerances:
  * against ``F.rms_norm`` and its autograd on the same device: outputs 2^-8 relative
    for a bf16 output (one bf16 ulp), 1e-5 for f32; dx 1e-5 and dweight 1e-4
    max-normalised for f32 rows (dweight sums 4096 rows in another order).
  * against float64 maths: f32 1e-5, bf16 output 4e-3, max-normalised.
"""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def maxrel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).abs().max() / b.abs().max()).item()


@pytest.mark.parametrize("rows,d", [(4096, 768), (333, 1024), (5, 12), (100, 1536), (64, 4096)])
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.bfloat16), (torch.float32, torch.float32),
                                     (torch.bfloat16, torch.bfloat16)])
def test_norm_matches_torch_and_float64(m3, dev, rows, d, xdt, ydt):
    K = m3.kernels
    g = torch.Generator().manual_seed(rows + d)
    x = (3 * torch.randn(rows, d, generator=g)).to(xdt).to(dev)
    w = (1 + 0.3 * torch.randn(d, generator=g)).to(dev)
    dy = torch.randn(rows, d, generator=g).to(ydt).to(dev)
    y, rstd = K.rms_forward(x, w, 1e-5, ydt)
    xr = x.detach().clone().requires_grad_(True)
    wr = w.detach().clone().requires_grad_(True)
    ref = F.rms_norm(xr.float(), (d,), wr, 1e-5).to(ydt)
    tol = 2.0 ** -8 if ydt == torch.bfloat16 else 1e-5
    assert maxrel(y, ref) <= tol
    ref.backward(dy)
    dx, dw = K.rms_backward(x, w, rstd, dy)
    assert dx.dtype == xdt and dw.dtype == torch.float32
    assert maxrel(dx, xr.grad) <= (1e-5 if xdt == torch.float32 else 2.0 ** -7)
    assert maxrel(dw, wr.grad) <= 1e-4
    # float64 maths
    x64 = x.double().cpu().requires_grad_(True)
    w64 = w.double().cpu().requires_grad_(True)
    y64 = x64 * torch.rsqrt(x64.square().mean(-1, keepdim=True) + 1e-5) * w64
    assert maxrel(y.cpu(), y64) <= (4e-3 if ydt == torch.bfloat16 else 1e-5)
    y64.backward(dy.double().cpu())
    assert maxrel(dx.cpu(), x64.grad) <= (1e-5 if xdt == torch.float32 else 8e-3)
    assert maxrel(dw.cpu(), w64.grad) <= 1e-4


def test_norm_node_in_the_model_and_empty_rows(m3, dev):
    K = m3.kernels
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 70, 256, generator=g).to(dev).requires_grad_(True)
    w = (1 + 0.1 * torch.randn(256, generator=g)).to(dev).requires_grad_(True)
    y = m3.model._norm(x, w, 1e-5, torch.bfloat16)
    ref = F.rms_norm(x.float(), (256,), w, 1e-5).to(torch.bfloat16)
    assert maxrel(y, ref) <= 2.0 ** -8
    dy = torch.randn(y.shape, generator=g).to(dev).to(torch.bfloat16)
    got = torch.autograd.grad(y, (x, w), dy)
    want = torch.autograd.grad(ref, (x, w), dy)
    assert maxrel(got[0], want[0]) <= 1e-5 and maxrel(got[1], want[1]) <= 1e-4
    e = torch.empty(0, 64, device=dev)
    y0, r0 = K.rms_forward(e, torch.ones(64, device=dev), 1e-5, torch.bfloat16)
    assert y0.shape == (0, 64) and r0.shape == (0,)


@pytest.mark.parametrize("rows,d", [(4096, 768), (333, 1024), (5, 12), (64, 4096)])
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.bfloat16), (torch.float32, torch.float32),
                                     (torch.bfloat16, torch.bfloat16)])
def test_residual_form_equals_add_then_norm(m3, dev, rows, d, xdt, ydt):
    """`m3s_rms_fwd` / `m3s_rms_bwd` with a residual: the sum and the normalised rows are
    bit-identical to the add followed by the plain kernel (the same roundings), and the
    cotangents of x, of the added block output and of the gain match autograd of
    ``x + y`` into the plain norm node with the sum's outside cotangent (dx, dy
    within one rounding of the add: 1e-6 max-normalised in f32, 2^-7 in bf16)."""
    K = m3.kernels
    g = torch.Generator().manual_seed(3 * rows + d)
    x = (2 * torch.randn(rows, d, generator=g)).to(xdt).to(dev)
    y = torch.randn(rows, d, generator=g).to(ydt).to(dev)
    w = (1 + 0.3 * torch.randn(d, generator=g)).to(dev)
    n, rstd, s = K.rms_forward(x, w, 1e-5, ydt, add=y)
    s_ref = x + y
    assert s.dtype == xdt and torch.equal(s, s_ref)
    n_ref, rstd_ref = K.rms_forward(s_ref, w, 1e-5, ydt)
    assert torch.equal(n, n_ref) and torch.equal(rstd, rstd_ref)
    dn = torch.randn(rows, d, generator=g).to(ydt).to(dev)
    ds = torch.randn(rows, d, generator=g).to(xdt).to(dev)
    for dsum in (ds, None):
        dx, dw, dadd = K.rms_backward(s, w, rstd, dn, dsum=dsum, add_dtype=ydt)
        xr = x.detach().clone().requires_grad_(True)
        yr = y.detach().clone().requires_grad_(True)
        wr = w.detach().clone().requires_grad_(True)
        sr = xr + yr
        nr = m3.model._NormFn.apply(sr, wr, 1e-5, ydt)
        outs, grads = [nr], [dn]
        if dsum is not None:
            outs.append(sr)
            grads.append(dsum)
        gx, gy, gw = torch.autograd.grad(outs, (xr, yr, wr), grads)
        tol = 1e-6 if xdt == torch.float32 else 2.0 ** -7
        assert dx.dtype == xdt and dadd.dtype == ydt
        assert maxrel(dx, gx) <= tol
        assert maxrel(dadd, gy) <= (tol if ydt == torch.float32 else 2.0 ** -7)
        assert torch.equal(dw, gw)


def test_add_norm_in_the_model_matches_the_composed_ops(m3, dev):
    """`model._add_norm` (one node) against ``x + y`` into `model._norm`: same outputs
    bit for bit, gradients of x, y and the gain within float rounding."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 96, 512, generator=g).to(dev).requires_grad_(True)
    y = torch.randn(2, 96, 512, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    w = (1 + 0.1 * torch.randn(512, generator=g)).to(dev).requires_grad_(True)
    s, h = m3.model._add_norm(x, y, w, 1e-5, torch.bfloat16)
    s2 = x + y
    h2 = m3.model._norm(s2, w, 1e-5, torch.bfloat16)
    assert torch.equal(s, s2) and torch.equal(h, h2)
    ds = torch.randn(s.shape, generator=g).to(dev)
    dh = torch.randn(h.shape, generator=g).to(torch.bfloat16).to(dev)
    got = torch.autograd.grad((s, h), (x, y, w), (ds, dh))
    want = torch.autograd.grad((s2, h2), (x, y, w), (ds, dh))
    assert maxrel(got[0], want[0]) <= 1e-6
    assert got[1].dtype == torch.bfloat16 and maxrel(got[1], want[1]) <= 2.0 ** -7
    assert maxrel(got[2], want[2]) <= 1e-6
