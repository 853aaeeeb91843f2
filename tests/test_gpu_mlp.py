"""GPU parity of the gated-MLP gate kernels (`m3s_swiglu_fwd` / `m3s_swiglu_bwd`) against
the composed framework ops they replace, `value * silu(gate)` and its autograd, on the
same device and dtype, and against float64 maths.

Tolerances:
  * against the composed ops (same rounding points): bf16 within one bf16 ulp
    (2^-8 relative) and at least 99% of elements bit-identical; f32 within 1e-6
    relative.
  * against float64 maths: bf16 4e-3 and f32 1e-6, max-normalised.
"""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def composed(h, width):
    value, gate = h.split(width, dim=-1)
    return value * F.silu(gate)


def inputs(rows, width, dtype, dev, seed):
    g = torch.Generator().manual_seed(seed)
    h = (2.5 * torch.randn(rows, 2 * width, generator=g)).to(dtype).to(dev)
    da = torch.randn(rows, width, generator=g).to(dtype).to(dev)
    return h, da


def close_to_composed(got, want, dtype):
    got, want = got.float(), want.float()
    rel = ((got - want).abs() / want.abs().clamp_min(1e-30)).max().item()
    if dtype == torch.bfloat16:
        assert rel <= 2.0 ** -8, rel
        assert (got == want).float().mean().item() >= 0.99
    else:
        assert rel <= 1e-6 or (got - want).abs().max().item() <= 1e-6 * want.abs().max().item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,width", [(4096, 1536), (333, 96), (64, 12), (7, 5)])
def test_gate_matches_composed_ops(m3, dev, dtype, rows, width):
    K = m3.kernels
    h, da = inputs(rows, width, dtype, dev, rows + width)
    close_to_composed(K.swiglu_forward(h, width), composed(h, width), dtype)
    hr = h.clone().requires_grad_(True)
    composed(hr, width).backward(da)
    close_to_composed(K.swiglu_backward(h, da, width), hr.grad, dtype)


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 4e-3), (torch.float32, 1e-6)])
def test_gate_matches_float64_maths(m3, dev, dtype, tol):
    K = m3.kernels
    h, da = inputs(512, 256, dtype, dev, 7)
    h64 = h.double().cpu().requires_grad_(True)
    want = composed(h64, 256)
    want.backward(da.double().cpu())
    got = K.swiglu_forward(h, 256).double().cpu()
    assert ((got - want).abs().max() / want.abs().max()).item() <= tol
    dh = K.swiglu_backward(h, da, 256).double().cpu()
    assert ((dh - h64.grad).abs().max() / h64.grad.abs().max()).item() <= tol


def test_gate_in_the_mlp_node_and_empty_rows(m3, dev):
    """`model.gated_mlp` through the kernel node equals the composed form, gradients
    included; zero rows is a no-op."""
    K = m3.kernels
    M = m3.model
    g = torch.Generator().manual_seed(3)
    fc1 = (torch.randn(64, 2 * 40, generator=g) / 8).to(dev).requires_grad_(True)
    fc2 = (torch.randn(40, 64, generator=g) / 6).to(dev).requires_grad_(True)
    x = torch.randn(3, 50, 64, generator=g).to(dev).requires_grad_(True)
    p = M.MLPParams(fc1=fc1, fc2=fc2)
    out = M.gated_mlp(p, x, torch.float32)
    ref = composed(x @ fc1, 40) @ fc2
    assert ((out - ref).abs().max() / ref.abs().max()).item() <= 1e-6
    dy = torch.randn(out.shape, generator=g).to(dev)
    got = torch.autograd.grad(out, (x, fc1, fc2), dy)
    want = torch.autograd.grad(ref, (x, fc1, fc2), dy)
    for a, b in zip(got, want):
        assert ((a - b).abs().max() / b.abs().max()).item() <= 1e-5
    h = torch.empty(0, 16, device=dev, dtype=torch.bfloat16)
    assert K.swiglu_forward(h, 8).shape == (0, 8)
    assert K.swiglu_backward(h, torch.empty(0, 8, device=dev, dtype=torch.bfloat16), 8).shape == (0, 16)
