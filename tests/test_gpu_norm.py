"""GPU parity of the BCNorm kernels (m3s_norm_fwd / m3s_norm_bwd) against the oracle's
``rms_norm`` (``layer.py:190-198``) and its float64 autograd, of the weight-layout kernel
(m3s_transpose, exact against torch's transpose + cast), and of the fused layer path
(`_LayerFn`) against the composed one.

Tolerances: the forward output is stored in the input dtype, so it must sit within one
rounding of the float64 value (2^-8 relative for bf16, 2e-6 for f32); rstd to 2e-6
relative. The backward is checked against float64 autograd of the oracle applied to the
same cotangent rounded to the input dtype (the primal-dtype cast the kernel reproduces):
max-normalised error <= 1e-2 for bf16 gradients (one bf16 rounding of dx plus f32
accumulation), p95 <= 2e-5 for f32; the gain gradient (an f32 sum over B*L rows) to
1e-4 max-normalised.
"""

import pytest
import torch

from helpers import BF16, F32, F64, assert_maxrel, cpu
from oracle import siso_oracle as O

pytestmark = pytest.mark.gpu


def strided_pair(b, l, n, dtype, seed, extra=24):
    """B and C as (B, L, N) slices of one wider buffer, like the projection's slices."""
    g = torch.Generator().manual_seed(seed)
    vec = 16 // torch.empty((), dtype=dtype).element_size()
    width = 2 * n + extra * vec
    buf = (torch.randn(b, l, width, generator=g) * 1.7).to(dtype)
    off = 2 * vec
    return buf, (off, off + n)


@pytest.mark.parametrize("dtype,n,count", [
    (BF16, 128, 2), (BF16, 64, 2), (BF16, 96, 1),   # 96: 12 active lanes of a 16-lane group
    (F32, 16, 2), (F32, 128, 1),
])
def test_norm_forward_and_backward_match_oracle(m3, dev, dtype, n, count):
    b, l, eps = 3, 77, 1e-5
    buf, offs = strided_pair(b, l, n, dtype, seed=n + count)
    g = torch.Generator().manual_seed(9)
    weights = [torch.rand(n, generator=g) + 0.5 for _ in range(count)]
    dbuf = buf.cuda()
    xs = [dbuf[..., o:o + n] for o in offs[:count]]
    ys, rstds = m3.kernels.bcnorm_forward(xs, [w.cuda() for w in weights], eps)
    one_ulp = 2.0 ** -8 if dtype == BF16 else 2e-6
    cots = [torch.randn(b, l, n, generator=g) for _ in range(count)]
    dxbuf = torch.full_like(dbuf, float("nan"))
    dxs = [dxbuf[..., o:o + n] for o in offs[:count]]
    dws = m3.kernels.bcnorm_backward(xs, [w.cuda() for w in weights], rstds,
                                     [c.cuda() for c in cots], dxs)
    for i in range(count):
        xo = buf[..., offs[i]:offs[i] + n].double().requires_grad_(True)
        wo = weights[i].double().requires_grad_(True)
        yo = O.rms_norm(xo, wo, eps)
        rstd_o = torch.rsqrt((xo.detach() ** 2).mean(-1) + eps)
        assert ys[i].dtype == dtype and ys[i].is_contiguous()
        err = ((cpu(ys[i]) - yo.detach()).abs() / yo.detach().abs().clamp_min(1e-3)).max()
        assert float(err) <= one_ulp * 1.01, (i, float(err))
        torch.testing.assert_close(cpu(rstds[i]), rstd_o, rtol=2e-6, atol=0)
        cot = cots[i].to(dtype).double()          # the primal-dtype cast
        yo.backward(cot)
        if dtype == BF16:
            assert_maxrel(dxs[i], xo.grad, 1e-2, f"dx[{i}]")
        else:
            assert O.rel_error(cpu(dxs[i]), xo.grad) <= 2e-5
        assert O.max_rel(cpu(dws[i]), wo.grad) <= 1e-4, (i, O.max_rel(cpu(dws[i]), wo.grad))
    # the kernels touched exactly the slices they were given
    mask = torch.zeros(dbuf.shape[-1], dtype=torch.bool)
    for o in offs[:count]:
        mask[o:o + n] = True
    assert torch.isnan(cpu(dxbuf)[..., ~mask]).all()
    assert not torch.isnan(cpu(dxbuf)[..., mask]).any()


def test_norm_rejects_misaligned_rows(m3, dev):
    x = torch.randn(2, 8, 136, device=dev).to(BF16)[..., 3:131]   # 6-byte offset
    with pytest.raises(ValueError, match="aligned"):
        m3.kernels.bcnorm_forward([x], [torch.ones(128, device=dev)], 1e-5)


def run_layer(m3, cfg, p_cpu, u, gy, fused, monkeypatch, with_state_loss=True):
    params = m3.SISOParams(*(t.cuda().requires_grad_(True) for t in p_cpu))
    ud = u.cuda().requires_grad_(True)
    with monkeypatch.context() as mp:
        if not fused:
            mp.setattr(m3.layer, "_fused_ok", lambda *a, **k: False)
        else:
            assert m3.layer._fused_ok(ud, cfg, None)
        y, st = m3.mamba3_siso_layer(params, ud, cfg)
        loss = (y.float() * gy.cuda().float()).sum()
        if with_state_loss:   # cotangents on every carried output: dfs, dfk, dfv, dphi_final
            loss = loss + 0.3 * st.ssm.sum() + 0.7 * st.k.square().sum() \
                + 0.5 * st.v.sum() + st.phi.sin().sum()
        loss.backward()
    grads = {f: getattr(params, f).grad for f in p_cpu._fields}
    grads["u"] = ud.grad
    return y, st, grads


@pytest.mark.parametrize("policy", ["bf16", "f32"])
def test_fused_layer_matches_composed_path(m3, dev, monkeypatch, policy):
    """The fused node (padded GEMMs, HIP BCNorm, in-place gradient slices) against the
    composed autograd path, outputs and every gradient, final-state cotangents included."""
    if policy == "bf16":
        cfg = m3.SISOConfig(d_model=256, d_state=128, headdim=64, expand=2, chunk=128)
        dt = BF16
    else:
        cfg = m3.SISOConfig(d_model=64, d_state=16, headdim=16, expand=1, chunk=64,
                            policy_name="f32")
        dt = F32
    p_cpu = m3.init_params(cfg, 11)
    g = torch.Generator().manual_seed(12)
    p_cpu = p_cpu._replace(b_norm_weight=torch.rand(cfg.d_state, generator=g) + 0.5,
                           c_norm_weight=torch.rand(cfg.d_state, generator=g) + 0.5)
    u = torch.randn(2, 384, cfg.d_model, generator=g).to(dt)
    gy = torch.randn(2, 384, cfg.d_model, generator=g).to(dt)
    y1, s1, g1 = run_layer(m3, cfg, p_cpu, u, gy, True, monkeypatch)
    y0, s0, g0 = run_layer(m3, cfg, p_cpu, u, gy, False, monkeypatch)
    tol = 2e-2 if policy == "bf16" else 2e-5
    assert_maxrel(y1, cpu(y0), tol, "y")
    for name in ("ssm", "k", "v"):
        assert_maxrel(getattr(s1, name), cpu(getattr(s0, name)), tol, name)
    assert O.rel_error(cpu(s1.phi), cpu(s0.phi), angle=True) <= 1e-5
    gtol = 3e-2 if policy == "bf16" else 2e-4
    for name, gv in g1.items():
        assert gv is not None, name
        assert gv.dtype == g0[name].dtype, name
        assert_maxrel(gv, cpu(g0[name]), gtol, f"d{name}")


def test_fused_layer_without_grad_saves_nothing(m3, dev):
    cfg = m3.SISOConfig(d_model=256, d_state=128, headdim=64, expand=2, chunk=128)
    params = m3.SISOParams(*(t.cuda() for t in m3.init_params(cfg, 2)))
    u = torch.randn(1, 256, 256, device=dev).to(BF16)
    with torch.no_grad():
        y, st = m3.mamba3_siso_layer(params, u, cfg)
    assert y.shape == (1, 256, 256) and y.dtype == BF16 and not y.requires_grad
    assert st.ssm.shape == (1, cfg.nheads, 64, 128)


@pytest.mark.parametrize("src,dst,rows,cols,out_rows,stride_pad", [
    (BF16, BF16, 1024, 4480, 4608, 0),     # the configs[1] in_proj layout (8-element runs)
    (BF16, BF16, 2048, 1024, 1024, 0),     # out_proj
    (F32, BF16, 1536, 768, 768, 0),        # an LM out_proj from float32 parameters
    (F32, BF16, 200, 136, 256, 8),         # 8-element runs over ragged tiles, strided input
    (F32, BF16, 200, 133, 256, 5),         # element-wise: ragged tiles, strided input
    (F32, F32, 64, 64, 64, 0),
    (BF16, F32, 70, 1, 8, 3),
])
def test_transpose_pad_matches_torch_exactly(m3, dev, src, dst, rows, cols, out_rows, stride_pad):
    g = torch.Generator().manual_seed(rows + cols)
    base = torch.randn(rows, cols + stride_pad, generator=g).to(src).to(dev)
    w = base[:, :cols]
    got = m3.kernels.transpose_pad(w, dst, out_rows)
    want = torch.zeros(out_rows, rows, dtype=dst, device=dev)
    want[:cols] = w.t().to(dst)
    assert got.shape == (out_rows, rows) and got.dtype == dst and got.is_contiguous()
    assert torch.equal(got, want)
