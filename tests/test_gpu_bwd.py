"""Reverse-scan backward (m3s_bwd + the epilogue) vs autograd of the float64 oracle --
the way the reference checks its VJP against ``jax.grad`` (``tests.py:573-612``)."""

import math

import pytest
import torch

from helpers import (assert_f32, BF16, BF16_GRAD_MAXREL, BF16_MAXREL, GRAD_F32_P95, STATE_MAXABS,
                     assert_maxabs, assert_maxrel, assert_p95, boundary_inputs, fwd_args,
                     phi_strips_of, report)
from oracle import siso_oracle as O

pytestmark = pytest.mark.gpu

NAMES = ("q", "k", "v", "adt", "gamma", "scale", "phi", "q_bias", "k_bias", "d_skip", "z",
         "seed_ssm", "seed_k", "seed_v", "seed_coef")
GRAD_FIELD = dict(q="dq", k="dk", v="dv", adt="dadt", gamma="dgamma", scale="dscale",
                  phi="dphi", q_bias="dq_bias", k_bias="dk_bias", d_skip="dd_skip", z="dz",
                  seed_ssm="dseed_ssm", seed_k="dseed_k", seed_v="dseed_v",
                  seed_coef="dseed_coef")


def run_case(m3, b, h, L, n, p, nr, chunk, policy, seeds, dfin, seed=0):
    c, d = boundary_inputs(b, h, L, n, p, nr, policy, seed=seed, seeds=seeds)
    g = torch.Generator().manual_seed(seed + 77)
    dfs = dfk = dfv = None
    if dfin:
        dfs = torch.randn(b, h, p, n, generator=g, dtype=torch.float64).float().double()
        dfk = torch.randn(b, h, n, generator=g, dtype=torch.float64).float().double()
        dfv = torch.randn(b, h, p, generator=g, dtype=torch.float64).float().double()
    want = O.boundary_grads({k_: c[k_] for k_ in NAMES if k_ in c}, c["dy"], dfs, dfk, dfv,
                            chunk=chunk)
    out = m3.siso_forward(*fwd_args(d), chunk=chunk, dtype_policy=policy, save_residuals=True)
    res = out[4]
    dev = lambda t: None if t is None else t.float().cuda()  # noqa: E731
    gr = m3.siso_backward(d["dy"], d["q"], d["k"], d["v"], d["adt"], d["gamma"], d["scale"],
                          d["phi"], d["q_bias"], d["k_bias"], res.ybar, res.chunk_states,
                          d["d_skip"], d["z"], d.get("seed_ssm"), d.get("seed_k"),
                          d.get("seed_v"), d.get("seed_coef"), dev(dfs), dev(dfk), dev(dfv),
                          chunk=chunk, dtype_policy=policy)
    return want, gr


@pytest.mark.parametrize("b,h,L,n,p,nr,chunk,seeds,dfin", [
    (1, 4, 512, 16, 16, 4, 64, False, False),    # cfg1 kernel shapes
    (1, 2, 64, 32, 16, 8, 32, True, True),
    (2, 3, 128, 32, 16, 8, 64, False, False),
    (1, 2, 128, 128, 64, 32, 32, True, True),
    (2, 2, 128, 64, 64, 16, 64, True, False),
])
def test_backward_f32_matches_autograd_of_oracle(m3, b, h, L, n, p, nr, chunk, seeds, dfin):
    want, gr = run_case(m3, b, h, L, n, p, nr, chunk, "f32", seeds, dfin)
    for name, w in want.items():
        assert_f32(getattr(gr, GRAD_FIELD[name]), w, "grad", f"d{name}")


@pytest.mark.parametrize("chunk,seeds,dfin", [(128, True, True), (64, False, False), (32, True, False)])
def test_backward_bf16_matches_autograd_of_oracle(m3, chunk, seeds, dfin):
    want, gr = run_case(m3, 2, 2, 256, 128, 64, 32, chunk, "bf16", seeds, dfin)
    assert gr.dv.dtype == BF16 and gr.dz.dtype == BF16
    for name, w in want.items():
        assert_maxrel(getattr(gr, GRAD_FIELD[name]), w, BF16_MAXREL, f"d{name}")


@pytest.mark.parametrize("n,chunk", [(64, 64), (128, 128)])
def test_backward_bf16_state64_and_no_gate(m3, n, chunk):
    """The bf16 backward at state_dim 64, and without the gate z and skip D."""
    want, gr = run_case(m3, 2, 2, 256, n, 64, n // 4, chunk, "bf16", True, True)
    for name, w in want.items():
        assert_maxrel(getattr(gr, GRAD_FIELD[name]), w, BF16_MAXREL, f"d{name}")
    c, d = boundary_inputs(1, 3, 256, 128, 64, 32, "bf16", seed=5)
    for t in (c, d):
        t.pop("d_skip"), t.pop("z")
    want = O.boundary_grads({k_: c[k_] for k_ in NAMES if k_ in c}, c["dy"], None, None, None,
                            chunk=chunk)
    out = m3.siso_forward(*fwd_args(d), chunk=chunk, dtype_policy="bf16", save_residuals=True)
    gr = m3.siso_backward(d["dy"], d["q"], d["k"], d["v"], d["adt"], d["gamma"], d["scale"],
                          d["phi"], d["q_bias"], d["k_bias"], out[4].ybar, out[4].chunk_states,
                          chunk=chunk, dtype_policy="bf16")
    assert gr.dz is None and gr.dd_skip is None
    for name, w in want.items():
        assert_maxrel(getattr(gr, GRAD_FIELD[name]), w, BF16_MAXREL, f"d{name} (no gate)")


@pytest.mark.parametrize("policy,n,p,chunk", [
    ("bf16", 64, 64, 128), ("bf16", 64, 64, 32), ("bf16", 32, 16, 128), ("bf16", 16, 16, 128),
    ("f32", 64, 64, 32), ("f32", 32, 16, 128), ("f32", 16, 16, 128),
])
def test_backward_every_table_shape(m3, policy, n, p, chunk):
    """Instantiations of the kernel table not covered above, against autograd of the
    float64 oracle."""
    want, gr = run_case(m3, 2, 2, 256, n, p, n // 4, chunk, policy, True, True, seed=19)
    for name, w in want.items():
        got = getattr(gr, GRAD_FIELD[name])
        if policy == "f32":
            assert_f32(got, w, "grad", f"d{name}")
        else:
            assert_maxrel(got, w, BF16_GRAD_MAXREL, f"d{name}")


@pytest.mark.parametrize("policy,n,p,chunk", [
    ("bf16", 128, 64, 128), ("bf16", 64, 64, 64), ("bf16", 32, 16, 32),
    ("f32", 128, 64, 32), ("f32", 16, 16, 64),
])
def test_backward_with_phi_built_in_the_kernel(m3, policy, n, p, chunk):
    """phi_strips mode of the backward: every gradient (dphi included, which the caller
    turns into theta and angle gradients) against autograd of the float64 oracle, with
    the seeds and final-state cotangents on."""
    c, d = boundary_inputs(2, 2, 256, n, p, n // 4, policy, seed=29, seeds=True)
    g = torch.Generator().manual_seed(101)
    dfs = torch.randn(2, 2, p, n, generator=g, dtype=torch.float64).float().double()
    dfk = torch.randn(2, 2, n, generator=g, dtype=torch.float64).float().double()
    dfv = torch.randn(2, 2, p, generator=g, dtype=torch.float64).float().double()
    want = O.boundary_grads({k_: c[k_] for k_ in NAMES if k_ in c}, c["dy"], dfs, dfk, dfv,
                            chunk=chunk)
    args = fwd_args(d)
    args[6] = phi_strips_of(c, m3)
    out = m3.siso_forward(*args, chunk=chunk, dtype_policy=policy, save_residuals=True)
    dev = lambda t: t.float().cuda()  # noqa: E731
    gr = m3.siso_backward(d["dy"], *args[:9], out[4].ybar, out[4].chunk_states, d["d_skip"],
                          d["z"], d["seed_ssm"], d["seed_k"], d["seed_v"], d["seed_coef"],
                          dev(dfs), dev(dfk), dev(dfv), chunk=chunk, dtype_policy=policy)
    for name, w in want.items():
        got = getattr(gr, GRAD_FIELD[name])
        if policy == "f32":
            assert_f32(got, w, "grad", f"d{name}")
        else:
            assert_maxrel(got, w, BF16_GRAD_MAXREL, f"d{name}")


@pytest.mark.parametrize("policy,n,p,chunk,compact", [
    ("bf16", 128, 64, 128, False), ("bf16", 128, 64, 128, True), ("bf16", 32, 16, 64, False),
    ("f32", 128, 64, 32, False), ("f32", 64, 64, 64, True),
])
def test_backward_is_bit_reproducible(m3, policy, n, p, chunk, compact):
    """Every gradient, the head-summed dq/dk, the bias and the dadt shares included, is
    bit-identical between two runs on the same inputs: the cross-wave sums are taken in
    wave order, not by float atomics in arrival order."""
    c, d = boundary_inputs(2, 8, 512, n, p, n // 4, policy, seed=5)
    phi = phi_strips_of(c, m3) if compact else d["phi"]
    a = fwd_args(dict(d, phi=phi))
    out = m3.siso_forward(*a, chunk=chunk, dtype_policy=policy, save_residuals=True)
    runs = [m3.siso_backward(d["dy"], *a[:9], out[4].ybar, out[4].chunk_states,
                             d_skip=d["d_skip"], z=d["z"], chunk=chunk, dtype_policy=policy)
            for _ in range(3)]
    for name in runs[0]._fields:
        x = getattr(runs[0], name)
        if isinstance(x, torch.Tensor):
            for r in runs[1:]:
                assert torch.equal(x, getattr(r, name)), name


@pytest.mark.parametrize("policy,n,p,chunk,compact", [("bf16", 128, 128, 128, False),
                                                    ("f32", 32, 48, 64, True)])
def test_forward_and_backward_with_sub_heads(m3, policy, n, p, chunk, compact):
    """A head width with no kernel runs as sub-heads of a compiled width: forward outputs
    and every gradient (the shared inputs' summed over sub-heads) against the oracle,
    with seeds and final-state cotangents, and dv / dz written into caller buffers laid
    out like the layer's (B, L, H*P) projection gradient."""
    want, gr = run_case(m3, 2, 2, 256, n, p, n // 4, chunk, policy, True, True, seed=3)
    c, d = boundary_inputs(2, 2, 256, n, p, n // 4, policy, seed=3, seeds=True)
    for name, w in want.items():
        g_ = getattr(gr, GRAD_FIELD[name])
        if policy == "f32":
            assert_f32(g_, w, "grad", f"d{name}")
        else:
            assert_maxrel(g_, w, BF16_GRAD_MAXREL, f"d{name}")
    # in place into (B, L, H*P) buffers, phi built in the kernel
    phi = phi_strips_of(c, m3) if compact else d["phi"]
    a = fwd_args(dict(d, phi=phi))
    out = m3.siso_forward(*a, chunk=chunk, dtype_policy=policy, save_residuals=True)
    mt = d["v"].dtype
    buf = torch.zeros(2, 256, 2 * 2 * p, device="cuda", dtype=mt)
    dv_out = buf[..., :2 * p].unflatten(-1, (2, p)).permute(0, 2, 1, 3)
    dz_out = buf[..., 2 * p:].unflatten(-1, (2, p)).permute(0, 2, 1, 3)
    g2 = m3.siso_backward(d["dy"], *a[:9], out[4].ybar, out[4].chunk_states,
                          d_skip=d["d_skip"], z=d["z"], seed_ssm=d["seed_ssm"],
                          seed_k=d["seed_k"], seed_v=d["seed_v"], seed_coef=d["seed_coef"],
                          chunk=chunk, dtype_policy=policy, dv_out=dv_out, dz_out=dz_out)
    assert g2.dv.data_ptr() == dv_out.data_ptr() and g2.dz.data_ptr() == dz_out.data_ptr()
    ref = m3.siso_backward(d["dy"], *a[:9], out[4].ybar, out[4].chunk_states,
                           d_skip=d["d_skip"], z=d["z"], seed_ssm=d["seed_ssm"],
                           seed_k=d["seed_k"], seed_v=d["seed_v"], seed_coef=d["seed_coef"],
                           chunk=chunk, dtype_policy=policy)
    assert torch.equal(g2.dv, ref.dv) and torch.equal(g2.dz, ref.dz)
    assert torch.equal(g2.dq, ref.dq) and torch.equal(g2.dadt, ref.dadt)


@pytest.mark.parametrize("policy,n,p,chunk", [("bf16", 128, 64, 128), ("f32", 32, 16, 64)])
def test_backward_writes_only_its_output_views(m3, policy, n, p, chunk):
    """dv / dz written into column views of a NaN-filled (B, L, W) buffer laid out like the
    layer's projection gradient (dz, dx, then 24 padding columns per token): every entry of
    the two views is finite and equal to the kernel's own allocation, and the padding
    columns are still NaN afterwards, so the kernel wrote exactly its views."""
    b, h, L = 2, 3, 256
    c, d = boundary_inputs(b, h, L, n, p, n // 4, policy, seed=37)
    a = fwd_args(d)
    out = m3.siso_forward(*a, chunk=chunk, dtype_policy=policy, save_residuals=True)
    mt = d["v"].dtype
    hp = h * p
    buf = torch.full((b, L, 2 * hp + 24), float("nan"), device="cuda", dtype=mt)
    dz_out = buf[..., :hp].unflatten(-1, (h, p)).permute(0, 2, 1, 3)
    dv_out = buf[..., hp:2 * hp].unflatten(-1, (h, p)).permute(0, 2, 1, 3)
    g2 = m3.siso_backward(d["dy"], *a[:9], out[4].ybar, out[4].chunk_states,
                          d_skip=d["d_skip"], z=d["z"], chunk=chunk, dtype_policy=policy,
                          dv_out=dv_out, dz_out=dz_out)
    ref = m3.siso_backward(d["dy"], *a[:9], out[4].ybar, out[4].chunk_states,
                           d_skip=d["d_skip"], z=d["z"], chunk=chunk, dtype_policy=policy)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(buf[..., :2 * hp].float()).all())
    assert bool(torch.isnan(buf[..., 2 * hp:].float()).all())
    assert torch.equal(g2.dv, ref.dv) and torch.equal(g2.dz, ref.dz)


def test_backward_matches_finite_differences_of_the_kernel_forward(m3):
    """Central differences of the HIP forward itself (f32, tiny): the VJP is checked
    against the function it differentiates, as tests.py:614-645 does."""
    c, d = boundary_inputs(1, 1, 64, 16, 16, 4, "f32", seed=9)
    dy = d["dy"]

    def loss(args):
        y, fs, fk, fv = m3.siso_forward(*args, chunk=32, dtype_policy="f32")
        return float((y.double() * dy.double()).sum())

    out = m3.siso_forward(*fwd_args(d), chunk=32, dtype_policy="f32", save_residuals=True)
    gr = m3.siso_backward(dy, d["q"], d["k"], d["v"], d["adt"], d["gamma"], d["scale"], d["phi"],
                          d["q_bias"], d["k_bias"], out[4].ybar, out[4].chunk_states, d["d_skip"],
                          d["z"], chunk=32, dtype_policy="f32")
    gen = torch.Generator().manual_seed(3)
    for idx, name, field, eps in ((0, "q", "dq", 1e-2), (2, "v", "dv", 1e-2), (3, "adt", "dadt", 1e-3),
                                  (6, "phi", "dphi", 1e-3), (5, "scale", "dscale", 1e-3)):
        base = fwd_args(d)
        t = base[idx]
        for i in torch.randperm(t.numel(), generator=gen)[:3].tolist():
            plus, minus = list(base), list(base)
            tp, tm = t.clone().reshape(-1), t.clone().reshape(-1)
            tp[i] += eps
            tm[i] -= eps
            plus[idx], minus[idx] = tp.reshape(t.shape), tm.reshape(t.shape)
            fd = (loss(plus) - loss(minus)) / (2 * eps)
            got = float(getattr(gr, field).reshape(-1)[i])
            assert abs(got - fd) <= 2e-2 * max(1.0, abs(fd)), (name, i, got, fd)


def test_backward_full_size_cfg3_head_slices_and_head_sum(m3):
    """cfg3 shapes (B=8, L=8192, H=32, bf16, chunk 128). Per-head gradients of a head
    slice match the oracle run on that slice alone (heads only couple through the
    head-summed dq/dk); the head sum is checked by linearity: the full run's dq/dk
    equals the sum of the kernel's dq/dk over disjoint head groups."""
    B, L, H, N, P, Nr = 8, 8192, 32, 128, 64, 32
    g = torch.Generator(device="cuda").manual_seed(21)

    def rn(*s):
        return torch.randn(*s, generator=g, device="cuda")

    def norm_rows(t):
        return t * torch.rsqrt(t.square().mean(-1, keepdim=True) + 1e-6)

    q = norm_rows(rn(B, L, N)).to(BF16)
    k = norm_rows(rn(B, L, N)).to(BF16)
    v, z, dy = rn(B, H, L, P).to(BF16), rn(B, H, L, P).to(BF16), rn(B, H, L, P).to(BF16)
    dt_raw = torch.log(torch.expm1(torch.exp(torch.rand(B, L, H, generator=g, device="cuda")
                                             * (math.log(0.1) - math.log(0.001)) + math.log(0.001))))
    pre, _ = m3.preprocess(dt_raw, rn(B, L, H), rn(B, L, H), 0.5 * rn(B, L, Nr),
                           torch.zeros(H, device="cuda"))
    qb, kb, dsk = 0.1 * rn(H, N), 0.1 * rn(H, N), rn(H)

    def grads(hs):
        a = [q, k, v[:, hs], pre.adt[:, hs], pre.gamma[:, hs], pre.scale[:, hs], pre.phi[:, hs],
             qb[hs], kb[hs], dsk[hs], z[:, hs]]
        out = m3.siso_forward(*a, chunk=128, save_residuals=True)
        return m3.siso_backward(dy[:, hs], *a[:9], out[4].ybar, out[4].chunk_states,
                                d_skip=dsk[hs], z=z[:, hs], chunk=128)

    full = grads(slice(None))
    parts = [grads(slice(i, i + 8)) for i in range(0, H, 8)]
    dq_sum = sum(p_.dq for p_ in parts)
    dk_sum = sum(p_.dk for p_ in parts)
    assert O.max_rel(full.dq.cpu(), dq_sum.cpu()) <= 1e-5
    assert O.max_rel(full.dk.cpu(), dk_sum.cpu()) <= 1e-5
    for name in ("dv", "dz", "dadt", "dscale", "dphi"):
        assert bool(torch.isfinite(getattr(full, name).float()).all()), name
    # per-head gradients of one batch element on a 2-head slice vs the oracle
    b_, hs = 3, [2, 29]
    sl = lambda t: t[b_:b_ + 1, hs].double().cpu()  # noqa: E731
    inputs = dict(q=q[b_:b_ + 1].double().cpu(), k=k[b_:b_ + 1].double().cpu(), v=sl(v),
                  adt=sl(pre.adt), gamma=sl(pre.gamma), scale=sl(pre.scale), phi=sl(pre.phi),
                  q_bias=qb[hs].double().cpu(), k_bias=kb[hs].double().cpu(),
                  d_skip=dsk[hs].double().cpu(), z=sl(z))
    want = O.boundary_grads(inputs, sl(dy), chunk=128)
    got = dict(v=full.dv, z=full.dz, adt=full.dadt, gamma=full.dgamma, scale=full.dscale,
               phi=full.dphi)
    for name, t in got.items():
        report(f"cfg3 d{name} (slice) vs float64", t[b_:b_ + 1, hs], want[name])
        assert_maxrel(t[b_:b_ + 1, hs], want[name], BF16_GRAD_MAXREL, f"d{name} (slice)")
    # the same two heads through the kernel alone, at the full length: the head-summed
    # dq/dk, the bias and skip gradients and the seed adjoint are then the oracle's too
    a = [q[b_:b_ + 1], k[b_:b_ + 1], v[b_:b_ + 1, hs], pre.adt[b_:b_ + 1, hs],
         pre.gamma[b_:b_ + 1, hs], pre.scale[b_:b_ + 1, hs], pre.phi[b_:b_ + 1, hs], qb[hs],
         kb[hs], dsk[hs], z[b_:b_ + 1, hs]]
    out = m3.siso_forward(*a, chunk=128, save_residuals=True)
    two = m3.siso_backward(dy[b_:b_ + 1, hs], *a[:9], out[4].ybar, out[4].chunk_states,
                           d_skip=dsk[hs], z=z[b_:b_ + 1, hs], chunk=128)
    for name in ("q", "k", "q_bias", "k_bias", "d_skip", "v", "adt", "phi"):
        report(f"cfg3 d{name} (2-head run) vs float64", getattr(two, GRAD_FIELD[name]), want[name])
        assert_maxrel(getattr(two, GRAD_FIELD[name]), want[name], BF16_GRAD_MAXREL,
                      f"d{name} (2-head run)")
    assert_maxabs(out[1], O.siso_boundary_forward(**inputs, chunk=128)[1], STATE_MAXABS,
                  "final ssm (2-head run)")
