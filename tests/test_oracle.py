"""Pins the CPU oracle (oracle/siso_oracle.py) before anything is checked against it.

Each check is chosen so a plausible mistake in the restatement (a dropped term, a
wrong sign, a transposed operand, an off-by-one shift) fails it: golden vectors
from the reference's own torch code, closed forms, brute-force equivalences in
float64, and finite differences.
"""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import siso_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
f64 = torch.float64


def _perm_last(x, n):
    return x[..., O.deinterleave_perm(n)]


# ---------------------------------------------------------------------------------
# Rotary helpers and the permutation
# ---------------------------------------------------------------------------------


@pytest.mark.parametrize("n,nr", [(16, 4), (16, 8), (128, 32), (128, 64)])
def test_perm_commutes_with_rotation(n, nr):
    """perm(interleaved_rope(u)) == halfsplit_rope(perm(u)) (layout.py:315-317)."""
    g = torch.Generator().manual_seed(n + nr)
    u = torch.randn(5, n, generator=g, dtype=f64)
    phi = torch.rand(5, nr, generator=g, dtype=f64) * 6.0
    inter = O.rope_apply_interleaved(u, torch.cos(phi), torch.sin(phi))
    cos, sin = O.rope_cos_sin(phi, n)
    half = O.rope_apply(_perm_last(u, n), cos, sin)
    assert torch.equal(_perm_last(inter, n), half)
    # the inverse permutation really is the inverse
    assert torch.equal(_perm_last(u, n)[..., O.interleave_perm(n)], u)


def test_rotation_is_orthogonal_and_dphi_is_its_derivative():
    g = torch.Generator().manual_seed(3)
    n, nr = 32, 8
    u = torch.randn(7, n, generator=g, dtype=f64)
    dx = torch.randn(7, n, generator=g, dtype=f64)
    phi = torch.rand(7, nr, generator=g, dtype=f64) * 6.0
    cos, sin = O.rope_cos_sin(phi, n)
    x = O.rope_apply(u, cos, sin)
    torch.testing.assert_close(x.norm(dim=-1), u.norm(dim=-1), rtol=1e-14, atol=0)
    # R^T = R(-phi): pulling back undoes the rotation
    torch.testing.assert_close(O.rope_apply(x, cos, -sin), u, rtol=0, atol=1e-13)
    # d/dphi_j <dx, R(phi) u> == rope_dphi(R u, dx)_j, by central differences
    eps = 1e-6
    fd = torch.empty(7, nr, dtype=f64)
    for j in range(nr):
        e = torch.zeros(nr, dtype=f64)
        e[j] = eps
        cp, sp = O.rope_cos_sin(phi + e, n)
        cm, sm = O.rope_cos_sin(phi - e, n)
        fd[:, j] = ((O.rope_apply(u, cp, sp) - O.rope_apply(u, cm, sm)) * dx).sum(-1) / (2 * eps)
    torch.testing.assert_close(O.rope_dphi(x, dx, nr), fd, rtol=1e-7, atol=1e-8)


# ---------------------------------------------------------------------------------
# Preprocess closed forms
# ---------------------------------------------------------------------------------


def test_preprocess_closed_forms():
    x = torch.tensor([-3.0, -1.0, -0.25, 0.0, 0.5, 2.0], dtype=f64)
    want = torch.tensor([1 / 4, 1 / 2, 1 / 1.25, 1.0, 1.5, 3.0], dtype=f64)
    torch.testing.assert_close(O.heavy_tail(x), want, rtol=0, atol=1e-15)

    b, seqlen, h, nr = 2, 9, 3, 4
    g = torch.Generator().manual_seed(0)
    dt_raw = torch.randn(b, seqlen, h, generator=g, dtype=f64)
    a_raw = torch.randn(b, seqlen, h, generator=g, dtype=f64)
    trap = torch.randn(b, seqlen, h, generator=g, dtype=f64)
    ang = torch.randn(b, seqlen, nr, generator=g, dtype=f64) * 3
    bias = torch.randn(h, generator=g, dtype=f64)
    pre, phi_fin = O.preprocess(dt_raw, a_raw, trap, ang, bias, a_floor=1e-4)
    dt = torch.log1p(torch.exp(dt_raw + bias)).transpose(1, 2)
    lam = (1 / (1 + torch.exp(-trap))).transpose(1, 2)
    a = -torch.where(a_raw >= 0, 1 + a_raw, 1 / (1 - a_raw)).transpose(1, 2)
    a = torch.minimum(a, torch.tensor(-1e-4, dtype=f64))
    torch.testing.assert_close(pre.dt, dt)
    torch.testing.assert_close(pre.adt, a * dt)
    torch.testing.assert_close(pre.gamma, dt * lam)
    # scale_t = gamma_t + dt_{t+1}(1 - lam_{t+1}); the last position has no successor
    torch.testing.assert_close(pre.scale[..., :-1], (dt * lam)[..., :-1] + dt[..., 1:] * (1 - lam[..., 1:]))
    torch.testing.assert_close(pre.scale[..., -1], (dt * lam)[..., -1])
    # phi is the wrapped running sum of tanh(angle)*pi*dt, per head
    theta = torch.tanh(ang)[:, None] * math.pi * dt[..., None]
    raw = torch.cumsum(theta, dim=2)
    assert bool(((pre.phi >= 0) & (pre.phi < 2 * math.pi)).all())
    d = torch.remainder(pre.phi - raw + math.pi, 2 * math.pi) - math.pi
    assert float(d.abs().max()) < 1e-12
    assert torch.equal(phi_fin, pre.phi[:, :, -1])


# ---------------------------------------------------------------------------------
# Golden vectors from the reference's torch code
# ---------------------------------------------------------------------------------


def _load(name):
    return dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))


def _golden_kernel_inputs(fx):
    t = {k: torch.from_numpy(v).to(f64) for k, v in fx.items() if v.dtype != bool and v.ndim > 0}
    n = t["q"].shape[-1]
    b, seqlen = t["q"].shape[:2]
    h = t["v"].shape[2]
    nr = t["angles"].shape[-1]
    perm = O.deinterleave_perm(n)
    lam = torch.sigmoid(t["trap"])
    angles_h = t["angles"][:, None].expand(b, h, seqlen, nr)
    phi, _ = O.cumulative_angles(angles_h, t["dt"])
    with_dz = bool(fx["with_dz"])
    return dict(
        q=t["q"][..., perm], k=t["k"][..., perm], v=t["v"].permute(0, 2, 1, 3),
        adt=t["adt"], dt=t["dt"], lam=lam, phi=phi,
        q_bias=t["q_bias"][:, perm], k_bias=t["k_bias"][:, perm],
        d_skip=t["d"] if with_dz else None,
        z=t["z"].permute(0, 2, 1, 3) if with_dz else None,
    ), t, perm


@pytest.mark.parametrize("name", ["torch_ref_kernel_gated", "torch_ref_kernel_plain"])
def test_recurrent_matches_reference_torch_golden(name):
    fx = _load(name)
    x, t, perm = _golden_kernel_inputs(fx)
    y, st = O.siso_recurrent(**x)
    want_y = t["out"].permute(0, 2, 1, 3)
    assert O.max_rel(y, want_y) < 2e-5, O.max_rel(y, want_y)
    assert O.max_rel(st.ssm, t["ssm_state"][..., perm]) < 2e-5
    assert O.max_rel(st.k, t["k_state"][..., perm]) < 2e-5
    assert O.max_rel(st.v, t["v_state"]) == 0.0
    assert O.rel_error(st.phi, t["angle_state"], angle=True) < 1e-5


@pytest.mark.parametrize("name,chunk", [("torch_ref_kernel_gated", 32), ("torch_ref_kernel_plain", 16)])
def test_chunked_matches_reference_torch_golden(name, chunk):
    fx = _load(name)
    x, t, perm = _golden_kernel_inputs(fx)
    gamma, scale = O.trapezoid_coeffs(x["dt"], x["lam"])
    y, st = O.siso_chunked(x["q"], x["k"], x["v"], x["adt"], gamma, scale, x["phi"],
                           x["q_bias"], x["k_bias"], x["d_skip"], x["z"], chunk=chunk)
    assert O.max_rel(y, t["out"].permute(0, 2, 1, 3)) < 2e-5
    assert O.max_rel(st.ssm, t["ssm_state"][..., perm]) < 2e-5
    assert O.max_rel(st.k, t["k_state"][..., perm]) < 2e-5


def _layer_params_from_sd(fx):
    """Same mapping as convert.torch_to_jax (convert.py:92-149)."""
    sd = {k[4:].replace("__", "."): torch.from_numpy(v).to(f64)
          for k, v in fx.items() if k.startswith("sd__")}
    d_model, n, p, expand = (int(v) for v in fx["cfg"])
    d_inner = expand * d_model
    perm = O.deinterleave_perm(n)
    in_proj = sd["in_proj.weight"].T.clone()
    for start in (2 * d_inner, 2 * d_inner + n):
        in_proj[:, start:start + n] = in_proj[:, start:start + n][:, perm]
    return dict(
        in_proj=in_proj, out_proj=sd["out_proj.weight"].T.clone(), dt_bias=sd["dt_bias"],
        b_norm_weight=sd["B_norm_weight"][perm], c_norm_weight=sd["C_norm_weight"][perm],
        b_bias=sd["B_bias"][:, 0][:, perm], c_bias=sd["C_bias"][:, 0][:, perm],
        d_skip=sd["D"],
    ), (d_model, n, p, expand, float(fx["rope_fraction"]))


@pytest.mark.parametrize("name", ["torch_ref_layer_half", "torch_ref_layer_full"])
def test_layer_matches_reference_torch_golden(name):
    fx = _load(name)
    params, (d_model, n, p, expand, rf) = _layer_params_from_sd(fx)
    u = torch.from_numpy(fx["u"]).to(f64)
    y, _ = O.layer_forward(params, u, d_state=n, headdim=p, expand=expand, rope_fraction=rf,
                           chunk=16)
    want = torch.from_numpy(fx["y"]).to(f64)
    assert O.max_rel(y, want) < 1e-5, O.max_rel(y, want)
    assert O.rel_error(y, want) < 1e-4


# ---------------------------------------------------------------------------------
# Formulation equivalences in float64
# ---------------------------------------------------------------------------------


def _f64_case(b=2, h=3, seqlen=64, n=16, p=8, nr=4, seed=0):
    x = O.make_inputs(b, h, seqlen, n, p, nr, seed=seed)
    pre, _ = O.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"])
    return x, pre


@pytest.mark.parametrize("chunk", [8, 16, 64])
def test_chunked_equals_recurrent_f64(chunk):
    x, pre = _f64_case()
    yr, sr = O.siso_recurrent(x["q"], x["k"], x["v"], pre.adt, pre.dt, pre.lam, pre.phi,
                              x["q_bias"], x["k_bias"], x["d_skip"], x["z"])
    yc, sc = O.siso_chunked(x["q"], x["k"], x["v"], pre.adt, pre.gamma, pre.scale, pre.phi,
                            x["q_bias"], x["k_bias"], x["d_skip"], x["z"], chunk=chunk)
    assert O.max_rel(yc, yr) < 1e-10
    assert O.max_rel(sc.ssm, sr.ssm) < 1e-10
    assert O.max_rel(sc.k, sr.k) < 1e-12
    assert torch.equal(sc.v, sr.v)


def test_seeded_chunked_equals_recurrent_f64():
    """A carried state (ssm, k, v, phi) seeds the chunked form exactly."""
    x, _ = _f64_case(seqlen=32)
    g = torch.Generator().manual_seed(5)
    b, h, p, n, nr = 2, 3, 8, 16, 4
    st = O.SISOState(torch.randn(b, h, p, n, generator=g, dtype=f64),
                     torch.randn(b, h, n, generator=g, dtype=f64),
                     torch.randn(b, h, p, generator=g, dtype=f64),
                     torch.rand(b, h, nr, generator=g, dtype=f64) * 6)
    pre, _ = O.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"],
                          phi_init=st.phi)
    yr, sr = O.siso_recurrent(x["q"], x["k"], x["v"], pre.adt, pre.dt, pre.lam, pre.phi,
                              x["q_bias"], x["k_bias"], x["d_skip"], x["z"], state=st)
    yc, sc = O.siso_chunked(x["q"], x["k"], x["v"], pre.adt, pre.gamma, pre.scale, pre.phi,
                            x["q_bias"], x["k_bias"], x["d_skip"], x["z"], state=st,
                            seed_dt=pre.dt[:, :, 0], seed_lam=pre.lam[:, :, 0], chunk=8)
    assert O.max_rel(yc, yr) < 1e-10
    assert O.max_rel(sc.ssm, sr.ssm) < 1e-10


def test_rotation_parity_known_answer():
    """tests.py:451-513: only token 0 writes, no decay, phi advances pi per set bit,
    so y_t = (-1)^(running parity)."""
    b, h, seqlen, n, p, nr = 2, 1, 64, 16, 4, 4
    g = torch.Generator().manual_seed(0)
    bits = (torch.rand(b, seqlen, generator=g) < 0.5).to(f64)
    bits[:, 0] = 0
    parity = torch.cumsum(bits, 1) % 2
    atanh_one = math.atanh(1 - 1e-12)
    angles = torch.where(bits[:, :, None] > 0.5, atanh_one, 0.0) * torch.ones(1, 1, nr, dtype=f64)
    dt = torch.ones(b, h, seqlen, dtype=f64)
    lam = torch.ones(b, h, seqlen, dtype=f64)
    adt = torch.full((b, h, seqlen), -1e-12, dtype=f64)
    gamma, scale = O.trapezoid_coeffs(dt, lam)
    phi, _ = O.cumulative_angles(angles[:, None].expand(b, h, seqlen, nr), dt)
    q = torch.zeros(b, seqlen, n, dtype=f64)
    q[..., 0] = 1
    k = torch.zeros(b, seqlen, n, dtype=f64)
    k[:, 0, 0] = 1
    v = torch.ones(b, h, seqlen, p, dtype=f64)
    zb = torch.zeros(h, n, dtype=f64)
    want = torch.where(parity[:, None, :, None] > 0.5, -1.0, 1.0).to(f64).expand(b, h, seqlen, p)
    yr, _ = O.siso_recurrent(q, k, v, adt, dt, lam, phi, zb, zb)
    yc, _ = O.siso_chunked(q, k, v, adt, gamma, scale, phi, zb, zb, chunk=16)
    for y in (yr, yc):
        assert torch.equal(torch.sign(y), want)
        assert float((y - want).abs().max()) < 1e-9


def test_segments_chain_equals_single_call():
    x, _ = _f64_case(seqlen=64)
    args = ("q", "k")
    full_y, full_st = O.siso_segment(*[x[a] for a in args], x["v"], x["dt_raw"], x["a_raw"],
                                     x["trap_raw"], x["angles"], x["dt_bias"], x["q_bias"],
                                     x["k_bias"], x["d_skip"], x["z"], chunk=16)

    def seg(sl, state=None):
        return O.siso_segment(x["q"][:, sl], x["k"][:, sl], x["v"][:, :, sl], x["dt_raw"][:, sl],
                              x["a_raw"][:, sl], x["trap_raw"][:, sl], x["angles"][:, sl],
                              x["dt_bias"], x["q_bias"], x["k_bias"], x["d_skip"],
                              x["z"][:, :, sl], state=state, chunk=16)

    y1, s1 = seg(slice(0, 32))
    y2, s2 = seg(slice(32, 64), s1)
    assert O.max_rel(torch.cat([y1, y2], 2), full_y) < 1e-10
    assert O.max_rel(s2.ssm, full_st.ssm) < 1e-10
    assert O.max_rel(s2.k, full_st.k) < 1e-12
    assert O.rel_error(s2.phi, full_st.phi, angle=True) < 1e-10


def test_step_chain_equals_prefill_and_handoff():
    x, pre = _f64_case(b=1, h=2, seqlen=32)
    b, h, p, n, nr = 1, 2, 8, 16, 4
    st = O.zero_state(b, h, p, n, nr)
    ys = []
    for t in range(32):
        y, st = O.siso_step(x["q"][:, t], x["k"][:, t], x["v"][:, :, t], pre.adt[:, :, t],
                            pre.dt[:, :, t], pre.lam[:, :, t], x["angles"][:, t], x["q_bias"],
                            x["k_bias"], st, x["d_skip"], x["z"][:, :, t])
        ys.append(y)
    y_pre, s_pre = O.siso_chunked(x["q"], x["k"], x["v"], pre.adt, pre.gamma, pre.scale, pre.phi,
                                  x["q_bias"], x["k_bias"], x["d_skip"], x["z"], chunk=8)
    assert O.max_rel(torch.stack(ys, 2), y_pre) < 1e-10
    assert O.max_rel(st.ssm, s_pre.ssm) < 1e-10
    assert O.max_rel(st.k, s_pre.k) < 1e-12
    # prefill the first half, then decode the rest from the handed-over carry
    y_a, s_a = O.siso_segment(x["q"][:, :16], x["k"][:, :16], x["v"][:, :, :16],
                              x["dt_raw"][:, :16], x["a_raw"][:, :16], x["trap_raw"][:, :16],
                              x["angles"][:, :16], x["dt_bias"], x["q_bias"], x["k_bias"],
                              x["d_skip"], x["z"][:, :, :16], chunk=8)
    st = s_a
    pre2, _ = O.preprocess(x["dt_raw"][:, 16:], x["a_raw"][:, 16:], x["trap_raw"][:, 16:],
                           x["angles"][:, 16:], x["dt_bias"], phi_init=s_a.phi)
    ys = []
    for t in range(16):
        y, st = O.siso_step(x["q"][:, 16 + t], x["k"][:, 16 + t], x["v"][:, :, 16 + t],
                            pre2.adt[:, :, t], pre2.dt[:, :, t], pre2.lam[:, :, t],
                            x["angles"][:, 16 + t], x["q_bias"], x["k_bias"], st,
                            x["d_skip"], x["z"][:, :, 16 + t])
        ys.append(y)
    assert O.max_rel(torch.cat([y_a, torch.stack(ys, 2)], 2), y_pre) < 1e-10


def test_step_matches_reference_torch_golden_first_tokens():
    """One decode step from a zero state is the first token of upstream's recurrence."""
    fx = _load("torch_ref_kernel_gated")
    x, t, perm = _golden_kernel_inputs(fx)
    b, h, p, n = 2, 3, 16, 16
    st = O.zero_state(b, h, p, n, 4)
    angles = t["angles"]
    for tt in range(3):
        y, st = O.siso_step(x["q"][:, tt], x["k"][:, tt], x["v"][:, :, tt], x["adt"][:, :, tt],
                            x["dt"][:, :, tt], x["lam"][:, :, tt], angles[:, tt], x["q_bias"],
                            x["k_bias"], st, x["d_skip"], x["z"][:, :, tt])
        assert O.max_rel(y, t["out"][:, tt].to(f64)) < 2e-5


# ---------------------------------------------------------------------------------
# Gradients: autograd of the chunked form vs finite differences
# ---------------------------------------------------------------------------------


def test_boundary_grads_match_finite_differences():
    b, h, seqlen, n, p, nr = 1, 2, 16, 8, 4, 2
    x = O.make_inputs(b, h, seqlen, n, p, nr, seed=4)
    pre, _ = O.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"])
    g = torch.Generator().manual_seed(9)
    inputs = dict(q=x["q"], k=x["k"], v=x["v"], adt=pre.adt, gamma=pre.gamma, scale=pre.scale,
                  phi=pre.phi, q_bias=x["q_bias"], k_bias=x["k_bias"], d_skip=x["d_skip"],
                  z=x["z"], seed_ssm=torch.randn(b, h, p, n, generator=g, dtype=f64),
                  seed_k=torch.randn(b, h, n, generator=g, dtype=f64),
                  seed_v=torch.randn(b, h, p, generator=g, dtype=f64),
                  seed_coef=torch.rand(b, h, generator=g, dtype=f64))
    dy = x["dy"]
    dfs = torch.randn(b, h, p, n, generator=g, dtype=f64)
    dfk = torch.randn(b, h, n, generator=g, dtype=f64)
    dfv = torch.randn(b, h, p, generator=g, dtype=f64)
    grads = O.boundary_grads(inputs, dy, dfs, dfk, dfv, chunk=8)

    def loss(inp):
        y, fs, fk, fv = O.siso_boundary_forward(**inp, chunk=8)
        return float((y * dy).sum() + (fs * dfs).sum() + (fk * dfk).sum() + (fv * dfv).sum())

    eps = 1e-6
    gen = torch.Generator().manual_seed(1)
    for name, grad in grads.items():
        base = inputs[name]
        flat = base.reshape(-1)
        picks = torch.randperm(flat.numel(), generator=gen)[:6]
        for i in picks.tolist():
            plus = dict(inputs)
            minus = dict(inputs)
            bp = flat.clone()
            bm = flat.clone()
            bp[i] += eps
            bm[i] -= eps
            plus[name] = bp.reshape(base.shape)
            minus[name] = bm.reshape(base.shape)
            fd = (loss(plus) - loss(minus)) / (2 * eps)
            got = float(grad.reshape(-1)[i])
            assert abs(got - fd) <= 1e-6 + 1e-6 * abs(fd), (name, i, got, fd)
