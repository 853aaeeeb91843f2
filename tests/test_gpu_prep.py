"""GPU parity of the HIP preprocessing (m3s_prep_fwd / m3s_prep_bwd) against the oracle's
``preprocess`` (``reference.py:160-199``) and its autograd.

Forward: the (B, H, L) scalars to 2e-6 relative (elementwise transcendental rounding of
f32 device math vs the CPU's). phi against the float64 oracle: p95 circular error at
most max(2e-5 rad, 5x the error of the same oracle run in float32). The reference sums
in f32 too, and before the wrap phi reaches 10^2-10^3 rad, where one f32 ulp is up to
~1e-4; an indexing or offset mistake in the scan costs O(theta) >= 1e-3 instead.
Backward: gradients against float64 autograd of the oracle, p95 relative <= 1e-4
(f32 raw inputs), max-normalised <= 2e-2 for bf16 raw slices.
"""

import pytest
import torch

from oracle import siso_oracle as O

pytestmark = pytest.mark.gpu

F64 = torch.float64


def raw_inputs(b, l, h, nr, seed, dtype=torch.float32, zeros=False, big=False):
    x = O.make_inputs(b, h, l, 16, 16, nr, seed=seed)
    dt_raw, a_raw, trap_raw, ang = x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"]
    g = torch.Generator().manual_seed(seed + 100)
    dt_bias = 0.3 * torch.randn(h, generator=g, dtype=F64)
    if zeros:   # exact zeros hit both heavy_tail masks; large dt_raw the softplus threshold
        a_raw = a_raw.clone()
        a_raw[:, ::7] = 0.0
    if big:
        dt_raw = dt_raw.clone()
        dt_raw[:, ::11] = 25.0
    cast = [t.to(dtype).to(F64) for t in (dt_raw, a_raw, trap_raw, ang)]   # identical values
    return cast + [dt_bias.float().to(F64)]


def phi_limit(dtr, ar, tr, ang, bias, a_floor=1e-4, phi0=None):
    """5x the p95 phi error of the oracle itself in float32, floored at 2e-5 rad."""
    f = [t.float() for t in (dtr, ar, tr, ang, bias)]
    r32, f32fin = O.preprocess(*f, a_floor=a_floor, phi_init=None if phi0 is None else phi0.float())
    r64, f64fin = O.preprocess(dtr, ar, tr, ang, bias, a_floor=a_floor, phi_init=phi0)
    return (max(2e-5, 5 * O.rel_error(r32.phi, r64.phi, angle=True)),
            max(2e-5, 5 * O.rel_error(f32fin, f64fin, angle=True)))


def as_proj(dev, dtype, *ts):
    """Lay the (B, L, X) inputs side by side in one (B, L, sum X) buffer, the way the
    layer hands the kernel slices of its fused projection."""
    buf = torch.cat([t.to(dtype) for t in ts], dim=-1).to(dev)
    out, o = [], 0
    for t in ts:
        out.append(buf[..., o:o + t.shape[-1]])
        o += t.shape[-1]
    return out


@pytest.mark.parametrize("b,l,h,nr,a_floor,init", [
    (2, 40, 3, 4, 1e-4, True),
    (1, 1000, 4, 6, 1e-4, False),    # Nr not a multiple of 4; ragged time ranges
    (2, 256, 8, 32, 0.5, True),      # a_floor = 0.5 makes the clamp active
    (1, 64, 2, 0, 1e-4, False),      # no rotary angles
])
def test_prep_forward_matches_oracle(m3, dev, b, l, h, nr, a_floor, init):
    dtr, ar, tr, ang, bias = raw_inputs(b, l, h, nr, seed=l + nr, zeros=True, big=True)
    g = torch.Generator().manual_seed(3)
    phi0 = (torch.rand(b, h, nr, generator=g, dtype=F64) * 6.0) if init else None
    ref, rfin = O.preprocess(dtr, ar, tr, ang, bias, a_floor=a_floor, phi_init=phi0)
    d_dt, d_a, d_tr, d_ang = as_proj(dev, torch.float32, dtr, ar, tr, ang)
    pre, fin = m3.preprocess(d_dt, d_a, d_tr, d_ang, bias.float().to(dev), a_floor=a_floor,
                             phi_init=None if phi0 is None else phi0.float().to(dev))
    for name in ("adt", "gamma", "scale", "lam", "dt"):
        got, want = getattr(pre, name).cpu().double(), getattr(ref, name)
        torch.testing.assert_close(got, want, rtol=2e-6, atol=1e-9, msg=name)
    assert pre.phi.shape == (b, h, l, nr)
    if nr:
        lim, lim_fin = phi_limit(dtr, ar, tr, ang, bias, a_floor, phi0)
        assert O.rel_error(pre.phi, ref.phi, angle=True) <= lim
        assert O.rel_error(fin, rfin, angle=True) <= lim_fin
        assert float(pre.phi.min()) >= 0.0 and float(pre.phi.max()) < 2 * torch.pi + 1e-6
        torch.testing.assert_close(fin, pre.phi[:, :, -1], rtol=0, atol=0)


def test_prep_forward_full_length(m3, dev):
    """configs[1] length (L = 8192, H = 32, Nr = 32) from bf16 projection slices."""
    b, l, h, nr = 2, 8192, 32, 32
    dtr, ar, tr, ang, bias = raw_inputs(b, l, h, nr, seed=5, dtype=torch.bfloat16)
    ref, rfin = O.preprocess(dtr, ar, tr, ang, bias)
    d_dt, d_a, d_tr, d_ang = as_proj(dev, torch.bfloat16, dtr, ar, tr, ang)
    pre, fin = m3.preprocess(d_dt, d_a, d_tr, d_ang, bias.float().to(dev))
    for name in ("adt", "gamma", "scale", "lam", "dt"):
        torch.testing.assert_close(getattr(pre, name).cpu().double(), getattr(ref, name),
                                   rtol=2e-6, atol=1e-9, msg=name)
    lim, lim_fin = phi_limit(dtr, ar, tr, ang, bias)
    assert O.rel_error(pre.phi, ref.phi, angle=True) <= lim
    assert O.rel_error(fin, rfin, angle=True) <= lim_fin


@pytest.mark.parametrize("b,l,h,nr,a_floor,init,raw_dtype", [
    (2, 40, 3, 4, 1e-4, True, torch.float32),
    (1, 200, 4, 6, 1e-4, False, torch.float32),
    (1, 150, 5, 12, 1e-4, True, torch.float32),    # 3 angle groups, padded to 4
    (2, 130, 8, 32, 0.5, True, torch.float32),
    (2, 256, 4, 16, 1e-4, True, torch.bfloat16),
])
def test_prep_backward_matches_oracle_autograd(m3, dev, b, l, h, nr, a_floor, init, raw_dtype):
    dtr, ar, tr, ang, bias = raw_inputs(b, l, h, nr, seed=7 + l, dtype=raw_dtype, zeros=True,
                                        big=True)
    g = torch.Generator().manual_seed(11)
    phi0 = (torch.rand(b, h, nr, generator=g, dtype=F64) * 6.0) if init else None
    cot = {k: torch.randn(b, h, l, generator=g, dtype=F64)
           for k in ("adt", "gamma", "scale", "lam", "dt")}
    cot["phi"] = torch.randn(b, h, l, nr, generator=g, dtype=F64)
    cot["fin"] = torch.randn(b, h, nr, generator=g, dtype=F64)

    leaves = [t.clone().requires_grad_(True) for t in (dtr, ar, tr, ang, bias)]
    p0 = phi0.clone().requires_grad_(True) if init else None
    ref, rfin = O.preprocess(*leaves, a_floor=a_floor, phi_init=p0)
    loss = sum((getattr(ref, k) * cot[k]).sum() for k in ("adt", "gamma", "scale", "lam", "dt"))
    loss = loss + (ref.phi * cot["phi"]).sum() + (rfin * cot["fin"]).sum()
    want = torch.autograd.grad(loss, leaves + ([p0] if init else []))

    d_in = as_proj(dev, raw_dtype, dtr, ar, tr, ang)
    d_in = [t.detach().requires_grad_(True) for t in d_in]
    d_bias = bias.float().to(dev).requires_grad_(True)
    d_p0 = phi0.float().to(dev).requires_grad_(True) if init else None
    pre, fin = m3.preprocess(*d_in, d_bias, a_floor=a_floor, phi_init=d_p0)
    dl = sum((getattr(pre, k) * cot[k].float().to(dev)).sum()
             for k in ("adt", "gamma", "scale", "lam", "dt"))
    dl = dl + (pre.phi * cot["phi"].float().to(dev)).sum() + (fin * cot["fin"].float().to(dev)).sum()
    got = torch.autograd.grad(dl, d_in + [d_bias] + ([d_p0] if init else []))
    names = ["dt_raw", "a_raw", "trap_raw", "angles", "dt_bias", "phi_init"]
    for name, gv, wv in zip(names, got, want):
        assert gv.dtype == (raw_dtype if name in names[:4] else torch.float32), name
        if raw_dtype == torch.float32:
            assert O.rel_error(gv, wv) < 1e-4, (name, O.rel_error(gv, wv))
        else:
            assert O.max_rel(gv, wv) < 2e-2, (name, O.max_rel(gv, wv))


@pytest.mark.parametrize("h,nr", [(32, 32), (64, 32), (5, 12)])
def test_prep_backward_is_bit_reproducible(m3, dev, h, nr):
    """The raw-slice gradients are bit-identical between runs: the angle cotangent's sum
    over heads is taken in wave order at the end of each run of tokens (one and two
    rounds of heads per workgroup, and a padded angle-group count)."""
    dtr, ar, tr, ang, bias = raw_inputs(2, 300, h, nr, seed=3)
    g = torch.Generator().manual_seed(4)
    cot = {k: torch.randn(2, h, 300, generator=g).to(dev)
           for k in ("adt", "gamma", "scale", "lam", "dt")}
    cphi = torch.randn(2, h, 300, nr, generator=g).to(dev)
    d_in = [t.detach().requires_grad_(True) for t in as_proj(dev, torch.float32, dtr, ar, tr, ang)]
    d_bias = bias.float().to(dev).requires_grad_(True)
    runs = []
    for _ in range(3):
        pre, fin = m3.preprocess(*d_in, d_bias)
        dl = sum((getattr(pre, k) * cot[k]).sum() for k in cot) + (pre.phi * cphi).sum()
        runs.append(torch.autograd.grad(dl, d_in + [d_bias]))
    for r in runs[1:]:
        for name, x, y in zip(["dt_raw", "a_raw", "trap_raw", "angles", "dt_bias"], runs[0], r):
            assert torch.equal(x, y), name


def test_prep_backward_with_partial_cotangents(m3, dev):
    """Only some outputs receive a gradient (the others arrive as None)."""
    b, l, h, nr = 1, 96, 4, 8
    dtr, ar, tr, ang, bias = raw_inputs(b, l, h, nr, seed=21)
    leaves = [t.clone().requires_grad_(True) for t in (dtr, ar, tr, ang, bias)]
    ref, _ = O.preprocess(*leaves)
    want = torch.autograd.grad((ref.phi.sin()).sum() + ref.scale.sum(), leaves, allow_unused=True)
    want = [torch.zeros_like(x) if w is None else w for w, x in zip(want, leaves)]  # a_raw: unused
    d_in = [t.detach().requires_grad_(True) for t in as_proj(dev, torch.float32, dtr, ar, tr, ang)]
    d_bias = bias.float().to(dev).requires_grad_(True)
    pre, _ = m3.preprocess(*d_in, d_bias)
    got = torch.autograd.grad((pre.phi.sin()).sum() + pre.scale.sum(), d_in + [d_bias])
    for gv, wv in zip(got, want):
        assert O.rel_error(gv, wv) < 1e-4
        assert O.max_abs(gv, wv) <= 1e-4 * max(1.0, float(wv.abs().max()))


def test_prep_backward_final_phi_only(m3, dev):
    """A loss on the carried phi and on adt only: dphi arrives as None, dphi_final not."""
    b, l, h, nr = 2, 100, 3, 8
    dtr, ar, tr, ang, bias = raw_inputs(b, l, h, nr, seed=31)
    g = torch.Generator().manual_seed(4)
    phi0 = torch.rand(b, h, nr, generator=g, dtype=F64) * 6.0
    leaves = [t.clone().requires_grad_(True) for t in (dtr, ar, tr, ang, bias)]
    p0 = phi0.clone().requires_grad_(True)
    ref, rfin = O.preprocess(*leaves, phi_init=p0)
    want = torch.autograd.grad(rfin.cos().sum() + ref.adt.sum(), leaves + [p0], allow_unused=True)
    want = [torch.zeros_like(x) if w is None else w for w, x in zip(want, leaves + [p0])]
    d_in = [t.detach().requires_grad_(True) for t in as_proj(dev, torch.float32, dtr, ar, tr, ang)]
    d_bias = bias.float().to(dev).requires_grad_(True)
    d_p0 = phi0.float().to(dev).requires_grad_(True)
    pre, fin = m3.preprocess(*d_in, d_bias, phi_init=d_p0)
    got = torch.autograd.grad(fin.cos().sum() + pre.adt.sum(), d_in + [d_bias, d_p0])
    for gv, wv in zip(got, want):
        assert O.max_abs(gv, wv) <= 1e-4 * max(1.0, float(wv.abs().max()))


@pytest.mark.parametrize("b,l,h,nr,init", [(2, 256, 8, 32, True), (1, 1024, 4, 6, False),
                                           (2, 64, 3, 4, True)])
def test_prep_compact_phi_matches_oracle(m3, dev, b, l, h, nr, init):
    """The compact phi (kernels.PhiStrips): the table is tanh(angles) pi, dt is the
    preprocess's dt, and strip s holds the angle entering token 16 s -- the oracle's
    phi at token 16 s - 1, or phi_init for the first strip. Rebuilt per token with the
    same rule the scan kernels use, it reproduces the oracle's phi."""
    dtr, ar, tr, ang, bias = raw_inputs(b, l, h, nr, seed=l + nr + 1)
    g = torch.Generator().manual_seed(4)
    phi0 = (torch.rand(b, h, nr, generator=g, dtype=F64) * 6.0) if init else None
    ref, rfin = O.preprocess(dtr, ar, tr, ang, bias, phi_init=phi0)
    lim, lim_fin = phi_limit(dtr, ar, tr, ang, bias, phi0=phi0)
    d_dt, d_a, d_tr, d_ang = as_proj(dev, torch.float32, dtr, ar, tr, ang)
    out = m3.scan_prep.prep_forward_launch(
        d_dt, d_a, d_tr, d_ang, bias.float().to(dev).contiguous(),
        None if phi0 is None else phi0.float().to(dev).contiguous(), 1e-4, compact=True)
    adt, gamma, scale, lam, dt, ph, fin = out
    assert isinstance(ph, m3.kernels.PhiStrips)
    torch.testing.assert_close(ph.table.cpu().double(), torch.tanh(ang) * torch.pi,
                               rtol=2e-6, atol=2e-6)
    assert ph.dt is dt
    want = torch.zeros(b, h, l // 16, nr, dtype=F64)
    want[:, :, 1:] = ref.phi[:, :, 15:-1:16]
    if phi0 is not None:
        want[:, :, 0] = phi0
    assert O.rel_error(ph.strips.cpu().double(), want, angle=True) <= lim
    assert O.rel_error(fin.cpu().double(), rfin, angle=True) <= lim_fin
    # the per-token rule of the scan kernels
    theta = ph.table.cpu().double()[:, None] * dt.cpu().double()[..., None]   # (B, H, L, Nr)
    within = torch.cumsum(theta.reshape(b, h, l // 16, 16, nr), dim=3).reshape(b, h, l, nr)
    rebuilt = ph.strips.cpu().double().repeat_interleave(16, dim=2) + within
    assert O.rel_error(rebuilt, ref.phi, angle=True) <= lim
    assert O.rel_error(ph.last().cpu().double(), rebuilt[:, :, -1], angle=True, pct=100.0) <= 1e-5
