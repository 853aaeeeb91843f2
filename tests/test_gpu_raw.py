"""Raw mode of the forward (the preprocess inside the BCNorm and scan launches): the rotary
table and theta strip totals that ``m3s_norm_fwd`` writes, and ``m3s_fwd`` reading the
projection's raw dt / a / trap slices and carrying phi itself -- against the float64 oracle
(`siso_segment` on the same raw slices, ``siso.py:154-216`` with ``reference.py:160-199``)
and against the same scan fed by the preprocess launches."""

import math

import pytest
import torch

from helpers import (BF16, BF16_MODEL_P95, BF16_OUT_MODEL_P95, BF16_Y_MAXREL, F32, F64,
                     STATE_MAXABS, assert_bf16_bound, assert_f32, assert_maxabs, assert_maxrel,
                     assert_p95, cpu, report)
from oracle import siso_oracle as O

pytestmark = pytest.mark.gpu


def raw_case(b, h, L, n, p, nr, seed, gate=True, phi_init=False, scale_dt=1.0, mt=BF16):
    """Seeded raw inputs, rounded to the operand dtype ``mt`` where the kernels read it:
    the dt / a / trap slices live in one (B, L, 3H + 8) buffer (as in the projection), the
    angles in a (B, L, Nr + 8) one; q and k are BCNorm outputs of random rows (the launch
    under test writes them with the angle outputs). Returns (cpu float64 dict, device
    dict)."""
    x = O.make_inputs(b, h, L, n, p, nr, seed=seed)
    g = torch.Generator().manual_seed(seed + 5)
    bias = torch.randn(h, generator=g, dtype=F64).float().double() * 0.5
    sc = torch.zeros(b, L, 3 * h + 8, dtype=F64)
    sc[..., :h] = x["dt_raw"] + math.log(scale_dt) - bias
    sc[..., h:2 * h] = x["a_raw"]
    sc[..., 2 * h:3 * h] = x["trap_raw"]
    sc = sc.to(mt)
    ang = torch.zeros(b, L, nr + 8, dtype=F64)
    ang[..., :nr] = x["angles"] * 2.0
    ang = ang.to(mt)
    wb = (torch.rand(n, generator=g, dtype=F64) + 0.5).float()
    wc = (torch.rand(n, generator=g, dtype=F64) + 0.5).float()
    kr = torch.randn(b, L, n, generator=g).to(mt)
    qr = torch.randn(b, L, n, generator=g).to(mt)
    dev = dict(sc=sc.cuda(), ang=ang.cuda(), bias=bias.float().cuda(), wb=wb.cuda(),
               wc=wc.cuda(), kr=kr.cuda(), qr=qr.cuda(),
               v=x["v"].to(mt).cuda(), z=x["z"].to(mt).cuda() if gate else None,
               qb=x["q_bias"].float().cuda(), kb=x["k_bias"].float().cuda(),
               d=x["d_skip"].float().cuda() if gate else None)
    if phi_init:
        dev["phi_init"] = (torch.rand(b, h, nr, generator=g) * 6.2).cuda()
    scd = sc.double()
    c = dict(dt_raw=scd[..., :h], a_raw=scd[..., h:2 * h], trap_raw=scd[..., 2 * h:3 * h],
             angles=ang.double()[..., :nr], bias=bias, v=x["v"].to(mt).double(),
             z=x["z"].to(mt).double() if gate else None, qb=x["q_bias"].float().double(),
             kb=x["k_bias"].float().double(), d=x["d_skip"].float().double() if gate else None,
             phi_init=dev["phi_init"].double().cpu() if phi_init else None)
    return c, dev


def views(dev, h, nr):
    sc = dev["sc"]
    return sc[..., :h], sc[..., h:2 * h], sc[..., 2 * h:3 * h], dev["ang"][..., :nr]


def run_raw(m3, dev, h, nr, chunk, a_floor=1e-4, policy="bf16"):
    K = m3.kernels
    dtr, ar, trr, ang = views(dev, h, nr)
    (k, q), _, angs = K.bcnorm_forward([dev["kr"], dev["qr"]], [dev["wb"], dev["wc"]], 1e-5,
                                       theta=(ang, dtr, dev["bias"], chunk))
    out = K.siso_forward_raw(q, k, dev["v"], dtr, ar, trr, angs, dev["bias"], dev["qb"],
                             dev["kb"], d_skip=dev["d"], z=dev["z"],
                             phi_init=dev.get("phi_init"), a_floor=a_floor, chunk=chunk,
                             dtype_policy=policy)
    return q, k, angs, out


def oracle(c, q, k, chunk, mm=None):
    st = None
    if c["phi_init"] is not None:
        b, h, nr = c["phi_init"].shape
        n, p = q.shape[-1], c["v"].shape[-1]
        st = O.SISOState(torch.zeros(b, h, p, n, dtype=F64), torch.zeros(b, h, n, dtype=F64),
                         torch.zeros(b, h, p, dtype=F64), c["phi_init"])
    return O.siso_segment(cpu(q), cpu(k), c["v"], c["dt_raw"], c["a_raw"], c["trap_raw"],
                          c["angles"], c["bias"], c["qb"], c["kb"], d_skip=c["d"], z=c["z"],
                          state=st, chunk=chunk, mm_dtype=mm)


@pytest.mark.parametrize("chunk", [16, 48])
def test_bcnorm_theta_outputs_match_float64(m3, chunk):
    """The angle role of m3s_norm_fwd: table = tanh(angles) pi within f32 rounding; with
    the float64 strip sums S of table * softplus(dt_raw + dt_bias), each strip's prefix
    within its chunk and each chunk's total within 1e-5 of their max |ref|; the norms it
    shares the launch with are bit-identical to a launch without it. Chunks of 1 and 3
    strips (ragged to the 256-thread blocks) and H, Nr not powers of two."""
    b, h, L, n, nr = 2, 6, 96, 64, 12
    c, dev = raw_case(b, h, L, n, 64, nr, seed=3)
    K = m3.kernels
    dtr, _, _, ang = views(dev, h, nr)
    (k, q), rs, angs = K.bcnorm_forward([dev["kr"], dev["qr"]], [dev["wb"], dev["wc"]], 1e-5,
                                        theta=(ang, dtr, dev["bias"], chunk))
    (k0, q0), rs0 = K.bcnorm_forward([dev["kr"], dev["qr"]], [dev["wb"], dev["wc"]], 1e-5)
    assert torch.equal(k, k0) and torch.equal(q, q0) and torch.equal(rs[0], rs0[0])
    tab = torch.tanh(c["angles"]) * math.pi
    assert_maxabs(angs.table, tab, 4e-6, "theta table")
    dt = torch.nn.functional.softplus(c["dt_raw"] + c["bias"])            # (B, L, H)
    theta = tab[:, :, None, :] * dt[..., None]                            # (B, L, H, Nr)
    strips = theta.unflatten(1, (L // 16, 16)).sum(2).permute(0, 2, 1, 3)   # (B, H, L/16, Nr)
    per = strips.unflatten(2, (L // chunk, chunk // 16))                      # (B, H, nc, s, Nr)
    prefix = (per.cumsum(3) - per).flatten(2, 3)
    assert_maxrel(angs.prefix, prefix, 1e-5, "strip prefixes")
    assert_maxrel(angs.chunk_totals, per.sum(3), 1e-5, "chunk totals")


@pytest.mark.parametrize("chunk,n,nr,gate,phi_init", [
    (128, 128, 32, True, False),    # the headline shape
    (128, 128, 32, False, True),    # no gate / skip, a carried phi_init
    (64, 128, 32, True, True),      # 4 strips per chunk
    (128, 64, 16, True, False),     # state_dim 64
    (64, 64, 32, True, False),      # rope_fraction 1.0 at state_dim 64
])
def test_raw_forward_matches_oracle(m3, chunk, n, nr, gate, phi_init):
    """Raw-mode forward vs `siso_segment` on the same raw slices (float64): y against the
    bf16 rounding model (p95, and the elementwise bf16 bound) and the float64 maths, the
    final state to north_star's max-abs bound, the final k (f32 maths) and phi (the carried
    angle) tightly, the final v exactly."""
    b, h, L = 2, 3, 512
    c, dev = raw_case(b, h, L, n, 64, nr, seed=7 + chunk + n, gate=gate, phi_init=phi_init)
    if not m3.kernels.raw_forward_ok("bf16", chunk, n, 64, nr, L, h):
        pytest.skip("no raw-mode kernel for this shape")
    q, k, angs, (y, fs, fk, fv, phi_f) = run_raw(m3, dev, h, nr, chunk)
    yr, sr = oracle(c, q, k, chunk)
    ym, sm = oracle(c, q, k, chunk, mm=BF16)
    report(f"raw y (C {chunk}, N {n}) vs float64", y, yr)
    assert_p95(y, ym, BF16_OUT_MODEL_P95, "y vs bf16 model")
    assert_bf16_bound(y, ym, what="y vs bf16 model")
    assert_maxrel(y, yr, BF16_Y_MAXREL, "y")
    assert_maxabs(fs, sr.ssm, STATE_MAXABS, "final ssm")
    assert_maxrel(fs, sm.ssm, BF16_MODEL_P95, "final ssm vs bf16 model")
    assert_maxabs(fk, sr.k, 1e-4, "final k")
    assert torch.equal(fv.cpu(), sr.v.float())
    assert O.rel_error(cpu(phi_f), sr.phi, angle=True, pct=100.0) <= 2e-5


@pytest.mark.parametrize("policy,chunk,n,p,nr,phi_init", [
    ("f32", 64, 16, 16, 4, False),     # BASELINE configs[0]'s layer shapes
    ("f32", 32, 128, 64, 32, True),    # f32 at the headline's state and head widths
    ("bf16", 32, 32, 16, 8, True),     # bf16 shapes the generic kernel runs
    ("bf16", 128, 16, 16, 4, False),
])
def test_raw_forward_generic_kernel_matches_oracle(m3, policy, chunk, n, p, nr, phi_init):
    """Raw mode in the generic kernel (the f32 policy and the small bf16 shapes): the f32
    policy to its two float64 bars (p95 2e-5 and 1e-4 of max |ref| on y and the final state;
    phi within 1e-5), the bf16 shapes to the bf16 bars."""
    b, h, L = 2, 3, 256
    mt = F32 if policy == "f32" else BF16
    c, dev = raw_case(b, h, L, n, p, nr, seed=43 + n + p, phi_init=phi_init, mt=mt)
    assert m3.kernels.raw_forward_ok(policy, chunk, n, p, nr, L, h)
    q, k, angs, (y, fs, fk, fv, phi_f) = run_raw(m3, dev, h, nr, chunk, policy=policy)
    yr, sr = oracle(c, q, k, chunk)
    report(f"raw y ({policy}, C {chunk}, N {n}, P {p}) vs float64", y, yr)
    if policy == "f32":
        assert_f32(y, yr, "out", "y")
        assert_f32(fs, sr.ssm, "out", "final ssm")
        assert_f32(fk, sr.k, "out", "final k")
        assert O.rel_error(cpu(phi_f), sr.phi, angle=True, pct=100.0) <= 1e-5
    else:
        assert_maxrel(y, yr, BF16_Y_MAXREL, "y")
        assert_maxabs(fs, sr.ssm, STATE_MAXABS, "final ssm")
        assert_maxabs(fk, sr.k, 1e-4, "final k")
        assert O.rel_error(cpu(phi_f), sr.phi, angle=True, pct=100.0) <= 2e-5
    assert torch.equal(fv.cpu(), sr.v.float())


def test_raw_forward_equals_the_preprocess_path(m3):
    """The same scan fed by the preprocess launches (compact phi): the row scalars and the
    angle table agree to float rounding (library functions there, hardware exp2 / log2 /
    rcp here), and the phi carry differs in its summation order; the outputs agree far
    inside the bf16 bars."""
    b, h, L, n, nr, chunk = 2, 4, 1024, 128, 32, 128
    c, dev = raw_case(b, h, L, n, 64, nr, seed=21, scale_dt=3.0)
    q, k, angs, (y, fs, fk, fv, phi_f) = run_raw(m3, dev, h, nr, chunk)
    dtr, ar, trr, ang = views(dev, h, nr)
    adt, gam, scl, _, _, phi, phi_f2 = m3.scan_prep.prep_forward_launch(
        dtr, ar, trr, ang, dev["bias"], None, 1e-4, compact=True)
    y2, fs2, fk2, fv2 = m3.siso_forward(q, k, dev["v"], adt, gam, scl, phi, dev["qb"], dev["kb"],
                                        d_skip=dev["d"], z=dev["z"], chunk=chunk)
    # the BCNorm call's table comes from the hardware exp2 / rcp, the preprocess's from the
    # library tanh
    assert O.max_abs(angs.table.cpu(), phi.table.cpu()) <= 1e-6
    report("raw y vs preprocess path", y, cpu(y2))
    assert O.rel_error(cpu(y), cpu(y2)) <= 1e-3
    assert O.max_rel(cpu(y), cpu(y2)) <= 4e-3
    assert O.max_rel(cpu(fs), cpu(fs2)) <= 1e-3
    assert O.max_abs(cpu(fk), cpu(fk2)) <= 1e-4 and torch.equal(fv, fv2)
    assert O.rel_error(cpu(phi_f), cpu(phi_f2), angle=True, pct=100.0) <= 1e-5


def test_raw_forward_rejects_slices_of_different_buffers(m3):
    """The raw slices must be views of one projection row layout: a_raw taken from another
    buffer is refused with the ABI's error, before any launch."""
    b, h, L, n, nr = 1, 2, 128, 128, 32
    c, dev = raw_case(b, h, L, n, 64, nr, seed=2)
    K = m3.kernels
    dtr, ar, trr, ang = views(dev, h, nr)
    (k, q), _, angs = K.bcnorm_forward([dev["kr"], dev["qr"]], [dev["wb"], dev["wc"]], 1e-5,
                                       theta=(ang, dtr, dev["bias"], 128))
    other = ar.clone()
    with pytest.raises(ValueError, match="raw slices|fixed number"):
        K.siso_forward_raw(q, k, dev["v"], dtr, other, trr, angs, dev["bias"], dev["qb"],
                           dev["kb"], chunk=128)


def test_raw_forward_full_size_cfg2(m3):
    """BASELINE configs[1]'s scan at full size (B=8, L=8192, H=32, N=128, P=64, chunk 128)
    in raw mode: against the preprocess-fed scan everywhere (equal row scalars, phi carried
    in another summation order), and against the float64 oracle on two head slices --
    y to the bf16 bound, the final state to north_star's 2e-2 max-abs, phi at the last
    position (8192 steps of carry) within 2e-5 rad."""
    B, L, H, N, P, Nr = 8, 8192, 32, 128, 64, 32
    g = torch.Generator().manual_seed(31)
    dt = torch.exp(torch.rand(B, L, H, generator=g) * (math.log(0.1) - math.log(0.001))
                   + math.log(0.001))
    bias = (torch.randn(H, generator=g) * 0.3).float()
    sc = torch.zeros(B, L, 3 * H + 8)
    sc[..., :H] = torch.log(torch.expm1(dt)) - bias
    sc[..., H:2 * H] = torch.randn(B, L, H, generator=g)
    sc[..., 2 * H:3 * H] = torch.randn(B, L, H, generator=g)
    sc = sc.to(BF16).cuda()
    ang = (torch.randn(B, L, Nr, generator=g) * 0.5).to(BF16).cuda()
    kr, qr = (torch.randn(B, L, N, generator=g).to(BF16).cuda() for _ in range(2))
    ones = torch.ones(N, device="cuda")
    gd = torch.Generator(device="cuda").manual_seed(32)
    v = torch.randn(B, H, L, P, generator=gd, device="cuda").to(BF16)
    z = torch.randn(B, H, L, P, generator=gd, device="cuda").to(BF16)
    qb, kb = (0.1 * torch.randn(H, N, generator=gd, device="cuda") for _ in range(2))
    dsk = torch.randn(H, generator=gd, device="cuda")
    bias_d = bias.cuda()
    dtr, ar, trr = sc[..., :H], sc[..., H:2 * H], sc[..., 2 * H:3 * H]
    K = m3.kernels
    (k, q), _, angs = K.bcnorm_forward([kr, qr], [ones, ones], 1e-5,
                                       theta=(ang, dtr, bias_d, 128))
    y, fs, fk, fv, phi_f = K.siso_forward_raw(q, k, v, dtr, ar, trr, angs, bias_d, qb, kb,
                                              d_skip=dsk, z=z, chunk=128)
    adt, gam, scl, _, _, phi, phi_f2 = m3.scan_prep.prep_forward_launch(
        dtr, ar, trr, ang, bias_d, None, 1e-4, compact=True)
    y2, fs2, fk2, fv2 = m3.siso_forward(q, k, v, adt, gam, scl, phi, qb, kb, d_skip=dsk, z=z,
                                        chunk=128)
    assert bool(torch.isfinite(y.float()).all()) and bool(torch.isfinite(fs).all())
    assert O.rel_error(y.float().cpu()[::2], y2.float().cpu()[::2]) <= BF16_MODEL_P95
    # 8192 steps of bf16 k-hat operands: a phi that differs in its last bits flips some
    # of their roundings (measured 1.9e-3 of max |S|); the oracle slices below are the bar
    report("raw cfg2 final ssm vs preprocess path", fs, fs2.double())
    assert O.max_rel(fs.cpu(), fs2.cpu()) <= 5e-3 and torch.equal(fv, fv2)
    assert O.rel_error(phi_f.cpu(), phi_f2.cpu(), angle=True, pct=100.0) <= 2e-5
    scd = sc.double().cpu()
    for b_, hs in ((0, [0, 31]), (7, [5, 17])):
        sl = lambda t: t[b_:b_ + 1, hs].double().cpu()  # noqa: E731
        raw = [scd[b_:b_ + 1, :, off:off + H][..., hs] for off in (0, H, 2 * H)]
        args = (q[b_:b_ + 1].double().cpu(), k[b_:b_ + 1].double().cpu(), sl(v), *raw,
                ang[b_:b_ + 1].double().cpu(), bias[hs].double(), qb[hs].double().cpu(),
                kb[hs].double().cpu())
        kw = dict(d_skip=dsk[hs].double().cpu(), z=sl(z), chunk=128)
        ym, sm = O.siso_segment(*args, mm_dtype=BF16, **kw)
        yr, sr = O.siso_segment(*args, **kw)
        tag = f"b={b_} heads={hs}"
        report(f"raw cfg2 y {tag} vs float64", y[b_:b_ + 1, hs], yr)
        assert_bf16_bound(y[b_:b_ + 1, hs], ym, what=f"y {tag} vs bf16 model")
        assert_maxrel(y[b_:b_ + 1, hs], yr, BF16_Y_MAXREL, f"y {tag}")
        assert_maxabs(fs[b_:b_ + 1, hs], sr.ssm, STATE_MAXABS, f"final ssm {tag}")
        assert_maxabs(fk[b_:b_ + 1, hs], sr.k, 1e-4, f"final k {tag}")
        assert O.rel_error(phi_f[b_:b_ + 1, hs].cpu(), sr.phi, angle=True, pct=100.0) <= 2e-5
