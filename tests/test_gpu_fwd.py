"""Chunked forward kernel (m3s_fwd) vs the CPU oracle on identical inputs."""

import math

import pytest
import torch

from helpers import (assert_f32, BF16, BF16_MAXREL, BF16_MODEL_P95, BF16_OUT_MODEL_P95, BF16_P95,
                     BF16_Y_MAXREL, F32, FWD_F32_P95, STATE_MAXABS, assert_bf16_bound,
                     assert_maxabs, assert_maxrel, assert_p95, boundary_inputs, cpu, fwd_args,
                     phi_strips_of, report)
from oracle import siso_oracle as O

pytestmark = pytest.mark.gpu


def oracle_fwd(c, chunk, mm=None, with_seed=False):
    kw = {}
    if with_seed:
        st = O.SISOState(c["seed_ssm"], c["seed_k"], c["seed_v"], None)
        kw = dict(state=st, seed_dt=c["seed_coef"], seed_lam=torch.zeros_like(c["seed_coef"]))
    return O.siso_chunked(c["q"], c["k"], c["v"], c["adt"], c["gamma"], c["scale"], c["phi"],
                          c["q_bias"], c["k_bias"], c.get("d_skip"), c.get("z"), chunk=chunk,
                          return_debug=True, mm_dtype=mm, **kw)


@pytest.mark.parametrize("b,h,L,n,p,nr,chunk", [
    (1, 4, 512, 16, 16, 4, 64),      # cfg1 kernel shapes
    (2, 3, 256, 128, 64, 32, 64),
    (1, 2, 128, 128, 64, 32, 32),
    (2, 2, 192, 32, 16, 8, 32),
])
def test_forward_f32_matches_oracle(m3, b, h, L, n, p, nr, chunk):
    """A chunk with no f32 kernel of its own (64 at N=128) runs as 32-token tiles: the
    states saved per tile are the oracle's states at the tile chunk, and every
    (chunk/tile)-th of them the state entering each requested chunk."""
    from mamba3_siso_tpu_amd import layout as LY
    tile = LY.kernel_chunk("f32", chunk, n, p)
    c, d = boundary_inputs(b, h, L, n, p, nr, "f32", seed=1)
    yr, sr, dbg = oracle_fwd(c, chunk)
    y, fs, fk, fv, res = m3.siso_forward(*fwd_args(d), chunk=chunk, dtype_policy="f32",
                                         save_residuals=True)
    assert_f32(y, yr, "out", "y")
    assert_f32(fs, sr.ssm, "out", "final ssm")
    assert_f32(fk, sr.k, "out", "final k")
    assert O.max_rel(cpu(fv), sr.v) == 0.0
    assert_f32(res.ybar, dbg["ybar"], "out", "ybar")
    assert tuple(res.chunk_states.shape) == (b, h, L // tile, p, n)
    assert_f32(res.chunk_states[:, :, ::chunk // tile], dbg["chunk_states"], "out",
               "chunk_states")
    if tile != chunk:
        _, _, dbg_t = oracle_fwd(c, tile)
        assert_f32(res.chunk_states, dbg_t["chunk_states"], "out", "tile states")


@pytest.mark.parametrize("chunk", [128, 64, 32])
def test_forward_bf16_matches_rounding_model_and_maths(m3, chunk):
    c, d = boundary_inputs(2, 3, 256, 128, 64, 32, "bf16", seed=2)
    yr, sr, dbg = oracle_fwd(c, chunk)
    ym, sm, dbgm = oracle_fwd(c, chunk, mm=BF16)
    y, fs, fk, fv, res = m3.siso_forward(*fwd_args(d), chunk=chunk, dtype_policy="bf16",
                                         save_residuals=True)
    assert y.dtype == BF16 and res.chunk_states.dtype == BF16
    # the kernel's own rounding model (reference kernel_fwd.py:133-187)
    assert_p95(res.ybar, dbgm["ybar"], BF16_OUT_MODEL_P95, "ybar vs bf16 model")
    assert_p95(fs, sm.ssm, BF16_MODEL_P95, "ssm vs bf16 model")
    # the float64 maths
    assert_p95(y, yr, BF16_P95, "y")
    assert_maxrel(y, yr, BF16_MAXREL, "y")
    assert_maxrel(fs, sr.ssm, BF16_MAXREL, "final ssm")
    assert_f32(fk, sr.k, "out", "final k (computed in f32)")


@pytest.mark.parametrize("n,chunk,gate", [(64, 64, True), (128, 128, False), (128, 64, False)])
def test_forward_bf16_other_shapes_and_no_gate(m3, n, chunk, gate):
    """The bf16 kernel's other compiled shapes (state_dim 64) and its path without the
    gate z and the skip D, against the rounding model and the float64 maths."""
    c, d = boundary_inputs(2, 3, 256, n, 64, n // 4, "bf16", seed=11)
    if not gate:
        c.pop("d_skip"), c.pop("z"), d.pop("d_skip"), d.pop("z")
    yr, sr, _ = oracle_fwd(c, chunk)
    ym, sm, dbgm = oracle_fwd(c, chunk, mm=BF16)
    y, fs, fk, fv, res = m3.siso_forward(*fwd_args(d), chunk=chunk, dtype_policy="bf16",
                                         save_residuals=True)
    assert_p95(res.ybar, dbgm["ybar"], BF16_OUT_MODEL_P95, "ybar vs bf16 model")
    assert_p95(fs, sm.ssm, BF16_MODEL_P95, "ssm vs bf16 model")
    # chunk states are stored in bf16: one more rounding of up to 2^-8 relative
    assert_p95(res.chunk_states, dbgm["chunk_states"], BF16_OUT_MODEL_P95, "chunk states vs bf16 model")
    assert_maxrel(y, yr, BF16_MAXREL, "y")
    assert_f32(fk, sr.k, "out", "final k")
    assert_f32(fv, sr.v, "out", "final v")


@pytest.mark.parametrize("policy,n,p,chunk", [
    ("bf16", 64, 64, 128), ("bf16", 64, 64, 32), ("bf16", 32, 16, 128), ("bf16", 16, 16, 128),
    ("f32", 64, 64, 32), ("f32", 32, 16, 128), ("f32", 16, 16, 128),
])
def test_forward_every_table_shape(m3, policy, n, p, chunk):
    """Instantiations of the kernel table not covered above, against the oracle."""
    c, d = boundary_inputs(2, 2, 256, n, p, n // 4, policy, seed=17)
    yr, sr, dbg = oracle_fwd(c, chunk)
    y, fs, fk, fv, res = m3.siso_forward(*fwd_args(d), chunk=chunk, dtype_policy=policy,
                                         save_residuals=True)
    if policy == "f32":
        assert_f32(y, yr, "out", "y")
        assert_f32(fs, sr.ssm, "out", "final ssm")
        assert_f32(res.chunk_states, dbg["chunk_states"], "out", "chunk_states")
    else:
        ym, sm, dbgm = oracle_fwd(c, chunk, mm=BF16)
        assert_p95(res.ybar, dbgm["ybar"], BF16_OUT_MODEL_P95, "ybar vs bf16 model")
        assert_p95(fs, sm.ssm, BF16_MODEL_P95, "ssm vs bf16 model")
        assert_maxrel(y, yr, BF16_Y_MAXREL, "y")
        assert_maxabs(fs, sr.ssm, STATE_MAXABS, "final ssm")
    assert_f32(fk, sr.k, "out", "final k")


@pytest.mark.parametrize("policy,n,p,chunk", [
    ("bf16", 128, 64, 128), ("bf16", 128, 64, 64), ("bf16", 64, 64, 64), ("bf16", 32, 16, 32),
    ("f32", 128, 64, 32), ("f32", 16, 16, 64),
])
def test_forward_with_phi_built_in_the_kernel(m3, policy, n, p, chunk):
    """phi_strips mode (the cumulative angle fused into the scan): the kernel rebuilds
    phi from tanh(angles) pi, dt and one angle per 16-token strip. Against the oracle
    with the same bars as when phi is read, and against the phi-reading run of the same
    kernel (the rebuilt phi differs from the read one by float rounding only)."""
    c, d = boundary_inputs(2, 3, 256, n, p, n // 4, policy, seed=23)
    yr, sr, dbg = oracle_fwd(c, chunk)
    args = fwd_args(d)
    base = m3.siso_forward(*args, chunk=chunk, dtype_policy=policy, save_residuals=True)
    args[6] = phi_strips_of(c, m3)
    y, fs, fk, fv, res = m3.siso_forward(*args, chunk=chunk, dtype_policy=policy,
                                         save_residuals=True)
    if policy == "f32":
        assert_f32(y, yr, "out", "y")
        assert_f32(fs, sr.ssm, "out", "final ssm")
        assert_f32(res.chunk_states, dbg["chunk_states"], "out", "chunk_states")
        assert_f32(y, cpu(base[0]), "out", "y vs phi read")
    else:
        ym, sm, dbgm = oracle_fwd(c, chunk, mm=BF16)
        assert_p95(res.ybar, dbgm["ybar"], BF16_OUT_MODEL_P95, "ybar vs bf16 model")
        assert_p95(fs, sm.ssm, BF16_MODEL_P95, "ssm vs bf16 model")
        assert_maxrel(y, yr, BF16_Y_MAXREL, "y")
        assert_maxabs(fs, sr.ssm, STATE_MAXABS, "final ssm")
        assert_p95(res.ybar, cpu(base[4].ybar), BF16_OUT_MODEL_P95, "ybar vs phi read")
    assert_f32(fk, sr.k, "out", "final k")
    assert O.max_rel(cpu(fv), cpu(base[3])) == 0.0


def test_forward_bf16_with_carried_state(m3):
    c, d = boundary_inputs(2, 2, 256, 128, 64, 32, "bf16", seed=13, seeds=True)
    yr, sr, _ = oracle_fwd(c, 128, with_seed=True)
    ym, sm, dbgm = oracle_fwd(c, 128, with_seed=True, mm=BF16)
    y, fs, fk, fv, res = m3.siso_forward(*fwd_args(d), chunk=128, dtype_policy="bf16",
                                         save_residuals=True)
    assert_p95(res.ybar, dbgm["ybar"], BF16_OUT_MODEL_P95, "ybar vs bf16 model (seeded)")
    assert_p95(fs, sm.ssm, BF16_MODEL_P95, "ssm vs bf16 model (seeded)")
    assert_maxrel(y, yr, BF16_MAXREL, "y (seeded)")


def test_forward_with_carried_state(m3):
    c, d = boundary_inputs(2, 2, 128, 128, 64, 32, "f32", seed=3, seeds=True)
    yr, sr, _ = oracle_fwd(c, 64, with_seed=True)
    y, fs, fk, fv = m3.siso_forward(*fwd_args(d), chunk=64, dtype_policy="f32")
    assert_f32(y, yr, "out", "y (seeded)")
    assert_f32(fs, sr.ssm, "out", "ssm (seeded)")


def test_forward_no_gate_no_skip(m3):
    c, d = boundary_inputs(1, 3, 128, 32, 16, 8, "f32", seed=4)
    c.pop("d_skip"), c.pop("z"), d.pop("d_skip"), d.pop("z")
    yr, sr, _ = oracle_fwd(c, 32)
    y, fs, _, _ = m3.siso_forward(*fwd_args(d), chunk=32, dtype_policy="f32")
    assert_f32(y, yr, "out", "y plain")


def test_forward_reads_strided_views_in_place(m3):
    """v/z as (B, L, H, P)-buffer views (the layer's layout) give bit-identical results
    to contiguous (B, H, L, P) copies, and y comes back in v's layout."""
    c, d = boundary_inputs(2, 4, 256, 128, 64, 32, "bf16", seed=5)
    vb = d["v"].permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    zb = d["z"].permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    a = fwd_args(d)
    y0, s0, _, _ = m3.siso_forward(*a, chunk=128)
    a[2], a[10] = vb, zb
    y1, s1, _, _ = m3.siso_forward(*a, chunk=128)
    assert y1.stride(2) > y1.stride(1)          # time-major like v
    assert torch.equal(y0, y1) and torch.equal(s0, s1)


@pytest.mark.parametrize("policy", ["f32", "bf16"])
def test_rotation_parity_known_answer(m3, policy):
    """tests.py:451-513 on the kernel: y_t = (-1)^(running parity) exactly in sign."""
    b, h, L, n, p, nr = 2, 1, 256, 128, 64, 32
    g = torch.Generator().manual_seed(0)
    bits = (torch.rand(b, L, generator=g) < 0.5).double()
    bits[:, 0] = 0
    parity = torch.cumsum(bits, 1) % 2
    atanh_one = math.atanh(1 - 1e-6)
    angles = torch.where(bits[:, :, None] > 0.5, atanh_one, 0.0) * torch.ones(1, 1, nr, dtype=torch.float64)
    dt = torch.ones(b, h, L, dtype=torch.float64)
    lam = torch.ones(b, h, L, dtype=torch.float64)
    adt = torch.full((b, h, L), -1e-6, dtype=torch.float64)
    gamma, scale = O.trapezoid_coeffs(dt, lam)
    phi, _ = O.cumulative_angles(angles[:, None].expand(b, h, L, nr), dt)
    q = torch.zeros(b, L, n, dtype=torch.float64)
    q[..., 0] = 1
    k = torch.zeros(b, L, n, dtype=torch.float64)
    k[:, 0, 0] = 1
    v = torch.ones(b, h, L, p, dtype=torch.float64)
    zb = torch.zeros(h, n)
    mt = BF16 if policy == "bf16" else F32
    y, _, _, _ = m3.siso_forward(q.to(mt).cuda(), k.to(mt).cuda(), v.to(mt).cuda(), adt.float().cuda(),
                                 gamma.float().cuda(), scale.float().cuda(), phi.float().cuda(),
                                 zb.cuda(), zb.cuda(), chunk=64, dtype_policy=policy)
    want = torch.where(parity[:, None, :, None] > 0.5, -1.0, 1.0).expand(b, h, L, p)
    yc = y.float().cpu().double()
    assert torch.equal(torch.sign(yc), want)
    assert float((yc - want).abs().max()) <= (1e-2 if policy == "bf16" else 1e-3)


def test_forward_full_size_cfg2_against_head_slices(m3):
    """cfg2 shapes (B=8, L=8192, H=32, N=128, P=64, bf16, chunk 128). The oracle checks
    a slice of heads exactly (heads are independent given the shared q/k); chunk 64 vs
    128 and finiteness cover the rest."""
    torch.manual_seed(0)
    B, L, H, N, P, Nr = 8, 8192, 32, 128, 64, 32
    g = torch.Generator(device="cuda").manual_seed(11)

    def rn(*s):
        return torch.randn(*s, generator=g, device="cuda")

    def norm_rows(t):
        return t * torch.rsqrt(t.square().mean(-1, keepdim=True) + 1e-6)

    q = norm_rows(rn(B, L, N)).to(BF16)
    k = norm_rows(rn(B, L, N)).to(BF16)
    v = rn(B, H, L, P).to(BF16)
    z = rn(B, H, L, P).to(BF16)
    dt_raw = torch.log(torch.expm1(torch.exp(torch.rand(B, L, H, generator=g, device="cuda")
                                             * (math.log(0.1) - math.log(0.001)) + math.log(0.001))))
    a_raw, trap_raw, ang = rn(B, L, H), rn(B, L, H), 0.5 * rn(B, L, Nr)
    pre, _ = m3.preprocess(dt_raw, a_raw, trap_raw, ang, torch.zeros(H, device="cuda"))
    qb, kb, dsk = 0.1 * rn(H, N), 0.1 * rn(H, N), rn(H)
    args = [q, k, v, pre.adt, pre.gamma, pre.scale, pre.phi, qb, kb, dsk, z]
    y, fs, fk, fv = m3.siso_forward(*args, chunk=128)
    y64, fs64, _, _ = m3.siso_forward(*args, chunk=64)
    assert bool(torch.isfinite(y.float()).all()) and bool(torch.isfinite(fs).all())
    assert O.rel_error(y64.float().cpu()[::3], y.float().cpu()[::3]) <= BF16_P95
    assert O.max_rel(fs64.cpu(), fs.cpu()) <= BF16_MAXREL
    # the headline forward's kernel: phi built from the compact form at full length, against
    # the phi-reading run (they differ by the float rounding of phi only) and the oracle
    # slices below
    compact = m3.scan_prep.prep_forward_launch(dt_raw, a_raw, trap_raw, ang,
                                               torch.zeros(H, device="cuda"), None, 1e-4,
                                               compact=True)[5]
    yc, fsc, fkc, fvc = m3.siso_forward(*args[:6], compact, *args[7:], chunk=128)
    report("cfg2 y, phi built vs read", yc, y.double())
    assert O.rel_error(yc.float().cpu()[::2], y.float().cpu()[::2]) <= BF16_MODEL_P95
    assert O.max_rel(fsc.cpu(), fs.cpu()) <= 1e-3
    assert O.max_rel(fkc.cpu(), fk.cpu()) <= 1e-4 and torch.equal(fvc, fv)
    for b_, hs in ((0, [0, 31]), (7, [5, 17])):
        sl = lambda t: t[b_:b_ + 1, hs].double().cpu()  # noqa: E731
        args_cpu = (q[b_:b_ + 1].double().cpu(), k[b_:b_ + 1].double().cpu(), sl(v),
                    sl(pre.adt), sl(pre.gamma), sl(pre.scale), sl(pre.phi),
                    qb[hs].double().cpu(), kb[hs].double().cpu(), dsk[hs].double().cpu(), sl(z))
        ym, sm = O.siso_chunked(*args_cpu, chunk=128, mm_dtype=BF16)
        yr, sr = O.siso_chunked(*args_cpu, chunk=128)
        tag = f"b={b_} heads={hs}"
        report(f"cfg2 y {tag} vs float64", y[b_:b_ + 1, hs], yr)
        report(f"cfg2 final ssm {tag} vs float64", fs[b_:b_ + 1, hs], sr.ssm)
        # the kernel's own rounding points
        assert_p95(y[b_:b_ + 1, hs], ym, BF16_OUT_MODEL_P95, f"y {tag} vs bf16 model")
        assert_bf16_bound(y[b_:b_ + 1, hs], ym, what=f"y {tag} vs bf16 model")
        assert_maxrel(fs[b_:b_ + 1, hs], sm.ssm, BF16_MODEL_P95, f"ssm {tag} vs bf16 model")
        # the float64 maths: north_star's max-abs bound on the float32 final state, the
        # reference's bf16 p95 bar on y (tests.py:533)
        assert_maxabs(fs[b_:b_ + 1, hs], sr.ssm, STATE_MAXABS, f"final ssm {tag}")
        assert_maxabs(fk[b_:b_ + 1, hs], sr.k, 1e-4, f"final k {tag}")
        assert_maxrel(y[b_:b_ + 1, hs], yr, BF16_Y_MAXREL, f"y {tag}")
        assert_p95(y[b_:b_ + 1, hs], yr, BF16_P95, f"y {tag}")
        assert_bf16_bound(yc[b_:b_ + 1, hs], ym, what=f"y {tag} (phi built) vs bf16 model")
        assert_maxabs(fsc[b_:b_ + 1, hs], sr.ssm, STATE_MAXABS, f"final ssm {tag} (phi built)")
        assert_maxrel(yc[b_:b_ + 1, hs], yr, BF16_Y_MAXREL, f"y {tag} (phi built)")


def _golden(name):
    import numpy as np
    from pathlib import Path
    fx = dict(np.load(Path(__file__).resolve().parent / "golden" / f"{name}.npz", allow_pickle=False))
    t = {k_: torch.from_numpy(v_).double() for k_, v_ in fx.items() if v_.dtype != bool and v_.ndim > 0}
    return fx, t


@pytest.mark.parametrize("name", ["torch_ref_kernel_gated", "torch_ref_kernel_plain"])
def test_forward_reproduces_reference_torch_golden(m3, name):
    """The reference's own upstream step reference (torch_ref.mamba3_siso_ref, interleaved
    layout) vs the HIP chunked forward, through the de-interleave permutation."""
    fx, t = _golden(name)
    b, L, n = t["q"].shape
    h, nr = t["v"].shape[2], t["angles"].shape[-1]
    perm = O.deinterleave_perm(n)
    phi, _ = O.cumulative_angles(t["angles"][:, None].expand(b, h, L, nr), t["dt"])
    gamma, scale = O.trapezoid_coeffs(t["dt"], torch.sigmoid(t["trap"]))
    with_dz = bool(fx["with_dz"])
    g = lambda x: x.float().cuda()  # noqa: E731
    y, fs, fk, fv = m3.siso_forward(
        g(t["q"][..., perm]), g(t["k"][..., perm]), g(t["v"].permute(0, 2, 1, 3)), g(t["adt"]),
        g(gamma), g(scale), g(phi), g(t["q_bias"][:, perm]), g(t["k_bias"][:, perm]),
        g(t["d"]) if with_dz else None, g(t["z"].permute(0, 2, 1, 3)) if with_dz else None,
        chunk=32, dtype_policy="f32")
    assert O.max_rel(cpu(y), t["out"].permute(0, 2, 1, 3)) <= 2e-5
    assert O.max_rel(cpu(fs), t["ssm_state"][..., perm]) <= 2e-5
    assert O.max_rel(cpu(fk), t["k_state"][..., perm]) <= 2e-5
    assert O.max_rel(cpu(fv), t["v_state"]) == 0.0
