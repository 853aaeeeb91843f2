"""Single-token decode kernel (m3s_decode) vs the oracle's three-term step, chains of
steps vs one chunked prefill, and the prefill -> decode handoff (tests.py:734-877)."""

import pytest
import torch

from helpers import (BF16, BF16_OUT_MODEL_P95, BF16_P95, F32, FWD_F32_P95, assert_f32, assert_maxrel,
                     assert_p95, cpu)
from oracle import siso_oracle as O

pytestmark = pytest.mark.gpu


def step_inputs(b, h, n, p, nr, policy, seed):
    x = O.make_inputs(b, h, 1, n, p, nr, seed=seed)
    pre, _ = O.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"])
    mt = BF16 if policy == "bf16" else F32
    g = torch.Generator().manual_seed(seed + 5)
    st = O.SISOState(torch.randn(b, h, p, n, generator=g, dtype=torch.float64).float().double() * 0.1,
                     torch.randn(b, h, n, generator=g, dtype=torch.float64).float().double(),
                     torch.randn(b, h, p, generator=g, dtype=torch.float64).float().double(),
                     (torch.rand(b, h, nr, generator=g, dtype=torch.float64) * 6).float().double())
    c = dict(q=x["q"][:, 0].to(mt).double(), k=x["k"][:, 0].to(mt).double(),
             v=x["v"][:, :, 0].to(mt).double(), z=x["z"][:, :, 0].to(mt).double(),
             adt=pre.adt[:, :, 0].float().double(), dt=pre.dt[:, :, 0].float().double(),
             lam=pre.lam[:, :, 0].float().double(), angles=x["angles"][:, 0].float().double(),
             q_bias=x["q_bias"].float().double(), k_bias=x["k_bias"].float().double(),
             d_skip=x["d_skip"].float().double())
    d = {k_: v_.to(mt if k_ in ("q", "k", "v", "z") else F32).cuda() for k_, v_ in c.items()}
    return c, d, st


def step_args(a, st):
    return (a["q"], a["k"], a["v"], a["adt"], a["dt"], a["lam"], a["angles"], a["q_bias"],
            a["k_bias"], st, a["d_skip"], a["z"])


@pytest.mark.parametrize("b,h,n,p,nr", [(2, 3, 128, 64, 32), (1, 4, 16, 16, 4), (3, 2, 64, 64, 16)])
def test_decode_step_f32_matches_oracle_in_place(m3, b, h, n, p, nr):
    c, d, st = step_inputs(b, h, n, p, nr, "f32", seed=1)
    yr, sr = O.siso_step(*step_args(c, st))
    gst = m3.SISOState(*(t.float().cuda() for t in st))
    ptrs = [t.data_ptr() for t in gst]
    y, s2 = m3.decode_step(*step_args(d, gst), dtype_policy="f32")
    assert [t.data_ptr() for t in s2] == ptrs        # donated: updated in place
    assert_f32(y, yr, "out", "y")
    assert_f32(s2.ssm, sr.ssm, "out", "ssm")
    assert_f32(s2.k, sr.k, "out", "k")
    assert O.max_rel(cpu(s2.v), sr.v) == 0.0
    assert O.rel_error(cpu(s2.phi), sr.phi, angle=True) <= 1e-4


def test_decode_step_bf16_matches_rounding_model(m3):
    c, d, st = step_inputs(4, 32, 128, 64, 32, "bf16", seed=2)
    ym, sm = O.siso_step(*step_args(c, st), mm_dtype=BF16)
    y, s2 = m3.decode_step(*step_args(d, m3.SISOState(*(t.float().cuda() for t in st))))
    assert y.dtype == BF16
    assert_p95(y, ym, BF16_OUT_MODEL_P95, "y vs bf16 readout model")
    assert_f32(s2.ssm, sm.ssm, "out", "ssm (f32 update)")


def test_decode_cfg4_batch_one_step(m3):
    """cfg4 sizes: B=256, H=32, P=64, N=128; state ~ N(0, 0.1)."""
    c, d, st = step_inputs(256, 32, 128, 64, 32, "bf16", seed=3)
    ym, sm = O.siso_step(*step_args(c, st), mm_dtype=BF16)
    y, s2 = m3.decode_step(*step_args(d, m3.SISOState(*(t.float().cuda() for t in st))))
    assert_p95(y, ym, BF16_OUT_MODEL_P95, "y")
    assert_maxrel(s2.ssm, sm.ssm, 1e-6, "ssm")


@pytest.mark.parametrize("policy", ["f32", "bf16"])
def test_decode_chain_equals_prefill_and_handoff(m3, policy):
    b, h, L, n, p, nr, chunk = 1, 2, 128, 128, 64, 32, 64
    mt = BF16 if policy == "bf16" else F32
    x = O.make_inputs(b, h, L, n, p, nr, seed=4)
    pre, _ = O.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"])
    g = lambda t, dt=F32: t.to(dt).cuda()  # noqa: E731
    q, k, v, z = g(x["q"], mt), g(x["k"], mt), g(x["v"], mt), g(x["z"], mt)
    adt, dtt, lam = g(pre.adt), g(pre.dt), g(pre.lam)
    qb, kb, dsk, ang = g(x["q_bias"]), g(x["k_bias"]), g(x["d_skip"]), g(x["angles"])
    y_pre, fs, fk, fv = m3.siso_forward(q, k, v, adt, g(pre.gamma), g(pre.scale), g(pre.phi), qb,
                                        kb, dsk, z, chunk=chunk, dtype_policy=policy)
    st = m3.zero_state(b, h, p, n, nr, device="cuda")
    y_dec, st = m3.decode_loop(q, k, v, adt, dtt, lam, ang, qb, kb, st, dsk, z, dtype_policy=policy)
    tol = FWD_F32_P95 if policy == "f32" else BF16_P95   # two rounding paths in bf16
    assert O.rel_error(cpu(y_dec), cpu(y_pre)) <= tol
    assert O.rel_error(cpu(st.ssm), cpu(fs)) <= tol
    assert O.rel_error(cpu(st.k), cpu(fk)) <= FWD_F32_P95
    # prefill the first half with the layer-level segment, decode the rest
    half = L // 2
    out = m3.siso_segment(q[:, :half], k[:, :half], v[:, :, :half], g(x["dt_raw"][:, :half]),
                          g(x["a_raw"][:, :half]), g(x["trap_raw"][:, :half]), ang[:, :half],
                          g(x["dt_bias"]), qb, kb, dsk, z[:, :, :half], chunk=chunk,
                          policy_name=policy)
    pre2, _ = m3.preprocess(g(x["dt_raw"][:, half:]), g(x["a_raw"][:, half:]),
                            g(x["trap_raw"][:, half:]), ang[:, half:], g(x["dt_bias"]),
                            phi_init=out.state.phi)
    carry = m3.SISOState(out.state.ssm.clone(), out.state.k.clone(), out.state.v.clone(),
                         out.state.phi.clone())
    y_b, _ = m3.decode_loop(q[:, half:], k[:, half:], v[:, :, half:], pre2.adt, pre2.dt, pre2.lam,
                            ang[:, half:], qb, kb, carry, dsk, z[:, :, half:], dtype_policy=policy)
    assert O.rel_error(cpu(torch.cat([out.y, y_b], dim=2)), cpu(y_pre)) <= tol


def test_decode_reproduces_reference_torch_golden(m3):
    """Token-by-token decode from a zero state vs upstream's step reference
    (torch_ref.mamba3_siso_ref) for the whole golden sequence."""
    import numpy as np
    from pathlib import Path
    fx = dict(np.load(Path(__file__).resolve().parent / "golden" / "torch_ref_kernel_gated.npz",
                      allow_pickle=False))
    t = {k_: torch.from_numpy(v_).float().cuda() for k_, v_ in fx.items() if v_.dtype != bool and v_.ndim > 0}
    b, L, n = t["q"].shape
    h, p, nr = t["v"].shape[2], t["v"].shape[3], t["angles"].shape[-1]
    perm = O.deinterleave_perm(n).cuda()
    st = m3.zero_state(b, h, p, n, nr, device="cuda")
    lam = torch.sigmoid(t["trap"])
    ys = []
    for tt in range(L):
        y, st = m3.decode_step(t["q"][:, tt][..., perm], t["k"][:, tt][..., perm], t["v"][:, tt],
                               t["adt"][:, :, tt], t["dt"][:, :, tt], lam[:, :, tt], t["angles"][:, tt],
                               t["q_bias"][:, perm], t["k_bias"][:, perm], st, t["d"], t["z"][:, tt],
                               dtype_policy="f32")
        ys.append(y)
    want = torch.from_numpy(fx["out"]).double()
    assert O.max_rel(cpu(torch.stack(ys, 1)), want) <= 2e-5
    assert O.max_rel(cpu(st.ssm), torch.from_numpy(fx["ssm_state"]).double()[..., perm.cpu()]) <= 2e-5
    assert O.rel_error(cpu(st.phi), torch.from_numpy(fx["angle_state"]).double(), angle=True) <= 1e-5


# ---- decode_scan: T steps in one launch --------------------------------------------------

def chain_inputs(b, h, T, n, p, nr, policy, seed):
    """A T-step run (time axis on every input) and a random carried state."""
    x = O.make_inputs(b, h, T, n, p, nr, seed=seed)
    pre, _ = O.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"])
    mt = BF16 if policy == "bf16" else F32
    g = torch.Generator().manual_seed(seed + 7)
    st = O.SISOState(torch.randn(b, h, p, n, generator=g, dtype=torch.float64).float().double() * 0.1,
                     torch.randn(b, h, n, generator=g, dtype=torch.float64).float().double(),
                     torch.randn(b, h, p, generator=g, dtype=torch.float64).float().double(),
                     (torch.rand(b, h, nr, generator=g, dtype=torch.float64) * 6).float().double())
    c = dict(q=x["q"].to(mt).double(), k=x["k"].to(mt).double(), v=x["v"].to(mt).double(),
             z=x["z"].to(mt).double(), adt=pre.adt.float().double(), dt=pre.dt.float().double(),
             lam=pre.lam.float().double(), angles=x["angles"].float().double(),
             q_bias=x["q_bias"].float().double(), k_bias=x["k_bias"].float().double(),
             d_skip=x["d_skip"].float().double())
    d = {k_: v_.to(mt if k_ in ("q", "k", "v", "z") else F32).cuda() for k_, v_ in c.items()}
    return c, d, st


def dev_state(st):
    return O.SISOState(*(t.float().cuda() for t in st))


def assert_same_run(a, b, what):
    (ya, sa), (yb, sb) = a, b
    assert torch.equal(ya, yb), f"{what}: y differs (max |d| {float((ya.float() - yb.float()).abs().max()):.3e})"
    for name, ta, tb in zip(("ssm", "k", "v", "phi"), sa, sb):
        assert torch.equal(ta, tb), f"{what}: {name} differs"


@pytest.mark.parametrize("policy,b,h,T,n,p,nr,gated", [
    ("bf16", 2, 3, 37, 128, 64, 32, True),
    ("bf16", 1, 2, 1, 128, 64, 32, True),
    ("bf16", 2, 2, 2, 128, 64, 32, False),
    ("bf16", 3, 2, 29, 64, 64, 16, True),
    ("bf16", 2, 3, 19, 16, 16, 4, False),
    ("bf16", 1, 2, 23, 256, 64, 64, True),
    ("bf16", 2, 2, 17, 128, 128, 32, True),    # headdim 128: two 64-wide sub-heads
    ("f32", 2, 3, 37, 128, 64, 32, True),
    ("f32", 2, 2, 21, 32, 16, 8, True),
    ("f32", 1, 3, 13, 128, 64, 0, False),      # no rotary angles
])
def test_decode_scan_is_decode_loop_bit_for_bit(m3, policy, b, h, T, n, p, nr, gated):
    """One launch for T steps gives exactly the T-launch chain's y and state."""
    _, d, st = chain_inputs(b, h, T, n, p, nr, policy, seed=11 + T)
    z = d["z"] if gated else None
    dsk = d["d_skip"] if gated else None
    args = (d["q"], d["k"], d["v"], d["adt"], d["dt"], d["lam"], d["angles"], d["q_bias"], d["k_bias"])
    s_loop, s_scan = dev_state(st), dev_state(st)
    ptrs = [t.data_ptr() for t in s_scan]
    ref = m3.decode_loop(*args, s_loop, dsk, z, dtype_policy=policy)
    got = m3.decode_scan(*args, s_scan, dsk, z, dtype_policy=policy)
    assert [t.data_ptr() for t in got[1]] == ptrs     # updated in place
    print(f"[decode_scan] {policy} b={b} h={h} T={T} n={n} p={p} nr={nr}", flush=True)
    assert_same_run(got, ref, f"{policy} T={T}")


@pytest.mark.parametrize("policy", ["f32", "bf16"])
def test_decode_scan_matches_chained_oracle_steps(m3, policy):
    """decode_scan vs T chained O.siso_step (float64; bf16 readout model for bf16)."""
    b, h, T, n, p, nr = 2, 4, 48, 128, 64, 32
    c, d, st = chain_inputs(b, h, T, n, p, nr, policy, seed=21)
    mm = BF16 if policy == "bf16" else None
    s, ys = st, []
    for t in range(T):
        y, s = O.siso_step(c["q"][:, t], c["k"][:, t], c["v"][:, :, t], c["adt"][:, :, t],
                           c["dt"][:, :, t], c["lam"][:, :, t], c["angles"][:, t], c["q_bias"],
                           c["k_bias"], s, c["d_skip"], c["z"][:, :, t], mm_dtype=mm)
        ys.append(y)
    yr = torch.stack(ys, dim=2)
    y, s2 = m3.decode_scan(d["q"], d["k"], d["v"], d["adt"], d["dt"], d["lam"], d["angles"],
                           d["q_bias"], d["k_bias"], dev_state(st), d["d_skip"], d["z"],
                           dtype_policy=policy)
    if policy == "f32":
        assert_f32(y, yr, "out", "y")
        assert_f32(s2.ssm, s.ssm, "out", "ssm")
        assert_f32(s2.k, s.k, "out", "k")
    else:
        assert y.dtype == BF16
        assert_p95(y, yr, BF16_OUT_MODEL_P95, "y vs bf16 readout model")
        assert_maxrel(y, yr, 2e-2, "y vs bf16 readout model (max-normalised)")
        assert_f32(s2.ssm, s.ssm, "out", "ssm (f32 update)")
    assert O.max_rel(cpu(s2.v), s.v) == 0.0
    assert O.rel_error(cpu(s2.phi), s.phi, angle=True) <= 1e-4


def test_decode_scan_golden_chain(m3):
    """The golden sequence (upstream's step reference, torch_ref.mamba3_siso_ref) as one
    decode_scan from a zero state: bit-identical to the step-by-step chain and within the
    f32 bar of the fixture."""
    import numpy as np
    from pathlib import Path
    fx = dict(np.load(Path(__file__).resolve().parent / "golden" / "torch_ref_kernel_gated.npz",
                      allow_pickle=False))
    t = {k_: torch.from_numpy(v_).float().cuda() for k_, v_ in fx.items() if v_.dtype != bool and v_.ndim > 0}
    b, L, n = t["q"].shape
    h, p, nr = t["v"].shape[2], t["v"].shape[3], t["angles"].shape[-1]
    perm = O.deinterleave_perm(n).cuda()
    lam = torch.sigmoid(t["trap"])
    args = (t["q"][..., perm], t["k"][..., perm], t["v"].transpose(1, 2), t["adt"], t["dt"], lam,
            t["angles"], t["q_bias"][:, perm], t["k_bias"][:, perm])
    loop = m3.decode_loop(*args, m3.zero_state(b, h, p, n, nr, device="cuda"), t["d"],
                          t["z"].transpose(1, 2), dtype_policy="f32")
    scan = m3.decode_scan(*args, m3.zero_state(b, h, p, n, nr, device="cuda"), t["d"],
                          t["z"].transpose(1, 2), dtype_policy="f32")
    assert_same_run(scan, loop, "golden chain")
    # the reference's `folded` switch (tests.py:814-824 checks both) selects the same step here
    unfolded = m3.decode_scan(*args, m3.zero_state(b, h, p, n, nr, device="cuda"), t["d"],
                              t["z"].transpose(1, 2), dtype_policy="f32", folded=False)
    assert_same_run(unfolded, loop, "golden chain, folded=False")
    y, st = scan
    want = torch.from_numpy(fx["out"]).double()
    assert O.max_rel(cpu(y.transpose(1, 2)), want) <= 2e-5
    assert O.max_rel(cpu(st.ssm), torch.from_numpy(fx["ssm_state"]).double()[..., perm.cpu()]) <= 2e-5
    assert O.rel_error(cpu(st.phi), torch.from_numpy(fx["angle_state"]).double(), angle=True) <= 1e-5


def test_decode_scan_cfg4_size(m3):
    """cfg4 sizes (B=256, H=32, P=64, N=128, Nr=32), 12 steps in one launch: the chain of
    12 single-step launches bit for bit, and chained float64 steps under the bf16 readout
    model on the first two batch rows."""
    c, d, st = chain_inputs(256, 32, 12, 128, 64, 32, "bf16", seed=31)
    args = (d["q"], d["k"], d["v"], d["adt"], d["dt"], d["lam"], d["angles"], d["q_bias"], d["k_bias"])
    ref = m3.decode_loop(*args, dev_state(st), d["d_skip"], d["z"])
    got = m3.decode_scan(*args, dev_state(st), d["d_skip"], d["z"])
    assert_same_run(got, ref, "cfg4")
    s, ys = O.SISOState(*(t[:2] for t in st)), []
    for t in range(12):
        y, s = O.siso_step(c["q"][:2, t], c["k"][:2, t], c["v"][:2, :, t], c["adt"][:2, :, t],
                           c["dt"][:2, :, t], c["lam"][:2, :, t], c["angles"][:2, t], c["q_bias"],
                           c["k_bias"], s, c["d_skip"], c["z"][:2, :, t], mm_dtype=BF16)
        ys.append(y)
    assert_p95(got[0][:2], torch.stack(ys, dim=2), BF16_OUT_MODEL_P95, "y vs bf16 readout model")
    assert_f32(got[1].ssm[:2], s.ssm, "out", "ssm (f32 update)")


def test_decode_scan_rejects_mismatched_shapes(m3):
    _, d, st = chain_inputs(1, 2, 4, 128, 64, 32, "bf16", seed=41)
    with pytest.raises(ValueError):
        m3.decode_scan(d["q"], d["k"], d["v"][:, :, :3], d["adt"], d["dt"], d["lam"], d["angles"],
                       d["q_bias"], d["k_bias"], dev_state(st))
    with pytest.raises(ValueError):
        m3.decode_scan(d["q"], d["k"], d["v"], d["adt"][:, :, :3], d["dt"], d["lam"], d["angles"],
                       d["q_bias"], d["k_bias"], dev_state(st))


def test_decode_scan_of_no_steps_keeps_the_state(m3):
    """A run of length 0 (``lax.scan`` with ``length=0`` in ``kernel_decode.py:474-533``):
    an empty ``(B, H, 0, P)`` output and the carried state unchanged; then a real run on
    that state still matches the step-by-step chain."""
    _, d, st = chain_inputs(2, 3, 5, 128, 64, 32, "bf16", seed=43)
    cut = {k_: (v_[:, :0] if k_ in ("q", "k", "angles") else
                v_[:, :, :0] if k_ in ("v", "z", "adt", "dt", "lam") else v_) for k_, v_ in d.items()}
    s0 = dev_state(st)
    y, s1 = m3.decode_scan(cut["q"], cut["k"], cut["v"], cut["adt"], cut["dt"], cut["lam"],
                           cut["angles"], cut["q_bias"], cut["k_bias"], s0, d_skip=cut["d_skip"],
                           z=cut["z"])
    assert tuple(y.shape) == (2, 3, 0, 64) and y.dtype == d["v"].dtype
    for name, a, b in zip(("ssm", "k", "v", "phi"), s1, dev_state(st)):
        assert torch.equal(a, b), f"{name} changed by an empty run"
    args = (d["q"], d["k"], d["v"], d["adt"], d["dt"], d["lam"], d["angles"], d["q_bias"], d["k_bias"])
    assert_same_run(m3.decode_scan(*args, s1, d_skip=d["d_skip"], z=d["z"]),
                    m3.kernels.decode_loop(*args, dev_state(st), d_skip=d["d_skip"], z=d["z"]),
                    "after an empty run")
