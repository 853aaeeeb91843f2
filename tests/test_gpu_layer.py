"""The layer on the GPU: BASELINE config 1 end to end (forward, final state, every
gradient), the reference's torch layer via convert, segmented prefill, bf16 layer
parity and the layer-level decode step -- all against the CPU oracle."""

from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import (assert_f32, BF16, BF16_GRAD_MAXREL, BF16_LAYER_MODEL_P95, BF16_MAXREL, BF16_Y_MAXREL,
                     GRAD_F32_P95, STATE_MAXABS, assert_bf16_bound, assert_maxabs,
                     assert_maxrel, assert_p95, cpu, report)
from oracle import siso_oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def params_dict(params, dtype=torch.float64):
    return {f: getattr(params, f).detach().cpu().to(dtype) for f in params._fields}


def cfg1(m3):
    return m3.SISOConfig(d_model=64, d_state=16, headdim=16, expand=1, chunk=64, policy_name="f32")


def test_cfg1_forward_state_and_all_gradients(m3):
    """B=1, L=512, d_model=64, H=4, P=16, N=16, chunk 64, fp32;
    params from init_params(seed=0); u ~ N(0,1) (seed 0); loss sum(y * g), g ~ N(0,1)
    (seed 1). Checks y, the final state and the gradients of u and all 8 params."""
    cfg = cfg1(m3)
    p_cpu = m3.init_params(cfg, 0)
    u = torch.randn(1, 512, 64, generator=torch.Generator().manual_seed(0))
    gy = torch.randn(1, 512, 64, generator=torch.Generator().manual_seed(1))
    # device run
    params = m3.SISOParams(*(t.cuda().requires_grad_(True) for t in p_cpu))
    ud = u.cuda().requires_grad_(True)
    y, st = m3.mamba3_siso_layer(params, ud, cfg)
    (y * gy.cuda()).sum().backward()
    # oracle run (float64, autograd)
    pd = {k_: v_.requires_grad_(True) for k_, v_ in params_dict(p_cpu).items()}
    uo = u.double().requires_grad_(True)
    yr, sr = O.layer_forward(pd, uo, d_state=16, headdim=16, expand=1, chunk=64)
    (yr * gy.double()).sum().backward()
    assert_f32(y, yr.detach(), "out", "y")
    assert_f32(st.ssm, sr.ssm.detach(), "out", "final ssm")
    assert_f32(st.k, sr.k.detach(), "out", "final k")
    assert O.rel_error(cpu(st.phi), sr.phi.detach(), angle=True) <= 1e-5
    assert_f32(ud.grad, uo.grad, "grad", "du")
    for f in p_cpu._fields:
        assert_f32(getattr(params, f).grad, pd[f].grad, "grad", f"d{f}")


@pytest.mark.parametrize("name", ["torch_ref_layer_half", "torch_ref_layer_full"])
def test_reference_torch_layer_via_convert_on_gpu(m3, name):
    fx = dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))
    sd = {k[4:].replace("__", "."): torch.from_numpy(v) for k, v in fx.items() if k.startswith("sd__")}
    d_model, n, p, expand = (int(v) for v in fx["cfg"])
    if not m3.kernels._lib.supported(0, 0, 32, n, p):
        pytest.skip(f"no f32 kernel for N={n} P={p}")
    cfg = m3.convert.config_from_state_dict(sd, headdim=p, chunk=32, policy_name="f32",
                                            rope_fraction=float(fx["rope_fraction"]))
    params = m3.convert.torch_to_jax(sd, cfg, device="cuda")
    y, _ = m3.mamba3_siso_layer(params, torch.from_numpy(fx["u"]).cuda(), cfg)
    assert O.max_rel(cpu(y), torch.from_numpy(fx["y"]).double()) <= 1e-4


def test_segmented_prefill_equals_one_call_with_gradients(m3):
    """tests.py:653-726 at layer level: two chained segments == one call, grads too."""
    cfg = m3.SISOConfig(d_model=64, d_state=16, headdim=16, expand=1, chunk=32, policy_name="f32")
    params = m3.SISOParams(*(t.cuda() for t in m3.init_params(cfg, 3)))
    g = torch.Generator().manual_seed(4)
    u = torch.randn(2, 256, 64, generator=g).cuda()
    gy = torch.randn(2, 256, 64, generator=g).cuda()
    u1 = u.clone().requires_grad_(True)
    y_full, st_full = m3.mamba3_siso_layer(params, u1, cfg)
    (y_full * gy).sum().backward()
    u2 = u.clone().requires_grad_(True)
    ya, sa = m3.mamba3_siso_layer(params, u2[:, :128], cfg)
    yb, sb = m3.mamba3_siso_layer(params, u2[:, 128:], cfg, state=sa)
    (torch.cat([ya, yb], 1) * gy).sum().backward()
    assert O.rel_error(cpu(torch.cat([ya, yb], 1)), cpu(y_full)) <= 2e-5
    assert O.rel_error(cpu(sb.ssm), cpu(st_full.ssm)) <= 2e-5
    assert O.rel_error(cpu(sb.phi), cpu(st_full.phi), angle=True) <= 1e-4
    assert O.rel_error(cpu(u2.grad), cpu(u1.grad)) <= GRAD_F32_P95


@pytest.mark.parametrize("d_model,batch,seqlen,seed", [(1024, 2, 512, 9), (256, 2, 512, 5)])
def test_layer_bf16_forward_and_grads(m3, d_model, batch, seqlen, seed):
    """The bf16 layer at BASELINE configs[1]/[2] widths (d_model 1024, H 32, N 128, P 64,
    chunk 128; short L so the float64 oracle stays quick) and at d_model 256: the output,
    the final state and the gradient of u and of every `SISOParams` field against autograd
    of the float64 layer; the output also against the bf16 layer's rounding model."""
    cfg = m3.SISOConfig(d_model=d_model, d_state=128, headdim=64, expand=2, chunk=128)
    p_cpu = m3.init_params(cfg, seed)
    g = torch.Generator().manual_seed(seed + 1)
    u = torch.randn(batch, seqlen, d_model, generator=g).to(BF16)
    gy = torch.randn(batch, seqlen, d_model, generator=g).to(BF16)
    params = m3.SISOParams(*(t.cuda().requires_grad_(True) for t in p_cpu))
    ud = u.cuda().requires_grad_(True)
    y, st = m3.mamba3_siso_layer(params, ud, cfg)
    assert y.dtype == BF16
    (y.float() * gy.cuda().float()).sum().backward()
    pd = {k_: v_.requires_grad_(True) for k_, v_ in params_dict(p_cpu).items()}
    uo = u.double().requires_grad_(True)
    yr, sr = O.layer_forward(pd, uo, d_state=128, headdim=64, expand=2, chunk=128)
    (yr * gy.double()).sum().backward()
    with torch.no_grad():
        ym, sm = O.layer_forward(params_dict(p_cpu), u.double(), d_state=128, headdim=64,
                                 expand=2, chunk=128, mm_dtype=BF16, act_dtype=BF16)
    report("layer y vs float64", y, yr.detach())
    report("layer y vs bf16 layer model", y, ym)
    report("layer final ssm vs float64", st.ssm, sr.ssm.detach())
    # the float64 maths
    assert_maxrel(y, yr.detach(), BF16_Y_MAXREL, "y")
    assert_maxabs(st.ssm, sr.ssm.detach(), STATE_MAXABS, "final ssm")
    assert_maxabs(st.k, sr.k.detach(), STATE_MAXABS * float(sr.k.detach().abs().max()), "final k")
    # the bf16 layer's own rounding points: weights cast per call and every stored
    # activation rounded (layer.py:233, 256). Against float64 the p95 of y sits at about
    # 5.2e-2, from outputs far below max|y| after those roundings; against the model it
    # is ~5e-3.
    assert_p95(y, ym, BF16_LAYER_MODEL_P95, "y vs bf16 layer model")
    assert_bf16_bound(y, ym, what="y vs bf16 layer model")
    assert_maxrel(st.ssm, sm.ssm, 2e-3, "final ssm vs bf16 layer model")   # measured ~9e-4
    report("layer du vs float64", ud.grad, uo.grad)
    assert_maxrel(ud.grad, uo.grad, BF16_GRAD_MAXREL, "du")
    for f in p_cpu._fields:
        report(f"layer d{f} vs float64", getattr(params, f).grad, pd[f].grad)
        assert_maxrel(getattr(params, f).grad, pd[f].grad, BF16_GRAD_MAXREL, f"d{f}")


def test_cfg1_layer_forward_without_gradients_in_raw_mode(m3, monkeypatch):
    """BASELINE configs[0]'s layer (f32 policy) without gradients runs raw mode (the generic
    kernel's): no preprocess launch; y and the final state within the f32 bars of the
    float64 layer, and phi within 1e-5."""
    cfg = cfg1(m3)
    p_cpu = m3.init_params(cfg, 0)
    params = m3.SISOParams(*(t.cuda() for t in p_cpu))
    u = torch.randn(1, 512, 64, generator=torch.Generator().manual_seed(0))
    with torch.no_grad(), monkeypatch.context() as mp:
        def refuse(*a, **k):
            raise AssertionError("the preprocess launch ran in raw mode")
        mp.setattr(m3.scan_prep, "prep_forward_launch", refuse)
        y, st = m3.mamba3_siso_layer(params, u.cuda(), cfg)
    yr, sr = O.layer_forward(params_dict(p_cpu), u.double(), d_state=16, headdim=16, expand=1,
                             chunk=64)
    report("raw-mode cfg1 layer y vs float64", y, yr)
    assert_f32(y, yr, "out", "y")
    assert_f32(st.ssm, sr.ssm, "out", "final ssm")
    assert_f32(st.k, sr.k, "out", "final k")
    assert O.rel_error(cpu(st.phi), sr.phi, angle=True, pct=100.0) <= 1e-5


@pytest.mark.parametrize("d_model,chunk,seqlen", [(1024, 128, 512), (256, 512, 1024),
                                                  (512, 64, 256)])
def test_layer_forward_without_gradients_runs_the_preprocess_in_the_scan(m3, monkeypatch,
                                                                         d_model, chunk, seqlen):
    """Under no_grad the bf16 layer runs raw mode (the BCNorm launch writes the rotary
    table and strip totals, the scan reads the raw dt / a / trap slices and carries phi):
    the preprocess launch is never called, and the output and final state agree with the
    path that materialises phi and the row scalars first (phi_in_kernel=False) and with the
    float64 layer and its bf16 rounding model."""
    cfg = m3.SISOConfig(d_model=d_model, d_state=128, headdim=64, expand=2, chunk=chunk)
    p_cpu = m3.init_params(cfg, 41)
    params = m3.SISOParams(*(t.cuda() for t in p_cpu))
    u = torch.randn(2, seqlen, d_model, generator=torch.Generator().manual_seed(42)).to(BF16)
    with torch.no_grad():
        y0, st0 = m3.mamba3_siso_layer(params, u.cuda(), cfg, phi_in_kernel=False)
        with monkeypatch.context() as mp:
            def refuse(*a, **k):
                raise AssertionError("the preprocess launch ran in raw mode")
            mp.setattr(m3.scan_prep, "prep_forward_launch", refuse)
            y, st = m3.mamba3_siso_layer(params, u.cuda(), cfg)
        # the rounding model at the chunk the kernel runs (a longer chunk runs as tiles)
        from mamba3_siso_tpu_amd import layout as LY
        tile = LY.kernel_chunk("bf16", chunk, 128, 64)
        ym, sm = O.layer_forward(params_dict(p_cpu), u.double(), d_state=128, headdim=64,
                                 expand=2, chunk=tile, mm_dtype=BF16, act_dtype=BF16)
        yr, sr = O.layer_forward(params_dict(p_cpu), u.double(), d_state=128, headdim=64,
                                 expand=2, chunk=chunk)
    report("raw-mode layer y vs phi materialised", y, cpu(y0))
    report("raw-mode layer final ssm vs phi materialised", st.ssm, cpu(st0.ssm))
    # the raw path's dt, gamma and scale come from hardware exp2 / log2 / rcp (a few 1e-5
    # relative), which moves some bf16 roundings of the operands
    assert O.rel_error(cpu(y), cpu(y0)) <= 1e-2
    assert O.max_rel(cpu(st.ssm), cpu(st0.ssm)) <= 5e-3
    assert torch.equal(st.v, st0.v)
    assert O.rel_error(cpu(st.phi), cpu(st0.phi), angle=True, pct=100.0) <= 1e-5
    report("raw-mode layer y vs bf16 layer model", y, ym)
    assert_p95(y, ym, BF16_LAYER_MODEL_P95, "y vs bf16 layer model")
    assert_bf16_bound(y, ym, what="y vs bf16 layer model")
    assert_maxrel(y, yr, BF16_Y_MAXREL, "y")
    assert_maxabs(st.ssm, sr.ssm, STATE_MAXABS, "final ssm")
    # the angles and dt come from the bf16 projection, whose entries the GEMM rounds
    # differently from the model in places (measured 1.2e-3 rad at L = 512)
    assert O.rel_error(cpu(st.phi), sm.phi, angle=True, pct=100.0) <= 5e-3


@pytest.mark.parametrize("policy,chunk", [("bf16", 256), ("bf16", 512), ("f32", 128),
                                          ("f32", 64)])
def test_layer_at_chunks_without_a_kernel_of_their_own(m3, policy, chunk):
    """The reference's chunks (a multiple of 128; its headline runs 512) and the f32
    policy at the default chunk run as compiled tiles (layout.kernel_chunk): the output,
    final state and every gradient against autograd of the float64 layer at the requested
    chunk, and bit-equal to the same layer configured at the tile itself."""
    from mamba3_siso_tpu_amd import layout as LY
    cfg = m3.SISOConfig(d_model=256, d_state=128, headdim=64, expand=2, chunk=chunk,
                        policy_name=policy)
    tile = LY.kernel_chunk(policy, chunk, 128, 64)
    assert tile < chunk
    cfg_t = m3.SISOConfig(d_model=256, d_state=128, headdim=64, expand=2, chunk=tile,
                          policy_name=policy)
    dt = BF16 if policy == "bf16" else torch.float32
    p_cpu = m3.init_params(cfg, 21)
    g = torch.Generator().manual_seed(22)
    u = torch.randn(2, 1024, 256, generator=g).to(dt)
    gy = torch.randn(2, 1024, 256, generator=g).to(dt)
    runs = []
    for c in (cfg, cfg_t):
        params = m3.SISOParams(*(t.cuda().requires_grad_(True) for t in p_cpu))
        ud = u.cuda().requires_grad_(True)
        y, st = m3.mamba3_siso_layer(params, ud, c)
        (y.float() * gy.cuda().float()).sum().backward()
        runs.append((y, st, ud.grad, params))
    (y, st, du, params), (y_t, st_t, du_t, params_t) = runs
    assert torch.equal(y, y_t) and torch.equal(st.ssm, st_t.ssm) and torch.equal(du, du_t)
    for f in p_cpu._fields:
        assert torch.equal(getattr(params, f).grad, getattr(params_t, f).grad), f
    pd = {k_: v_.requires_grad_(True) for k_, v_ in params_dict(p_cpu).items()}
    uo = u.double().requires_grad_(True)
    yr, sr = O.layer_forward(pd, uo, d_state=128, headdim=64, expand=2, chunk=chunk)
    (yr * gy.double()).sum().backward()
    report(f"layer y ({policy}, chunk {chunk} as {tile}) vs float64", y, yr.detach())
    if policy == "f32":
        assert_f32(y, yr.detach(), "out", "y")
        assert_f32(st.ssm, sr.ssm.detach(), "out", "final ssm")
        assert_f32(du, uo.grad, "grad", "du")
        for f in p_cpu._fields:
            assert_f32(getattr(params, f).grad, pd[f].grad, "grad", f"d{f}")
    else:
        assert_maxrel(y, yr.detach(), BF16_Y_MAXREL, "y")
        assert_maxabs(st.ssm, sr.ssm.detach(), STATE_MAXABS, "final ssm")
        assert_maxrel(du, uo.grad, BF16_GRAD_MAXREL, "du")
        for f in p_cpu._fields:
            assert_maxrel(getattr(params, f).grad, pd[f].grad, BF16_GRAD_MAXREL, f"d{f}")


@pytest.mark.parametrize("policy,n,p,chunk", [("bf16", 128, 128, 128), ("f32", 32, 32, 64),
                                            ("bf16", 64, 192, 64), ("bf16", 256, 64, 128),
                                            ("bf16", 256, 128, 128)])
def test_layer_with_heads_wider_than_a_kernel(m3, policy, n, p, chunk):
    """Head widths with no kernel of their own (a checkpoint with headdim 128) run as
    sub-heads of a compiled width (layout.kernel_headdim), and d_state 256 runs the
    generic kernels at 32-token tiles: the output, final state and every gradient
    against autograd of the float64 layer, then a decode step from the final state
    against the oracle's."""
    from mamba3_siso_tpu_amd import layout as LY
    cfg = m3.SISOConfig(d_model=2 * p, d_state=n, headdim=p, expand=2, chunk=chunk,
                        policy_name=policy)
    assert LY.kernel_headdim(policy, chunk, n, p) < p or LY.kernel_chunk(policy, chunk, n, p) < chunk
    dt = BF16 if policy == "bf16" else torch.float32
    p_cpu = m3.init_params(cfg, 31)
    g = torch.Generator().manual_seed(32)
    u = torch.randn(2, 256, cfg.d_model, generator=g).to(dt)
    gy = torch.randn(2, 256, cfg.d_model, generator=g).to(dt)
    params = m3.SISOParams(*(t.cuda().requires_grad_(True) for t in p_cpu))
    ud = u.cuda().requires_grad_(True)
    y, st = m3.mamba3_siso_layer(params, ud, cfg)
    (y.float() * gy.cuda().float()).sum().backward()
    pd = {k_: v_.requires_grad_(True) for k_, v_ in params_dict(p_cpu).items()}
    uo = u.double().requires_grad_(True)
    yr, sr = O.layer_forward(pd, uo, d_state=n, headdim=p, expand=2, chunk=chunk)
    (yr * gy.double()).sum().backward()
    report(f"layer y ({policy}, N {n}, P {p}) vs float64", y, yr.detach())
    if policy == "f32":
        assert_f32(y, yr.detach(), "out", "y")
        assert_f32(st.ssm, sr.ssm.detach(), "out", "final ssm")
        assert_f32(ud.grad, uo.grad, "grad", "du")
        for f in p_cpu._fields:
            assert_f32(getattr(params, f).grad, pd[f].grad, "grad", f"d{f}")
    else:
        assert_maxrel(y, yr.detach(), BF16_Y_MAXREL, "y")
        assert_maxabs(st.ssm, sr.ssm.detach(), STATE_MAXABS, "final ssm")
        assert_maxrel(ud.grad, uo.grad, BF16_GRAD_MAXREL, "du")
        for f in p_cpu._fields:
            assert_maxrel(getattr(params, f).grad, pd[f].grad, BF16_GRAD_MAXREL, f"d{f}")
    # bf16: the angles and dt come from the bf16 projection, 2^-9 relative per token
    assert O.rel_error(cpu(st.phi), sr.phi.detach(), angle=True) <= (1e-4 if policy == "f32" else 1e-2)
    # one decode step from the final state (composed path: sub-heads of the decode kernel)
    g2 = torch.Generator().manual_seed(33)
    u1 = torch.randn(2, cfg.d_model, generator=g2).to(dt)
    st_o = O.SISOState(*(t.detach().double() for t in (sr.ssm, sr.k, sr.v, sr.phi)))
    with torch.no_grad():
        y1, s1 = m3.mamba3_siso_decode_step(
            m3.SISOParams(*(t.detach() for t in params)), u1.cuda(), cfg,
            m3.SISOState(*(t.float().cuda().contiguous() for t in st_o)))
    y1r, s1r = O.layer_decode_step(params_dict(p_cpu), u1.double(), st_o, d_state=n, headdim=p,
                                   mm_dtype=BF16 if policy == "bf16" else None)
    if policy == "f32":
        assert_p95(y1, y1r, 1e-4, "decode y")
        assert_f32(s1.ssm, s1r.ssm, "out", "decode ssm")
    else:
        assert_maxrel(y1, y1r, BF16_MAXREL, "decode y")
        assert_maxrel(s1.ssm, s1r.ssm, BF16_MAXREL, "decode ssm")
    # bf16: the token's k row and angles come from the bf16 projection
    assert O.max_rel(cpu(s1.k), s1r.k) <= (1e-5 if policy == "f32" else BF16_MAXREL)
    assert O.rel_error(cpu(s1.phi), s1r.phi, angle=True) <= (1e-5 if policy == "f32" else 1e-2)


@pytest.mark.parametrize("policy", ["f32", "bf16"])
def test_layer_decode_step_matches_oracle(m3, policy):
    # decode does not depend on the chunk; f32 at N=128 is compiled at chunk 32
    cfg = m3.SISOConfig(d_model=256, d_state=128, headdim=64, expand=2,
                        chunk=128 if policy == "bf16" else 32, policy_name=policy)
    p_cpu = m3.init_params(cfg, 7)
    params = m3.SISOParams(*(t.cuda() for t in p_cpu))
    g = torch.Generator().manual_seed(8)
    B, H, P, N, Nr = 3, cfg.nheads, 64, 128, cfg.n_angles
    st = O.SISOState(torch.randn(B, H, P, N, generator=g, dtype=torch.float64).float().double() * 0.1,
                     torch.randn(B, H, N, generator=g, dtype=torch.float64).float().double(),
                     torch.randn(B, H, P, generator=g, dtype=torch.float64).float().double(),
                     (torch.rand(B, H, Nr, generator=g, dtype=torch.float64) * 6).float().double())
    mt = BF16 if policy == "bf16" else torch.float32
    u = torch.randn(B, 256, generator=g).to(mt)
    y, s2 = m3.mamba3_siso_decode_step(params, u.cuda(), cfg,
                                       m3.SISOState(*(t.float().cuda() for t in st)))
    yr, sr = O.layer_decode_step(params_dict(p_cpu), u.double(), st, d_state=N, headdim=P,
                                 mm_dtype=BF16 if policy == "bf16" else None)
    if policy == "f32":
        assert_p95(y, yr, 1e-4, "y")
        assert_f32(s2.ssm, sr.ssm, "out", "ssm")
    else:
        assert_maxrel(y, yr, BF16_MAXREL, "y")
        assert_maxrel(s2.ssm, sr.ssm, BF16_MAXREL, "ssm")


def test_layer_decode_step_at_cfg4_size(m3):
    """BASELINE configs[3] at its own size: B=256, d_model 1024 (H=32, P=64, N=128), bf16
    tokens, the carried state ~ N(0, 0.1) from seed 3 (k, v, phi seeded too); three chained
    layer steps (one m3s_decode_layer launch each between the projections) against the
    float64 oracle's step with the bf16 readout model, to the bf16 bars: y and the state
    within 2e-2 of max |ref|, the state also within north_star's 2e-2 max-abs."""
    cfg = m3.SISOConfig(d_model=1024, d_state=128, headdim=64, expand=2, chunk=128)
    p_cpu = m3.init_params(cfg, 0)
    params = m3.SISOParams(*(t.cuda() for t in p_cpu))
    B, H, P, N, Nr = 256, cfg.nheads, 64, 128, cfg.n_angles
    g = torch.Generator().manual_seed(3)
    st_o = O.SISOState(torch.randn(B, H, P, N, generator=g).double() * 0.1,
                       torch.randn(B, H, N, generator=g).double(),
                       torch.randn(B, H, P, generator=g).double(),
                       (torch.rand(B, H, Nr, generator=g) * 6).double())
    st = m3.SISOState(*(t.float().cuda() for t in st_o))
    pd = params_dict(p_cpu)
    for step in range(3):
        u = torch.randn(B, 1024, generator=torch.Generator().manual_seed(1000 + step)).to(BF16)
        print(f"[cfg4 decode] step {step}", flush=True)
        assert m3.layer._decode_fused_ok(u.cuda(), cfg)
        y, st = m3.mamba3_siso_decode_step(params, u.cuda(), cfg, st)
        yr, st_o = O.layer_decode_step(pd, u.double(), st_o, d_state=N, headdim=P,
                                       mm_dtype=BF16)
        report(f"cfg4 decode y step {step}", y, yr)
        assert_maxrel(y, yr, BF16_MAXREL, f"y step {step}")
        assert_maxrel(st.ssm, st_o.ssm, BF16_MAXREL, f"ssm step {step}")
        assert_maxabs(st.ssm, st_o.ssm, STATE_MAXABS, f"ssm step {step}")
        assert_maxrel(st.k, st_o.k, BF16_MAXREL, f"k step {step}")
        assert_maxrel(st.v, st_o.v, BF16_MAXREL, f"v step {step}")
        assert O.rel_error(cpu(st.phi), st_o.phi, angle=True) <= 1e-2


@pytest.mark.parametrize("policy", ["bf16", "f32"])
def test_layer_decode_fused_matches_composed_over_steps(m3, policy, monkeypatch):
    """The one-launch layer step (m3s_decode_layer) against the composed step (torch
    BCNorm / dt / lambda ops + m3s_decode) over 6 chained tokens, with non-unit norm
    gains, scaled inputs and a batch that is not a multiple of 8."""
    cfg = m3.SISOConfig(d_model=256, d_state=128, headdim=64, expand=2,
                        chunk=128 if policy == "bf16" else 32, policy_name=policy)
    p_cpu = m3.init_params(cfg, 9)
    g = torch.Generator().manual_seed(10)
    p_cpu = p_cpu._replace(b_norm_weight=torch.rand(128, generator=g) + 0.5,
                           c_norm_weight=torch.rand(128, generator=g) + 0.5)
    params = m3.SISOParams(*(t.cuda() for t in p_cpu))
    mt = BF16 if policy == "bf16" else torch.float32
    B, H, Nr = 5, cfg.nheads, cfg.n_angles

    def fresh_state():
        gs = torch.Generator().manual_seed(11)
        return m3.SISOState(torch.randn(B, H, 64, 128, generator=gs).cuda() * 0.1,
                            torch.randn(B, H, 128, generator=gs).cuda(),
                            torch.randn(B, H, 64, generator=gs).cuda(),
                            (torch.rand(B, H, Nr, generator=gs) * 6).cuda())

    toks = [(torch.randn(B, 256, generator=g) * 3).to(mt).cuda() for _ in range(6)]
    s1, s0 = fresh_state(), fresh_state()
    tol = BF16_MAXREL if policy == "bf16" else 2e-5
    for t in toks:
        assert m3.layer._decode_fused_ok(t, cfg)
        y1, s1 = m3.mamba3_siso_decode_step(params, t, cfg, s1)
        with monkeypatch.context() as mp:
            mp.setattr(m3.layer, "_decode_fused_ok", lambda *a: False)
            y0, s0 = m3.mamba3_siso_decode_step(params, t, cfg, s0)
        assert_maxrel(y1, cpu(y0), tol, "y")
    for name in ("ssm", "k", "v"):
        assert_maxrel(getattr(s1, name), cpu(getattr(s0, name)), tol, name)
    assert O.rel_error(cpu(s1.phi), cpu(s0.phi), angle=True) <= 1e-5


@pytest.mark.parametrize("policy", ["bf16", "f32"])
def test_layer_with_phi_built_in_the_kernels(m3, policy):
    """phi_in_kernel=True (the preprocess writes the compact phi, both scan kernels rebuild
    it per token) against the default (phi materialised): outputs, state and every
    gradient agree to float rounding, and the bf16 run stays within its float64 bars."""
    if policy == "bf16":
        cfg = m3.SISOConfig(d_model=256, d_state=128, headdim=64, expand=2, chunk=128)
        dt, tol = BF16, 2e-3
    else:
        cfg = m3.SISOConfig(d_model=64, d_state=16, headdim=16, expand=1, chunk=64,
                            policy_name="f32")
        dt, tol = torch.float32, 2e-5
    p_cpu = m3.init_params(cfg, 13)
    g = torch.Generator().manual_seed(14)
    u = torch.randn(2, 512, cfg.d_model, generator=g).to(dt)
    gy = torch.randn(2, 512, cfg.d_model, generator=g).to(dt)
    runs = []
    for flag in (False, True):
        params = m3.SISOParams(*(t.cuda().requires_grad_(True) for t in p_cpu))
        ud = u.cuda().requires_grad_(True)
        y, st = m3.mamba3_siso_layer(params, ud, cfg, phi_in_kernel=flag)
        (y.float() * gy.cuda().float()).sum().backward()
        runs.append((y, st, ud.grad, [getattr(params, f).grad for f in p_cpu._fields]))
    (y0, s0, du0, g0), (y1, s1, du1, g1) = runs
    if policy == "bf16":   # y is stored in bf16: a rounding may flip by one ulp
        assert_bf16_bound(y1, cpu(y0), rel=tol, what="y")
    else:
        assert_maxrel(y1, cpu(y0), tol, "y")
    assert_maxrel(s1.ssm, cpu(s0.ssm), tol, "ssm")
    assert O.rel_error(cpu(s1.phi), cpu(s0.phi), angle=True) <= 1e-5
    assert_maxrel(du1, cpu(du0), 10 * tol, "du")
    for f, a, b in zip(p_cpu._fields, g1, g0):
        assert_maxrel(a, cpu(b), 10 * tol, f"d{f}")


def test_recorded_gemm_solutions_change_only_gemm_rounding(m3):
    """gemm_tuning.enable() picks other library kernels for the projections; the layer's
    output and input gradient stay within bf16 rounding of the default solutions'."""
    from mamba3_siso_tpu_amd import gemm_tuning

    cfg = m3.SISOConfig(d_model=1024, d_state=128, headdim=64, expand=2, chunk=128)
    params = m3.SISOParams(*(t.cuda() for t in m3.init_params(cfg, 17)))
    g = torch.Generator().manual_seed(18)
    u = torch.randn(8, 8192, 1024, generator=g).to(BF16).cuda()   # a recorded shape
    outs = []
    for tuned in (False, True):
        if tuned:
            assert gemm_tuning.enable()
        try:
            ud = u.clone().requires_grad_(True)
            y, _ = m3.mamba3_siso_layer(params, ud, cfg)
            y.float().square().mean().backward()
            outs.append((y.detach(), ud.grad))
        finally:
            gemm_tuning.disable()
    assert_maxrel(outs[1][0], cpu(outs[0][0]), 1e-2, "y")
    assert_maxrel(outs[1][1], cpu(outs[0][1]), 2e-2, "du")


@pytest.mark.parametrize("m,p,q,dtype", [
    (65536, 2048, 1024, torch.bfloat16),   # configs[2] out_proj: 8 token slices
    (32768, 768, 520, torch.bfloat16),     # a strided column slice (in the layer: dproj[..., :d])
    (16384, 256, 96, torch.float32),       # float32 operands (the LM head)
    (1000, 64, 32, torch.bfloat16),        # tokens not a multiple of 32: one library product
    (64, 300, 40, torch.bfloat16),         # m3s_wgrad, one split (straight to C), P % 8 != 0
    (64, 296, 44, torch.bfloat16),         # m3s_wgrad, one split, Q % 8 != 0 on a padded stride
    (4096, 520, 1000, torch.bfloat16),     # m3s_wgrad, several splits, ragged tiles
])
def test_weight_grad_matches_float64(m3, dev, m, p, q, dtype):
    """`layer.weight_grad` (``a^T b`` over the tokens, float32 out) against float64: bf16
    operands go to ``m3s_wgrad`` (token splits whose float32 partials are added in split
    order), the others to the library split; 1e-5 of max |ref| (f32 accumulation over up
    to 65536 terms), bit-identical on a second call. Both operands are column slices of
    wider buffers whose row strides are multiples of 8 (as ``dproj[..., :d]`` in the layer),
    so a last 16-byte piece of a row reads past the slice's columns."""
    g = torch.Generator().manual_seed(m + p)
    pad = lambda n: (n + 7) // 8 * 8 + 8   # noqa: E731
    afull = torch.randn(m, pad(p), generator=g).to(dtype)
    bfull = torch.randn(m, pad(q), generator=g).to(dtype)
    ad, bd = afull.to(dev)[:, :p], bfull.to(dev)[:, :q]
    if dtype == torch.bfloat16 and m % 32 == 0:
        assert m3.kernels.wgrad_supported(ad, bd)
    got = m3.layer.weight_grad(ad, bd)
    ref = afull[:, :p].double().t() @ bfull[:, :q].double()
    assert got.dtype == torch.float32 and got.shape == (p, q)
    err = ((got.cpu().double() - ref).abs().max() / ref.abs().max()).item()
    assert err <= 1e-5, err
    assert torch.equal(got, m3.layer.weight_grad(ad, bd))


@pytest.mark.parametrize("m,k,n,ldw", [
    (1, 768, 3432, 3432),    # the LM's in_proj at one row
    (2, 1536, 768, 776),     # out_proj / fc2 widths, a padded weight row stride
    (1, 4096, 8, 8),         # the longest reduction the kernel takes
    (3, 40, 24, 24),         # three rows, fewer rows than the row lanes
    (4, 1000, 1000, 1000),   # four rows, ragged column tiles
])
def test_gemv_matches_float64(m3, dev, m, k, n, ldw):
    """``m3s_gemv`` (a decode step's projection) against float64: bf16 output, so within
    one bf16 rounding of max |ref| (2^-8), bit-identical on a second call."""
    g = torch.Generator().manual_seed(m + k + n)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    wfull = (torch.randn(k, ldw, generator=g) / k ** 0.5).to(torch.bfloat16)
    xd, wd = x.to(dev), wfull.to(dev)[:, :n]
    got = m3.kernels.gemv(xd, wd)
    ref = x.double() @ wfull[:, :n].double()
    assert got.dtype == torch.bfloat16 and got.shape == (m, n)
    err = ((got.cpu().double() - ref).abs().max() / ref.abs().max()).item()
    assert err <= 2 ** -8, err
    assert torch.equal(got, m3.kernels.gemv(xd, wd))


@pytest.mark.parametrize("m,k,n,ldx,ldw", [
    (256, 1024, 4480, 1024, 4480),   # the layer's in_proj at the decode batch (128-row tiles)
    (200, 128, 5000, 136, 5000),     # 128-row tiles, a partial one and ragged columns
    (1000, 192, 2056, 192, 2056),    # 128-row tiles over several rounds, ragged rows and columns
    (256, 2048, 1024, 2048, 1024),   # its out_proj
    (64, 768, 3432, 768, 3432),      # the LM's in_proj, ragged 64-column tiles
    (5, 1536, 768, 1544, 776),       # five rows (a partial row tile), padded row strides
    (300, 128, 40, 128, 40),         # a ragged row tile and 32-column tiles, N % 32 != 0
    (1024, 64, 256, 64, 256),        # the largest row count, one K step
])
def test_gemv_tiles_match_float64(m3, dev, m, k, n, ldx, ldw):
    """``m3s_gemv`` with more than four rows (its MFMA tiles) against float64: within one
    bf16 rounding of max |ref| (2^-8), rows and columns past the matrix untouched (the
    output is NaN-filled first), bit-identical on a second call."""
    g = torch.Generator().manual_seed(m + k + n)
    xfull = torch.randn(m, ldx, generator=g).to(torch.bfloat16)
    wfull = (torch.randn(k, ldw, generator=g) / k ** 0.5).to(torch.bfloat16)
    xd, wd = xfull.to(dev)[:, :k], wfull.to(dev)[:, :n]
    got = m3.kernels.gemv(xd, wd)
    ref = xfull[:, :k].double() @ wfull[:, :n].double()
    assert got.dtype == torch.bfloat16 and got.shape == (m, n)
    assert bool(torch.isfinite(got).all())
    err = ((got.cpu().double() - ref).abs().max() / ref.abs().max()).item()
    assert err <= 2 ** -8, err
    assert torch.equal(got, m3.kernels.gemv(xd, wd))
    # the layer routes its decode batch through the same tiles
    if m3.kernels.MATMUL_TILE_ROWS[0] <= m <= m3.kernels.MATMUL_TILE_ROWS[1]:
        assert torch.equal(m3.kernels.matmul(xd, wd), got)


def test_layer_forward_cfg2_full_size(m3):
    """BASELINE configs[1] at its own size, the headline path end to end: B=8, L=8192,
    d_model 1024 (H 32, N 128, P 64, chunk 128), init_params(seed=0), u ~ N(0, 1) in bf16;
    the inference forward (raw mode: BCNorm with the angle pass, the preprocess inside the
    scan), one sequence at a time, against the bf16 layer's rounding model (the reference's
    storage points: the projection, the normalised B and C and y in bf16): y to the model
    bars, the final state within north_star's 2e-2 max-abs and 5e-3 of max |ref| (measured
    2.4e-3); and y against the float32 maths (no activation rounding) within 1e-2 of
    max |ref|. The final state against those maths is printed, not bounded: the bf16
    projection's dt shifts the decay of a whole sequence's contributions, about 4e-2 of
    max |ref| at this length, for the reference's bf16 policy as for this one."""
    cfg = m3.SISOConfig(d_model=1024, d_state=128, headdim=64, expand=2, chunk=128)
    p_cpu = m3.init_params(cfg, 0)
    params = m3.SISOParams(*(t.to(BF16).cuda() if f in ("in_proj", "out_proj") else t.cuda()
                             for f, t in zip(p_cpu._fields, p_cpu)))
    B, L = 8, 8192
    u = torch.randn(B, L, 1024, generator=torch.Generator().manual_seed(0)).to(BF16)
    print("[cfg2 layer] GPU forward", flush=True)
    with torch.no_grad():
        y, st = m3.mamba3_siso_layer(params, u.cuda(), cfg)
    y, ssm, kf = cpu(y), cpu(st.ssm), cpu(st.k)
    # the oracle with the weights the bf16 layer multiplies by (rounded once, as cast)
    pd = params_dict(p_cpu, torch.float32)
    pd["in_proj"], pd["out_proj"] = (pd[k_].to(BF16).float() for k_ in ("in_proj", "out_proj"))
    torch.set_num_threads(min(16, torch.get_num_threads()))
    with torch.no_grad():
        for b in range(B):
            print(f"[cfg2 layer] oracle sequence {b}", flush=True)
            ub = u[b:b + 1].float()
            ym, sm = O.layer_forward(pd, ub, d_state=128, headdim=64, expand=2, chunk=128,
                                     mm_dtype=BF16, act_dtype=BF16)
            report(f"cfg2 layer y[{b}] vs bf16 layer model", y[b:b + 1], ym)
            report(f"cfg2 layer final ssm[{b}] vs bf16 layer model", ssm[b:b + 1], sm.ssm)
            assert_p95(y[b:b + 1], ym, BF16_LAYER_MODEL_P95, f"y[{b}] vs bf16 layer model")
            assert_bf16_bound(y[b:b + 1], ym, what=f"y[{b}] vs bf16 layer model")
            assert_maxabs(ssm[b:b + 1], sm.ssm, STATE_MAXABS, f"final ssm[{b}] vs bf16 layer model")
            assert_maxrel(ssm[b:b + 1], sm.ssm, 5e-3, f"final ssm[{b}] vs bf16 layer model")
            assert_maxrel(kf[b:b + 1], sm.k, 5e-3, f"final k[{b}] vs bf16 layer model")
            yr, sr = O.layer_forward(pd, ub, d_state=128, headdim=64, expand=2, chunk=128)
            report(f"cfg2 layer y[{b}] vs float32", y[b:b + 1], yr)
            report(f"cfg2 layer final ssm[{b}] vs float32", ssm[b:b + 1], sr.ssm)
            report(f"bf16 layer model final ssm[{b}] vs float32 (no kernel)", sm.ssm, sr.ssm)
            assert_maxrel(y[b:b + 1], yr, BF16_Y_MAXREL, f"y[{b}] vs float32")


def test_layer_gradients_cfg3_full_size(m3):
    """BASELINE configs[2] at its own size: the bf16 layer's forward and backward at B=8,
    L=8192, d_model 1024, init_params(seed=0), u ~ N(0, 1) in bf16 (seed 0), float32
    parameters cast per call as the layer does. The upstream gradient is N(0, 1) in bf16
    (seed 2) on sequences 0 and 7 and zero on the others, so that the float32 oracle, run
    with autograd through the bf16 layer's rounding model on those two sequences only,
    gives every parameter's whole gradient: du of sequences 0 and 7 and the gradient of
    each `SISOParams` field within 2e-2 of max |ref|; du of the other sequences exactly
    zero."""
    cfg = m3.SISOConfig(d_model=1024, d_state=128, headdim=64, expand=2, chunk=128)
    p_cpu = m3.init_params(cfg, 0)
    B, L, live = 8, 8192, (0, 7)
    u = torch.randn(B, L, 1024, generator=torch.Generator().manual_seed(0)).to(BF16)
    dy = torch.zeros(B, L, 1024, dtype=BF16)
    g2 = torch.Generator().manual_seed(2)
    for b in live:
        dy[b] = torch.randn(L, 1024, generator=g2).to(BF16)
    print("[cfg3 layer] GPU forward and backward", flush=True)
    params = m3.SISOParams(*(t.cuda().requires_grad_(True) for t in p_cpu))
    ud = u.cuda().requires_grad_(True)
    y, _ = m3.mamba3_siso_layer(params, ud, cfg)
    (y.float() * dy.cuda().float()).sum().backward()
    du = cpu(ud.grad)
    for b in range(B):
        if b not in live:
            assert float(du[b].abs().max()) == 0.0, f"du[{b}] without upstream gradient"
    pd = {k_: v_.requires_grad_(True) for k_, v_ in params_dict(p_cpu, torch.float32).items()}
    torch.set_num_threads(min(16, torch.get_num_threads()))
    for b in live:
        print(f"[cfg3 layer] oracle sequence {b}", flush=True)
        ub = u[b:b + 1].float().requires_grad_(True)
        yr, _ = O.layer_forward(pd, ub, d_state=128, headdim=64, expand=2, chunk=128,
                                mm_dtype=BF16, act_dtype=BF16)
        (yr * dy[b:b + 1].float()).sum().backward()
        report(f"cfg3 layer du[{b}] vs bf16 layer model", du[b:b + 1], ub.grad)
        assert_maxrel(du[b:b + 1], ub.grad, BF16_GRAD_MAXREL, f"du[{b}]")
        del yr, ub
    for f in p_cpu._fields:
        report(f"cfg3 layer d{f} vs bf16 layer model", getattr(params, f).grad, pd[f].grad)
        assert_maxrel(getattr(params, f).grad, pd[f].grad, BF16_GRAD_MAXREL, f"d{f}")
