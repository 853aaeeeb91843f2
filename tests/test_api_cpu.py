"""Host-side logic of the drop-in API, on the CPU: config rules, init, the split, the
weight-layout conversion (against the reference's own torch module, via golden
fixtures), the preprocessing, and loud failure when a kernel is handed CPU tensors."""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import siso_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_config_fields_defaults_and_rules(m3):
    cfg = m3.SISOConfig(d_model=1024)
    assert (cfg.d_state, cfg.headdim, cfg.expand, cfg.rope_fraction, cfg.chunk) == (128, 64, 2, 0.5, 128)
    assert (cfg.a_floor, cfg.norm_eps, cfg.dt_min, cfg.dt_max, cfg.dt_init_floor) == (1e-4, 1e-5, 1e-3, 0.1, 1e-4)
    assert cfg.policy_name == "bf16"
    # cfg2 dimensions (layer.py:69-95)
    assert (cfg.d_inner, cfg.nheads, cfg.n_angles, cfg.d_in_proj) == (2048, 32, 32, 4480)
    # cfg1: expand=1 gives H=4, Nr=4, d_in_proj=176
    c1 = m3.SISOConfig(d_model=64, d_state=16, headdim=16, expand=1, chunk=64, policy_name="f32")
    assert (c1.nheads, c1.n_angles, c1.d_in_proj) == (4, 4, 176)
    assert m3.SISOConfig(d_model=64, d_state=16, rope_fraction=1.0, headdim=16).n_angles == 8
    with pytest.raises(ValueError):
        m3.SISOConfig(d_model=64, chunk=100)
    with pytest.raises(ValueError):
        m3.SISOConfig(d_model=64, rope_fraction=0.25)
    with pytest.raises(ValueError):
        m3.SISOConfig(d_model=96, headdim=64, expand=1)
    with pytest.raises(ValueError):
        m3.SISOConfig(d_model=64, policy_name="fp8")


@pytest.mark.parametrize("kw,match", [
    (dict(d_model=1024, chunk=96), "multiple of 128"),     # neither a tile nor a 128 multiple
    (dict(d_model=1024, chunk=192), "multiple of 128"),
    (dict(d_model=1024, chunk=0), "multiple of 128"),
    (dict(d_model=1024, chunk=16), "multiple of 128"),
    (dict(d_model=256, d_state=256, policy_name="f32"), "forward/backward/decode"),
    (dict(d_model=256, headdim=32), "forward/backward/decode"),      # 32 < the compiled 64
    (dict(d_model=192, d_state=32, headdim=24), "forward/backward/decode"),
])
def test_config_rejects_shapes_without_compiled_kernels(m3, kw, match):
    """The reference rejects a bad chunk when the config is built (layer.py:97-99), and so
    does this one. A (policy, chunk, d_state, headdim) without forward, backward and decode
    kernels still builds (host-only work such as checkpoint conversion takes any shape),
    and `require_kernels` -- called by the layer entry points before a launch -- refuses it
    with an error naming the chunks that do exist."""
    if match == "multiple of 128":
        with pytest.raises(ValueError, match=match):
            m3.SISOConfig(**kw)
        return
    cfg = m3.SISOConfig(**kw)
    with pytest.raises(ValueError, match=match):
        cfg.require_kernels()
    u = torch.zeros(1, cfg.chunk, cfg.d_model)
    with pytest.raises(ValueError, match=match):   # refused before any device work
        m3.mamba3_siso_layer(m3.init_params(cfg, 0), u, cfg)


def test_config_accepts_every_compiled_shape(m3):
    from mamba3_siso_tpu_amd import layout as LY
    both = LY.KERNELS["forward"] & LY.KERNELS["backward"]
    for pol, c, n, p in sorted(both):
        if (pol, 0, n, p) in LY.KERNELS["decode"]:
            cfg = m3.SISOConfig(d_model=4 * p, d_state=n, headdim=p, chunk=c, policy_name=pol)
            cfg.require_kernels()
            assert (cfg.chunk, cfg.d_state, cfg.headdim) == (c, n, p)
    assert LY.compiled_chunks("f32", 128, 64) == (32,)
    assert LY.compiled_chunks("bf16", 128, 64) == (32, 64, 128)


@pytest.mark.parametrize("pol,n,p,width", [
    ("bf16", 128, 64, 64), ("bf16", 128, 128, 64), ("bf16", 128, 256, 64), ("f32", 128, 192, 64),
    ("bf16", 64, 128, 64), ("bf16", 32, 32, 16), ("f32", 16, 48, 16), ("bf16", 256, 128, 64),
])
def test_wide_heads_run_as_compiled_sub_heads(m3, pol, n, p, width):
    """A head width with no kernel of its own runs as sub-heads of the largest compiled
    width dividing it (the scan is independent across a head's v columns given its
    scores), for the scans and the decode alike."""
    from mamba3_siso_tpu_amd import layout as LY
    cfg = m3.SISOConfig(d_model=4 * p, d_state=n, headdim=p, chunk=64, policy_name=pol)
    assert cfg.headdim == p
    assert LY.kernel_headdim(pol, 64, n, p) == width
    assert LY.decode_headdim(pol, n, p) == width


@pytest.mark.parametrize("pol,chunk,n,p,tile", [
    ("bf16", 128, 128, 64, 128), ("bf16", 64, 128, 64, 64), ("bf16", 32, 128, 64, 32),
    ("bf16", 256, 128, 64, 128), ("bf16", 512, 128, 64, 128), ("bf16", 1024, 64, 64, 128),
    ("f32", 128, 128, 64, 32), ("f32", 64, 128, 64, 32),     # f32 backward only at 32
    ("f32", 512, 32, 16, 128), ("f32", 128, 64, 64, 64),
])
def test_long_chunks_run_as_compiled_tiles(m3, pol, chunk, n, p, tile):
    """The reference's chunks (any multiple of 128, layout.py:225-236; its headline runs
    chunk 512) and the f32 policy at the default chunk build, and the scans run them as
    the largest compiled tile dividing the chunk that has both a forward and a backward
    kernel, so the forward's per-tile states are the ones the backward reads."""
    from mamba3_siso_tpu_amd import layout as LY
    cfg = m3.SISOConfig(d_model=4 * p, d_state=n, headdim=p, chunk=chunk, policy_name=pol)
    assert cfg.chunk == chunk
    assert LY.kernel_chunk(pol, chunk, n, p) == tile
    assert (pol, tile, n, p) in LY.KERNELS["forward"] & LY.KERNELS["backward"]
    assert chunk % tile == 0


def test_init_params_distributions(m3):
    cfg = m3.SISOConfig(d_model=256, d_state=32, headdim=16)
    p = m3.init_params(cfg, 0)
    assert p.in_proj.shape == (256, cfg.d_in_proj) and p.out_proj.shape == (512, 256)
    assert float(p.in_proj.abs().max()) <= 1 / math.sqrt(256)
    assert float(p.out_proj.abs().max()) <= 1 / math.sqrt(512)
    dt = torch.nn.functional.softplus(p.dt_bias)
    assert bool(((dt >= 1e-3 - 1e-7) & (dt <= 0.1 + 1e-7)).all())
    for t in (p.b_norm_weight, p.c_norm_weight, p.b_bias, p.c_bias, p.d_skip):
        assert bool((t == 1).all())
    assert torch.equal(m3.init_params(cfg, 0).in_proj, p.in_proj)       # seeded
    assert not torch.equal(m3.init_params(cfg, 1).in_proj, p.in_proj)


def test_split_in_proj_order_and_views(m3):
    cfg = m3.SISOConfig(d_model=64, d_state=16, headdim=16, expand=1, chunk=64)
    proj = torch.arange(2 * 3 * cfg.d_in_proj, dtype=torch.float32).reshape(2, 3, cfg.d_in_proj)
    z, x, b, c, dt, a, tr, ang = m3.split_in_proj(proj, cfg)
    assert z.shape == (2, 3, 4, 16) and x.shape == (2, 3, 4, 16)
    assert b.shape == c.shape == (2, 3, 16) and dt.shape == a.shape == tr.shape == (2, 3, 4)
    assert ang.shape == (2, 3, 4)
    assert float(x[0, 0, 0, 0]) == 64 and float(b[0, 0, 0]) == 128 and float(c[0, 0, 0]) == 144
    assert float(dt[0, 0, 0]) == 160 and float(a[0, 0, 0]) == 164 and float(tr[0, 0, 0]) == 168
    assert float(ang[0, 0, 0]) == 172
    assert x.data_ptr() == proj.data_ptr() + 64 * 4   # a view, not a copy


def test_rms_norm_matches_oracle(m3):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 5, 16, generator=g).to(torch.bfloat16)
    w = torch.randn(16, generator=g)
    torch.testing.assert_close(m3.rms_norm(x, w, 1e-5), O.rms_norm(x, w, 1e-5), rtol=0, atol=0)


def test_preprocess_fails_loudly_on_cpu_tensors(m3):
    """preprocess is a HIP launch (m3s_prep_fwd); its parity with the oracle is
    tests/test_gpu_prep.py. On CPU tensors it raises instead of computing."""
    x = O.make_inputs(2, 3, 40, 16, 8, 4, seed=2, dtype=torch.float32)
    with pytest.raises(ValueError, match="ROCm device"):
        m3.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"])


def _golden_sd(name):
    fx = dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))
    sd = {k[4:].replace("__", "."): torch.from_numpy(v) for k, v in fx.items() if k.startswith("sd__")}
    return fx, sd


@pytest.mark.parametrize("name", ["torch_ref_layer_half", "torch_ref_layer_full"])
def test_convert_round_trip_and_golden_layer(m3, name):
    """convert.torch_to_jax/jax_to_torch (convert.py:92-176) on the reference module's own
    state dict: exact round trip (tests.py:908-915), and the converted params reproduce
    the reference torch layer's output through the CPU oracle layer."""
    fx, sd = _golden_sd(name)
    d_model, n, p, expand = (int(v) for v in fx["cfg"])
    rf = float(fx["rope_fraction"])
    cfg = m3.convert.config_from_state_dict(sd, headdim=p, chunk=32, policy_name="f32",
                                            rope_fraction=rf)
    assert (cfg.d_model, cfg.d_state, cfg.expand) == (d_model, n, expand)
    params = m3.convert.torch_to_jax(sd, cfg)
    back = m3.convert.jax_to_torch(params, cfg)
    for key, val in back.items():
        src = sd[key.replace("B_norm.weight", "B_norm_weight").replace("C_norm.weight", "C_norm_weight")]
        assert np.array_equal(val, src.numpy()), key
    pd = {f: getattr(params, f).double() for f in params._fields}
    y, _ = O.layer_forward(pd, torch.from_numpy(fx["u"]).double(), d_state=n, headdim=p,
                           expand=expand, rope_fraction=rf, chunk=16)
    assert O.max_rel(y, torch.from_numpy(fx["y"])) < 1e-5


def test_convert_rejects_mimo_and_bad_headdim(m3):
    _, sd = _golden_sd("torch_ref_layer_half")
    with pytest.raises(ValueError):
        m3.convert.config_from_state_dict(sd, headdim=12)
    sd2 = dict(sd)
    sd2["in_proj.weight"] = torch.zeros(sd["in_proj.weight"].shape[0] + 4, sd["in_proj.weight"].shape[1])
    with pytest.raises(ValueError, match="MIMO"):
        m3.convert.config_from_state_dict(sd2, headdim=16, chunk=32)
    cfg = m3.convert.config_from_state_dict(sd, headdim=16, chunk=32)
    sd3 = dict(sd)
    sd3["B_bias"] = torch.zeros(sd["B_bias"].shape[0], 2, sd["B_bias"].shape[-1])
    with pytest.raises(ValueError, match="mimo_rank"):
        m3.convert.torch_to_jax(sd3, cfg)


def test_kernels_fail_loudly_on_cpu_tensors(m3):
    x = O.make_inputs(1, 2, 64, 16, 16, 4, seed=0, dtype=torch.float32)
    pre, _ = O.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"])
    pre = {k: getattr(pre, k).float() for k in ("adt", "gamma", "scale", "phi", "dt", "lam")}
    with pytest.raises(ValueError, match="ROCm device"):
        m3.siso_forward(x["q"], x["k"], x["v"], pre["adt"], pre["gamma"], pre["scale"], pre["phi"],
                        x["q_bias"], x["k_bias"], chunk=64, dtype_policy="f32")
    st = m3.zero_state(1, 2, 16, 16, 4)
    with pytest.raises(ValueError, match="ROCm device"):
        m3.decode_step(x["q"][:, 0], x["k"][:, 0], x["v"][:, :, 0], pre["adt"][:, :, 0],
                       pre["dt"][:, :, 0], pre["lam"][:, :, 0], x["angles"][:, 0], x["q_bias"],
                       x["k_bias"], st, dtype_policy="f32")


def test_kernel_shape_errors_match_the_reference(m3):
    x = O.make_inputs(1, 2, 64, 16, 16, 4, seed=0, dtype=torch.float32)
    pre, _ = O.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"])
    a = (x["q"], x["k"], x["v"], pre.adt.float(), pre.gamma.float(), pre.scale.float(), pre.phi.float(),
         x["q_bias"], x["k_bias"])
    with pytest.raises(ValueError, match="multiple of chunk"):
        m3.siso_forward(*a, chunk=128)                       # L=64 (layout.py:500-506)
    with pytest.raises(ValueError, match="multiple of 128"):
        m3.siso_forward(*a, chunk=48)
    with pytest.raises(ValueError, match="must match"):
        m3.siso_forward(a[0], a[1][:, :, :8], *a[2:], chunk=64)   # kernel_fwd.py:255-256
    with pytest.raises(ValueError, match="given together"):
        m3.siso_forward(*a, seed_ssm=torch.zeros(1, 2, 16, 16), chunk=64)   # kernel_fwd.py:263-266
    with pytest.raises(ValueError, match="adt must be"):
        m3.siso_forward(*a[:3], a[3][:, :1], *a[4:], chunk=64)
