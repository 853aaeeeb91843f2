"""Host-side formats either side of the layer: the npz checkpoint (``checkpoint.py``) and
whole released-checkpoint conversion (``convert.py:179-356``), on the CPU.

Mirrors the reference's checkpoint and pretrained-format stages (``tests.py:930-1198``):
exact round trips, bf16 halving and widening, strict refusal of missing / extra /
misshapen arrays, vocab padding, MIMO / hybrid refusal, and the released key mapping
leaf by leaf (the mixer mapping itself is pinned by the layer golden vectors through
`convert.torch_to_jax`).
"""

import json
import os

import numpy as np
import pytest
import torch


def make_cfg(m3, tie=True, di=24, n_layers=2, vocab=64, d_model=32):
    scfg = m3.SISOConfig(d_model=d_model, d_state=16, headdim=16, expand=2, chunk=32,
                         policy_name="f32")
    return m3.model.LMConfig(vocab_size=vocab, n_layers=n_layers, siso=scfg, tie_head=tie,
                             d_intermediate=di)


def named(m3, params):
    return m3.checkpoint._named_leaves(params)


@pytest.mark.parametrize("tie,di", [(True, 24), (False, 24), (True, 0)])
def test_save_load_round_trip_is_exact(m3, tmp_path, tie, di):
    cfg = make_cfg(m3, tie, di)
    params = m3.model.init_lm(cfg, 3)
    path = m3.checkpoint.save(str(tmp_path / "model"), params, cfg)
    assert path.endswith(".npz") and os.path.exists(path)
    got, got_cfg = m3.checkpoint.load(path)
    assert got_cfg == cfg
    a, b = named(m3, params), named(m3, got)
    assert [n for n, _ in a] == [n for n, _ in b]
    for (n, x), (_, y) in zip(a, b):
        assert y.dtype == x.dtype and torch.equal(x, y), n
    # bare numpy can read it, and nothing in it is a pickle
    with np.load(path, allow_pickle=False) as z:
        meta = json.loads(bytes(z["__config__"]).decode())
        assert meta["format_version"] == 1 and meta["siso"]["d_model"] == 32
        assert "blocks.0.siso.in_proj" in z.files and z["embed"].shape == (64, 32)
        assert ("head" in z.files) == (not tie)


def test_template_matches_init(m3):
    for tie, di in ((True, 0), (False, 40)):
        cfg = make_cfg(m3, tie, di, n_layers=3)
        a = named(m3, m3.model.init_lm(cfg, 0))
        b = named(m3, m3.model.lm_template(cfg))
        assert [(n, tuple(t.shape)) for n, t in a] == [(n, tuple(t.shape)) for n, t in b]


def test_bf16_file_is_half_and_widens(m3, tmp_path):
    cfg = make_cfg(m3, di=256, vocab=256, d_model=128)     # big enough that headers vanish
    params = m3.model.init_lm(cfg, 4)
    p32 = m3.checkpoint.save(str(tmp_path / "f32.npz"), params, cfg)
    p16 = m3.checkpoint.save(str(tmp_path / "bf16.npz"), params, cfg, dtype=torch.bfloat16)
    ratio = os.path.getsize(p16) / os.path.getsize(p32)
    assert abs(ratio - 0.5) < 0.03, ratio
    with np.load(p16, allow_pickle=False) as z:
        assert z["embed"].dtype == np.dtype("V2")          # opaque 2-byte storage
    raw, _ = m3.checkpoint.load(p16)
    wide, _ = m3.checkpoint.load(p16, dtype=torch.float32)
    for (n, x), (_, r), (_, w) in zip(named(m3, params), named(m3, raw), named(m3, wide)):
        assert r.dtype == torch.bfloat16 and w.dtype == torch.float32, n
        assert torch.equal(w, x.to(torch.bfloat16).float()), n    # exactly the bf16 rounding


def test_load_is_strict(m3, tmp_path):
    cfg = make_cfg(m3)
    params = m3.model.init_lm(cfg, 5)
    path = m3.checkpoint.save(str(tmp_path / "ok.npz"), params, cfg)
    with np.load(path, allow_pickle=False) as z:
        files = {k: z[k] for k in z.files}

    def write(name, d):
        p = str(tmp_path / name)
        np.savez(p, **d)
        return p + ".npz"

    missing = dict(files)
    del missing["blocks.1.siso.dt_bias"]
    with pytest.raises(ValueError, match="missing array 'blocks.1.siso.dt_bias'"):
        m3.checkpoint.load(write("missing", missing))
    extra = dict(files, stray=np.zeros(3, np.float32))
    with pytest.raises(ValueError, match="unexpected arrays"):
        m3.checkpoint.load(write("extra", extra))
    bad = dict(files)
    bad["final_norm"] = np.zeros(31, np.float32)
    with pytest.raises(ValueError, match="shape"):
        m3.checkpoint.load(write("shape", bad))
    nocfg = {k: v for k, v in files.items() if k != "__config__"}
    with pytest.raises(ValueError, match="__config__"):
        m3.checkpoint.load(write("nocfg", nocfg))
    meta = json.loads(bytes(files["__config__"]).decode())
    meta["format_version"] = 99
    newer = dict(files, __config__=np.frombuffer(json.dumps(meta).encode(), np.uint8))
    with pytest.raises(ValueError, match="unsupported checkpoint layout"):
        m3.checkpoint.load(write("newer", newer))


# ---------------------------------------------------------------------------------
# released checkpoints
# ---------------------------------------------------------------------------------

CFG_JSON = {
    "d_model": 64, "d_intermediate": 96, "n_layer": 2, "vocab_size": 60,
    "pad_vocab_size_multiple": 16, "tie_embeddings": True, "attn_layer_idx": [],
    "attn_cfg": {},
    "ssm_cfg": {"layer": "Mamba3", "d_state": 16, "expand": 2, "headdim": 16,
                "ngroups": 1, "chunk_size": 64, "rope_fraction": 0.5, "A_floor": 2e-4},
}


def fake_released_sd(cfg, seed=0):
    """A state dict shaped like a released ``state-spaces/mamba3-siso-*`` checkpoint
    (``tests.py:1026-1056``): the key names, shapes and transposes; random values."""
    c = cfg.siso
    rng = np.random.default_rng(seed)
    n = lambda *s: (rng.normal(size=s) * 0.05).astype(np.float32)  # noqa: E731
    g = lambda k: (1.0 + 0.1 * rng.normal(size=k)).astype(np.float32)  # noqa: E731
    sd = {"backbone.embedding.weight": n(cfg.vocab_size, c.d_model),
          "backbone.norm_f.weight": g(c.d_model)}
    for i in range(cfg.n_layers):
        p = f"backbone.layers.{i}."
        sd[p + "norm.weight"] = g(c.d_model)
        sd[p + "mixer.in_proj.weight"] = n(c.d_in_proj, c.d_model)
        sd[p + "mixer.out_proj.weight"] = n(c.d_model, c.d_inner)
        sd[p + "mixer.dt_bias"] = n(c.nheads)
        sd[p + "mixer.B_bias"] = n(c.nheads, 1, c.d_state)
        sd[p + "mixer.C_bias"] = n(c.nheads, 1, c.d_state)
        sd[p + "mixer.B_norm.weight"] = g(c.d_state)
        sd[p + "mixer.C_norm.weight"] = g(c.d_state)
        sd[p + "mixer.D"] = n(c.nheads)
        if cfg.d_intermediate:
            sd[p + "norm2.weight"] = g(c.d_model)
            sd[p + "mlp.fc1.weight"] = n(2 * cfg.d_intermediate, c.d_model)
            sd[p + "mlp.fc2.weight"] = n(c.d_model, cfg.d_intermediate)
    sd["lm_head.weight"] = sd["backbone.embedding.weight"]
    return {k: torch.from_numpy(v) for k, v in sd.items()}


def test_config_from_hf(m3):
    CV = m3.convert
    cfg = CV.config_from_hf(CFG_JSON, policy_name="f32")
    assert cfg.vocab_size == 64                       # 60 padded to a multiple of 16
    assert cfg.siso.chunk == 128                      # the file's 64 is a tiling choice
    assert cfg.siso.a_floor == 2e-4 and cfg.d_intermediate == 96 and cfg.n_layers == 2
    assert CV.config_from_hf(CFG_JSON, chunk=64).siso.chunk == 64
    for bad, why in (({**CFG_JSON, "ssm_cfg": {**CFG_JSON["ssm_cfg"], "mimo": True}}, "MIMO"),
                     ({**CFG_JSON, "ssm_cfg": {**CFG_JSON["ssm_cfg"], "mimo_rank": 4}}, "MIMO"),
                     ({**CFG_JSON, "attn_layer_idx": [1]}, "attention"),
                     ({**CFG_JSON, "ssm_cfg": {**CFG_JSON["ssm_cfg"], "ngroups": 2}}, "ngroups"),
                     ({**CFG_JSON, "ssm_cfg": {**CFG_JSON["ssm_cfg"], "layer": "Mamba2"}},
                      "Mamba3")):
        with pytest.raises(ValueError, match=why):
            CV.config_from_hf(bad)


def test_load_lm_state_dict_maps_every_key(m3):
    CV = m3.convert
    cfg = CV.config_from_hf(CFG_JSON, chunk=64, policy_name="f32")
    sd = fake_released_sd(cfg)
    params = CV.load_lm_state_dict(sd, cfg)
    assert sum(t.numel() for t in m3.model.lm_leaves(params)) == cfg.param_count()
    assert params.head is None
    assert torch.equal(params.embed, sd["backbone.embedding.weight"])
    assert torch.equal(params.final_norm, sd["backbone.norm_f.weight"])
    for i, b in enumerate(params.blocks):
        p = f"backbone.layers.{i}."
        assert torch.equal(b.norm_gain, sd[p + "norm.weight"])
        assert torch.equal(b.mlp_norm_gain, sd[p + "norm2.weight"])
        assert torch.equal(b.mlp.fc1, sd[p + "mlp.fc1.weight"].t())
        assert torch.equal(b.mlp.fc2, sd[p + "mlp.fc2.weight"].t())
        mixer = {k[len(p + "mixer."):]: v for k, v in sd.items() if k.startswith(p + "mixer.")}
        for x, y in zip(b.siso, CV.torch_to_jax(mixer, cfg.siso)):
            assert torch.equal(x, y)
    # the inverse restores every tensor of the released dict
    back = CV.lm_state_dict(params, cfg)
    assert set(back) == set(sd)
    for k, v in sd.items():
        assert np.array_equal(back[k], v.numpy()), k


def test_load_lm_state_dict_bf16_and_errors(m3):
    CV = m3.convert
    cfg = CV.config_from_hf(CFG_JSON, chunk=64, policy_name="f32")
    sd = fake_released_sd(cfg, seed=1)
    bf16 = {k: v.to(torch.bfloat16) for k, v in sd.items()}
    rounded = {k: v.float() for k, v in bf16.items()}
    a = m3.model.lm_leaves(CV.load_lm_state_dict(bf16, cfg))
    b = m3.model.lm_leaves(CV.load_lm_state_dict(rounded, cfg))
    assert all(x.dtype == torch.float32 and torch.equal(x, y) for x, y in zip(a, b))
    missing = dict(sd)
    del missing["backbone.layers.1.norm2.weight"]
    with pytest.raises(KeyError, match="norm2"):
        CV.load_lm_state_dict(missing, cfg)
    narrow = dict(sd, **{"backbone.embedding.weight": sd["backbone.embedding.weight"][:60]})
    with pytest.raises(ValueError, match="pad_vocab_size_multiple"):
        CV.load_lm_state_dict(narrow, cfg)
    untied = CV.config_from_hf({**CFG_JSON, "tie_embeddings": False}, chunk=64)
    head = CV.load_lm_state_dict(sd, untied).head
    assert torch.equal(head, sd["lm_head.weight"].t())


@pytest.mark.parametrize("fmt", ["safetensors", "bin"])
def test_load_pretrained_from_local_dir(m3, tmp_path, fmt):
    CV = m3.convert
    cfg = CV.config_from_hf(CFG_JSON)
    sd = fake_released_sd(cfg, seed=2)
    (tmp_path / "config.json").write_text(json.dumps(CFG_JSON))
    store = {k: v.clone() for k, v in sd.items()}       # tied weights: distinct storage
    if fmt == "safetensors":
        from safetensors.torch import save_file
        save_file(store, str(tmp_path / "model.safetensors"))
    else:
        torch.save(store, str(tmp_path / "pytorch_model.bin"))
    params, got_cfg = CV.load_pretrained(str(tmp_path), chunk=64)
    assert got_cfg.siso.chunk == 64 and got_cfg.vocab_size == 64
    want = CV.load_lm_state_dict(sd, got_cfg)
    for x, y in zip(m3.model.lm_leaves(params), m3.model.lm_leaves(want)):
        assert torch.equal(x, y)
    with pytest.raises(ValueError, match="local"):
        CV.load_pretrained("state-spaces/mamba3-siso-1.5b")
