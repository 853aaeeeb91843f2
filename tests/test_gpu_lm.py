"""GPU parity of the LM stack (`model`, `train`) against the CPU oracle
(oracle/lm_oracle.py, float64), through the HIP layer kernels.

Tolerances:
  * f32 policy: logits max |got - ref| / max |ref| <= 1e-4; gradients of every
    parameter <= 1e-3 max-normalised (f32 GEMMs, f32 scan; ~30 accumulations deep).
  * bf16 policy (operands rounded to bf16 in every product): logits and gradients
    <= 3e-2 max-normalised against the float64 maths (the layer's bf16 bar of 2e-2 plus
    the stack's extra bf16 products).
  * decode vs prefill (same device, f32): 1e-4 max-normalised; graph replays vs eager
    steps: bit-identical.
  * optimizer: the device update against the oracle's on the same (device) gradients,
    1e-6 relative (float32 moments) after one update, 2e-6 after six.
"""

import numpy as np
import pytest
import torch

from helpers import assert_maxrel, cpu
from oracle import lm_oracle as LO

pytestmark = pytest.mark.gpu


def make_lm(m3, policy, d_intermediate=48, tie_head=True, n_layers=2, vocab=40, seed=0):
    if policy == "f32":
        scfg = m3.SISOConfig(d_model=64, d_state=16, headdim=16, expand=2, chunk=64,
                             policy_name="f32")
    elif policy == "bf16_cfg5":
        # BASELINE configs[4] widths: d_model 768, N 128, P 64, chunk 128 (the
        # <128, 128, 64> scan kernels and the MLP / norm kernels at widths 768 and 1536)
        scfg = m3.SISOConfig(d_model=768, d_state=128, headdim=64, expand=2, chunk=128)
    else:
        scfg = m3.SISOConfig(d_model=128, d_state=64, headdim=64, expand=2, chunk=64)
    cfg = m3.model.LMConfig(vocab_size=vocab, n_layers=n_layers, siso=scfg,
                            tie_head=tie_head, d_intermediate=d_intermediate)
    params = m3.model.init_lm(cfg, seed)
    g = torch.Generator().manual_seed(seed + 50)

    def jitter(t):   # move every tensor off its init (ones, zeros) so each one matters
        if t.dim() >= 2 and t.shape[0] != vocab:
            return t * (1 + 0.2 * torch.randn(t.shape, generator=g))
        return t + 0.2 * torch.randn(t.shape, generator=g)

    params = m3.model.lm_map(jitter, params)
    s = scfg
    lay = dict(d_state=s.d_state, headdim=s.headdim, expand=s.expand,
               rope_fraction=s.rope_fraction, chunk=s.chunk, a_floor=s.a_floor,
               norm_eps=s.norm_eps)
    return cfg, params, lay


def tokens_for(cfg, b, l, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, cfg.vocab_size, (b, l), generator=g)


@pytest.mark.parametrize("policy,tie,di,vocab,seqlen", [
    ("f32", True, 48, 40, 192), ("f32", False, 0, 40, 192), ("bf16", True, 96, 40, 192),
    ("bf16_cfg5", True, 1536, 256, 256)])
def test_lm_loss_and_grads_match_oracle(m3, dev, policy, tie, di, vocab, seqlen):
    cfg, params, lay = make_lm(m3, policy, d_intermediate=di, tie_head=tie, vocab=vocab)
    xs = tokens_for(cfg, 2, seqlen, 1)
    ys = tokens_for(cfg, 2, seqlen, 2)
    p_dev = m3.train.train_params(m3.model.lm_to(params, device=dev))
    logits = m3.model.lm_forward(p_dev, xs.to(dev), cfg)
    assert logits.dtype == torch.float32 and logits.shape == (2, seqlen, cfg.vocab_size)
    loss = m3.model.lm_loss(p_dev, xs.to(dev), ys.to(dev), cfg)
    loss.backward()

    ref = LO.from_lm_params(params)
    leaves = []

    def req(t):
        if t is not None:
            t.requires_grad_(True)
            leaves.append(t)

    req(ref["embed"]), req(ref["final_norm"]), req(ref["head"])
    for b in ref["blocks"]:
        req(b["norm_gain"])
        for f in LO.SISO_FIELDS:
            req(b["siso"][f])
        for f in ("mlp_norm_gain", "fc1", "fc2"):
            req(b.get(f))
    ref_logits = LO.lm_forward(ref, xs, lay)
    ref_loss = LO.lm_loss(ref, xs, ys, lay)
    ref_loss.backward()

    tol = 1e-4 if policy == "f32" else 3e-2
    gtol = 1e-3 if policy == "f32" else 3e-2
    assert_maxrel(logits.detach(), ref_logits.detach(), tol, "logits")
    assert abs(float(loss.detach()) - float(ref_loss.detach())) <= tol * abs(float(ref_loss.detach()))
    mine = m3.model.lm_leaves(p_dev)
    theirs = [ref["embed"]]
    for b in ref["blocks"]:
        theirs.append(b["norm_gain"])
        theirs.extend(b["siso"][f] for f in LO.SISO_FIELDS)
        if "fc1" in b:
            theirs.extend((b["mlp_norm_gain"], b["fc1"], b["fc2"]))
    theirs.append(ref["final_norm"])
    if ref["head"] is not None:
        theirs.append(ref["head"])
    assert len(mine) == len(theirs)
    for i, (a, r) in enumerate(zip(mine, theirs)):
        assert a.grad is not None and a.grad.dtype == torch.float32, i
        assert_maxrel(a.grad, r.grad, gtol, f"grad[{i}] {tuple(a.shape)}")


def test_decode_chain_matches_prefill_and_oracle(m3, dev):
    """Prefill of a whole chunk with a zero carry, then decode steps: logits at every
    position equal the no-state forward over the full sequence (f32), and the oracle's."""
    cfg, params, lay = make_lm(m3, "f32")
    p_dev = m3.model.lm_to(params, device=dev)
    toks = tokens_for(cfg, 3, 128, 9).to(dev)
    with torch.no_grad():
        full = m3.model.lm_forward(p_dev, toks, cfg)
        pre, states = m3.model.lm_forward(p_dev, toks[:, :64], cfg,
                                          states=m3.model.zero_states(cfg, 3, device=dev))
        assert_maxrel(pre, cpu(full[:, :64]), 1e-4, "prefill logits")
        steps = []
        for t in range(64, 128):
            lg, states = m3.model.lm_decode_step(p_dev, toks[:, t], states, cfg)
            steps.append(lg)
    dec = torch.stack(steps, dim=1)
    assert_maxrel(dec, cpu(full[:, 64:]), 1e-4, "decode vs forward")
    ref = LO.lm_forward(LO.from_lm_params(params), toks.cpu(), lay)
    assert_maxrel(dec, ref[:, 64:], 1e-4, "decode vs oracle")


def test_decode_matches_forward_with_bf16_params_under_f32_policy(m3, dev):
    """bf16 parameters give a bf16 embedding stream; under the f32 policy the block
    outputs are f32, and the forward's ``x + y`` promotes the stream to f32. The decode
    step's residual add must promote the same way (not round the block output to the
    stream's bf16), so decode equals the no-state forward at every position."""
    cfg, params, _ = make_lm(m3, "f32")
    p_dev = m3.model.lm_map(lambda t: t.to(torch.bfloat16), m3.model.lm_to(params, device=dev))
    toks = tokens_for(cfg, 2, 64, 12).to(dev)
    with torch.no_grad():
        full = m3.model.lm_forward(p_dev, toks, cfg)
        states = m3.model.zero_states(cfg, 2, device=dev)
        steps = []
        for t in range(toks.shape[1]):
            lg, states = m3.model.lm_decode_step(p_dev, toks[:, t], states, cfg)
            steps.append(lg)
    assert_maxrel(torch.stack(steps, dim=1), cpu(full), 1e-4, "decode vs forward (bf16 params)")


@pytest.mark.parametrize("policy", ["f32", "bf16"])
def test_decode_graph_replays_equal_eager_steps(m3, dev, policy):
    """Every replay of the recorded step equals the eager step bit for bit, with eager
    work and synchronisations between replays; the carried states agree too."""
    cfg, params, _ = make_lm(m3, policy)
    dp = m3.model.decode_params(m3.model.lm_to(params, device=dev), cfg)
    batch = 2
    dg = m3.train.DecodeGraph(dp, cfg, batch=batch)
    states = m3.model.zero_states(cfg, batch, device=dev)
    toks = tokens_for(cfg, batch, 12, 3).to(dev)
    with torch.no_grad():
        for t in range(toks.shape[1]):
            want, states = m3.model.lm_decode_step(dp, toks[:, t], states, cfg)
            torch.cuda.synchronize()
            got = dg.step(toks[:, t]).clone()
            _ = torch.randn(1000, device=dev).sum()     # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(got, want), t
    for a, b in zip(dg.states, states):
        for x, y in zip(a, b):
            assert torch.equal(x, y)


def test_decode_params_do_not_change_results(m3, dev):
    cfg, params, _ = make_lm(m3, "bf16")
    p_dev = m3.model.lm_to(params, device=dev)
    dp = m3.model.decode_params(p_dev, cfg)
    toks = tokens_for(cfg, 2, 4, 4).to(dev)
    s1 = m3.model.zero_states(cfg, 2, device=dev)
    s2 = m3.model.zero_states(cfg, 2, device=dev)
    with torch.no_grad():
        for t in range(4):
            a, s1 = m3.model.lm_decode_step(p_dev, toks[:, t], s1, cfg)
            b, s2 = m3.model.lm_decode_step(dp, toks[:, t], s2, cfg)
            assert torch.equal(a, b)


@pytest.mark.parametrize("prompt_len", [3, 150])
def test_generate_contract(m3, dev, prompt_len):
    """``tests.py:1172-1198``: the prompt is kept, n tokens follow, ids are in the vocab,
    a stop id ends generation; the graph and eager paths draw the same ids from the same
    seed, and greedy-like sampling (tiny top_p) picks the argmax of the oracle's logits
    wherever the oracle's top two are well separated."""
    cfg, params, lay = make_lm(m3, "f32")
    p_dev = m3.model.lm_to(params, device=dev)
    ids = [int(t) for t in tokens_for(cfg, 1, prompt_len, 6)[0]]
    out = m3.train.generate(p_dev, cfg, 0, ids, n_tokens=6, rep_penalty=1.0)
    assert out[:len(ids)] == ids and len(out) == len(ids) + 6
    assert all(0 <= t < cfg.vocab_size for t in out)
    eager = m3.train.generate(p_dev, cfg, 0, ids, n_tokens=6, rep_penalty=1.0, graph=False)
    assert eager == out
    stopped = m3.train.generate(p_dev, cfg, 0, ids, n_tokens=8,
                                stop_ids=set(range(cfg.vocab_size)))
    assert len(stopped) == len(ids) + 1
    greedy = m3.train.generate(p_dev, cfg, 1, ids, n_tokens=5, top_p=1e-6, rep_penalty=1.0)
    ref_p = LO.from_lm_params(params)
    states = LO.zero_states(ref_p, 1, lay)
    for pos, t in enumerate(greedy[:-1]):   # the oracle's own decode chain
        ref, states = LO.lm_decode_step(ref_p, torch.tensor([t]), states, lay)
        if pos < len(ids) - 1:
            continue
        top2 = torch.topk(ref[0], 2).values
        if float(top2[0] - top2[1]) > 1e-3 * float(ref[0].abs().max()):
            assert greedy[pos + 1] == int(torch.argmax(ref[0])), pos
    with pytest.raises(ValueError, match="empty"):
        m3.train.generate(p_dev, cfg, 0, [], n_tokens=1)


def test_pick_token_draws_from_the_filtered_distribution(m3, dev):
    """40,000 Gumbel-max draws land on each id with the probability of the softmax of
    the oracle's filtered logits (max deviation 0.01), and never outside the nucleus."""
    g = torch.Generator().manual_seed(8)
    vocab = 16
    lg = torch.randn(vocab, generator=g) * 2
    seen = torch.rand(vocab, generator=g) < 0.3
    filt = (0.8, 0.9, 1.2)
    want = torch.softmax(LO.filtered_logits(lg, seen, *filt), dim=0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    draws = m3.train._pick_token(lg.to(dev).expand(40000, vocab), seen.to(dev), gen, filt, vocab)
    freq = torch.bincount(draws.cpu(), minlength=vocab).double() / 40000
    assert float((freq - want).abs().max()) < 0.01
    assert bool((freq[want == 0] == 0).all())


def test_train_step_update_matches_oracle_and_memorizes(m3, dev):
    """One optimizer update on the device equals the oracle's clip + AdamW on the same
    gradients; then 40 steps on one fixed batch cut the loss by 4x
    (``tests.py:1228-1262``'s memorization check, on the whole stack)."""
    cfg, params, _ = make_lm(m3, "bf16", vocab=17)
    p_dev = m3.train.train_params(m3.model.lm_to(params, device=dev))
    opt = m3.train.make_optimizer(p_dev, lr=3e-3, warmup=2, steps=40)
    xs = tokens_for(cfg, 4, 128, 11).to(dev)
    ys = tokens_for(cfg, 4, 128, 12).to(dev)
    before = [t.detach().cpu().double() for t in m3.model.lm_leaves(p_dev)]
    loss = m3.model.lm_loss(p_dev, xs, ys, cfg)
    loss.backward()
    grads = [t.grad.detach().cpu().double() for t in m3.model.lm_leaves(p_dev)]
    opt.step()
    opt.zero_grad()
    clipped = LO.clip_by_global_norm(grads, 1.0)
    zeros = [torch.zeros_like(t) for t in before]
    want, _, _ = LO.adamw_update(before, clipped, zeros, zeros, 0, opt.schedule(0))
    for i, (a, w) in enumerate(zip(m3.model.lm_leaves(p_dev), want)):
        torch.testing.assert_close(a.detach().cpu().double(), w, rtol=1e-6, atol=1e-7,
                                   msg=lambda m: f"param {i}: {m}")
    # memorization: next token of a fixed random sequence, Adam 3e-3 (no decay, no clip)
    seq = tokens_for(cfg, 4, 129, 13).to(dev)
    xs, ys = seq[:, :-1], seq[:, 1:]
    p_dev = m3.train.train_params(m3.model.lm_to(params, device=dev))
    adam = m3.train.AdamW(m3.model.lm_leaves(p_dev), 3e-3, weight_decay=0.0, clip=None)
    step = m3.train.make_step(cfg, adam)
    first = last = None
    for i in range(40):
        loss, p_dev, adam = step(p_dev, adam, xs, ys)
        if i == 0:
            first = float(loss)
    last = float(loss)
    ratio = last / first
    assert np.isfinite(ratio) and ratio < 0.25, (first, last)


@pytest.mark.parametrize("clip", [None, 1.0])
def test_fused_adamw_matches_oracle_over_steps(m3, dev, clip):
    """`train.AdamW` on device float32 tensors (one m3s_adamw pass per update) against the
    oracle's clip + AdamW in float64 over 6 updates. 31 tensors (two launch groups) whose
    sizes cover whole 4096-element blocks, ragged tails, a single element, a tensor that
    is not 16-byte aligned (the element-wise path) and an empty one; gradients alternate
    between norms above and below the clip bound."""
    gen = torch.Generator().manual_seed(21)
    sizes = [1, 3, 4, 5, 4095, 4096, 4097, 8192, 12289, 0, 70000] + [
        int(x) for x in torch.randint(1, 20000, (20,), generator=gen)]
    base = [torch.randn(n, generator=gen, dtype=torch.float64) for n in sizes]
    flat = torch.zeros(sum(sizes) + 4 * len(sizes) + 1, device=dev)   # the first tensor sits at offset 1
    dev_params, off = [], 1
    for i, t in enumerate(base):
        if i > 0:
            off = (off + 3) // 4 * 4   # the others 16-byte aligned (the vector path)
        v = flat[off:off + t.numel()]
        v.copy_(t.to(dev))
        dev_params.append(v)
        off += t.numel()
    assert dev_params[0].data_ptr() % 16 != 0
    sched = m3.train.warmup_cosine_decay_schedule(1e-3, 1e-2, 2, 8, 1e-3)
    opt = m3.train.AdamW(dev_params, sched, weight_decay=0.1, clip=clip)
    ref = [t.clone() for t in base]
    mu = [torch.zeros_like(t) for t in base]
    nu = [torch.zeros_like(t) for t in base]
    for step in range(6):
        grads = [torch.randn(n, generator=gen, dtype=torch.float64) * (3.0 if step % 2 else 1e-3)
                 for n in sizes]
        opt.step([g.to(dev, torch.float32) for g in grads])
        # the oracle sees the same float32 gradients
        g32 = [g.float().double() for g in grads]
        used = LO.clip_by_global_norm(g32, clip) if clip is not None else g32
        ref, mu, nu = LO.adamw_update(ref, used, mu, nu, step, sched(step))
        for i, (a, w) in enumerate(zip(dev_params, ref)):
            torch.testing.assert_close(a.detach().cpu().double(), w, rtol=2e-6, atol=2e-7,
                                       msg=lambda m: f"step {step} tensor {i}: {m}")
        for i, (a, w) in enumerate(zip(opt.nu, nu)):
            torch.testing.assert_close(a.cpu().double(), w, rtol=2e-6, atol=1e-12,
                                       msg=lambda m: f"step {step} nu {i}: {m}")
    if clip is not None:
        assert opt.last_norm is not None and opt.last_norm.is_cuda


def test_released_checkpoint_runs_and_matches_oracle(m3, dev, tmp_path):
    """``tests.py:1058-1198`` on the device: a released-format checkpoint (config.json
    with vocab padding, gated MLP, tied head) loaded from a local directory runs through
    `lm_forward` to the oracle's logits, survives an npz save/load unchanged, and drives
    `generate` with non-byte token ids."""
    import json

    from test_checkpoint_cpu import CFG_JSON, fake_released_sd

    CV = m3.convert
    cfg = CV.config_from_hf(CFG_JSON, chunk=64, policy_name="f32")
    sd = fake_released_sd(cfg, seed=3)
    (tmp_path / "config.json").write_text(json.dumps(CFG_JSON))
    torch.save({k: v.clone() for k, v in sd.items()}, str(tmp_path / "pytorch_model.bin"))
    params, cfg = CV.load_pretrained(str(tmp_path), device=dev, chunk=64, policy_name="f32")
    toks = tokens_for(cfg, 2, 128, 21)
    got = m3.model.lm_forward(params, toks.to(dev), cfg)
    lay = dict(d_state=16, headdim=16, expand=2, rope_fraction=0.5, chunk=64, a_floor=2e-4,
               norm_eps=1e-5)
    ref = LO.lm_forward(LO.from_lm_params(params), toks, lay)
    assert_maxrel(got, ref, 1e-4, "released checkpoint logits")
    path = m3.checkpoint.save(str(tmp_path / "ckpt.npz"), params, cfg)
    again, cfg2 = m3.checkpoint.load(path, device=dev)
    assert cfg2 == cfg
    assert torch.equal(m3.model.lm_forward(again, toks.to(dev), cfg2), got)
    ids = [7, 11, 42]
    out = m3.train.generate(params, cfg, 0, ids, n_tokens=4, rep_penalty=1.0)
    assert out[:3] == ids and len(out) == 7 and all(0 <= t < cfg.vocab_size for t in out)
