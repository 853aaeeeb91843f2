"""Pins the LM-stack oracle (oracle/lm_oracle.py) and checks the package's host-side LM
logic (config, init, optimizer, schedule, sampler filter, data helpers) on the CPU.

Every oracle check is a known answer, a closed form, an invariant of the maths or a
library routine -- never the oracle's own formula retyped.
"""

import math

import numpy as np
import pytest
import torch

from oracle import lm_oracle as LO
from oracle import siso_oracle as O

f64 = torch.float64


def small_lm(m3, d_intermediate=24, tie_head=True, n_layers=2, vocab=11, seed=0):
    """A small float64 LM with every parameter perturbed away from its init."""
    scfg = m3.SISOConfig(d_model=32, d_state=16, headdim=16, expand=2, chunk=32,
                         policy_name="f32")
    cfg = m3.model.LMConfig(vocab_size=vocab, n_layers=n_layers, siso=scfg,
                            tie_head=tie_head, d_intermediate=d_intermediate)
    params = m3.model.init_lm(cfg, seed, dtype=torch.float64)
    g = torch.Generator().manual_seed(seed + 100)

    def jitter(t):
        if t.dim() == 2 and t.shape[0] != vocab:
            return t * (1 + 0.2 * torch.randn(t.shape, generator=g, dtype=t.dtype))
        return t + 0.3 * torch.randn(t.shape, generator=g, dtype=t.dtype)

    params = m3.model.lm_map(jitter, params)
    lay = dict(d_state=16, headdim=16, expand=2, rope_fraction=0.5, chunk=32, a_floor=1e-4,
               norm_eps=1e-5)
    return cfg, params, lay


# ---------------------------------------------------------------------------------
# oracle pins
# ---------------------------------------------------------------------------------


def test_gated_mlp_known_answer():
    """value = 2, gate = 3 -> 2 * 3 * sigmoid(3); swapping the halves would give
    3 * 2 * sigmoid(2), dropping the nonlinearity 6."""
    x = torch.tensor([[1.0]], dtype=f64)
    fc1 = torch.tensor([[2.0, 3.0]], dtype=f64)
    fc2 = torch.tensor([[1.0]], dtype=f64)
    want = 2.0 * 3.0 / (1.0 + math.exp(-3.0))
    assert abs(float(LO.gated_mlp(fc1, fc2, x)) - want) < 1e-14


@pytest.mark.parametrize("tie", [True, False])
def test_lm_forward_collapses_without_residual_branches(m3, tie):
    cfg, params, lay = small_lm(m3, tie_head=tie)
    p = LO.from_lm_params(params)
    for b in p["blocks"]:
        b["siso"]["out_proj"].zero_()
        b["fc2"].zero_()
    tokens = torch.tensor([[1, 5, 7, 2] * 8, [0, 10, 3, 3] * 8])
    got = LO.lm_forward(p, tokens, lay)
    x = p["embed"][tokens]
    rstd = 1.0 / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-5)
    head = p["embed"].t() if tie else p["head"]
    want = (x * rstd * p["final_norm"]) @ head
    torch.testing.assert_close(got, want, rtol=1e-13, atol=1e-13)


def _per_token_lm(p, tokens, lay, variant="reference"):
    """Known answer for `lm_forward` on a model whose state decays at once (every a_raw is
    thousands, so 2^{A_i - A_j} underflows to 0 for i > j and the carried state vanishes):
    the layer then maps each token on its own, ``y_t = [(D_h + gamma_t (u_t . w_t)) x_t
    silu(z_t)]_h @ out_proj`` (the scan's diagonal term, kernel_fwd.py:146-187; the rotation
    leaves u . w unchanged), and the whole stack is a per-token closed form.
    ``variant`` builds the stack in the block order of model.py:194-232 ("reference") or
    with one plausible mistake, to show that the known answer tells them apart."""
    eps = lay["norm_eps"]
    b = p["blocks"][0]
    sp = b["siso"]
    n, hd = lay["d_state"], lay["headdim"]

    def norm(x, g):
        return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * g

    def mixer(h):
        d_model = h.shape[-1]
        d_inner, nh, nr, _ = O.layer_dims(d_model, n, hd, lay["expand"], lay["rope_fraction"])
        proj = h @ sp["in_proj"]
        z, x, bb, cc, dt_raw, _, trap, _ = torch.split(
            proj, (d_inner, d_inner, n, n, nh, nh, nh, nr), dim=-1)
        u = norm(cc, sp["c_norm_weight"])[..., None, :] + sp["c_bias"]
        w = norm(bb, sp["b_norm_weight"])[..., None, :] + sp["b_bias"]
        dt = torch.nn.functional.softplus(dt_raw + sp["dt_bias"])
        gamma = dt * torch.sigmoid(trap)
        coef = sp["d_skip"] + gamma * (u * w).sum(-1)
        zz = z.unflatten(-1, (nh, hd))
        y = coef[..., None] * x.unflatten(-1, (nh, hd)) * zz * torch.sigmoid(zz)
        return y.flatten(-2) @ sp["out_proj"]

    def mlp(x):
        value, gate = (x @ b["fc1"]).chunk(2, dim=-1)
        return (value * gate * torch.sigmoid(gate)) @ b["fc2"]

    x = p["embed"][tokens]
    h = norm(x, b["norm_gain"])
    if variant == "post_norm":
        x1 = norm(x + mixer(x), b["norm_gain"])
    elif variant == "residual_from_normed":
        x1 = h + mixer(h)
    else:
        x1 = x + mixer(h)
    if variant == "mlp_reads_mixer_gain":
        x2 = x1 + mlp(norm(x1, b["norm_gain"]))
    elif variant == "mlp_before_residual":
        x2 = x1 + mlp(norm(x, b["mlp_norm_gain"]))
    else:
        x2 = x1 + mlp(norm(x1, b["mlp_norm_gain"]))
    head = p["embed"].t() if p["head"] is None else p["head"]
    return norm(x2, p["final_norm"]) @ head


def test_lm_forward_block_order_known_answer(m3):
    """`lm_forward`'s block order (model.py:194-232: pre-norm with the block's gain, residual
    add of the raw stream, then the MLP on its own norm of the updated stream, the final
    norm, the tied head) against `_per_token_lm`'s closed form on a one-layer model whose
    mixer and MLP branches are both nonzero; each swapped order lands far from it."""
    cfg, params, lay = small_lm(m3, n_layers=1)
    p = LO.from_lm_params(params)
    g = torch.Generator().manual_seed(41)
    blk = p["blocks"][0]
    p["embed"] = 0.5 + torch.rand(p["embed"].shape, generator=g, dtype=f64)   # positive rows
    for key in ("norm_gain", "mlp_norm_gain"):
        blk[key] = 0.5 + torch.rand(blk[key].shape, generator=g, dtype=f64)
    p["final_norm"] = 0.5 + torch.rand(p["final_norm"].shape, generator=g, dtype=f64)
    # a_raw = 1e4 * sum(h) with h > 0: adt ~ -1e2 per token, the decay 2^(A_i - A_j) is 0
    d_inner, nh, _, _ = O.layer_dims(32, 16, 16, 2, 0.5)
    a0 = 2 * d_inner + 2 * 16 + nh
    blk["siso"]["in_proj"][:, a0:a0 + nh] = 1e4
    tokens = torch.tensor([[1, 5, 7, 2] * 8, [0, 10, 3, 3] * 8])
    got = LO.lm_forward(p, tokens, lay)
    want = _per_token_lm(p, tokens, lay)
    mixer_scale = float((want - _per_token_lm({**p, "blocks": [
        {**blk, "siso": {**blk["siso"], "out_proj": torch.zeros_like(blk["siso"]["out_proj"])}}]},
        tokens, lay)).abs().max())
    assert mixer_scale > 1e-2, "the mixer branch must be nonzero for the check to mean anything"
    torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)
    for variant in ("post_norm", "residual_from_normed", "mlp_reads_mixer_gain",
                    "mlp_before_residual"):
        wrong = _per_token_lm(p, tokens, lay, variant)
        assert O.max_rel(wrong, got) > 1e-3, variant


def test_lm_decode_chain_reproduces_forward(m3):
    """Token-by-token decode through the stack equals the chunked prefill's logits at
    every position, and the carried states agree (both in float64)."""
    cfg, params, lay = small_lm(m3)
    p = LO.from_lm_params(params)
    g = torch.Generator().manual_seed(5)
    tokens = torch.randint(0, cfg.vocab_size, (2, 64), generator=g)
    logits, st_f = LO.lm_forward(p, tokens, lay, states=LO.zero_states(p, 2, lay))
    states = LO.zero_states(p, 2, lay)
    for t in range(tokens.shape[1]):
        lg, states = LO.lm_decode_step(p, tokens[:, t], states, lay)
        torch.testing.assert_close(lg, logits[:, t], rtol=1e-9, atol=1e-10)
    for a, b in zip(states, st_f):
        torch.testing.assert_close(a.ssm, b.ssm, rtol=1e-9, atol=1e-10)
        torch.testing.assert_close(O.rel_error(a.phi, b.phi, angle=True), 0.0, rtol=0,
                                   atol=1e-9)


def test_adamw_matches_torch_adamw():
    g = torch.Generator().manual_seed(2)
    shapes = [(5, 3), (7,), (2, 2, 2)]
    params = [torch.randn(s, generator=g, dtype=f64) for s in shapes]
    ref = [p.clone().requires_grad_(True) for p in params]
    opt = torch.optim.AdamW(ref, lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1,
                            foreach=False)
    mu = [torch.zeros_like(p) for p in params]
    nu = [torch.zeros_like(p) for p in params]
    for step in range(6):
        lr = 1e-2 * (1 + step) / 3
        grads = [torch.randn(s, generator=g, dtype=f64) * (10 ** (step - 3)) for s in shapes]
        params, mu, nu = LO.adamw_update(params, grads, mu, nu, step, lr)
        for r, gr in zip(ref, grads):
            r.grad = gr.clone()
        opt.param_groups[0]["lr"] = lr
        opt.step()
        for a, b in zip(params, ref):
            torch.testing.assert_close(a, b.detach(), rtol=1e-12, atol=1e-14)


def test_clip_by_global_norm_known_answers():
    g = [torch.tensor([3.0], dtype=f64), torch.tensor([4.0], dtype=f64)]
    out = LO.clip_by_global_norm(g, 1.0)
    assert torch.allclose(torch.cat(out), torch.tensor([0.6, 0.8], dtype=f64), atol=1e-15)
    same = LO.clip_by_global_norm(g, 10.0)
    assert torch.equal(torch.cat(same), torch.tensor([3.0, 4.0], dtype=f64))


def test_warmup_cosine_closed_forms():
    s = lambda c: LO.warmup_cosine(c, 0.1, 1.0, 10, 110, 0.05)  # noqa: E731
    assert s(0) == 0.1
    assert abs(s(5) - 0.55) < 1e-15
    assert abs(s(10) - 1.0) < 1e-15
    assert abs(s(60) - (1.0 + 0.05) / 2) < 1e-15
    assert abs(s(110) - 0.05) < 1e-15 and abs(s(500) - 0.05) < 1e-15


def test_filtered_logits_known_answers():
    lg = torch.tensor([1.0, 2.0, 3.0, 0.0], dtype=f64)
    none = torch.zeros(4, dtype=torch.bool)
    # softmax sorted: .644, .237, .087, .032 -> mass before: 0, .644, .881, .968
    out = LO.filtered_logits(lg, none, 1.0, 0.9, 1.0)
    assert torch.equal(torch.isinf(out), torch.tensor([False, False, False, True]))
    assert torch.equal(out[:3], lg[:3])
    tiny = LO.filtered_logits(lg, none, 1.0, 1e-9, 1.0)
    assert torch.equal(torch.isfinite(tiny), torch.tensor([False, False, True, False]))
    pen = LO.filtered_logits(torch.tensor([2.0, -2.0, 0.5], dtype=f64),
                             torch.tensor([True, True, False]), 0.5, 1.0, 1.25)
    torch.testing.assert_close(pen, torch.tensor([3.2, -5.0, 1.0], dtype=f64))


# ---------------------------------------------------------------------------------
# host-side package logic
# ---------------------------------------------------------------------------------


@pytest.mark.parametrize("di,tie", [(0, True), (24, True), (24, False)])
def test_param_count_matches_init(m3, di, tie):
    cfg, params, _ = small_lm(m3, d_intermediate=di, tie_head=tie)
    n = sum(t.numel() for t in m3.model.lm_leaves(params))
    assert n == cfg.param_count()


def test_cfg5_param_count(m3):
    """The training benchmark's model: 8 layers, d_model 768, MLP 1536 -> 59.1M."""
    scfg = m3.SISOConfig(d_model=768, d_state=128, headdim=64, chunk=128)
    cfg = m3.model.LMConfig(vocab_size=256, n_layers=8, siso=scfg, d_intermediate=1536)
    assert abs(cfg.param_count() - 59.10e6) < 0.01e6


def test_schedule_matches_oracle(m3):
    T = m3.train
    s = T.warmup_cosine_decay_schedule(1e-4, 1e-3, 100, 2000, 1e-4)
    for c in (0, 1, 50, 99, 100, 101, 777, 1999, 2000, 5000):
        assert abs(s(c) - LO.warmup_cosine(c, 1e-4, 1e-3, 100, 2000, 1e-4)) < 1e-18


def test_adamw_and_clip_match_oracle(m3):
    T = m3.train
    g = torch.Generator().manual_seed(4)
    shapes = [(6, 4), (9,)]
    params = [torch.randn(s, generator=g, dtype=f64) for s in shapes]
    mine = [p.clone() for p in params]
    sched = T.warmup_cosine_decay_schedule(1e-3, 1e-2, 2, 6, 1e-3)
    opt = T.AdamW(mine, sched, weight_decay=0.1, clip=1.0)
    mu = [torch.zeros_like(p) for p in params]
    nu = [torch.zeros_like(p) for p in params]
    for step in range(5):
        grads = [torch.randn(s, generator=g, dtype=f64) * (0.1 if step % 2 else 3.0)
                 for s in shapes]
        opt.step([gr.clone() for gr in grads])
        clipped = LO.clip_by_global_norm(grads, 1.0)
        params, mu, nu = LO.adamw_update(params, clipped, mu, nu, step, sched(step))
        for a, b in zip(mine, params):
            torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-15)


def test_filtered_logits_matches_oracle(m3):
    g = torch.Generator().manual_seed(7)
    for trial in range(20):
        lg = torch.randn(40, generator=g) * 3
        seen = torch.rand(40, generator=g) < 0.3
        args = (0.7 + 0.1 * (trial % 5), 0.5 + 0.02 * trial, 1.0 + 0.05 * (trial % 4))
        got = m3.train._filtered_logits(lg, seen, *args)
        want = LO.filtered_logits(lg, seen, *args)
        assert torch.equal(torch.isinf(got), torch.isinf(want)), trial
        fin = torch.isfinite(want)
        torch.testing.assert_close(got[fin].double(), want[fin], rtol=1e-6, atol=1e-6)


def test_zipf_bytes_and_bigram(m3):
    T = m3.train
    data = T.zipf_bytes(200_000, s=1.1, seed=3)
    assert data.dtype == np.uint8 and data.shape == (200_000,)
    assert np.array_equal(data, T.zipf_bytes(200_000, s=1.1, seed=3))
    p = np.arange(1, 257, dtype=np.float64) ** -1.1
    p /= p.sum()
    freq = np.bincount(data, minlength=256) / data.size
    assert np.abs(freq - p).max() < 5e-3
    # i.i.d. bytes: the smoothed bigram's cross-entropy is close to the unigram entropy
    h = -(p * np.log(p)).sum()
    assert abs(T.bigram_baseline(data) - h) < 0.2
    xs, ys = next(T.batches(data, 4, 64, seed=1))
    assert xs.shape == ys.shape == (4, 64) and xs.dtype == torch.int64
    assert torch.equal(xs[:, 1:], ys[:, :-1])


def test_repetition_window_tracks_the_last_ids(m3):
    """The sampler's penalty set is exactly the ids among the last ``window`` tokens
    (prompt included), as a brute-force recount over the history says after each push,
    and a zero window penalises nothing."""
    RI = m3.train._RecentIds
    g = torch.Generator().manual_seed(3)
    history = torch.randint(0, 12, (9,), generator=g).tolist()
    win = 5
    rec = RI(win, 12, "cpu", history)
    hist = list(history)
    for tok in torch.randint(0, 12, (40,), generator=g).tolist():
        want = torch.zeros(12, dtype=torch.bool)
        want[list(set(hist[-win:]))] = True
        assert torch.equal(rec.mask, want), hist[-win:]
        rec.push(tok)
        hist.append(tok)
    off = RI(0, 12, "cpu", history)
    off.push(3)
    assert not bool(off.mask.any())
