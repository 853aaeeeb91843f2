"""Torch-CPU restatement of the reference's byte-LM stack, optimizer and sampler
(TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and ``bench.py``'s CPU leg, never by
the package).

Each function cites the reference file:line it restates. Parameters are plain dicts of
CPU tensors (see `from_lm_params`); pass float64 for the tight checks. The layer itself
is `siso_oracle.layer_forward` / `layer_decode_step`.

How each function is pinned (``tests/test_lm_oracle.py``):

* ``gated_mlp`` -- a hand-computed known answer that fails if the value and gate halves
  are swapped or the gate's nonlinearity is dropped.
* ``lm_forward`` -- with every residual branch zeroed (``out_proj = fc2 = 0``) the stack
  collapses to ``rms_norm(embed[t]) @ embed.T`` (closed form); and a chain of
  ``lm_decode_step`` calls reproduces ``lm_forward``'s logits at every position (the
  recurrent decode against the chunked prefill, ``tests.py:734-877``'s invariant lifted
  to the stack).
* ``adamw_update`` -- equal to ``torch.optim.AdamW`` (float64, single-tensor path) over
  several steps with a changing learning rate (a library routine).
* ``clip_by_global_norm`` -- known answers (``[3, 4]`` clipped to norm 1 is
  ``[0.6, 0.8]``; below the bound it is untouched).
* ``warmup_cosine`` -- the closed-form values at 0, mid-warmup, the peak, the cosine
  midpoint and the end.
* ``filtered_logits`` -- known answers: the nucleus of ``softmax([1, 2, 3, 0])`` at
  ``top_p = 0.9`` keeps exactly the top three; a vanishing ``top_p`` keeps the argmax
  only; the repetition penalty divides positive and multiplies negative logits.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

from . import siso_oracle as O

Tensor = torch.Tensor

SISO_FIELDS = ("in_proj", "out_proj", "dt_bias", "b_norm_weight", "c_norm_weight", "b_bias",
               "c_bias", "d_skip")


def from_lm_params(params, dtype=torch.float64) -> dict:
    """A package ``LMParams`` tree -> the oracle's dict of CPU tensors in ``dtype``."""
    c = lambda t: None if t is None else t.detach().to("cpu", dtype)  # noqa: E731
    blocks = []
    for b in params.blocks:
        blk = {"norm_gain": c(b.norm_gain),
               "siso": {f: c(getattr(b.siso, f)) for f in SISO_FIELDS}}
        if b.mlp is not None:
            blk.update(mlp_norm_gain=c(b.mlp_norm_gain), fc1=c(b.mlp.fc1), fc2=c(b.mlp.fc2))
        blocks.append(blk)
    return {"embed": c(params.embed), "blocks": blocks, "final_norm": c(params.final_norm),
            "head": c(params.head)}


def gated_mlp(fc1: Tensor, fc2: Tensor, x: Tensor) -> Tensor:
    """``model.py:128-141``: ``fc2(value * silu(gate))``; value = first half of fc1's
    columns, gate = second half."""
    value, gate = (x @ fc1.to(x.dtype)).chunk(2, dim=-1)
    return (value * F.silu(gate)) @ fc2.to(x.dtype)


def _head(params: dict) -> Tensor:
    return params["embed"].t() if params["head"] is None else params["head"]


def lm_forward(params: dict, tokens: Tensor, lay: dict, states: Optional[list] = None,
               mm_dtype=None):
    """``model.py:194-232``: embed -> per block ``x += siso(rms_norm(x))`` then (with an
    MLP) ``x += mlp(rms_norm2(x))`` -> ``rms_norm(x) @ head``. ``lay`` holds the layer
    hyperparameters (d_state, headdim, expand, rope_fraction, chunk, a_floor, norm_eps).
    Returns logits, or ``(logits, states)`` when ``states`` is given."""
    eps = lay["norm_eps"]
    x = params["embed"][tokens]
    new_states = []
    for i, b in enumerate(params["blocks"]):
        h = O.rms_norm(x, b["norm_gain"], eps)
        y, st = O.layer_forward(b["siso"], h, lay["d_state"], lay["headdim"], lay["expand"],
                                lay["rope_fraction"], lay["chunk"], lay["a_floor"], eps,
                                state=None if states is None else states[i],
                                mm_dtype=mm_dtype)
        new_states.append(st)
        x = x + y
        if "fc1" in b:
            x = x + gated_mlp(b["fc1"], b["fc2"], O.rms_norm(x, b["mlp_norm_gain"], eps))
    logits = O.rms_norm(x, params["final_norm"], eps) @ _head(params).to(x.dtype)
    return (logits, new_states) if states is not None else logits


def lm_loss(params: dict, xs: Tensor, ys: Tensor, lay: dict, mm_dtype=None) -> Tensor:
    """``train.py:414-416``: mean softmax cross-entropy with integer labels."""
    logits = lm_forward(params, xs, lay, mm_dtype=mm_dtype)
    return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), ys.reshape(-1))


def zero_states(params: dict, batch: int, lay: dict, dtype=torch.float64) -> list:
    """``model.py:235-241``."""
    out = []
    for b in params["blocks"]:
        d_model = b["norm_gain"].shape[0]
        _, h, nr, _ = O.layer_dims(d_model, lay["d_state"], lay["headdim"], lay["expand"],
                                   lay["rope_fraction"])
        out.append(O.zero_state(batch, h, lay["headdim"], lay["d_state"], nr, dtype))
    return out


def lm_decode_step(params: dict, token: Tensor, states: list, lay: dict, mm_dtype=None):
    """``model.py:244-296``: one token ``(B,)`` through the stack -> ``((B, vocab),
    states)`` using the layer's per-token step."""
    eps = lay["norm_eps"]
    x = params["embed"][token]
    out_states = []
    for i, b in enumerate(params["blocks"]):
        h = O.rms_norm(x, b["norm_gain"], eps)
        y, st = O.layer_decode_step(b["siso"], h, states[i], lay["d_state"], lay["headdim"],
                                    lay["expand"], lay["rope_fraction"], lay["a_floor"], eps,
                                    mm_dtype=mm_dtype)
        out_states.append(st)
        x = x + y
        if "fc1" in b:
            x = x + gated_mlp(b["fc1"], b["fc2"], O.rms_norm(x, b["mlp_norm_gain"], eps))
    logits = O.rms_norm(x, params["final_norm"], eps) @ _head(params).to(x.dtype)
    return logits, out_states


# ------------------------------------------------------------------------------------
# optimizer (optax chain of train.py:799-805)
# ------------------------------------------------------------------------------------


def warmup_cosine(count: int, init: float, peak: float, warmup: int, decay_steps: int,
                  end: float) -> float:
    """optax ``warmup_cosine_decay_schedule`` (``train.py:799-802``): linear
    ``init -> peak`` over ``warmup`` updates, then ``end + (peak - end) * (1 +
    cos(pi * s / (decay_steps - warmup))) / 2`` with ``s`` clipped to the decay span."""
    if count < warmup:
        return init + (peak - init) * count / warmup
    span = decay_steps - warmup
    s = min(count - warmup, span)
    return end + (peak - end) * 0.5 * (1.0 + math.cos(math.pi * s / span))


def clip_by_global_norm(grads: list, max_norm: float) -> list:
    """optax ``clip_by_global_norm``: ``g * max_norm / ||g||`` when ``||g|| >= max_norm``."""
    norm = math.sqrt(sum(float((g.double() ** 2).sum()) for g in grads))
    if norm < max_norm:
        return [g.clone() for g in grads]
    return [g * (max_norm / norm) for g in grads]


def adamw_update(params: list, grads: list, mu: list, nu: list, count: int, lr: float,
                 b1=0.9, b2=0.999, eps=1e-8, weight_decay=0.1):
    """optax ``adamw`` for update number ``count + 1``: returns ``(params, mu, nu)``.
    ``update = mu_hat / (sqrt(nu_hat) + eps) + weight_decay * p``; ``p -= lr * update``."""
    t = count + 1
    new_p, new_mu, new_nu = [], [], []
    for p, g, m, v in zip(params, grads, mu, nu):
        m = b1 * m + (1 - b1) * g
        v = b2 * v + (1 - b2) * g * g
        upd = (m / (1 - b1 ** t)) / (torch.sqrt(v / (1 - b2 ** t)) + eps) + weight_decay * p
        new_p.append(p - lr * upd)
        new_mu.append(m)
        new_nu.append(v)
    return new_p, new_mu, new_nu


# ------------------------------------------------------------------------------------
# sampler (train.py:454-500)
# ------------------------------------------------------------------------------------


def filtered_logits(logits: Tensor, seen: Tensor, temperature: float, top_p: float,
                    rep_penalty: float) -> Tensor:
    """``train.py:454-500`` before the draw, for one ``(vocab,)`` row: penalty on seen
    entries (divide positive logits, multiply negative ones), temperature, then keep the
    sorted entries whose preceding probability mass is below ``top_p``."""
    lg = logits.double().clone()
    for i in range(lg.shape[0]):
        if bool(seen[i]):
            lg[i] = lg[i] / rep_penalty if lg[i] > 0 else lg[i] * rep_penalty
    lg = lg / temperature
    order = sorted(range(lg.shape[0]), key=lambda i: -float(lg[i]))
    probs = torch.softmax(lg[order], dim=0)
    out = torch.full_like(lg, float("-inf"))
    before = 0.0
    for rank, i in enumerate(order):
        if before < top_p:
            out[i] = lg[i]
        before += float(probs[rank])
    return out
