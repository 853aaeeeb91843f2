"""Training step, optimizer, sampler and generation for the byte LM (``train.py`` surface).

* `warmup_cosine_decay_schedule`, `clip_by_global_norm_` and `AdamW` restate the optax
  chain the reference trains with (``train.py:799-805``): a global-norm clip at
  ``CLIP_NORM`` before decoupled-weight-decay Adam (b1 0.9, b2 0.999, eps 1e-8, decay on
  every tensor), with a linear warmup into a cosine decay. The clip and the update run as
  multi-tensor (``torch._foreach_*``) launches with no host synchronisation.
* `make_step` is ``train.py:382-451``'s one-device step: loss and gradients through
  `model.lm_forward` (the fused HIP layer), then the optimizer, params updated in place.
* `_pick_token`, `generate` and `sample` are ``train.py:454-624``: chunked prefill, then
  `model.lm_decode_step` per token, sampling with repetition penalty, temperature and
  nucleus (top-p) filtering. `DecodeGraph` records one decode step of the whole stack as
  a HIP graph (one replay per token instead of ~10 launches per layer).
* `zipf_bytes`, `batches` and `bigram_baseline` are the synthetic data side: i.i.d.
  Zipf-distributed bytes for the training benchmark, the random-window batcher of
  ``train.py:273-281`` and the smoothed-bigram entropy of ``train.py:284-295``.
"""

from __future__ import annotations

import codecs
import collections
import math
import sys
from typing import Any, Callable, Iterable, Optional

import numpy as np
import torch
import torch.nn.functional as F

from . import kernels as K
from . import model as M

Tensor = torch.Tensor

#: Global gradient-norm clip, applied before AdamW (``train.py:102``).
CLIP_NORM = 1.0


# ------------------------------------------------------------------------------------
# data
# ------------------------------------------------------------------------------------


def zipf_bytes(n_bytes: int, s: float = 1.1, seed: int = 0) -> np.ndarray:
    """``n_bytes`` i.i.d. bytes with ``P(byte = v) ∝ (v + 1)^-s`` over the 256 values,
    from a seeded numpy generator (the synthetic corpus of the training benchmark)."""
    p = np.arange(1, 257, dtype=np.float64) ** -s
    p /= p.sum()
    rng = np.random.default_rng(seed)
    return rng.choice(256, size=n_bytes, p=p).astype(np.uint8)


def batches(data: np.ndarray, batch: int, seqlen: int, seed: int = 0, device=None):
    """Infinite stream of ``(inputs, targets)``, both ``(batch, seqlen)`` int64, from
    random windows of ``data`` (``train.py:273-281``); targets are inputs shifted by one."""
    n = len(data) - seqlen - 1
    if n <= 0:
        raise ValueError(f"corpus of {len(data)} bytes is too short for seqlen {seqlen}")
    rng = np.random.default_rng(seed)
    while True:
        idx = rng.integers(0, n, size=batch)
        xs = np.stack([data[i:i + seqlen] for i in idx]).astype(np.int64)
        ys = np.stack([data[i + 1:i + seqlen + 1] for i in idx]).astype(np.int64)
        yield torch.from_numpy(xs).to(device), torch.from_numpy(ys).to(device)


def bigram_baseline(data: np.ndarray) -> float:
    """Cross-entropy in nats of a Laplace-smoothed bigram model fitted on ``data``
    (``train.py:284-295``)."""
    counts = np.ones((256, 256), np.float64)
    np.add.at(counts, (data[:-1], data[1:]), 1.0)
    probs = counts / counts.sum(axis=1, keepdims=True)
    return float(-np.mean(np.log(probs[data[:-1], data[1:]])))


# ------------------------------------------------------------------------------------
# optimizer
# ------------------------------------------------------------------------------------


def warmup_cosine_decay_schedule(init_value: float, peak_value: float, warmup_steps: int,
                                 decay_steps: int, end_value: float = 0.0) -> Callable:
    """Learning rate at update ``count`` (0-based): linear from ``init_value`` to
    ``peak_value`` over ``warmup_steps``, then a cosine from ``peak_value`` to
    ``end_value`` reached at ``decay_steps`` (total, warmup included), constant after.
    The schedule ``train.py:799-802`` builds with optax."""

    def sched(count: int) -> float:
        if warmup_steps > 0 and count < warmup_steps:
            return init_value + (peak_value - init_value) * count / warmup_steps
        span = max(decay_steps - warmup_steps, 1)
        t = min(max(count - warmup_steps, 0), span) / span
        return end_value + (peak_value - end_value) * 0.5 * (1.0 + math.cos(math.pi * t))

    return sched


def global_norm(grads: list) -> Tensor:
    """``sqrt(sum_i ||g_i||^2)`` over a list of tensors, as a device scalar in float32
    (float64 if any gradient is float64)."""
    norms = torch._foreach_norm(grads)
    dt = torch.float64 if any(n.dtype == torch.float64 for n in norms) else torch.float32
    return torch.linalg.vector_norm(torch.stack([n.to(dt) for n in norms]))


def clip_by_global_norm_(grads: list, max_norm: float) -> Tensor:
    """Scale ``grads`` in place by ``max_norm / norm`` when their global norm reaches
    ``max_norm`` (optax ``clip_by_global_norm``: no epsilon, untouched below the bound).
    Returns the pre-clip norm; no host synchronisation."""
    norm = global_norm(grads)
    scale = torch.where(norm < max_norm, torch.ones_like(norm), max_norm / norm)
    torch._foreach_mul_(grads, scale)
    return norm


class AdamW:
    """Clip-then-AdamW over a fixed list of float tensors, updated in place.

    Per update ``t = 1, 2, ...`` with ``lr = schedule(t - 1)``:
    ``mu = b1 mu + (1 - b1) g``; ``nu = b2 nu + (1 - b2) g^2``;
    ``p -= lr * ((mu / (1 - b1^t)) / (sqrt(nu / (1 - b2^t)) + eps) + weight_decay * p)``
    -- optax's ``chain(clip_by_global_norm, adamw)`` as used by ``train.py:803-805``.
    Moments are float32 (the master weights' dtype). ``clip=None`` disables the clip."""

    def __init__(self, params: list, schedule: Callable | float, b1: float = 0.9,
                 b2: float = 0.999, eps: float = 1e-8, weight_decay: float = 0.1,
                 clip: Optional[float] = CLIP_NORM):
        self.params = list(params)
        for p in self.params:
            if not p.is_floating_point():
                raise ValueError("AdamW needs floating-point parameters")
        self.schedule = schedule if callable(schedule) else (lambda _c, v=float(schedule): v)
        self.b1, self.b2, self.eps, self.weight_decay, self.clip = b1, b2, eps, weight_decay, clip
        self.mu = [torch.zeros_like(p) for p in self.params]
        self.nu = [torch.zeros_like(p) for p in self.params]
        self.count = 0
        self.last_norm: Optional[Tensor] = None

    @torch.no_grad()
    def step(self, grads: Optional[list] = None) -> None:
        """One update from ``grads`` (default: each parameter's ``.grad``)."""
        if grads is None:
            grads = [p.grad for p in self.params]
        if any(g is None for g in grads):
            raise ValueError("a parameter has no gradient")
        grads = [g if g.dtype == p.dtype else g.to(p.dtype) for g, p in zip(grads, self.params)]
        lr = float(self.schedule(self.count))
        self.count += 1
        t = self.count
        if all(p.is_cuda and p.dtype == torch.float32 for p in self.params):
            # device float32 (the master weights): the clip factor stays on the device and
            # the update is one m3s_adamw pass over every tensor
            scale = None
            if self.clip is not None:
                norm = global_norm(grads)
                self.last_norm = norm
                scale = torch.where(norm < self.clip, torch.ones_like(norm),
                                    self.clip / norm).float()
            K.adamw_update(self.params, [g.contiguous() for g in grads], self.mu, self.nu,
                           lr, self.b1, self.b2, self.eps, self.weight_decay, t, scale)
            return
        if self.clip is not None:
            self.last_norm = clip_by_global_norm_(grads, self.clip)
        torch._foreach_lerp_(self.mu, grads, 1.0 - self.b1)
        torch._foreach_mul_(self.nu, self.b2)
        torch._foreach_addcmul_(self.nu, grads, grads, value=1.0 - self.b2)
        denom = torch._foreach_sqrt(self.nu)
        torch._foreach_div_(denom, math.sqrt(1.0 - self.b2 ** t))
        torch._foreach_add_(denom, self.eps)
        if self.weight_decay:
            torch._foreach_mul_(self.params, 1.0 - lr * self.weight_decay)
        torch._foreach_addcdiv_(self.params, self.mu, denom, value=-lr / (1.0 - self.b1 ** t))

    def zero_grad(self) -> None:
        for p in self.params:
            p.grad = None


def make_optimizer(params: M.LMParams, lr: float = 1e-3, warmup: int = 100,
                   steps: int = 2000, weight_decay: float = 0.1,
                   clip: Optional[float] = CLIP_NORM) -> AdamW:
    """The reference's training optimizer (``train.py:799-805``): warmup from ``lr/10`` to
    ``lr``, cosine back to ``lr/10`` at ``steps``; clip 1.0; AdamW with decay 0.1."""
    sched = warmup_cosine_decay_schedule(lr * 0.1, lr, warmup, max(steps, warmup + 1), lr * 0.1)
    return AdamW(M.lm_leaves(params), sched, weight_decay=weight_decay, clip=clip)


def make_step(cfg: M.LMConfig, opt: AdamW, interpret: Any = False):
    """One training step (``train.py:382-426``, one device): ``step(params, opt_state,
    xs, ys) -> (loss, params, opt_state)``. The parameters must be the optimizer's
    (``requires_grad`` leaves); they are updated in place and returned, as is the
    optimizer (its own state). ``loss`` is a device scalar (no host synchronisation)."""

    def step(params: M.LMParams, opt_state: AdamW, xs: Tensor, ys: Tensor):
        loss = M.lm_loss(params, xs, ys, cfg)
        loss.backward()
        opt_state.step()
        opt_state.zero_grad()
        return loss.detach(), params, opt_state

    return step


def train_params(params: M.LMParams) -> M.LMParams:
    """Detached float32 copies of ``params`` that require grad (master weights)."""
    return M.lm_map(lambda t: t.detach().float().clone().requires_grad_(True), params)


# ------------------------------------------------------------------------------------
# sampling and generation
# ------------------------------------------------------------------------------------


def _filtered_logits(logits: Tensor, seen: Tensor, temperature: float, top_p: float,
                     rep_penalty: float) -> Tensor:
    """``train.py:454-500`` up to the draw: sign-aware repetition penalty on ``seen``
    entries, temperature, then nucleus filtering -- keep the smallest prefix of the
    descending distribution whose mass before each entry is below ``top_p`` (the top
    entry is always kept); the rest becomes ``-inf``. Float32, same shape."""
    lg = logits.float()
    penalized = torch.where(lg > 0, lg / rep_penalty, lg * rep_penalty)
    lg = torch.where(seen, penalized, lg) / temperature
    srt, order = torch.sort(lg, dim=-1, descending=True)
    probs = torch.softmax(srt, dim=-1)
    keep = (torch.cumsum(probs, dim=-1) - probs) < top_p
    masked = torch.where(keep, srt, torch.full_like(srt, float("-inf")))
    return torch.full_like(lg, float("-inf")).scatter(-1, order, masked)


def _pick_token(logits: Tensor, seen: Tensor, generator: Optional[torch.Generator],
                params, vocab: int) -> Tensor:
    """Penalty + temperature + top-p, then one categorical draw (``train.py:454-500``).
    ``params`` is ``(temperature, top_p, rep_penalty)``. The draw is Gumbel-max over the
    filtered logits with uniforms from ``generator``; returns a 0-dim int64 tensor."""
    temperature, top_p, rep_penalty = (float(v) for v in params)
    lg = _filtered_logits(logits, seen, temperature, top_p, rep_penalty)
    u = torch.rand(lg.shape, generator=generator, device=lg.device, dtype=torch.float32)
    gumbel = -torch.log(-torch.log(u.clamp_min(torch.finfo(torch.float32).tiny)))
    return torch.argmax(lg + gumbel, dim=-1) % vocab


class DecodeGraph:
    """One `model.lm_decode_step` of the whole stack recorded as a HIP graph.

    The graph owns static buffers: the input token ``(batch,)``, the per-layer states
    and the float32 logits. `load_states` copies a carry in; `step(token)` copies the
    token in, replays, and returns the logits buffer (overwritten by the next replay).
    Every kernel of the step writes device memory only (the decode kernel updates the
    states in place); nothing is cleared with a memset, so replays are exact repeats of
    the eager step."""

    def __init__(self, params: M.LMParams, cfg: M.LMConfig, batch: int = 1, warmup: int = 2):
        dev = params.embed.device
        if dev.type != "cuda":
            raise ValueError("DecodeGraph needs parameters on the ROCm device")
        self.params, self.cfg = params, cfg
        self.token = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.states = M.zero_states(cfg, batch, device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(warmup):   # first calls load code objects and cached weights
                M.lm_decode_step(params, self.token, self.states, cfg)
        torch.cuda.current_stream(dev).wait_stream(side)
        for s in self.states:
            for t in s:
                t.zero_()
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.logits, _ = M.lm_decode_step(params, self.token, self.states, cfg)

    def load_states(self, states: list) -> None:
        for dst, src in zip(self.states, states):
            for d, s in zip(dst, src):
                d.copy_(s)

    def step(self, token: Tensor) -> Tensor:
        self.token.copy_(token.reshape(-1))
        self.graph.replay()
        return self.logits


def _as_generator(key: Any, device) -> torch.Generator:
    if isinstance(key, torch.Generator):
        return key
    g = torch.Generator(device=device)
    g.manual_seed(int(key))
    return g


@torch.no_grad()
def generate(params: M.LMParams, cfg: M.LMConfig, key: Any, prompt_ids,
             n_tokens: int = 192, temperature: float = 0.9, top_p: float = 0.95,
             rep_penalty: float = 1.15, rep_window: int = 64,
             stop_ids: Optional[Iterable[int]] = None, interpret: Any = False,
             on_token: Optional[Callable[[int], None]] = None, graph: bool = True) -> list:
    """Token ids: chunked prefill, then one decode step per token (``train.py:503-582``).

    The prompt's whole ``chunk`` blocks (keeping at least one token back) go through
    `model.lm_forward` with a zero carry; the remainder and every generated token go
    through the decode step (a `DecodeGraph` replay with ``graph=True``). Sampling keeps
    a ``rep_window``-token window of recent ids for the repetition penalty. Generation
    stops early after emitting an id in ``stop_ids``. ``key`` is an int seed or a device
    ``torch.Generator``. Returns the prompt ids followed by the generated ones."""
    ids = [int(t) for t in np.asarray(prompt_ids).reshape(-1)]
    if not ids:
        raise ValueError("prompt_ids is empty; at least one token is needed")
    dev = params.embed.device
    gen = _as_generator(key, dev)
    params = M.decode_params(params, cfg)
    chunk = cfg.siso.chunk
    n_whole = (len(ids) - 1) // chunk * chunk
    if graph:
        dg = DecodeGraph(params, cfg, batch=1)
        step = lambda tok: (dg.step(tok), None)  # noqa: E731
        states = None
    else:
        states = M.zero_states(cfg, 1, device=dev)
        step = lambda tok: M.lm_decode_step(params, tok, states, cfg)  # noqa: E731
    last = None
    if n_whole:
        logits, pre = M.lm_forward(params, torch.tensor([ids[:n_whole]], device=dev), cfg,
                                   states=M.zero_states(cfg, 1, device=dev))
        last = logits[0, -1]
        if graph:
            dg.load_states(pre)
        else:
            for dst, src in zip(states, pre):
                for d, s in zip(dst, src):
                    d.copy_(s)
    for t in ids[n_whole:]:
        logits, _ = step(torch.tensor([t], device=dev))
        last = logits[0]
    stops = frozenset(int(s) for s in stop_ids) if stop_ids else frozenset()
    penalty = _RecentIds(rep_window, cfg.vocab_size, dev, ids)
    out = list(ids)
    filt = (temperature, top_p, rep_penalty)
    for _ in range(n_tokens):
        nxt_t = _pick_token(last, penalty.mask, gen, filt, cfg.vocab_size)
        nxt = int(nxt_t)
        out.append(nxt)
        if on_token is not None:
            on_token(nxt)
        if nxt in stops:
            break
        penalty.push(nxt)
        logits, _ = step(nxt_t.reshape(1))
        last = logits[0]
    return out


class _RecentIds:
    """The ids the repetition penalty applies to: those among the last ``window``
    tokens. Host-side counts over a bounded deque decide membership; the device mask
    that `_pick_token` reads changes only when an id enters or leaves the window."""

    def __init__(self, window: int, vocab: int, device, history) -> None:
        self.window = max(0, int(window))
        self.mask = torch.zeros(vocab, dtype=torch.bool, device=device)
        self.recent: collections.deque = collections.deque()
        self.count: collections.Counter = collections.Counter()
        for t in list(history)[-self.window:] if self.window else []:
            self.push(t)

    def push(self, tok: int) -> None:
        if not self.window:
            return
        self.recent.append(tok)
        self.count[tok] += 1
        if self.count[tok] == 1:
            self.mask[tok] = True
        if len(self.recent) > self.window:
            old = self.recent.popleft()
            self.count[old] -= 1
            if self.count[old] == 0:
                del self.count[old]
                self.mask[old] = False


def sample(params: M.LMParams, cfg: M.LMConfig, key: Any, prompt: bytes = b"the ",
           n_tokens: int = 192, temperature: float = 0.9, top_p: float = 0.95,
           rep_penalty: float = 1.15, rep_window: int = 64, interpret: Any = False,
           stream: bool = True) -> bytes:
    """Byte-level wrapper over `generate` (``train.py:585-624``); ``stream`` prints bytes
    as they arrive."""
    emit = None
    if stream:
        # bytes arrive one at a time; an incremental decoder holds back the leading
        # bytes of a multi-byte character until it is complete
        text = codecs.getincrementaldecoder("utf-8")(errors="replace")
        sys.stdout.write(text.decode(prompt))
        sys.stdout.flush()

        def emit(t: int) -> None:
            sys.stdout.write(text.decode(bytes((t,))))
            sys.stdout.flush()

    ids = generate(params, cfg, key, np.frombuffer(prompt, dtype=np.uint8), n_tokens=n_tokens,
                   temperature=temperature, top_p=top_p, rep_penalty=rep_penalty,
                   rep_window=rep_window, on_token=emit)
    if stream:
        sys.stdout.write(text.decode(b"", final=True) + "\n")
        sys.stdout.flush()
    return bytes(ids)
