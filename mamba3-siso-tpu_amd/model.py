"""A stacked Mamba-3 SISO language model (``model.py`` surface).

``n_layers`` SISO layers in a pre-norm residual stack with an embedding and an output
head (``model.py:1-22``):

    x = embed[tokens]
    for each block:  x = x + siso(rms_norm(x))
                     x = x + mlp(rms_norm2(x))        # only with d_intermediate > 0
    logits = rms_norm(x) @ head                       # head = embed.T when tied

Names, fields, defaults and initialisation follow ``model.py:39-296``. Precision: the
residual stream stays in the embedding's dtype (float32 master weights give a float32
stream, as in the reference), and every matrix product takes its operands in the
layer policy's operand dtype -- under ``"bf16"`` that is the bf16 operand rounding the
reference gets from the TPU's default matmul precision (``layout.py:243-291``). The
SISO mixer is `layer.mamba3_siso_layer` (one fused autograd node around the HIP scan
when no state is carried); per-token decode goes through the one-launch
`layer.mamba3_siso_decode_step`, which updates each layer's state in place.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any, NamedTuple, Optional

import torch
import torch.nn.functional as F

from . import kernels as K
from . import layer as LY
from . import layout as L
from .scan_prep import SISOState, zero_state

Tensor = torch.Tensor


@dataclasses.dataclass(frozen=True)
class LMConfig:
    """Model shape (``model.py:39-92``). ``siso`` is the per-layer config shared by every
    block; ``d_intermediate = 0`` means no MLP."""

    vocab_size: int
    n_layers: int
    siso: LY.SISOConfig
    tie_head: bool = True
    d_intermediate: int = 0

    @property
    def d_model(self) -> int:
        return self.siso.d_model

    def param_count(self) -> int:
        """Analytic parameter count (``model.py:65-92``). Exact for this build's trees:
        `init_lm` creates exactly these tensors."""
        c = self.siso
        per_layer = (c.d_model * c.d_in_proj + c.d_inner * c.d_model + c.nheads * 2
                     + c.d_state * 2 + c.nheads * c.d_state * 2 + c.d_model)
        if self.d_intermediate:
            per_layer += (c.d_model * 2 * self.d_intermediate
                          + self.d_intermediate * c.d_model + c.d_model)
        head = 0 if self.tie_head else self.d_model * self.vocab_size
        return self.vocab_size * self.d_model + self.n_layers * per_layer + self.d_model + head


class MLPParams(NamedTuple):
    """Gated MLP (``model.py:95-107``): ``fc1`` ``(d_model, 2*d_intermediate)`` produces
    the value half (first ``d_intermediate`` columns) and the gate half together."""

    fc1: Tensor
    fc2: Tensor


class BlockParams(NamedTuple):
    """One residual block (``model.py:110-116``)."""

    norm_gain: Tensor
    siso: LY.SISOParams
    mlp_norm_gain: Optional[Tensor] = None
    mlp: Optional[MLPParams] = None


class LMParams(NamedTuple):
    """Weights (``model.py:119-125``); ``blocks`` is a list of `BlockParams`."""

    embed: Tensor
    blocks: list
    final_norm: Tensor
    head: Optional[Tensor]


def _mm_dtype(cfg: LMConfig) -> torch.dtype:
    return L.policy(cfg.siso.policy_name).matmul


class _MatmulFn(torch.autograd.Function):
    """``x.to(dt) @ w.to(dt)`` as one autograd node whose weight gradient is
    `layer.weight_grad` (split over the tokens, float32 out) instead of one library GEMM
    with too few output tiles for the GPU; the input gradient is the usual product."""

    @staticmethod
    def forward(ctx, x, w, dt):
        xd, wd = x.to(dt), w.to(dt)
        ctx.save_for_backward(xd, wd)
        ctx.x_dtype, ctx.w_dtype = x.dtype, w.dtype
        return K.matmul(xd, wd)

    @staticmethod
    def backward(ctx, dy):
        xd, wd = ctx.saved_tensors
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = (dy @ wd.t()).to(ctx.x_dtype)
        if ctx.needs_input_grad[1]:
            dw = LY.weight_grad(xd.reshape(-1, xd.shape[-1]),
                                dy.reshape(-1, dy.shape[-1]).to(xd.dtype)).to(ctx.w_dtype)
        return dx, dw, None


def _mm(x: Tensor, w: Tensor, dt: torch.dtype) -> Tensor:
    """A matrix product with both operands in the policy's operand dtype (`_MatmulFn`)."""
    return _MatmulFn.apply(x, w, dt)


class _GateFn(torch.autograd.Function):
    """``value * silu(gate)`` of the fc1 product ``h`` = value | gate as one autograd node:
    one HIP pass each way (``m3s_swiglu_fwd`` / ``m3s_swiglu_bwd``), whose backward writes
    both halves' cotangents into one dense ``dh`` (the composed ops' backward builds them
    apart and concatenates)."""

    @staticmethod
    def forward(ctx, h, width):
        ctx.save_for_backward(h)
        ctx.width = width
        return K.swiglu_forward(h, width)

    @staticmethod
    def backward(ctx, da):
        (h,) = ctx.saved_tensors
        return K.swiglu_backward(h, da, ctx.width), None


def gated_mlp(p: MLPParams, x: Tensor, mm_dtype: Optional[torch.dtype] = None) -> Tensor:
    """``fc2(value * silu(gate))`` (``model.py:125-140``); value is the first half of
    ``fc1``'s output, gate the second (upstream's ``chunk(2, dim=-1)`` order). Products
    run in ``mm_dtype`` (default: ``x``'s dtype); the result is in that dtype. The gate
    runs as one HIP kernel each way (`_GateFn`)."""
    dt = x.dtype if mm_dtype is None else mm_dtype
    h = _mm(x, p.fc1, dt)
    return _mm(_GateFn.apply(h.contiguous(), p.fc1.shape[1] // 2), p.fc2, dt)


def init_lm(cfg: LMConfig, key: Any = 0, dtype=torch.float32, device=None) -> LMParams:
    """Fresh weights (``model.py:141-191``): embedding ``N(0, 0.02^2)``; each block's SISO
    weights from `layer.init_params` with ``out_proj`` scaled by ``1/sqrt(2 n_layers)``;
    ``fc1`` ``N(0, 1/d_model)``, ``fc2`` ``N(0, 1/d_intermediate)`` times the same residual
    scale; norm gains ones; an untied head ``N(0, 0.02^2)``.

    ``key`` is an int seed or a ``torch.Generator``; the draws happen on the CPU (JAX's
    threefry stream is not reproduced, only the distributions), then move to ``device``.
    """
    gen = key if isinstance(key, torch.Generator) else torch.Generator().manual_seed(int(key))
    d, di = cfg.d_model, cfg.d_intermediate
    embed = torch.randn(cfg.vocab_size, d, generator=gen) * 0.02
    resid = 1.0 / math.sqrt(2.0 * cfg.n_layers)
    blocks = []
    for _ in range(cfg.n_layers):
        p = LY.init_params(cfg.siso, gen, dtype)
        p = p._replace(out_proj=p.out_proj * resid)
        mlp = mlp_norm = None
        if di:
            fc1 = torch.randn(d, 2 * di, generator=gen) / math.sqrt(d)
            fc2 = torch.randn(di, d, generator=gen) / math.sqrt(di) * resid
            mlp = MLPParams(fc1=fc1.to(dtype), fc2=fc2.to(dtype))
            mlp_norm = torch.ones(d, dtype=dtype)
        blocks.append(BlockParams(torch.ones(d, dtype=dtype), p, mlp_norm, mlp))
    head = None if cfg.tie_head else (torch.randn(d, cfg.vocab_size, generator=gen) * 0.02).to(dtype)
    params = LMParams(embed.to(dtype), blocks, torch.ones(d, dtype=dtype), head)
    return params if device is None else lm_to(params, device=device)


def lm_template(cfg: LMConfig) -> LMParams:
    """The tree `init_lm` builds, as storage-less ``meta`` tensors of the same shapes
    (for loaders that only need the structure)."""
    e = lambda *shape: torch.empty(*shape, device="meta")  # noqa: E731
    c, d, di = cfg.siso, cfg.d_model, cfg.d_intermediate
    blocks = []
    for _ in range(cfg.n_layers):
        siso = LY.SISOParams(e(d, c.d_in_proj), e(c.d_inner, d), e(c.nheads), e(c.d_state),
                             e(c.d_state), e(c.nheads, c.d_state), e(c.nheads, c.d_state),
                             e(c.nheads))
        mlp = MLPParams(e(d, 2 * di), e(di, d)) if di else None
        blocks.append(BlockParams(e(d), siso, e(d) if di else None, mlp))
    return LMParams(e(cfg.vocab_size, d), blocks, e(d),
                    None if cfg.tie_head else e(d, cfg.vocab_size))


def lm_map(fn, params: LMParams) -> LMParams:
    """Apply ``fn`` to every tensor of the tree, keeping its structure (``None`` stays)."""
    f = lambda t: None if t is None else fn(t)  # noqa: E731
    blocks = [BlockParams(f(b.norm_gain), LY.SISOParams(*(f(t) for t in b.siso)),
                          f(b.mlp_norm_gain),
                          None if b.mlp is None else MLPParams(f(b.mlp.fc1), f(b.mlp.fc2)))
              for b in params.blocks]
    return LMParams(f(params.embed), blocks, f(params.final_norm), f(params.head))


def lm_to(params: LMParams, device=None, dtype=None) -> LMParams:
    return lm_map(lambda t: t.to(device=device, dtype=dtype), params)


def lm_leaves(params: LMParams) -> list:
    """The tree's tensors in a fixed order (embed, per block: norm, the eight SISO fields,
    MLP norm, fc1, fc2; final norm, head), ``None`` entries skipped."""
    out = [params.embed]
    for b in params.blocks:
        out.append(b.norm_gain)
        out.extend(b.siso)
        if b.mlp is not None:
            out.extend((b.mlp_norm_gain, b.mlp.fc1, b.mlp.fc2))
    out.append(params.final_norm)
    if params.head is not None:
        out.append(params.head)
    return out


def decode_params(params: LMParams, cfg: LMConfig) -> LMParams:
    """``params`` with each block's projection matrices (in_proj, out_proj, fc1, fc2) cast
    once to the policy's operand dtype. Every product casts them to that dtype anyway, so
    results are bit-identical; a per-token step then reads half the weight bytes and
    launches no casts. The embedding (which sets the residual stream's dtype), the head
    and the vectors are unchanged."""
    dt = _mm_dtype(cfg)
    blocks = [b._replace(siso=b.siso._replace(in_proj=b.siso.in_proj.detach().to(dt),
                                              out_proj=b.siso.out_proj.detach().to(dt)),
                         mlp=None if b.mlp is None else MLPParams(b.mlp.fc1.detach().to(dt),
                                                                  b.mlp.fc2.detach().to(dt)))
              for b in params.blocks]
    return params._replace(blocks=blocks)


def _head(params: LMParams, cfg: LMConfig) -> Tensor:
    return params.embed.t() if cfg.tie_head else params.head


def _logits(x: Tensor, params: LMParams, cfg: LMConfig) -> Tensor:
    """``rms_norm(x) @ head`` with float32 logits. Under a bf16 policy both operands are
    rounded to bf16 and accumulated in float32 (the head is about 0.3% of the model's
    flops, so a float32 product of the rounded operands costs nothing measurable)."""
    dt = _mm_dtype(cfg)
    return _head_logits(_norm(x, params.final_norm, cfg.siso.norm_eps, dt), params, cfg)


def _head_logits(xn: Tensor, params: LMParams, cfg: LMConfig) -> Tensor:
    """The head product of `_logits` on the already normalised rows."""
    return _mm(xn.float(), _head(params, cfg).to(_mm_dtype(cfg)), torch.float32)


class _NormFn(torch.autograd.Function):
    """The block norm as one autograd node over ``m3s_rms_fwd`` / ``m3s_rms_bwd``: the
    stream row in, the normalised row out in the next product's dtype, and back, each one
    HBM pass (the backward takes dy in that dtype, with no cast pass)."""

    @staticmethod
    def forward(ctx, x, gain, eps, dt):
        y, rstd = K.rms_forward(x, gain, eps, dt)
        ctx.save_for_backward(x, gain, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, gain, rstd = ctx.saved_tensors
        dx, dw = K.rms_backward(x, gain, rstd, dy)
        return dx, dw.to(gain.dtype), None, None


class _AddNormFn(torch.autograd.Function):
    """The residual add and the next norm as one autograd node: ``s = x + y`` (the stream
    after a block, in x's dtype) and ``rms_norm(s)`` in ``dt``, one ``m3s_rms_fwd`` pass;
    backward, the cotangent of ``s`` from the rest of the network plus the norm's
    pullback, returned for x and (in y's dtype) for y, one ``m3s_rms_bwd`` pass. The
    same values as `_add_residual` followed by `_norm`, without the add, its backward
    and the cast of its cotangent."""

    @staticmethod
    def forward(ctx, x, y, gain, eps, dt):
        n, rstd, s = K.rms_forward(x, gain, eps, dt, add=y)
        ctx.save_for_backward(s, gain, rstd)
        ctx.y_dtype = y.dtype
        ctx.set_materialize_grads(False)
        return s, n

    @staticmethod
    def backward(ctx, ds, dn):
        s, gain, rstd = ctx.saved_tensors
        if dn is None:
            dn = torch.zeros(s.shape, device=s.device, dtype=ctx.y_dtype)
        dx, dw, dy = K.rms_backward(s, gain, rstd, dn, dsum=ds, add_dtype=ctx.y_dtype)
        return dx, dy, dw.to(gain.dtype), None, None


def _add_norm(x: Tensor, y: Tensor, gain: Tensor, eps: float, dt: torch.dtype):
    """``(x + y, rms_norm(x + y, gain, eps) in dt)`` for the residual stream ``x`` and a
    block output ``y``: one HIP pass each way (`_AddNormFn`) when the sum keeps x's dtype
    and y is already in ``dt``, else the add and `_norm`."""
    d = x.shape[-1]
    if (x.is_cuda and y.is_cuda and x.shape == y.shape and y.dtype == dt
            and torch.promote_types(x.dtype, y.dtype) == x.dtype and d % 4 == 0 and d <= 4096
            and x.dtype in (torch.float32, torch.bfloat16)):
        return _AddNormFn.apply(x, y, gain, eps, dt)
    s = _add_residual(x, y)
    return s, _norm(s, gain, eps, dt)


def _norm(x: Tensor, gain: Tensor, eps: float, dt: torch.dtype) -> Tensor:
    """``rms_norm(x, gain, eps)`` (``layer.py:190-198``: float32 statistics, gain after
    scaling) returned in ``dt``, as the next product takes it: one HIP pass each way
    (`_NormFn`). Rows wider than 4096 or not a multiple of 4 go through ``F.rms_norm``."""
    d = x.shape[-1]
    if x.is_cuda and d % 4 == 0 and d <= 4096 and x.dtype in (torch.float32, torch.bfloat16):
        return _NormFn.apply(x, gain, eps, dt)
    return F.rms_norm(x.float(), (d,), gain.float(), eps).to(dt)


def _embed(table: Tensor, tokens: Tensor) -> Tensor:
    """``table[tokens]``. Through ``F.embedding``, whose backward reduces duplicate ids in
    parallel partial segments; the plain-indexing backward sums each id's rows serially,
    which for byte data (256 ids, Zipf-skewed) costs ~5 ms per training step."""
    return F.embedding(tokens, table)


def lm_forward(params: LMParams, tokens: Tensor, cfg: LMConfig, interpret: Any = False,
               device_kind: str | None = None, states: Optional[list] = None):
    """``(B, L)`` int tokens -> ``(B, L, vocab)`` float32 logits (``model.py:194-232``).

    With ``states`` (a per-layer carry-in, e.g. `zero_states`) the per-layer carry-out is
    returned as well: ``(logits, states)`` -- the segmented prefill of generation.
    ``interpret`` and ``device_kind`` are accepted for signature compatibility."""
    dt = _mm_dtype(cfg)
    x = _embed(params.embed, tokens)
    new_states = []
    eps = cfg.siso.norm_eps
    blocks = params.blocks
    # each residual add is fused with the norm that reads the sum next (the next sublayer's,
    # or the head's); the first block's norm reads the embedding alone
    h = _norm(x, blocks[0].norm_gain, eps, dt) if blocks else None
    for i, b in enumerate(blocks):
        y, st = LY.mamba3_siso_layer(b.siso, h, cfg.siso,
                                     state=None if states is None else states[i])
        new_states.append(st)
        nxt = blocks[i + 1].norm_gain if i + 1 < len(blocks) else params.final_norm
        if b.mlp is not None:
            x, h = _add_norm(x, y, b.mlp_norm_gain, eps, dt)
            y = gated_mlp(b.mlp, h, dt)
        x, h = _add_norm(x, y, nxt, eps, dt)
    logits = _head_logits(h, params, cfg) if blocks else _logits(x, params, cfg)
    return (logits, new_states) if states is not None else logits


def lm_loss(params: LMParams, xs: Tensor, ys: Tensor, cfg: LMConfig) -> Tensor:
    """Mean next-token cross-entropy of `lm_forward`'s logits against ``ys``
    (``train.py:414-416``)."""
    logits = lm_forward(params, xs, cfg)
    return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), ys.reshape(-1))


def zero_states(cfg: LMConfig, batch: int, dtype=torch.float32, device=None) -> list:
    """A fresh per-layer carry (``model.py:235-241``)."""
    c = cfg.siso
    out = []
    for _ in range(cfg.n_layers):
        s = zero_state(batch, c.nheads, c.headdim, c.d_state, c.n_angles, dtype)
        out.append(SISOState(*(t.to(device) for t in s)) if device is not None else s)
    return out


def _add_residual(x: Tensor, y: Tensor) -> Tensor:
    """``x + y`` for a one-token step, with PyTorch's type promotion: both operands are
    cast to the promoted dtype first, then added. That is what the mixed-dtype add
    computes (a bf16 stream plus an f32 block output becomes an f32 stream, as the
    reference's JAX add promotes), but the mixed-dtype add kernel needs scratch memory and
    costs ~40 us per launch on ROCm whatever its size, against a few us for a cast and a
    plain add."""
    if x.dtype == y.dtype:
        return x + y
    wide = torch.promote_types(x.dtype, y.dtype)
    return x.to(wide) + y.to(wide)


def lm_decode_step(params: LMParams, token: Tensor, states: list, cfg: LMConfig,
                   interpret: Any = False):
    """One token through the stack (``model.py:244-296``): ``(B,)`` -> ``((B, vocab)
    float32 logits, states)``. Each layer between its projections is one
    ``m3s_decode_layer`` launch, which updates that layer's state in place (the
    reference donates it); the returned list holds the same state tensors."""
    dt = _mm_dtype(cfg)
    c = cfg.siso
    eps = c.norm_eps
    x = _embed(params.embed, token)
    out_states = []
    blocks = params.blocks
    # as in lm_forward: each residual add fused with the norm that reads the sum next
    h = _norm(x, blocks[0].norm_gain, eps, dt) if blocks else None
    for i, b in enumerate(blocks):
        y, st = LY.mamba3_siso_decode_step(b.siso, h, c, states[i])
        out_states.append(st)
        nxt = blocks[i + 1].norm_gain if i + 1 < len(blocks) else params.final_norm
        if b.mlp is not None:
            x, h = _add_norm(x, y, b.mlp_norm_gain, eps, dt)
            y = gated_mlp(b.mlp, h, dt)
        x, h = _add_norm(x, y, nxt, eps, dt)
    logits = _head_logits(h, params, cfg) if blocks else _logits(x, params, cfg)
    return logits, out_states
