"""The Mamba-3 SISO layer: projections around the HIP scan (``layer.py`` surface).

``SISOConfig`` / ``SISOParams`` / ``init_params`` / ``split_in_proj`` / ``rms_norm`` /
``mamba3_siso_layer`` keep the reference's names, fields, defaults and semantics
(``layer.py:39-262``). ``mamba3_siso_decode_step`` is the per-token layer step the
reference inlines in ``model.lm_decode_step`` (``model.py:266-289``), minus the block
norm, residual and MLP.

Layer structure: ``in_proj -> [z, x, B, C, dd_dt, dd_A, trap, angles]``; B, C ->
RMSNorm; scan with ``q = C``, ``k = B``, gated by ``silu(z)``; ``out_proj``.

Layout: the scan reads ``x`` and ``z`` in place from the fused projection
``(B, L, d_in_proj)`` (strided ``(B, H, L, P)`` views) and writes ``y`` as a
``(B, L, H, P)`` buffer, so no transpose is ever materialised (the reference pays three,
``layer.py:240,249,258``).

Two execution paths, same results:

* `_LayerFn` (no carried state): the whole layer as one autograd node. The projection
  is computed ``(B, L, D_pad)`` wide, D_pad = d_in_proj rounded up to 256 columns, from
  a transposed, zero-padded copy of ``in_proj`` (the layout hipBLASLt runs fastest at
  these shapes; the padding columns are never read). BCNorm is one HIP launch
  (``m3s_norm_fwd``). In the backward every kernel writes its slice of one projection
  gradient buffer in place -- dz, dx from the scan, dB, dC from ``m3s_norm_bwd``, the
  raw-scalar and angle slices from ``m3s_prep_bwd`` -- so no concatenation is needed.
* the composed path (a carried ``state``, or shapes the in-place kernels cannot
  address): torch autograd over `rms_norm`, the differentiable `preprocess` and `siso`.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any, NamedTuple, Optional

import torch
import torch.nn.functional as F

from . import kernels as K
from . import layout as LY
from . import scan_prep as SP
from .scan_prep import SISOState, heavy_tail
from .siso import siso_segment

Tensor = torch.Tensor


@dataclasses.dataclass(frozen=True)
class SISOConfig:
    """Shapes and hyperparameters (``layer.py:39-99``); same fields and defaults.

    ``chunk`` follows the reference's rule (a positive multiple of 128) widened to the
    shorter kernel tiles 32 and 64 (`layout.validate_chunk`); a chunk with no kernel of
    its own is scanned in tiles of the largest compiled chunk dividing it
    (`layout.kernel_chunk`: the chunked form is exact for any chunk length). Construction
    makes the reference's checks only (``layer.py:74-99``), so host-only work -- checkpoint
    conversion, the CPU oracle -- takes any shape. Whether forward, backward and decode
    kernels are compiled for its (policy, chunk, d_state, headdim) is checked by
    `require_kernels`, which the layer's entry points call before their first launch.
    """

    d_model: int
    d_state: int = 128
    headdim: int = 64
    expand: int = 2
    rope_fraction: float = 0.5
    chunk: int = 128
    a_floor: float = 1e-4
    norm_eps: float = 1e-5
    dt_min: float = 0.001
    dt_max: float = 0.1
    dt_init_floor: float = 1e-4
    policy_name: str = "bf16"

    @property
    def d_inner(self) -> int:
        return self.expand * self.d_model

    @property
    def nheads(self) -> int:
        if self.d_inner % self.headdim != 0:
            raise ValueError(f"d_inner {self.d_inner} not divisible by headdim {self.headdim}")
        return self.d_inner // self.headdim

    @property
    def n_angles(self) -> int:
        """Rotary pairs (``layer.py:80-91``): even-floored ``d_state*rope_fraction``/2."""
        if self.rope_fraction not in (0.5, 1.0):
            raise ValueError(f"rope_fraction must be 0.5 or 1.0, got {self.rope_fraction}")
        width = int(self.d_state * self.rope_fraction)
        if width % 2:
            width -= 1
        n = width // 2
        if n <= 0:
            raise ValueError("rope_fraction too small: no rotary angles")
        return n

    @property
    def d_in_proj(self) -> int:
        """``layer.py:93-95``; order fixed by `split_in_proj`."""
        return 2 * self.d_inner + 2 * self.d_state + 3 * self.nheads + self.n_angles

    def __post_init__(self):
        LY.validate_chunk(self.chunk)
        LY.policy(self.policy_name)
        _ = self.nheads, self.n_angles

    def require_kernels(self) -> None:
        """``ValueError`` naming the missing kernels (and the chunks that are compiled)
        unless this (policy, chunk, d_state, headdim) can run on the device
        (`layout.validate_kernel_shape`)."""
        LY.validate_kernel_shape(self.policy_name, self.chunk, self.d_state, self.headdim)


class SISOParams(NamedTuple):
    """``layer.py:102-124``. in_proj ``(d_model, d_in_proj)``; out_proj
    ``(d_inner, d_model)``; dt_bias ``(H,)``; b/c_norm_weight ``(N,)`` and b/c_bias
    ``(H, N)`` in the permuted rotary layout; d_skip ``(H,)``."""

    in_proj: Tensor
    out_proj: Tensor
    dt_bias: Tensor
    b_norm_weight: Tensor
    c_norm_weight: Tensor
    b_bias: Tensor
    c_bias: Tensor
    d_skip: Tensor


def init_params(cfg: SISOConfig, key: Any = 0, dtype=torch.float32, device=None) -> SISOParams:
    """Fresh weights with upstream's initialisation (``layer.py:127-160``).

    ``key`` is an int seed or a ``torch.Generator`` (the reference takes a JAX PRNG key;
    JAX's threefry stream is not reproduced, only the distributions): in_proj
    ``U(+-1/sqrt(d_model))``, out_proj ``U(+-1/sqrt(d_inner))``, ``dt_bias`` the inverse
    softplus of a log-uniform ``dt`` in ``[dt_min, dt_max]`` floored at ``dt_init_floor``;
    norm gains, B/C biases and D are ones. Drawn on the CPU, then moved to ``device``.
    """
    gen = key if isinstance(key, torch.Generator) else torch.Generator().manual_seed(int(key))
    s_in = 1.0 / math.sqrt(cfg.d_model)
    s_out = 1.0 / math.sqrt(cfg.d_inner)
    in_proj = (torch.rand(cfg.d_model, cfg.d_in_proj, generator=gen) * 2 - 1) * s_in
    out_proj = (torch.rand(cfg.d_inner, cfg.d_model, generator=gen) * 2 - 1) * s_out
    dt = torch.exp(torch.rand(cfg.nheads, generator=gen)
                   * (math.log(cfg.dt_max) - math.log(cfg.dt_min)) + math.log(cfg.dt_min))
    dt = torch.clamp(dt, min=cfg.dt_init_floor)
    dt_bias = dt + torch.log(-torch.expm1(-dt))   # inverse softplus
    ones = lambda *s: torch.ones(*s, dtype=dtype)  # noqa: E731
    p = SISOParams(
        in_proj=in_proj.to(dtype), out_proj=out_proj.to(dtype), dt_bias=dt_bias.float(),
        b_norm_weight=ones(cfg.d_state), c_norm_weight=ones(cfg.d_state),
        b_bias=ones(cfg.nheads, cfg.d_state), c_bias=ones(cfg.nheads, cfg.d_state),
        d_skip=ones(cfg.nheads))
    return SISOParams(*(t.to(device) for t in p)) if device is not None else p


def split_in_proj(proj: Tensor, cfg: SISOConfig):
    """``layer.py:163-187``: ``(z, x, B, C, dt_raw, a_raw, trap_raw, angles)`` with z, x
    ``(B, L, H, P)``, B, C ``(B, L, N)``, scalars ``(B, L, H)``, angles ``(B, L, Nr)``.
    All are views of ``proj``."""
    sizes = (cfg.d_inner, cfg.d_inner, cfg.d_state, cfg.d_state,
             cfg.nheads, cfg.nheads, cfg.nheads, cfg.n_angles)
    z, x, b, c, dt_raw, a_raw, trap_raw, angles = torch.split(proj, sizes, dim=-1)
    z = z.unflatten(-1, (cfg.nheads, cfg.headdim))
    x = x.unflatten(-1, (cfg.nheads, cfg.headdim))
    return z, x, b, c, dt_raw, a_raw, trap_raw, angles


def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """``layer.py:190-198``: RMSNorm in f32, gain, no bias, cast back to x.dtype."""
    xf = x.float()
    rstd = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (xf * rstd * weight.float()).to(x.dtype)


_PROJ_PAD = 256


def _padded_width(d: int) -> int:
    return (d + _PROJ_PAD - 1) // _PROJ_PAD * _PROJ_PAD


def _fused_ok(u: Tensor, cfg: SISOConfig, state) -> bool:
    """Whether `_LayerFn` can run this call: no carried state, the policy's operand dtype
    equals ``u``'s, and every slice of the padded projection the kernels address in place
    starts on a 16-byte boundary (z, x, B, C; the scalar slices are read elementwise)."""
    if state is not None or not u.is_cuda or u.dim() != 3:
        return False
    if u.dtype not in (torch.bfloat16, torch.float32) or LY.policy(cfg.policy_name).matmul != u.dtype:
        return False
    vec = 16 // u.element_size()
    n = cfg.d_state
    return (cfg.d_inner % vec == 0 and cfg.headdim % vec == 0 and n % vec == 0
            and n // vec <= 64)


def weight_grad(a: Tensor, b: Tensor) -> Tensor:
    """``a^T b`` in float32 for ``(M, P)`` and ``(M, Q)`` operands over the M tokens: the
    weight gradient of a projection. Its output is small (P x Q) and its reduction long
    (M = B*L), so one library GEMM has too few output tiles to fill the GPU.

    bf16 device operands that `kernels.wgrad_supported` takes go to ``m3s_wgrad`` (MFMA
    tiles over token splits sized to fill the CUs, partials added in a fixed order). Else,
    with M a multiple of 8 and at least 16384, the tokens are cut into 8 slices, one
    batched GEMM forms the 8 partial products (float32 out) and they are summed in slice
    order. The right operand is never a transposed view (a column slice is a strided row
    view)."""
    m = a.shape[0]
    if a.dtype != b.dtype or a.dim() != 2 or b.dim() != 2 or b.shape[0] != m:
        raise ValueError("weight_grad: a (M, P) and b (M, Q) of one dtype")
    if K.wgrad_supported(a, b):
        return K.wgrad(a, b)
    if m % 8 or m < 16384 or not a.is_cuda:
        if a.dtype == torch.float32 or not a.is_cuda:
            return (a.t() @ b).float()
        return torch.mm(a.t(), b, out_dtype=torch.float32)
    a3, b3 = a.unflatten(0, (8, m // 8)), b.unflatten(0, (8, m // 8))
    if a.dtype == torch.float32:
        return torch.bmm(a3.transpose(1, 2), b3).sum(0)
    return torch.bmm(a3.transpose(1, 2), b3, out_dtype=torch.float32).sum(0)


class _LayerFn(torch.autograd.Function):
    """``layer.py:201-262`` with state=None as one autograd node (see the module notes).
    Outputs: out (B, L, d_model), final ssm, final k, final v, final phi."""

    @staticmethod
    def forward(ctx, u, in_proj, out_proj, dt_bias, b_norm_weight, c_norm_weight, b_bias,
                c_bias, d_skip, cfg, phi_in_kernel=None):
        dt = u.dtype
        batch, seqlen, dm = u.shape
        m = batch * seqlen
        d, dp = cfg.d_in_proj, _padded_width(cfg.d_in_proj)
        if tuple(in_proj.shape) != (dm, d) or tuple(out_proj.shape) != (cfg.d_inner, dm):
            raise ValueError(f"in_proj must be {(dm, d)} and out_proj {(cfg.d_inner, dm)}")
        # the reference casts the weights per call (layer.py:233, 256); this lays them out too
        w_t = K.transpose_pad(in_proj, dt, dp)
        u2 = u.reshape(m, dm)
        proj = (u2 @ w_t.t()).view(batch, seqlen, dp)
        z, x, b, c, dt_raw, a_raw, trap_raw, angles = split_in_proj(proj[..., :d], cfg)
        bias = dt_bias.float().contiguous()
        need = any(ctx.needs_input_grad[:9])   # all False under no_grad
        # Without gradients the preprocess runs inside the other launches (raw mode): the
        # BCNorm launch also writes the rotary table and per-strip theta totals, and the scan
        # reads the raw dt / a / trap slices in place and carries phi itself. With gradients
        # the preprocess materialises the row scalars the backward reads, and phi either as
        # (B, H, L, Nr) or compact (kernels.PhiStrips: the scans rebuild it per row).
        raw = (not need and phi_in_kernel is not False
               and K.raw_forward_ok(cfg.policy_name, cfg.chunk, cfg.d_state, cfg.headdim,
                                    cfg.n_angles, seqlen, cfg.nheads))
        if raw:
            tile = LY.kernel_chunk(cfg.policy_name, cfg.chunk, cfg.d_state, cfg.headdim)
            (k, q), (rk, rq), angs = K.bcnorm_forward(
                [b, c], [b_norm_weight, c_norm_weight], cfg.norm_eps,
                theta=(angles, dt_raw, bias, tile))
            outs = K.siso_forward_raw(q, k, x.permute(0, 2, 1, 3), dt_raw, a_raw, trap_raw, angs,
                                      bias, c_bias, b_bias, d_skip=d_skip,
                                      z=z.permute(0, 2, 1, 3), a_floor=cfg.a_floor,
                                      chunk=cfg.chunk, dtype_policy=cfg.policy_name)
            phi_final = outs[4]
        else:
            (k, q), (rk, rq) = K.bcnorm_forward([b, c], [b_norm_weight, c_norm_weight],
                                                cfg.norm_eps)
            compact = (not need) if phi_in_kernel is None else bool(phi_in_kernel)
            adt, gamma, scale, _, _, phi, phi_final = SP.prep_forward_launch(
                dt_raw, a_raw, trap_raw, angles, bias, None, cfg.a_floor, compact=compact)
            outs = K.siso_forward(q, k, x.permute(0, 2, 1, 3), adt, gamma, scale, phi, c_bias,
                                  b_bias, d_skip=d_skip, z=z.permute(0, 2, 1, 3),
                                  chunk=cfg.chunk, dtype_policy=cfg.policy_name,
                                  save_residuals=need)
        y, fs, fk, fv = outs[:4]
        y2 = y.permute(0, 2, 1, 3).reshape(m, cfg.d_inner)
        wo_t = K.transpose_pad(out_proj, dt, dm)
        out = (y2 @ wo_t.t()).view(batch, seqlen, dm)
        if need:
            res = outs[4]
            phis = tuple(phi) if isinstance(phi, K.PhiStrips) else (phi,)
            ctx.n_phi = len(phis)
            ctx.save_for_backward(u, proj, q, k, rk, rq, adt, gamma, scale, y, res.ybar,
                                  res.chunk_states, in_proj, out_proj, bias, b_norm_weight,
                                  c_norm_weight, b_bias, c_bias, d_skip, *phis)
        ctx.cfg = cfg
        ctx.set_materialize_grads(False)
        return out, fs, fk, fv, phi_final

    @staticmethod
    def backward(ctx, dout, dfs, dfk, dfv, dphi_final):
        saved = ctx.saved_tensors
        (u, proj, q, k, rk, rq, adt, gamma, scale, y, ybar, cstates, in_proj, out_proj,
         bias, wb, wc, b_bias, c_bias, d_skip) = saved[:-ctx.n_phi]
        phis = saved[-ctx.n_phi:]
        phi = K.PhiStrips(*phis) if ctx.n_phi == 3 else phis[0]
        cfg = ctx.cfg
        dt = u.dtype
        batch, seqlen, dm = u.shape
        m = batch * seqlen
        d, dp = cfg.d_in_proj, _padded_width(cfg.d_in_proj)
        H, P = cfg.nheads, cfg.headdim
        needs = ctx.needs_input_grad
        z, x, b, c, dt_raw, a_raw, trap_raw, angles = split_in_proj(proj[..., :d], cfg)
        y2 = y.permute(0, 2, 1, 3).reshape(m, cfg.d_inner)
        d_out_proj = None
        if dout is not None:
            dout2 = dout.reshape(m, dm).to(dt)
            dy2 = dout2 @ out_proj.to(dt).t()
            if needs[2]:
                d_out_proj = weight_grad(y2, dout2).to(out_proj.dtype)
            dys = dy2.view(batch, seqlen, H, P).permute(0, 2, 1, 3)
        else:
            dys = torch.zeros_like(y)
        # every slice of the projection gradient is written by exactly one kernel below
        dproj = K.empty(batch, seqlen, dp, device=u.device, dtype=dt)
        dz_v, dx_v, db_v, dc_v, ddt_v, da_v, dtr_v, dang_v = split_in_proj(dproj[..., :d], cfg)
        g = K.siso_backward(
            dys, q, k, x.permute(0, 2, 1, 3), adt, gamma, scale, phi, c_bias, b_bias, ybar,
            cstates, d_skip=d_skip, z=z.permute(0, 2, 1, 3), dfinal_ssm=dfs, dfinal_k=dfk,
            dfinal_v=dfv, chunk=cfg.chunk, dtype_policy=cfg.policy_name,
            dv_out=dx_v.permute(0, 2, 1, 3), dz_out=dz_v.permute(0, 2, 1, 3))
        dwb, dwc = K.bcnorm_backward([b, c], [wb, wc], [rk, rq], [g.dk, g.dq], [db_v, dc_v])
        d_bias = K.empty(H, device=u.device, dtype=torch.float32)
        SP.prep_backward_launch(dt_raw, a_raw, trap_raw, angles, bias, cfg.a_floor,
                                (g.dadt, g.dgamma, g.dscale, None, None, g.dphi, dphi_final),
                                ddt_v, da_v, dtr_v, dang_v, d_bias, None)
        dp2 = dproj.view(m, dp)[:, :d]
        du = d_in_proj = None
        if needs[0]:
            du = (dp2 @ in_proj.to(dt).t()).view(batch, seqlen, dm)
        if needs[1]:
            d_in_proj = weight_grad(u.reshape(m, dm), dp2).to(in_proj.dtype)

        def like(t, p_):
            return None if (t is None or p_ is None) else t.to(p_.dtype)

        return (du, d_in_proj, d_out_proj, like(d_bias, bias), like(dwb, wb), like(dwc, wc),
                like(g.dk_bias, b_bias), like(g.dq_bias, c_bias), like(g.dd_skip, d_skip), None,
                None)


def mamba3_siso_layer(params: SISOParams, u: Tensor, cfg: SISOConfig,
                      state: Optional[SISOState] = None, interpret: Any = False,
                      device_kind: str | None = None, phi_in_kernel: Optional[bool] = None):
    """Forward of one layer (``layer.py:201-262``). ``u`` is ``(B, L, d_model)`` on the
    ROCm device; returns ``(out (B, L, d_model), SISOState)``. Differentiable w.r.t.
    ``u`` and every `SISOParams` field through torch autograd.

    ``phi_in_kernel`` (no counterpart in the reference; same results to float rounding):
    when True the cumulative rotary angle is not materialised as ``(B, H, L, Nr)``; the
    scan kernels rebuild it per token from the head-shared ``tanh(angles) pi`` table, dt
    and one angle per 16 tokens, which moves 1/16 of phi's bytes. Without gradients
    (``None`` or True) the whole preprocess then runs inside the BCNorm and scan launches
    (`kernels.siso_forward_raw`) where a raw-mode kernel exists for the shape. With
    gradients ``None`` (the default) materialises phi, whose backward scan is faster, and
    True keeps it compact. False always materialises phi and the row scalars first."""
    cfg.require_kernels()
    if _fused_ok(u, cfg, state):
        out, fs, fk, fv, phi_final = _LayerFn.apply(
            u, params.in_proj, params.out_proj, params.dt_bias, params.b_norm_weight,
            params.c_norm_weight, params.b_bias, params.c_bias, params.d_skip, cfg,
            phi_in_kernel)
        return out, SISOState(ssm=fs, k=fk, v=fv, phi=phi_final)
    batch, seqlen, _ = u.shape
    proj = u @ params.in_proj.to(u.dtype)
    z, x, b, c, dt_raw, a_raw, trap_raw, angles = split_in_proj(proj, cfg)
    b = rms_norm(b, params.b_norm_weight, cfg.norm_eps)
    c = rms_norm(c, params.c_norm_weight, cfg.norm_eps)
    out = siso_segment(
        q=c, k=b, v=x.permute(0, 2, 1, 3), dt_raw=dt_raw, a_raw=a_raw, trap_raw=trap_raw,
        angles=angles, dt_bias=params.dt_bias, q_bias=params.c_bias, k_bias=params.b_bias,
        d_skip=params.d_skip, z=z.permute(0, 2, 1, 3), state=state, a_floor=cfg.a_floor,
        chunk=cfg.chunk, policy_name=cfg.policy_name)
    y = out.y.permute(0, 2, 1, 3).reshape(batch, seqlen, cfg.d_inner)
    return y.to(u.dtype) @ params.out_proj.to(u.dtype), out.state


def _decode_fused_ok(u: Tensor, cfg: SISOConfig) -> bool:
    """Whether the decode step runs as one ``m3s_decode_layer`` launch: ``u`` on the
    device in the policy's operand dtype, and a decode kernel of the head's own width
    (otherwise the composed step casts as needed and runs sub-heads)."""
    return (u.is_cuda and u.dtype == LY.policy(cfg.policy_name).matmul
            and LY.decode_headdim(cfg.policy_name, cfg.d_state, cfg.headdim) == cfg.headdim)


def mamba3_siso_decode_step(params: SISOParams, u: Tensor, cfg: SISOConfig,
                            state: SISOState):
    """One token through the layer (``model.py:266-289`` without block norm/residual):
    ``u`` ``(B, d_model)`` -> ``(out (B, d_model), next_state)``. The state is updated in
    place by the decode kernel (the reference donates it). When ``u`` is in the policy's
    operand dtype, everything between the two projections (BCNorm, dt / lambda / a, the
    state update and readout) is one ``m3s_decode_layer`` launch on the projection rows."""
    cfg.require_kernels()
    proj = K.matmul(u, params.in_proj.to(u.dtype))
    if _decode_fused_ok(u, cfg):
        y, st = K.decode_layer_step(
            proj, state, nheads=cfg.nheads, headdim=cfg.headdim, state_dim=cfg.d_state,
            n_angles=cfg.n_angles, b_norm_weight=params.b_norm_weight,
            c_norm_weight=params.c_norm_weight, dt_bias=params.dt_bias, q_bias=params.c_bias,
            k_bias=params.b_bias, d_skip=params.d_skip, a_floor=cfg.a_floor,
            norm_eps=cfg.norm_eps)
    else:
        z, x, b, c, dt_raw, a_raw, trap_raw, angles = split_in_proj(proj[:, None, :], cfg)
        b = rms_norm(b, params.b_norm_weight, cfg.norm_eps)[:, 0]
        c = rms_norm(c, params.c_norm_weight, cfg.norm_eps)[:, 0]
        dt = F.softplus(dt_raw[:, 0].float() + params.dt_bias.float())
        a = torch.clamp(-heavy_tail(a_raw[:, 0].float()), max=-cfg.a_floor)
        lam = torch.sigmoid(trap_raw[:, 0].float())
        y, st = K.decode_step(c, b, x[:, 0], a * dt, dt, lam, angles[:, 0], params.c_bias,
                              params.b_bias, state, d_skip=params.d_skip, z=z[:, 0],
                              dtype_policy=cfg.policy_name)
    out = K.matmul(y.reshape(u.shape[0], cfg.d_inner).to(u.dtype), params.out_proj.to(u.dtype))
    return out, st
