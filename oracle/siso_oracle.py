"""Torch-CPU restatement of the reference's Mamba-3 SISO maths (test oracle only).

Every function cites the reference file:line it restates. All tensors are CPU
tensors; pass float64 for the tight checks, float32 for the baseline timing. The
``mm_dtype`` switch of `siso_chunked` additionally rounds the matmul operands to
bfloat16 at exactly the points the reference's bf16 kernel does
(``kernel_fwd.py:133-187``), so a bf16 GPU kernel can be compared against its own
rounding model as well as against the float32 maths.

State-axis tensors are in the permuted half-split rotary layout
(``layout.py:299-337``) unless a function says otherwise.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import NamedTuple, Optional

import torch
import torch.nn.functional as F

TWO_PI = 2.0 * math.pi
LOG2_E = 1.4426950408889634

Tensor = torch.Tensor


# ------------------------------------------------------------------------------------
# layout.py helpers
# ------------------------------------------------------------------------------------


def deinterleave_perm(n: int) -> Tensor:
    """``layout.py:299-320``: new[j] = old[2j], new[n/2+j] = old[2j+1]."""
    if n % 2:
        raise ValueError(f"state dim must be even, got {n}")
    return torch.cat([torch.arange(0, n, 2), torch.arange(1, n, 2)])


def interleave_perm(n: int) -> Tensor:
    """``layout.py:323-326``: inverse of `deinterleave_perm`."""
    return torch.argsort(deinterleave_perm(n))


def rope_cos_sin(phi: Tensor, n: int) -> tuple[Tensor, Tensor]:
    """``layout.py:345-372``: angles padded with zeros to N/2, doubled to N."""
    half = n // 2
    nr = phi.shape[-1]
    if nr > half:
        raise ValueError("n_angles exceeds N/2")
    if nr < half:
        phi = torch.cat([phi, phi.new_zeros(*phi.shape[:-1], half - nr)], dim=-1)
    full = torch.cat([phi, phi], dim=-1)
    return torch.cos(full), torch.sin(full)


def rope_apply(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """``layout.py:375-398``: ``x*cos + [-x_hi, x_lo]*sin``."""
    half = x.shape[-1] // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * cos + rot * sin


def rope_dphi(x_rot: Tensor, dx_rot: Tensor, nr: int) -> Tensor:
    """``layout.py:414-428``: ``dphi_j = dhi_j*lo_j - dlo_j*hi_j`` for j < Nr."""
    half = x_rot.shape[-1] // 2
    lo, hi = x_rot[..., :half], x_rot[..., half:]
    dlo, dhi = dx_rot[..., :half], dx_rot[..., half:]
    return (dhi * lo - dlo * hi)[..., :nr]


def rope_apply_interleaved(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """``torch_ref.py:42-61``: upstream's adjacent-pair rotation; ``cos``/``sin`` are
    per pair (``(..., Nr)``), padded with cos=1, sin=0 to N/2 pairs."""
    pairs = x.reshape(*x.shape[:-1], -1, 2)
    t0, t1 = pairs[..., 0], pairs[..., 1]
    if cos.shape[-1] < t0.shape[-1]:
        pad = t0.shape[-1] - cos.shape[-1]
        cos = F.pad(cos, (0, pad), value=1.0)
        sin = F.pad(sin, (0, pad), value=0.0)
    return torch.stack([t0 * cos - t1 * sin, t0 * sin + t1 * cos], dim=-1).reshape(x.shape)


# ------------------------------------------------------------------------------------
# reference.py: state and preprocessing
# ------------------------------------------------------------------------------------


class SISOState(NamedTuple):
    """``reference.py:46-63``: ssm (B,H,P,N), k (B,H,N) rotated-unscaled, v (B,H,P),
    phi (B,H,Nr)."""

    ssm: Tensor
    k: Tensor
    v: Tensor
    phi: Tensor


def zero_state(b, h, p, n, nr, dtype=torch.float64) -> SISOState:
    """``reference.py:66-74``."""
    return SISOState(
        torch.zeros(b, h, p, n, dtype=dtype),
        torch.zeros(b, h, n, dtype=dtype),
        torch.zeros(b, h, p, dtype=dtype),
        torch.zeros(b, h, nr, dtype=dtype),
    )


@dataclass
class Preprocessed:
    """``reference.py:82-101``."""

    adt: Tensor
    gamma: Tensor
    scale: Tensor
    phi: Tensor
    lam: Tensor
    dt: Tensor


def heavy_tail(x: Tensor) -> Tensor:
    """``reference.py:202-209``: ``max(x,0) + 1/(1 - min(x,0))``."""
    return torch.clamp(x, min=0.0) + torch.reciprocal(1.0 - torch.clamp(x, max=0.0))


def trapezoid_coeffs(dt: Tensor, lam: Tensor) -> tuple[Tensor, Tensor]:
    """``reference.py:104-131``: gamma = dt*lam; scale = gamma + dt_{t+1}(1-lam_{t+1})
    with the successor of the last position taken as zero."""
    gamma = dt * lam
    dt_next = torch.cat([dt[..., 1:], torch.zeros_like(dt[..., :1])], dim=-1)
    lam_next = torch.cat([lam[..., 1:], torch.zeros_like(lam[..., :1])], dim=-1)
    return gamma, gamma + dt_next * (1.0 - lam_next)


def wrap_angle(phi: Tensor) -> Tensor:
    """``reference.py:156``: ``phi - 2*pi*floor(phi / 2*pi)``."""
    return phi - TWO_PI * torch.floor(phi / TWO_PI)


def cumulative_angles(angles_h: Tensor, dt: Tensor, phi_init: Optional[Tensor] = None):
    """``reference.py:134-157``. angles_h (B,H,L,Nr), dt (B,H,L)."""
    theta = torch.tanh(angles_h) * math.pi * dt[..., None]
    phi = torch.cumsum(theta, dim=2)
    if phi_init is not None:
        phi = phi + phi_init[:, :, None, :]
    phi = wrap_angle(phi)
    return phi, phi[:, :, -1, :]


def preprocess(dt_raw, a_raw, trap_raw, angles, dt_bias, a_floor=1e-4, phi_init=None):
    """``reference.py:160-199``. Raw slices are (B,L,H); angles (B,L,Nr)."""
    dt = F.softplus(dt_raw + dt_bias).transpose(1, 2)
    a = -heavy_tail(a_raw).transpose(1, 2)
    a = torch.clamp(a, max=-a_floor)
    lam = torch.sigmoid(trap_raw).transpose(1, 2)
    gamma, scale = trapezoid_coeffs(dt, lam)
    h = dt.shape[1]
    angles_h = angles[:, None].expand(angles.shape[0], h, angles.shape[1], angles.shape[2])
    phi, phi_final = cumulative_angles(angles_h, dt, phi_init)
    return Preprocessed(adt=a * dt, gamma=gamma, scale=scale, phi=phi, lam=lam, dt=dt), phi_final


# ------------------------------------------------------------------------------------
# reference.py: the three formulations
# ------------------------------------------------------------------------------------


def siso_recurrent(q, k, v, adt, dt, lam, phi, q_bias, k_bias, d_skip=None, z=None, state=None):
    """``reference.py:217-287``: explicit three-term trapezoidal scan, token by token."""
    b, seqlen, n = q.shape
    h, p = v.shape[1], v.shape[3]
    nr = phi.shape[-1]
    if state is None:
        state = zero_state(b, h, p, n, nr, dtype=v.dtype)
    ssm, k_prev, v_prev = state.ssm, state.k, state.v
    ys = []
    for t in range(seqlen):
        u = q[:, t][:, None, :] + q_bias[None]
        w = k[:, t][:, None, :] + k_bias[None]
        cos, sin = rope_cos_sin(phi[:, :, t, :], n)
        q_rot = rope_apply(u, cos, sin)
        k_rot = rope_apply(w, cos, sin)
        alpha = torch.exp(adt[:, :, t])
        beta = (1.0 - lam[:, :, t]) * dt[:, :, t] * alpha
        gamma = dt[:, :, t] * lam[:, :, t]
        v_t = v[:, :, t, :]
        ssm = (
            alpha[..., None, None] * ssm
            + beta[..., None, None] * (v_prev[..., :, None] * k_prev[..., None, :])
            + gamma[..., None, None] * (v_t[..., :, None] * k_rot[..., None, :])
        )
        y = torch.einsum("bhpn,bhn->bhp", ssm, q_rot.to(ssm.dtype))
        if d_skip is not None:
            y = y + d_skip[None, :, None] * v_t
        if z is not None:
            z_t = z[:, :, t, :]
            y = y * (z_t * torch.sigmoid(z_t))
        ys.append(y)
        k_prev, v_prev = k_rot, v_t
    y = torch.stack(ys, dim=2)
    return y, SISOState(ssm, k_prev, v_prev, phi[:, :, -1, :])


def _bf16(x: Tensor) -> Tensor:
    """Round to bfloat16 (round-to-nearest-even) and widen back."""
    return x.to(torch.bfloat16).to(x.dtype)


def siso_chunked(
    q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip=None, z=None, state=None,
    seed_dt=None, seed_lam=None, chunk=128, return_debug=False, mm_dtype=None,
):
    """``reference.py:295-434``: chunked linear-attention form (the gradient oracle).

    ``mm_dtype=torch.bfloat16`` rounds q~, khat, v, the chunk-start state, the masked
    score matrix and the decay-scaled v to bf16 before each product, as the reference
    kernel does (``kernel_fwd.py:136-187``); products still accumulate in the working
    precision.
    """
    b, seqlen, n = q.shape
    h, p = v.shape[1], v.shape[3]
    if seqlen % chunk:
        raise ValueError(f"seqlen ({seqlen}) must be a multiple of chunk ({chunk})")
    nc = seqlen // chunk
    rnd = _bf16 if mm_dtype == torch.bfloat16 else (lambda x: x)
    dtype = adt.dtype
    v = v.to(dtype)
    if state is None:
        s0 = torch.zeros(b, h, p, n, dtype=dtype)
    else:
        if seed_dt is None or seed_lam is None:
            raise ValueError("seed_dt and seed_lam are required when passing a state")
        seed = (seed_dt * (1.0 - seed_lam))[..., None, None]
        s0 = state.ssm.to(dtype) + seed * (state.v.to(dtype)[..., :, None] * state.k.to(dtype)[..., None, :])

    u = q.to(dtype)[:, None] + q_bias[None, :, None, :]
    w = k.to(dtype)[:, None] + k_bias[None, :, None, :]
    cos, sin = rope_cos_sin(phi, n)
    q_rot = rope_apply(u, cos, sin)
    k_rot = rope_apply(w, cos, sin)
    k_hat = k_rot * scale[..., None]
    qk_diag = (u * w).sum(-1) * gamma

    qc = rnd(q_rot).reshape(b, h, nc, chunk, n)
    kc = rnd(k_hat).reshape(b, h, nc, chunk, n)
    vc = v.reshape(b, h, nc, chunk, p)
    vmc = rnd(v).reshape(b, h, nc, chunk, p)
    adtc = adt.reshape(b, h, nc, chunk)
    diagc = qk_diag.reshape(b, h, nc, chunk)
    idx = torch.arange(chunk)
    strict = idx[:, None] > idx[None, :]

    ssm = s0
    outs, states = [], []
    for c in range(nc):
        A = torch.cumsum(adtc[:, :, c], dim=-1)
        A_last = A[..., -1:]
        qb_, kb_, vb_, vmb = qc[:, :, c], kc[:, :, c], vc[:, :, c], vmc[:, :, c]
        out = torch.einsum("bhtn,bhpn->bhtp", qb_, rnd(ssm)) * torch.exp(A)[..., None]
        s = torch.einsum("bhtn,bhsn->bhts", qb_, kb_)
        s = s * torch.exp(torch.clamp(A[..., :, None] - A[..., None, :], max=0.0))
        s = torch.where(strict, s, torch.zeros_like(s))
        out = out + torch.einsum("bhts,bhsp->bhtp", rnd(s), vmb)
        coeff = diagc[:, :, c]
        if d_skip is not None:
            coeff = coeff + d_skip[None, :, None]
        out = out + coeff[..., None] * vb_
        v_scaled = rnd(vb_ * torch.exp(A_last - A)[..., None])
        states.append(ssm)
        ssm = ssm * torch.exp(A_last)[..., None] + torch.einsum("bhtp,bhtn->bhpn", v_scaled, kb_)
        outs.append(out)
    ybar = torch.stack(outs, dim=2).reshape(b, h, seqlen, p)
    y = ybar * (z.to(dtype) * torch.sigmoid(z.to(dtype))) if z is not None else ybar
    final = SISOState(ssm, k_rot[:, :, -1, :], v[:, :, -1, :], phi[:, :, -1, :])
    if not return_debug:
        return y, final
    debug = {
        "ybar": ybar,
        "chunk_states": torch.stack(states, dim=2),
        "q_rot": q_rot,
        "k_rot": k_rot,
        "k_hat": k_hat,
        "qk_diag": qk_diag,
        "uw": (u * w).sum(-1),
        "seeded_state": s0,
    }
    return y, final, debug


def siso_step(q, k, v, adt, dt, lam, angles, q_bias, k_bias, state, d_skip=None, z=None,
              mm_dtype=None):
    """``reference.py:442-490`` (three-term decode step). With ``mm_dtype=bf16`` the
    readout ``S' q~`` rounds both operands to bf16 as ``kernel_decode.py:216-222``."""
    n = q.shape[-1]
    rnd = _bf16 if mm_dtype == torch.bfloat16 else (lambda x: x)
    phi = wrap_angle(state.phi + torch.tanh(angles)[:, None, :] * math.pi * dt[..., None])
    u = q[:, None, :] + q_bias[None]
    w = k[:, None, :] + k_bias[None]
    cos, sin = rope_cos_sin(phi, n)
    q_rot = rope_apply(u, cos, sin)
    k_rot = rope_apply(w, cos, sin)
    alpha = torch.exp(adt)
    beta = alpha * dt * (1.0 - lam)
    gamma = dt * lam
    ssm = (
        alpha[..., None, None] * state.ssm
        + beta[..., None, None] * (state.v[..., :, None] * state.k[..., None, :])
        + gamma[..., None, None] * (v[..., :, None] * k_rot[..., None, :])
    )
    y = torch.einsum("bhpn,bhn->bhp", rnd(ssm), rnd(q_rot).to(ssm.dtype))
    if d_skip is not None:
        y = y + d_skip[None, :, None] * v
    if z is not None:
        y = y * (z * torch.sigmoid(z))
    return y, SISOState(ssm, k_rot, v, phi)


# ------------------------------------------------------------------------------------
# siso.py: segment wrapper (preprocess + seeding)
# ------------------------------------------------------------------------------------


def siso_segment(q, k, v, dt_raw, a_raw, trap_raw, angles, dt_bias, q_bias, k_bias,
                 d_skip=None, z=None, state=None, a_floor=1e-4, chunk=128, mm_dtype=None,
                 return_debug=False):
    """``siso.py:154-216``: preprocess this segment's raw inputs (``phi_init`` from the
    carry), seed from the carried state, run the chunked form."""
    pre, _ = preprocess(dt_raw, a_raw, trap_raw, angles, dt_bias, a_floor,
                        phi_init=None if state is None else state.phi)
    kw = {}
    if state is not None:
        kw = dict(state=state, seed_dt=pre.dt[:, :, 0], seed_lam=pre.lam[:, :, 0])
    res = siso_chunked(q, k, v, pre.adt, pre.gamma, pre.scale, pre.phi, q_bias, k_bias,
                       d_skip, z, chunk=chunk, mm_dtype=mm_dtype,
                       return_debug=return_debug, **kw)
    y, fin = res[0], res[1]
    out_state = SISOState(fin.ssm, fin.k, fin.v, pre.phi[:, :, -1, :])
    if return_debug:
        return y, out_state, res[2], pre
    return y, out_state


# ------------------------------------------------------------------------------------
# layer.py
# ------------------------------------------------------------------------------------


def layer_dims(d_model, d_state=128, headdim=64, expand=2, rope_fraction=0.5):
    """``layer.py:69-95``: (d_inner, nheads, n_angles, d_in_proj)."""
    d_inner = expand * d_model
    h = d_inner // headdim
    width = int(d_state * rope_fraction)
    width -= width % 2
    nr = width // 2
    return d_inner, h, nr, 2 * d_inner + 2 * d_state + 3 * h + nr


def split_in_proj(proj, d_inner, n, h, nr, p):
    """``layer.py:163-187``: ``[z, x, B, C, dd_dt, dd_A, trap, angles]``."""
    sizes = (d_inner, d_inner, n, n, h, h, h, nr)
    z, x, bb, cc, dt_raw, a_raw, trap_raw, angles = torch.split(proj, sizes, dim=-1)
    bsz, seqlen = proj.shape[0], proj.shape[1]
    return (z.reshape(bsz, seqlen, h, p), x.reshape(bsz, seqlen, h, p), bb, cc,
            dt_raw, a_raw, trap_raw, angles)


def rms_norm(x, weight, eps):
    """``layer.py:190-198``: f32-or-wider inside, cast back to x.dtype."""
    xf = x.to(torch.float64) if x.dtype == torch.float64 else x.float()
    rstd = torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps)
    return (xf * rstd * weight.to(xf.dtype)).to(x.dtype)


def layer_forward(params: dict, u: Tensor, d_state, headdim, expand=2, rope_fraction=0.5,
                  chunk=128, a_floor=1e-4, norm_eps=1e-5, state=None, mm_dtype=None,
                  act_dtype=None):
    """``layer.py:201-262``: in_proj -> split -> BCNorm -> siso_segment -> out_proj.

    ``params`` holds the reference's `SISOParams` fields by name, permuted layout.

    ``act_dtype=torch.bfloat16`` is the layer's bf16 rounding model, computed in the
    working precision of ``u`` (float64 for the checks): the projection weights are
    rounded as ``params.in_proj.astype(u.dtype)`` rounds them (``layer.py:233, 256``),
    and every activation the bf16 layer stores is rounded where it is stored -- the
    projection output, the normalised B and C (``rms_norm`` casts back,
    ``layer.py:196``), the scan output y (``v.dtype``, ``kernel_fwd.py:193``) and the
    layer output. Pair it with ``mm_dtype=torch.bfloat16`` for the scan's own MFMA
    operand roundings."""
    bsz, seqlen, d_model = u.shape
    d_inner, h, nr, _ = layer_dims(d_model, d_state, headdim, expand, rope_fraction)
    act = _bf16 if act_dtype == torch.bfloat16 else (lambda x: x)
    proj = act(act(u) @ act(params["in_proj"].to(u.dtype)))
    z, x, bb, cc, dt_raw, a_raw, trap_raw, angles = split_in_proj(
        proj, d_inner, d_state, h, nr, headdim)
    bb = act(rms_norm(bb, params["b_norm_weight"], norm_eps))
    cc = act(rms_norm(cc, params["c_norm_weight"], norm_eps))
    f = torch.float64 if u.dtype == torch.float64 else torch.float32
    y, st = siso_segment(
        cc, bb, x.permute(0, 2, 1, 3), dt_raw.to(f), a_raw.to(f), trap_raw.to(f),
        angles.to(f), params["dt_bias"].to(f), params["c_bias"].to(f), params["b_bias"].to(f),
        d_skip=params["d_skip"].to(f), z=z.permute(0, 2, 1, 3),
        state=state, a_floor=a_floor, chunk=chunk, mm_dtype=mm_dtype)
    y = act(y.permute(0, 2, 1, 3).reshape(bsz, seqlen, d_inner))
    return act(y.to(u.dtype) @ act(params["out_proj"].to(u.dtype))), st


def layer_decode_step(params: dict, token_embed: Tensor, state: SISOState, d_state, headdim,
                      expand=2, rope_fraction=0.5, a_floor=1e-4, norm_eps=1e-5, mm_dtype=None):
    """The per-token layer step inlined in ``model.py:266-289`` (without the block norm,
    residual and MLP): in_proj matvec, split, BCNorm, dt/a/lambda, `siso_step`,
    out_proj. ``token_embed`` is (B, d_model)."""
    bsz, d_model = token_embed.shape
    d_inner, h, nr, _ = layer_dims(d_model, d_state, headdim, expand, rope_fraction)
    proj = token_embed @ params["in_proj"].to(token_embed.dtype)
    z, x, bb, cc, dt_raw, a_raw, trap_raw, angles = split_in_proj(
        proj[:, None, :], d_inner, d_state, h, nr, headdim)
    bb = rms_norm(bb, params["b_norm_weight"], norm_eps)[:, 0]
    cc = rms_norm(cc, params["c_norm_weight"], norm_eps)[:, 0]
    f = state.ssm.dtype
    dt = F.softplus(dt_raw[:, 0].to(f) + params["dt_bias"].to(f))
    a = torch.clamp(-heavy_tail(a_raw[:, 0].to(f)), max=-a_floor)
    lam = torch.sigmoid(trap_raw[:, 0].to(f))
    y, st = siso_step(cc.to(f), bb.to(f), x[:, 0].to(f), a * dt, dt, lam, angles[:, 0].to(f),
                      params["c_bias"].to(f), params["b_bias"].to(f), state,
                      d_skip=params["d_skip"].to(f), z=z[:, 0].to(f), mm_dtype=mm_dtype)
    if mm_dtype is not None:
        y = y.to(token_embed.dtype)
    out = y.reshape(bsz, d_inner).to(token_embed.dtype) @ params["out_proj"].to(token_embed.dtype)
    return out, st


# ------------------------------------------------------------------------------------
# kernel_bwd.py epilogue semantics: gradients at the kernel boundary
# ------------------------------------------------------------------------------------


SISO_ARG_NAMES = ("q", "k", "v", "adt", "gamma", "scale", "phi", "q_bias", "k_bias",
                  "d_skip", "z", "seed_ssm", "seed_k", "seed_v", "seed_coef")


def siso_boundary_forward(q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip=None,
                          z=None, seed_ssm=None, seed_k=None, seed_v=None, seed_coef=None,
                          chunk=128, mm_dtype=None):
    """The differentiable core ``siso.siso`` (``siso.py:39-91``) as a plain function:
    returns ``(y, final_ssm, final_k, final_v)``. The seed is folded in exactly as
    ``kernel_fwd.py:97-111`` (``S0 = seed_ssm + seed_coef * v_prev (x) k_prev``)."""
    b, seqlen, n = q.shape
    h, p = v.shape[1], v.shape[3]
    dtype = adt.dtype
    if seed_ssm is not None:
        st = SISOState(seed_ssm, seed_k, seed_v, torch.zeros(b, h, 1, dtype=dtype))
        # siso_chunked computes seed as seed_dt*(1-seed_lam); pass (seed_coef, 0).
        y, fin = siso_chunked(q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip, z,
                              state=st, seed_dt=seed_coef, seed_lam=torch.zeros_like(seed_coef),
                              chunk=chunk, mm_dtype=mm_dtype)
    else:
        y, fin = siso_chunked(q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip, z,
                              chunk=chunk, mm_dtype=mm_dtype)
    return y, fin.ssm, fin.k, fin.v


def boundary_grads(inputs: dict, dy, dfinal_ssm=None, dfinal_k=None, dfinal_v=None,
                   chunk=128):
    """Autograd of `siso_boundary_forward` -- the gradient oracle for the kernel VJP,
    as ``tests.py:573-612`` takes ``jax.grad`` of ``siso_chunked``. Returns a dict of
    gradients for every tensor in ``inputs`` that is not None."""
    leaves = {}
    for name in SISO_ARG_NAMES:
        t = inputs.get(name)
        if t is not None:
            leaves[name] = t.detach().clone().requires_grad_(True)
    args = {name: leaves.get(name) for name in SISO_ARG_NAMES}
    y, fs, fk, fv = siso_boundary_forward(**args, chunk=chunk)
    loss = (y * dy).sum()
    if dfinal_ssm is not None:
        loss = loss + (fs * dfinal_ssm).sum()
    if dfinal_k is not None:
        loss = loss + (fk * dfinal_k).sum()
    if dfinal_v is not None:
        loss = loss + (fv * dfinal_v).sum()
    names = list(leaves)
    grads = torch.autograd.grad(loss, [leaves[n_] for n_ in names], allow_unused=True)
    return {n_: (g if g is not None else torch.zeros_like(leaves[n_])) for n_, g in zip(names, grads)}


# ------------------------------------------------------------------------------------
# Test-input generator (the shapes and magnitudes of tests.py:179-212)
# ------------------------------------------------------------------------------------


def make_inputs(b, h, seqlen, n, p, nr, seed=0, dtype=torch.float64):
    """Kernel-boundary inputs with the magnitudes of ``tests.py:179-212``: q/k RMS
    normalised, dt log-uniform in [1e-3, 1e-1] (dt_raw its inverse softplus, bias 0),
    a/trap ~ N(0,1), angles ~ 0.5 N(0,1), biases ~ 0.1 N(0,1), D, z, v, dy ~ N(0,1).
    Draws come from a seeded torch generator, not JAX's threefry."""
    g = torch.Generator().manual_seed(seed)

    def rn(*shape):
        return torch.randn(*shape, generator=g, dtype=torch.float64)

    def norm_rows(x):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6)

    dt = torch.exp(torch.rand(b, seqlen, h, generator=g, dtype=torch.float64)
                   * (math.log(0.1) - math.log(0.001)) + math.log(0.001))
    out = {
        "q": norm_rows(rn(b, seqlen, n)),
        "k": norm_rows(rn(b, seqlen, n)),
        "v": rn(b, h, seqlen, p),
        "z": rn(b, h, seqlen, p),
        "dt_raw": torch.log(torch.expm1(dt)),
        "a_raw": rn(b, seqlen, h),
        "trap_raw": rn(b, seqlen, h),
        "angles": rn(b, seqlen, nr) * 0.5,
        "dt_bias": torch.zeros(h, dtype=torch.float64),
        "q_bias": rn(h, n) * 0.1,
        "k_bias": rn(h, n) * 0.1,
        "d_skip": rn(h),
        "dy": rn(b, h, seqlen, p),
    }
    return {k_: v_.to(dtype) for k_, v_ in out.items()}


def rel_error(got, ref, mag_floor=1e-2, pct=95.0, angle=False) -> float:
    """``tests.py:60-88``: p95 relative error over |ref| >= 1e-2 (circular absolute
    error for angles)."""
    g = torch.as_tensor(got).detach().to(torch.float64).cpu()
    r = torch.as_tensor(ref).detach().to(torch.float64).cpu()
    if g.shape != r.shape:
        raise AssertionError(f"shape mismatch: {tuple(g.shape)} vs {tuple(r.shape)}")
    if angle:
        d = torch.abs(torch.remainder(g - r + math.pi, 2 * math.pi) - math.pi)
        return float(torch.quantile(d.flatten(), pct / 100.0)) if d.numel() else 0.0
    mask = r.abs() >= mag_floor
    if not bool(mask.any()):
        return 0.0
    e = (g - r).abs()[mask] / r.abs()[mask]
    return float(_percentile(e, pct))


def _percentile(x: Tensor, pct: float) -> float:
    x = x.flatten()
    if x.numel() > 1_000_000:  # torch.quantile caps input size
        x = x[torch.randperm(x.numel(), generator=torch.Generator().manual_seed(0))[:1_000_000]]
    return float(torch.quantile(x, pct / 100.0))


def max_rel(got, ref) -> float:
    """``tests.py:91-96``: max |got-ref| normalised by max |ref|."""
    g = torch.as_tensor(got).detach().to(torch.float64).cpu()
    r = torch.as_tensor(ref).detach().to(torch.float64).cpu()
    return float((g - r).abs().max() / max(float(r.abs().max()), 1e-30))


def max_abs(got, ref) -> float:
    g = torch.as_tensor(got).detach().to(torch.float64).cpu()
    r = torch.as_tensor(ref).detach().to(torch.float64).cpu()
    return float((g - r).abs().max())

