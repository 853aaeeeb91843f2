"""Autograd glue tying the HIP forward and backward together (``siso.py`` surface).

The differentiable boundary sits where the reference puts it (``siso.py:39-151``):
at ``(q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip, z, seed_ssm, seed_kv,
seed_coef)``. `preprocess` runs in front of it as its own differentiable HIP step
(``scan_prep._PrepFn``), which carries ``dgamma``/``dscale``/``dphi`` back to
``dt``/``lambda``/``angles`` where the reference relies on ``jax.grad``.
"""

from __future__ import annotations

from typing import Any, NamedTuple, Optional

import torch

from . import kernels as K
from . import layout as LY
from .scan_prep import SISOState, preprocess

Tensor = torch.Tensor


class SISOOutput(NamedTuple):
    """``siso.py:27-36``: y ``(B, H, L, P)`` gated output, and the carry."""

    y: Tensor
    state: SISOState


def _split_kv(seed_kv: Optional[Tensor], n: int):
    if seed_kv is None:
        return None, None
    return seed_kv[..., :n], seed_kv[..., n:]


class _SisoFn(torch.autograd.Function):
    """``jax.custom_vjp`` of ``siso.py:39-148`` as a torch autograd Function."""

    @staticmethod
    def forward(ctx, q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip, z,
                seed_ssm, seed_kv, seed_coef, chunk, policy_name):
        n = q.shape[-1]
        seed_k, seed_v = _split_kv(seed_kv, n)
        need_res = any(ctx.needs_input_grad[:14])
        outs = K.siso_forward(
            q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip=d_skip, z=z,
            seed_ssm=seed_ssm, seed_k=seed_k, seed_v=seed_v, seed_coef=seed_coef,
            chunk=chunk, dtype_policy=policy_name, save_residuals=need_res)
        y, fs, fk, fv = outs[:4]
        if need_res:
            res = outs[4]
            ctx.save_for_backward(q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip, z,
                                  seed_ssm, seed_kv, seed_coef, res.ybar, res.chunk_states)
        ctx.chunk, ctx.policy_name = chunk, policy_name
        ctx.set_materialize_grads(False)  # unused final-state cotangents arrive as None
        return y, fs, fk, fv

    @staticmethod
    def backward(ctx, dy, dfs, dfk, dfv):
        (q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip, z,
         seed_ssm, seed_kv, seed_coef, ybar, chunk_states) = ctx.saved_tensors
        n = q.shape[-1]
        seed_k, seed_v = _split_kv(seed_kv, n)
        if dy is None:
            dy = torch.zeros_like(v)
        g = K.siso_backward(
            dy, q, k, v, adt, gamma, scale, phi, q_bias, k_bias, ybar, chunk_states,
            d_skip=d_skip, z=z, seed_ssm=seed_ssm, seed_k=seed_k, seed_v=seed_v,
            seed_coef=seed_coef, dfinal_ssm=dfs, dfinal_k=dfk, dfinal_v=dfv,
            chunk=ctx.chunk, dtype_policy=ctx.policy_name)
        dseed_kv = (torch.cat([g.dseed_k, g.dseed_v], dim=-1)
                    if seed_kv is not None else None)

        # Cast back to each primal's dtype, as siso.py:140-148 does.
        def like(x, p_):
            return None if (p_ is None or x is None) else x.to(p_.dtype)

        return (like(g.dq, q), like(g.dk, k), like(g.dv, v), like(g.dadt, adt),
                like(g.dgamma, gamma), like(g.dscale, scale), like(g.dphi, phi),
                like(g.dq_bias, q_bias), like(g.dk_bias, k_bias), like(g.dd_skip, d_skip),
                like(g.dz, z), like(g.dseed_ssm, seed_ssm), like(dseed_kv, seed_kv),
                like(g.dseed_coef, seed_coef), None, None)


def siso(q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip, z, seed_ssm, seed_kv,
         seed_coef, chunk: int = 128, policy_name: str = "bf16", interpret: Any = False,
         device_kind: str | None = None):
    """Differentiable chunked SISO scan (``siso.py:39-91``).

    Returns ``(y, final_ssm, final_k, final_v)``; ``final_k`` is rotated, unscaled.
    ``y`` (and, in the backward, ``dv``/``dz``) take ``v``'s memory layout.
    """
    return _SisoFn.apply(q, k, v, adt, gamma, scale, phi, q_bias, k_bias, d_skip, z,
                         seed_ssm, seed_kv, seed_coef, chunk, LY.policy(policy_name).name)


def siso_segment(q, k, v, dt_raw, a_raw, trap_raw, angles, dt_bias, q_bias, k_bias,
                 d_skip=None, z=None, state: Optional[SISOState] = None, a_floor: float = 1e-4,
                 chunk: int = 128, policy_name: str = "bf16", interpret: Any = False,
                 device_kind: str | None = None) -> SISOOutput:
    """``siso.py:154-216``: preprocess this segment's own raw inputs (``phi_init`` from
    the carry -- never slice a whole-sequence ``scale``), seed from the carried state,
    run the scan, return the carry."""
    pre, phi_final = preprocess(dt_raw, a_raw, trap_raw, angles, dt_bias, a_floor=a_floor,
                                phi_init=None if state is None else state.phi)
    if state is None:
        seed_ssm = seed_kv = seed_coef = None
    else:
        seed_ssm = state.ssm
        seed_kv = torch.cat([state.k.float(), state.v.float()], dim=-1)
        seed_coef = pre.dt[:, :, 0] * (1.0 - pre.lam[:, :, 0])
    y, fs, fk, fv = siso(q, k, v, pre.adt, pre.gamma, pre.scale, pre.phi, q_bias, k_bias,
                         d_skip, z, seed_ssm, seed_kv, seed_coef, chunk, policy_name)
    return SISOOutput(y=y, state=SISOState(ssm=fs, k=fk, v=fv, phi=phi_final))
