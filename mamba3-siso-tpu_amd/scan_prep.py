"""The carried state and the per-token preprocessing (``reference.py`` product half).

``SISOState`` / ``zero_state`` / ``preprocess`` and its helpers keep the reference's
names and semantics (``reference.py:46-209``). The preprocessing is cheap elementwise
algebra plus one cumulative sum over time; it runs as torch ops on the device and
its autograd supplies the cotangents of ``dt``/``lambda``/``angles`` from the kernel's
``dgamma``/``dscale``/``dphi``, exactly as the reference leaves it to ``jax.grad``
(``siso.py:1-11``).
"""

from __future__ import annotations

import dataclasses
import math
from typing import NamedTuple, Optional

import torch
import torch.nn.functional as F

TWO_PI = 2.0 * math.pi
Tensor = torch.Tensor


class SISOState(NamedTuple):
    """Carry between segments and between prefill and decode (``reference.py:46-63``).

    ssm ``(B, H, P, N)`` f32; k ``(B, H, N)`` previous token's rotated, *unscaled* key;
    v ``(B, H, P)`` previous token's value; phi ``(B, H, Nr)`` cumulative angle mod 2pi.
    """

    ssm: Tensor
    k: Tensor
    v: Tensor
    phi: Tensor


def zero_state(batch: int, nheads: int, headdim: int, state_dim: int, n_angles: int,
               dtype=torch.float32, device=None) -> SISOState:
    """``reference.py:66-74``."""
    return SISOState(
        ssm=torch.zeros(batch, nheads, headdim, state_dim, dtype=torch.float32, device=device),
        k=torch.zeros(batch, nheads, state_dim, dtype=dtype, device=device),
        v=torch.zeros(batch, nheads, headdim, dtype=dtype, device=device),
        phi=torch.zeros(batch, nheads, n_angles, dtype=torch.float32, device=device),
    )


@dataclasses.dataclass(frozen=True)
class Preprocessed:
    """``reference.py:82-101``: adt, gamma, scale, lam, dt are ``(B, H, L)``; phi is
    ``(B, H, L, Nr)``."""

    adt: Tensor
    gamma: Tensor
    scale: Tensor
    phi: Tensor
    lam: Tensor
    dt: Tensor


def heavy_tail(x: Tensor) -> Tensor:
    """``reference.py:202-209``: ``1 + x`` for x >= 0, ``1/(1 - x)`` for x < 0."""
    return torch.clamp(x, min=0.0) + torch.reciprocal(1.0 - torch.clamp(x, max=0.0))


def trapezoid_coeffs(dt: Tensor, lam: Tensor) -> tuple[Tensor, Tensor]:
    """``reference.py:104-131``: ``gamma = dt lam``; ``scale_t = gamma_t +
    dt_{t+1}(1 - lam_{t+1})``, the last position having no successor."""
    gamma = dt * lam
    dt_next = F.pad(dt[..., 1:], (0, 1))
    lam_next = F.pad(lam[..., 1:], (0, 1))
    return gamma, gamma + dt_next * (1.0 - lam_next)


def wrap_angle(phi: Tensor) -> Tensor:
    """``phi - 2 pi floor(phi / 2 pi)``; ``floor`` has zero derivative, so autograd
    passes straight through (``reference.py:150-156``)."""
    return phi - TWO_PI * torch.floor(phi / TWO_PI).detach()


def cumulative_angles(angles: Tensor, dt: Tensor, phi_init: Optional[Tensor] = None):
    """``reference.py:134-157``: ``phi_t = (phi_init + sum_{i<=t} tanh(angles_i) pi dt_i)
    mod 2 pi``. ``angles`` is ``(B, H, L, Nr)`` (or ``(B, 1, L, Nr)`` -- broadcast)."""
    theta = torch.tanh(angles.float()) * math.pi * dt[..., None]
    phi = torch.cumsum(theta, dim=2)
    if phi_init is not None:
        phi = phi + phi_init[:, :, None, :].float()
    phi = wrap_angle(phi)
    return phi, phi[:, :, -1, :]


def preprocess(dt_raw: Tensor, a_raw: Tensor, trap_raw: Tensor, angles: Tensor,
               dt_bias: Tensor, a_floor: float = 1e-4, phi_init: Optional[Tensor] = None):
    """``reference.py:160-199``. Raw slices ``(B, L, H)``, angles ``(B, L, Nr)``.

    Returns ``(Preprocessed, phi_final)``; every output is f32.
    """
    dt = F.softplus(dt_raw.float() + dt_bias.float()).transpose(1, 2)
    a = -heavy_tail(a_raw.float()).transpose(1, 2)
    a = torch.clamp(a, max=-a_floor)  # negate first, then clamp (torch_ref.py:212-217)
    lam = torch.sigmoid(trap_raw.float()).transpose(1, 2)
    gamma, scale = trapezoid_coeffs(dt, lam)
    phi, phi_final = cumulative_angles(angles[:, None], dt, phi_init)
    return Preprocessed(adt=(a * dt).contiguous(), gamma=gamma.contiguous(),
                        scale=scale.contiguous(), phi=phi.contiguous(), lam=lam, dt=dt), phi_final
