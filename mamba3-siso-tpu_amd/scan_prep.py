"""The carried state and the per-token preprocessing (``reference.py`` product half).

``SISOState`` / ``zero_state`` / ``preprocess`` and its helpers keep the reference's
names and semantics (``reference.py:46-209``).

`preprocess` -- elementwise algebra plus the cumulative angle sum over time -- runs on
the device through ``m3s_prep_fwd``, and its backward (``m3s_prep_bwd``: the suffix sum
of ``dphi``, the head sum of the angle cotangent, the raw-slice cotangents) is wired
in as a `torch.autograd.Function`, where the reference leaves it to ``jax.grad``
(``siso.py:1-11``). The small helpers `heavy_tail`, `trapezoid_coeffs`, `wrap_angle`
and `cumulative_angles` stay plain torch functions for callers that use them
directly; the layer does not.
"""

from __future__ import annotations

import ctypes
import dataclasses
import math
from typing import NamedTuple, Optional

import torch
import torch.nn.functional as F

from . import _lib
from . import kernels as K

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


def _raw_dtype(*ts) -> torch.dtype:
    dts = {t.dtype for t in ts}
    if len(dts) == 1 and dts <= {torch.bfloat16, torch.float32}:
        return dts.pop()
    return torch.float32


def _raw_operand(t: Tensor, dt: torch.dtype) -> Tensor:
    """A (B, L, X) operand the kernel reads in place: unit stride on X."""
    if t.dtype != dt:
        t = t.to(dt)
    return t if (t.stride(2) == 1 or t.shape[2] <= 1) else t.contiguous()


def _check_device(*ts) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(
                "preprocess runs on the ROCm device only; got a CPU tensor "
                "(move inputs to 'cuda' -- there is no CPU fallback)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _f32c(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None else t.to(torch.float32).contiguous()


def prep_forward_launch(r_dt: Tensor, r_a: Tensor, r_tr: Tensor, r_ang: Tensor,
                        bias: Tensor, init: Optional[Tensor], a_floor: float,
                        compact: bool = False):
    """One ``m3s_prep_fwd`` call on raw ``(B, L, X)`` operands with a unit last stride and
    one dtype (bf16 or f32); ``bias`` and ``init`` f32 contiguous. Returns fresh
    ``(adt, gamma, scale, lam, dt, phi, phi_final)``. With ``compact`` (needs
    ``L % 16 == 0``) phi is not materialised: the sixth entry is a `kernels.PhiStrips`
    (the head-shared ``tanh(angles) pi`` table, dt and the angle entering each 16-token
    strip), which the scan kernels take in place of phi."""
    from .kernels import PhiStrips

    batch, seqlen, nheads = r_dt.shape
    n_angles = r_ang.shape[-1]
    dev = r_dt.device
    f32 = dict(device=dev, dtype=torch.float32)
    adt, gamma, scale, lam, dt = (K.empty(batch, nheads, seqlen, **f32) for _ in range(5))
    phi_final = K.empty(batch, nheads, n_angles, **f32)
    lib = _lib.load()
    ws = K.empty(lib.m3s_prep_fwd_workspace_bytes(batch, seqlen, nheads, n_angles),
                     device=dev, dtype=torch.uint8)
    a = _lib.PrepFwdArgs()
    a.struct_size = ctypes.sizeof(_lib.PrepFwdArgs)
    a.batch, a.seqlen, a.nheads, a.n_angles = batch, seqlen, nheads, n_angles
    a.dtype = _lib.dtype_code(r_dt.dtype)
    a.has_phi_init = int(init is not None)
    a.a_floor = float(a_floor)
    a.dt_raw, a.a_raw, a.trap_raw, a.angles = (_lib.blx(t) for t in (r_dt, r_a, r_tr, r_ang))
    a.dt_bias, a.phi_init = bias.data_ptr(), _lib.ptr(init)
    a.adt, a.gamma, a.scale, a.lam, a.dt = (t.data_ptr() for t in (adt, gamma, scale, lam, dt))
    if compact:
        table = K.empty(batch, seqlen, n_angles, **f32)
        strips = K.empty(batch, nheads, seqlen // 16, n_angles, **f32)
        a.theta_table, a.phi_strips = table.data_ptr(), strips.data_ptr()
        phi = PhiStrips(table, dt, strips)
    else:
        phi = K.empty(batch, nheads, seqlen, n_angles, **f32)
        a.phi = phi.data_ptr()
    a.phi_final = phi_final.data_ptr()
    a.workspace = ws.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(lib.m3s_prep_fwd(ctypes.byref(a), _lib.stream_handle(dev)), "m3s_prep_fwd")
    return adt, gamma, scale, lam, dt, phi, phi_final


def prep_backward_launch(r_dt: Tensor, r_a: Tensor, r_tr: Tensor, r_ang: Tensor, bias: Tensor,
                         a_floor: float, cots, d_dt: Tensor, d_a: Tensor, d_tr: Tensor,
                         d_ang: Tensor, d_bias: Tensor, d_init: Optional[Tensor]) -> None:
    """One ``m3s_prep_bwd`` call. ``cots`` = (dadt, dgamma, dscale, dlam, ddt, dphi,
    dphi_final), each a tensor or None. The raw cotangents are written into ``d_dt``,
    ``d_a``, ``d_tr``, ``d_ang`` (any ``(B, L, X)`` strides with a unit last stride, in
    the raw operands' dtype -- e.g. slices of the projection's gradient)."""
    batch, seqlen, nheads = r_dt.shape
    n_angles = r_ang.shape[-1]
    dev = r_dt.device
    ins = [_f32c(t) for t in cots]
    lib = _lib.load()
    ws = K.empty(lib.m3s_prep_bwd_workspace_bytes(batch, seqlen, nheads, n_angles),
                     device=dev, dtype=torch.uint8)
    a = _lib.PrepBwdArgs()
    a.struct_size = ctypes.sizeof(_lib.PrepBwdArgs)
    a.batch, a.seqlen, a.nheads, a.n_angles = batch, seqlen, nheads, n_angles
    a.dtype = _lib.dtype_code(r_dt.dtype)
    a.a_floor = float(a_floor)
    a.dt_raw, a.a_raw, a.trap_raw, a.angles = (_lib.blx(t) for t in (r_dt, r_a, r_tr, r_ang))
    a.dt_bias = bias.data_ptr()
    (a.dadt, a.dgamma, a.dscale, a.dlam, a.ddt, a.dphi,
     a.dphi_final) = (_lib.ptr(t) for t in ins)
    a.ddt_raw, a.da_raw, a.dtrap_raw, a.dangles = (_lib.blx(t) for t in (d_dt, d_a, d_tr, d_ang))
    a.ddt_bias, a.dphi_init = d_bias.data_ptr(), _lib.ptr(d_init)
    a.workspace = ws.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(lib.m3s_prep_bwd(ctypes.byref(a), _lib.stream_handle(dev)), "m3s_prep_bwd")


class _PrepFn(torch.autograd.Function):
    """``reference.preprocess`` with its backward (``jax.grad`` in the reference) as
    two HIP launches. Outputs: adt, gamma, scale, phi, lam, dt, phi_final."""

    @staticmethod
    def forward(ctx, dt_raw, a_raw, trap_raw, angles, dt_bias, phi_init, a_floor):
        dev = _check_device(dt_raw, a_raw, trap_raw, angles, dt_bias, phi_init)
        batch, seqlen, nheads = dt_raw.shape
        n_angles = angles.shape[-1]
        for name, t in (("a_raw", a_raw), ("trap_raw", trap_raw)):
            if tuple(t.shape) != (batch, seqlen, nheads):
                raise ValueError(f"{name} must be (B, L, H) = {(batch, seqlen, nheads)}, "
                                 f"got {tuple(t.shape)}")
        if tuple(angles.shape[:2]) != (batch, seqlen) or angles.dim() != 3:
            raise ValueError(f"angles must be (B, L, Nr), got {tuple(angles.shape)}")
        if tuple(dt_bias.shape) != (nheads,):
            raise ValueError(f"dt_bias must be (H,) = ({nheads},), got {tuple(dt_bias.shape)}")
        if phi_init is not None and tuple(phi_init.shape) != (batch, nheads, n_angles):
            raise ValueError(f"phi_init must be (B, H, Nr) = {(batch, nheads, n_angles)}, "
                             f"got {tuple(phi_init.shape)}")
        rdt = _raw_dtype(dt_raw, a_raw, trap_raw, angles)
        r_dt, r_a, r_tr, r_ang = (_raw_operand(t, rdt) for t in (dt_raw, a_raw, trap_raw, angles))
        bias = _f32c(dt_bias)
        adt, gamma, scale, lam, dt, phi, phi_final = prep_forward_launch(
            r_dt, r_a, r_tr, r_ang, bias, _f32c(phi_init), a_floor)
        ctx.save_for_backward(r_dt, r_a, r_tr, r_ang, bias)
        ctx.a_floor = float(a_floor)
        ctx.in_dtypes = (dt_raw.dtype, a_raw.dtype, trap_raw.dtype, angles.dtype, dt_bias.dtype,
                         None if phi_init is None else phi_init.dtype)
        ctx.set_materialize_grads(False)
        return adt, gamma, scale, phi, lam, dt, phi_final

    @staticmethod
    def backward(ctx, dadt, dgamma, dscale, dphi, dlam, ddt, dphi_final):
        r_dt, r_a, r_tr, r_ang, bias = ctx.saved_tensors
        batch, seqlen, nheads = r_dt.shape
        n_angles = r_ang.shape[-1]
        dev = r_dt.device
        rdt = r_dt.dtype
        d_dt = K.empty(batch, seqlen, nheads, device=dev, dtype=rdt)
        d_a = K.empty_like(d_dt)
        d_tr = K.empty_like(d_dt)
        d_ang = K.empty(batch, seqlen, n_angles, device=dev, dtype=rdt)
        d_bias = K.empty(nheads, device=dev, dtype=torch.float32)
        want_init = ctx.in_dtypes[5] is not None and ctx.needs_input_grad[5]
        d_init = (K.empty(batch, nheads, n_angles, device=dev, dtype=torch.float32)
                  if want_init else None)
        prep_backward_launch(r_dt, r_a, r_tr, r_ang, bias, ctx.a_floor,
                             (dadt, dgamma, dscale, dlam, ddt, dphi, dphi_final),
                             d_dt, d_a, d_tr, d_ang, d_bias, d_init)
        dts = ctx.in_dtypes

        def cast(t, d):
            return None if (t is None or d is None) else t.to(d)

        return (cast(d_dt, dts[0]), cast(d_a, dts[1]), cast(d_tr, dts[2]), cast(d_ang, dts[3]),
                cast(d_bias, dts[4]), cast(d_init, dts[5]), None)


def preprocess(dt_raw: Tensor, a_raw: Tensor, trap_raw: Tensor, angles: Tensor,
               dt_bias: Tensor, a_floor: float = 1e-4, phi_init: Optional[Tensor] = None):
    """``reference.py:160-199``. Raw slices ``(B, L, H)``, angles ``(B, L, Nr)`` (any
    strides with a unit last stride -- e.g. slices of the fused projection); all on the
    ROCm device.

    Returns ``(Preprocessed, phi_final)``; every output is f32 and differentiable
    w.r.t. the raw slices, ``dt_bias`` and ``phi_init``.
    """
    adt, gamma, scale, phi, lam, dt, phi_final = _PrepFn.apply(
        dt_raw, a_raw, trap_raw, angles, dt_bias, phi_init, a_floor)
    return Preprocessed(adt=adt, gamma=gamma, scale=scale, phi=phi, lam=lam, dt=dt), phi_final
