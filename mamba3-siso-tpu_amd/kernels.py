"""Python entry points over the HIP kernels, with the reference's kernel signatures.

* `siso_forward`   -- ``kernel_fwd.siso_forward``   (kernel_fwd.py:204-388)
* `siso_backward_kernel` / `siso_backward` -- ``kernel_bwd.py:358-669``
* `siso_decode`, `siso_decode_folded`, `decode_step`, `decode_scan`, `decode_loop`
  -- ``kernel_decode.py:252-573``

Each validates shapes with the reference's ``ValueError`` conditions, then calls the
C ABI (``include/m3s.h``) on the current torch stream. Nothing here computes on the
CPU: every tensor must already be on the ROCm device, and a missing library raises.
``interpret`` and ``device_kind`` are accepted for signature compatibility and ignored.
"""

from __future__ import annotations

import ctypes
import math
from typing import Any, NamedTuple, Optional

import torch

from . import _lib
from . import layout as LY

Tensor = torch.Tensor

#: Test-only switch (no counterpart in the reference): when True, `empty` and
#: `empty_like` -- which allocate every kernel output and workspace in this package --
#: fill the new memory with all-ones bytes (NaN for float32, bfloat16 and float16), so a
#: region a kernel fails to write, or scratch it reads before writing, surfaces as a
#: non-finite value in the parity checks. The product path never sets it.
POISON_OUTPUTS = False


def empty(*size, device=None, dtype=None) -> Tensor:
    """``torch.empty`` for kernel outputs and workspaces (see `POISON_OUTPUTS`)."""
    t = torch.empty(*size, device=device, dtype=dtype)
    if POISON_OUTPUTS:
        t.view(torch.uint8).fill_(255) if t.numel() else None
    return t


def empty_like(x: Tensor) -> Tensor:
    """``torch.empty_like`` for kernel outputs (see `POISON_OUTPUTS`)."""
    return empty(x.shape, device=x.device, dtype=x.dtype)


class PhiStrips(NamedTuple):
    """phi in the compact form the scan kernels rebuild it from (the cumulative angle of
    ``reference.py:134-157`` fused into the scan): ``phi[t] = strips[t // 16] +
    sum_{16 (t // 16) <= t' <= t} table[t'] * dt[t']`` taken mod 2 pi. ``table`` is
    ``tanh(angles) pi`` ``(B, L, Nr)`` (shared by the heads), ``dt`` ``(B, H, L)``,
    ``strips`` ``(B, H, L / 16, Nr)`` the wrapped angle entering each 16-token strip. The
    kernels accept it wherever they take ``phi``; it is 1/16 of phi's bytes plus the
    head-shared table."""

    table: Tensor
    dt: Tensor
    strips: Tensor

    @property
    def shape(self):
        b, h, l = self.dt.shape
        return (b, h, l, self.table.shape[-1])

    def last(self) -> Tensor:
        """phi at the last position, ``(B, H, Nr)`` in [0, 2 pi)."""
        theta = torch.einsum("bln,bhl->bhn", self.table[:, -16:].float(), self.dt[:, :, -16:].float())
        return torch.remainder(self.strips[:, :, -1, :] + theta, 2 * math.pi)


def _phi_fields(a, phi, dev) -> list:
    """Fill ``a.phi`` or the three ``phi_strips`` fields of an args struct; returns the
    converted tensors, which must stay alive until the launch."""
    if isinstance(phi, PhiStrips):
        tab, dt, st = _f32c(phi.table), _f32c(phi.dt), _f32c(phi.strips)
        _device_of(tab, dt, st)
        a.phi = None
        a.theta_table, a.phi_dt, a.phi_strips = tab.data_ptr(), dt.data_ptr(), st.data_ptr()
        return [tab, dt, st]
    ph = _f32c(phi)
    a.phi = ph.data_ptr()
    return [ph]


class ForwardResiduals(NamedTuple):
    """``kernel_fwd.py:41-52``. ``chunk_states`` is the logical ``(B, H, nc, P, N)``
    view of an N-major ``(B, H, nc, N, P)`` buffer (the layout the backward reads).
    ``ybar`` is in the policy's matmul dtype (bf16 under the bf16 policy; the reference
    keeps it float32): the backward only uses it in ``dz``, where its bf16 rounding is far
    inside the gradient tolerance, and it halves the residual's bytes."""

    ybar: Tensor
    chunk_states: Tensor


def _device_of(*ts) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(
                "the Mamba-3 SISO kernels run on the ROCm device only; got a CPU tensor "
                "(move inputs to 'cuda' -- there is no CPU fallback)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _f32c(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None else t.to(torch.float32).contiguous()


def _mt(t: Optional[Tensor], mt: torch.dtype) -> Optional[Tensor]:
    return None if t is None else t.to(mt).contiguous()


def _bhlp_operand(t: Optional[Tensor], mt: torch.dtype) -> Optional[Tensor]:
    """Keep a strided (B, H, L, P) view if the kernel can read it in place."""
    if t is None:
        return None
    if t.dtype != mt:
        t = t.to(mt)
    vec = 16 // t.element_size()
    ok = (t.stride(3) == 1 and t.data_ptr() % 16 == 0
          and all(t.stride(i) % vec == 0 for i in range(3)))
    return t if ok else t.contiguous()


def _empty_like_layout(v: Tensor, dtype: torch.dtype) -> Tensor:
    """A new ``(B, H, L, P)`` tensor laid out like ``v``: if ``v`` is a time-major view
    (a ``(B, L, H, P)`` buffer, e.g. a slice of the fused in_proj output), the result
    is the same permuted view of a fresh ``(B, L, H, P)`` buffer, so the layer can
    reshape it to ``(B, L, H*P)`` for free."""
    b, h, l, p = v.shape
    if v.stride(2) > v.stride(1):
        return empty(b, l, h, p, device=v.device, dtype=dtype).permute(0, 2, 1, 3)
    return empty(b, h, l, p, device=v.device, dtype=dtype)


def _tile(pol: LY.DtypePolicy, chunk: int, state_dim: int, headdim: int, role: str) -> int:
    """`layout.kernel_chunk`, or the error naming what is compiled."""
    tile = LY.kernel_chunk(pol.name, chunk, state_dim, headdim)
    if tile is None:
        raise ValueError(
            f"no {role} kernel for policy={pol.name} chunk={chunk} d_state={state_dim} "
            f"headdim={headdim}; chunks compiled for this shape: "
            f"{list(LY.compiled_chunks(pol.name, state_dim, headdim))}")
    return tile


def _width(pol: LY.DtypePolicy, chunk: int, state_dim: int, headdim: int, role: str) -> int:
    """`layout.kernel_headdim`, or the error naming the shape."""
    width = LY.kernel_headdim(pol.name, chunk, state_dim, headdim)
    if width is None:
        raise ValueError(
            f"no {role} kernel for policy={pol.name} chunk={chunk} d_state={state_dim} "
            f"headdim={headdim}; chunks compiled for this shape: "
            f"{list(LY.compiled_chunks(pol.name, state_dim, headdim))}")
    return width


# A head of width P runs as r = P / P' sub-heads of a compiled width P' (layout.kernel_headdim):
# sub-head h*r + s takes columns s*P'.. of head h and shares every other input of head h.
def _rep(t: Optional[Tensor], r: int, dim: int = 1) -> Optional[Tensor]:
    """A per-head input, repeated for each of the head's r sub-heads."""
    return None if t is None else t.repeat_interleave(r, dim=dim)


def _split_cols(t: Optional[Tensor], r: int) -> Optional[Tensor]:
    """``(B, H, L, P)`` -> ``(B, H*r, L, P/r)``: a view when a head's columns are adjacent in
    memory (the layer's ``(B, L, H*P)`` layout), else a copy."""
    if t is None:
        return None
    b, h, l, p = t.shape
    return t.unflatten(3, (r, p // r)).permute(0, 1, 3, 2, 4).reshape(b, h * r, l, p // r)


def _merge_cols(t: Tensor, r: int) -> Tensor:
    """Inverse of `_split_cols`: ``(B, H*r, L, P')`` -> ``(B, H, L, r*P')``."""
    b, hr, l, pp = t.shape
    return t.unflatten(1, (hr // r, r)).permute(0, 1, 3, 2, 4).reshape(b, hr // r, l, r * pp)


def _rep_phi(phi, r: int):
    if isinstance(phi, PhiStrips):
        return PhiStrips(phi.table, _rep(phi.dt, r), _rep(phi.strips, r))
    return _rep(phi, r)


def _head_sum(t: Tensor, r: int, dim: int = 1) -> Tensor:
    """Sum a per-sub-head gradient over each head's r sub-heads (in sub-head order)."""
    return t.unflatten(dim, (t.shape[dim] // r, r)).sum(dim + 1)


def siso_forward(
    q: Tensor, k: Tensor, v: Tensor, adt: Tensor, gamma: Tensor, scale: Tensor,
    phi: Tensor, q_bias: Tensor, k_bias: Tensor, d_skip: Optional[Tensor] = None,
    z: Optional[Tensor] = None, seed_ssm: Optional[Tensor] = None,
    seed_k: Optional[Tensor] = None, seed_v: Optional[Tensor] = None,
    seed_coef: Optional[Tensor] = None, chunk: int = 128,
    dtype_policy: LY.DtypePolicy | str = LY.BF16, save_residuals: bool = False,
    interpret: Any = False, device_kind: str | None = None,
):
    """Chunked forward (``kernel_fwd.py:204-248``).

    Returns ``(y, final_ssm, final_k, final_v)`` and, with ``save_residuals``, a
    `ForwardResiduals`. ``y`` has ``v``'s memory layout (see `_empty_like_layout`).
    A ``chunk`` with no kernel of its own runs as tiles of `layout.kernel_chunk`; the
    residual ``chunk_states`` are then per tile.
    """
    pol = LY.policy(dtype_policy)
    LY.validate_chunk(chunk)
    batch, seqlen, state_dim = q.shape
    nheads, headdim = v.shape[1], v.shape[3]
    n_angles = phi.shape[-1]
    LY.num_chunks(seqlen, chunk)
    width = _width(pol, chunk, state_dim, headdim, "forward")
    if width != headdim and tuple(v.shape) == (batch, nheads, seqlen, headdim):
        r = headdim // width
        sd = lambda t, *s: None if t is None else t.reshape(batch, nheads * r, *s)  # noqa: E731
        outs = siso_forward(
            q, k, _split_cols(v, r), _rep(adt, r), _rep(gamma, r), _rep(scale, r),
            _rep_phi(phi, r), _rep(q_bias, r, 0), _rep(k_bias, r, 0), _rep(d_skip, r, 0),
            _split_cols(z, r), sd(seed_ssm, width, state_dim), _rep(seed_k, r),
            sd(seed_v, width), _rep(seed_coef, r), chunk=chunk, dtype_policy=pol,
            save_residuals=save_residuals)
        y, fs, fk, fv = outs[:4]
        res = (_merge_cols(y, r), fs.reshape(batch, nheads, headdim, state_dim),
               fk[:, ::r].contiguous(), fv.reshape(batch, nheads, headdim))
        if save_residuals:
            cs = outs[4].chunk_states   # (B, H*r, nc, P', N)
            cs = cs.unflatten(1, (nheads, r)).permute(0, 1, 3, 2, 4, 5).reshape(
                batch, nheads, cs.shape[2], headdim, state_dim)
            res += (ForwardResiduals(ybar=_merge_cols(outs[4].ybar, r), chunk_states=cs),)
        return res
    chunk = _tile(pol, chunk, state_dim, headdim, "forward")
    nc = seqlen // chunk
    if q.shape != k.shape:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} must match")
    if tuple(v.shape) != (batch, nheads, seqlen, headdim):
        raise ValueError(f"unexpected v shape {tuple(v.shape)}")
    for name, t in (("adt", adt), ("gamma", gamma), ("scale", scale)):
        if tuple(t.shape) != (batch, nheads, seqlen):
            raise ValueError(
                f"{name} must be (B, H, L) = {(batch, nheads, seqlen)}, got {tuple(t.shape)}")
    seeds = (seed_ssm, seed_k, seed_v, seed_coef)
    has_seed = any(s is not None for s in seeds)
    if has_seed and not all(s is not None for s in seeds):
        raise ValueError("seed_ssm, seed_k, seed_v and seed_coef must be given together")
    if tuple(phi.shape) != (batch, nheads, seqlen, n_angles):
        raise ValueError(
            f"phi must be (B, H, L, Nr) = {(batch, nheads, seqlen, n_angles)}, got {tuple(phi.shape)}")
    if z is not None and tuple(z.shape) != tuple(v.shape):
        raise ValueError(f"z shape {tuple(z.shape)} must match v {tuple(v.shape)}")
    dev = _device_of(q, k, v, adt, gamma, scale, q_bias, k_bias, d_skip, z, *seeds,
                     *(phi if isinstance(phi, PhiStrips) else (phi,)))
    mt = pol.matmul
    dcode = _lib.dtype_code(mt)
    if not _lib.supported(0, dcode, chunk, state_dim, headdim):
        raise ValueError(
            f"no forward kernel for policy={pol.name} chunk={chunk} d_state={state_dim} "
            f"headdim={headdim} (see layout.SUPPORTED_CHUNKS and the library's config table)")

    qc, kc = _mt(q, mt), _mt(k, mt)
    vc, zc = _bhlp_operand(v, mt), _bhlp_operand(z, mt)
    adt_c, gam_c, scl_c = _f32c(adt), _f32c(gamma), _f32c(scale)
    qb_c, kb_c, d_c = _f32c(q_bias), _f32c(k_bias), _f32c(d_skip)
    s_ssm, s_k, s_v, s_c = (_f32c(s) for s in seeds)

    y_dtype = v.dtype if v.dtype in (torch.bfloat16, torch.float32) else mt
    y = _empty_like_layout(vc, mt)
    f32 = dict(device=dev, dtype=torch.float32)
    final_ssm = empty(batch, nheads, headdim, state_dim, **f32)
    final_k = empty(batch, nheads, state_dim, **f32)
    final_v = empty(batch, nheads, headdim, **f32)
    if save_residuals:
        ybar = empty(batch, nheads, seqlen, headdim, device=dev, dtype=mt)
        cstates = empty(batch, nheads, nc, state_dim, headdim, device=dev, dtype=mt)
    else:
        ybar = cstates = None

    a = _lib.FwdArgs()
    a.struct_size = ctypes.sizeof(_lib.FwdArgs)
    a.batch, a.seqlen, a.nheads, a.headdim = batch, seqlen, nheads, headdim
    a.state_dim, a.n_angles, a.chunk = state_dim, n_angles, chunk
    a.dtype = dcode
    a.has_d, a.has_z, a.has_seed = int(d_c is not None), int(zc is not None), int(has_seed)
    a.save_residuals = int(save_residuals)
    a.q, a.k = qc.data_ptr(), kc.data_ptr()
    a.v, a.z = _lib.bhlp(vc), _lib.bhlp(zc)
    a.adt, a.gamma, a.scale = (t.data_ptr() for t in (adt_c, gam_c, scl_c))
    keep = _phi_fields(a, phi, dev)  # noqa: F841  (alive until the launch)
    a.q_bias, a.k_bias, a.d_skip = qb_c.data_ptr(), kb_c.data_ptr(), _lib.ptr(d_c)
    a.seed_ssm, a.seed_k, a.seed_v, a.seed_coef = (_lib.ptr(s) for s in (s_ssm, s_k, s_v, s_c))
    a.y = _lib.bhlp(y)
    a.ybar, a.chunk_states = _lib.ptr(ybar), _lib.ptr(cstates)
    a.final_ssm, a.final_k, a.final_v = final_ssm.data_ptr(), final_k.data_ptr(), final_v.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.load().m3s_fwd(ctypes.byref(a), _lib.stream_handle(dev)), "m3s_fwd")

    if y.dtype != y_dtype:
        y = y.to(y_dtype)
    outs = (y, final_ssm, final_k, final_v)
    if save_residuals:
        return outs + (ForwardResiduals(ybar=ybar, chunk_states=cstates.transpose(-1, -2)),)
    return outs


class RawAngles(NamedTuple):
    """The rotary angles' per-token work that `siso_forward_raw` reads, written by
    `bcnorm_forward` (``theta=``) in the BCNorm launch for scans at ``chunk``: ``table`` =
    ``tanh(angles) pi`` ``(B, L, Nr)`` (shared by the heads); with ``theta[t, h] = table[t]
    dt[t, h]`` summed over each 16-token strip, ``prefix`` ``(B, H, L / 16, Nr)`` the sum of
    the strips before each one within its chunk and ``chunk_totals`` ``(B, H, L / chunk,
    Nr)`` each chunk's sum."""

    table: Tensor
    prefix: Tensor
    chunk_totals: Tensor
    chunk: int


def raw_forward_ok(pol: LY.DtypePolicy | str, chunk: int, state_dim: int, headdim: int,
                   n_angles: int, seqlen: int, nheads: int = 1) -> bool:
    """Whether `siso_forward_raw` runs this shape: a raw-mode kernel of the head's own
    width at the chunk's tile, ``n_angles % 4 == 0``, ``seqlen % 16 == 0``, and the BCNorm
    call's angle kernel's per-chunk tables within its 64 KiB of LDS."""
    pol = LY.policy(pol)
    if n_angles <= 0 or n_angles % 4 or seqlen % 16:
        return False
    try:
        tile = LY.kernel_chunk(pol.name, chunk, state_dim, headdim)
    except ValueError:
        return False
    if seqlen % tile or (tile * (nheads + n_angles) + tile // 16 * nheads * n_angles) * 4 > 65536:
        return False
    return _lib.raw_supported(_lib.dtype_code(pol.matmul), tile, state_dim, headdim, n_angles)


def siso_forward_raw(
    q: Tensor, k: Tensor, v: Tensor, dt_raw: Tensor, a_raw: Tensor, trap_raw: Tensor,
    angles: RawAngles, dt_bias: Tensor, q_bias: Tensor, k_bias: Tensor,
    d_skip: Optional[Tensor] = None, z: Optional[Tensor] = None,
    phi_init: Optional[Tensor] = None, a_floor: float = 1e-4, chunk: int = 128,
    dtype_policy: LY.DtypePolicy | str = LY.BF16,
):
    """`reference.preprocess` (``reference.py:160-199``) and ``kernel_fwd.siso_forward``
    (``kernel_fwd.py:204-248``) in one scan launch, without residuals (inference): the
    kernel reads the projection's raw ``dt_raw``, ``a_raw``, ``trap_raw`` ``(B, L, H)``
    slices in place and computes dt, a, lambda, adt, gamma and the trapezoid's t+1 scale
    shift as it loads each chunk, and carries the cumulative angle phi across its strips
    and chunks from ``angles`` (`RawAngles`, from `bcnorm_forward`), starting at
    ``phi_init`` (zero when None). Returns ``(y, final_ssm, final_k, final_v, phi_final)``;
    ``y`` has ``v``'s layout. The three raw slices must be views of one projection
    buffer (shared strides, a and trap after dt in each row)."""
    pol = LY.policy(dtype_policy)
    LY.validate_chunk(chunk)
    batch, seqlen, state_dim = q.shape
    nheads, headdim = v.shape[1], v.shape[3]
    n_angles = angles.table.shape[-1]
    LY.num_chunks(seqlen, chunk)
    if not raw_forward_ok(pol, chunk, state_dim, headdim, n_angles, seqlen, nheads):
        raise ValueError(
            f"no raw-mode forward for policy={pol.name} chunk={chunk} d_state={state_dim} "
            f"headdim={headdim} n_angles={n_angles} seqlen={seqlen}")
    chunk = _tile(pol, chunk, state_dim, headdim, "forward")
    if q.shape != k.shape:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} must match")
    if tuple(v.shape) != (batch, nheads, seqlen, headdim):
        raise ValueError(f"unexpected v shape {tuple(v.shape)}")
    for name, t in (("dt_raw", dt_raw), ("a_raw", a_raw), ("trap_raw", trap_raw)):
        if tuple(t.shape) != (batch, seqlen, nheads):
            raise ValueError(f"{name} must be (B, L, H) = {(batch, seqlen, nheads)}, got {tuple(t.shape)}")
    if (tuple(angles.table.shape) != (batch, seqlen, n_angles)
            or tuple(angles.prefix.shape) != (batch, nheads, seqlen // 16, n_angles)
            or tuple(angles.chunk_totals.shape) != (batch, nheads, seqlen // chunk, n_angles)
            or angles.chunk != chunk):
        raise ValueError(
            f"angles must come from bcnorm_forward for this shape at the scan's chunk {chunk}: "
            "table (B, L, Nr), prefix (B, H, L / 16, Nr), chunk_totals (B, H, L / chunk, Nr)")
    if z is not None and tuple(z.shape) != tuple(v.shape):
        raise ValueError(f"z shape {tuple(z.shape)} must match v {tuple(v.shape)}")
    mt = pol.matmul
    dev = _device_of(q, k, v, dt_raw, a_raw, trap_raw, angles.table, angles.prefix, angles.chunk_totals, dt_bias,
                     q_bias, k_bias, d_skip, z, phi_init)
    if dt_raw.dtype != mt or a_raw.dtype != mt or trap_raw.dtype != mt:
        raise ValueError(f"the raw slices must be in the policy's operand dtype {mt}")
    qc, kc = _mt(q, mt), _mt(k, mt)
    vc, zc = _bhlp_operand(v, mt), _bhlp_operand(z, mt)
    qb_c, kb_c, d_c = _f32c(q_bias), _f32c(k_bias), _f32c(d_skip)
    tab, pre, ctot, bias = (_f32c(t) for t in (angles.table, angles.prefix, angles.chunk_totals,
                                                dt_bias))
    pinit = _f32c(phi_init)
    y = _empty_like_layout(vc, mt)
    f32 = dict(device=dev, dtype=torch.float32)
    final_ssm = empty(batch, nheads, headdim, state_dim, **f32)
    final_k = empty(batch, nheads, state_dim, **f32)
    final_v = empty(batch, nheads, headdim, **f32)
    phi_final = empty(batch, nheads, n_angles, **f32)

    a = _lib.FwdArgs()
    a.struct_size = ctypes.sizeof(_lib.FwdArgs)
    a.batch, a.seqlen, a.nheads, a.headdim = batch, seqlen, nheads, headdim
    a.state_dim, a.n_angles, a.chunk = state_dim, n_angles, chunk
    a.dtype = _lib.dtype_code(mt)
    a.has_d, a.has_z, a.has_seed = int(d_c is not None), int(zc is not None), 0
    a.save_residuals = 0
    a.q, a.k = qc.data_ptr(), kc.data_ptr()
    a.v, a.z = _lib.bhlp(vc), _lib.bhlp(zc)
    a.theta_table = tab.data_ptr()
    a.q_bias, a.k_bias, a.d_skip = qb_c.data_ptr(), kb_c.data_ptr(), _lib.ptr(d_c)
    a.y = _lib.bhlp(y)
    a.final_ssm, a.final_k, a.final_v = final_ssm.data_ptr(), final_k.data_ptr(), final_v.data_ptr()
    a.raw, a.a_floor = 1, float(a_floor)
    a.dt_raw, a.a_raw, a.trap_raw = _lib.blx(dt_raw), _lib.blx(a_raw), _lib.blx(trap_raw)
    a.dt_bias, a.theta_prefix, a.theta_chunk_totals = bias.data_ptr(), pre.data_ptr(), ctot.data_ptr()
    a.phi_init, a.phi_final = _lib.ptr(pinit), phi_final.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.load().m3s_fwd(ctypes.byref(a), _lib.stream_handle(dev)), "m3s_fwd")
    return y, final_ssm, final_k, final_v, phi_final


# ======================================================================================
# Decode (kernel_decode.py:252-573)
# ======================================================================================


def _state_buf(t: Tensor, shape, dev) -> Tensor:
    """The decode kernel updates the carried state in place; reuse the caller's buffer
    when it already is f32, contiguous and on the device (the donation of
    ``kernel_decode.py:350-352``), else work on a converted copy."""
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"state tensor has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.dtype == torch.float32 and t.is_contiguous() and t.device == dev:
        return t
    return t.to(device=dev, dtype=torch.float32).contiguous()


def siso_decode(q: Tensor, k: Tensor, v: Tensor, adt: Tensor, dt: Tensor, lam: Tensor,
                angles: Tensor, q_bias: Tensor, k_bias: Tensor, state,
                d_skip: Optional[Tensor] = None, z: Optional[Tensor] = None,
                dtype_policy: LY.DtypePolicy | str = LY.BF16, interpret: Any = False):
    """One decode step (``kernel_decode.py:252-360``).

    q, k ``(B, N)``; v, z ``(B, H, P)``; adt, dt, lam ``(B, H)``; angles ``(B, Nr)`` raw
    (pre-tanh). Returns ``(y (B, H, P), next_state)``. The state's four buffers are
    updated **in place** and returned (the reference donates them): the input state is
    consumed.
    """
    from .scan_prep import SISOState

    pol = LY.policy(dtype_policy)
    batch, state_dim = q.shape
    nheads, headdim = v.shape[1], v.shape[2]
    n_angles = angles.shape[-1]
    if tuple(k.shape) != (batch, state_dim):
        raise ValueError(f"k shape {tuple(k.shape)} must match q {tuple(q.shape)}")
    for name, t in (("adt", adt), ("dt", dt), ("lam", lam)):
        if tuple(t.shape) != (batch, nheads):
            raise ValueError(f"{name} must be (B, H) = {(batch, nheads)}, got {tuple(t.shape)}")
    if z is not None and tuple(z.shape) != tuple(v.shape):
        raise ValueError("z must match v")
    dev = _device_of(q, k, v, adt, dt, lam, angles, q_bias, k_bias, d_skip, z, *state)
    mt = pol.matmul
    dcode = _lib.dtype_code(mt)
    width = LY.decode_headdim(pol.name, state_dim, headdim)
    if width is None:
        raise ValueError(f"no decode kernel for policy={pol.name} d_state={state_dim} headdim={headdim}")
    if width != headdim:   # sub-heads (see _split_cols): ssm and v update in place as views
        r = headdim // width
        ssm = _state_buf(state.ssm, (batch, nheads, headdim, state_dim), dev)
        vst = _state_buf(state.v, (batch, nheads, headdim), dev)
        kst = _state_buf(state.k, (batch, nheads, state_dim), dev)
        phist = _state_buf(state.phi, (batch, nheads, n_angles), dev)
        sub = SISOState(ssm=ssm.view(batch, nheads * r, width, state_dim), k=_rep(kst, r),
                        v=vst.view(batch, nheads * r, width), phi=_rep(phist, r))
        cut = lambda t: None if t is None else t.reshape(batch, nheads * r, width)  # noqa: E731
        y, st = siso_decode(q, k, cut(v), _rep(adt, r), _rep(dt, r), _rep(lam, r), angles,
                            _rep(q_bias, r, 0), _rep(k_bias, r, 0), sub,
                            d_skip=_rep(d_skip, r, 0), z=cut(z), dtype_policy=pol)
        kst.copy_(st.k[:, ::r])
        phist.copy_(st.phi[:, ::r])
        return y.reshape(batch, nheads, headdim), SISOState(ssm=ssm, k=kst, v=vst, phi=phist)
    ssm = _state_buf(state.ssm, (batch, nheads, headdim, state_dim), dev)
    kst = _state_buf(state.k, (batch, nheads, state_dim), dev)
    vst = _state_buf(state.v, (batch, nheads, headdim), dev)
    phist = _state_buf(state.phi, (batch, nheads, n_angles), dev)
    qc, kc, vc, zc = _mt(q, mt), _mt(k, mt), _mt(v, mt), _mt(z, mt)
    adt_c, dt_c, lam_c, ang_c = _f32c(adt), _f32c(dt), _f32c(lam), _f32c(angles)
    qb_c, kb_c, d_c = _f32c(q_bias), _f32c(k_bias), _f32c(d_skip)
    y = empty(batch, nheads, headdim, device=dev, dtype=mt)

    a = _lib.DecodeArgs()
    a.struct_size = ctypes.sizeof(_lib.DecodeArgs)
    a.batch, a.nheads, a.headdim, a.state_dim, a.n_angles = batch, nheads, headdim, state_dim, n_angles
    a.dtype = dcode
    a.has_d, a.has_z = int(d_c is not None), int(zc is not None)
    a.q, a.k, a.v, a.z = qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), _lib.ptr(zc)
    a.adt, a.dt, a.lam, a.angles = adt_c.data_ptr(), dt_c.data_ptr(), lam_c.data_ptr(), ang_c.data_ptr()
    a.q_bias, a.k_bias, a.d_skip = qb_c.data_ptr(), kb_c.data_ptr(), _lib.ptr(d_c)
    a.ssm, a.k_state, a.v_state, a.phi_state = (t.data_ptr() for t in (ssm, kst, vst, phist))
    a.y = y.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.load().m3s_decode(ctypes.byref(a), _lib.stream_handle(dev)), "m3s_decode")
    y_dtype = v.dtype if v.dtype in (torch.bfloat16, torch.float32) else mt
    if y.dtype != y_dtype:
        y = y.to(y_dtype)
    return y, SISOState(ssm=ssm, k=kst, v=vst, phi=phist)


def decode_layer_step(proj: Tensor, state, *, nheads: int, headdim: int, state_dim: int,
                      n_angles: int, b_norm_weight: Tensor, c_norm_weight: Tensor,
                      dt_bias: Tensor, q_bias: Tensor, k_bias: Tensor,
                      d_skip: Optional[Tensor], a_floor: float, norm_eps: float):
    """The layer's decode step from its in_proj output (``model.py:266-289`` without the
    block norm): ``proj`` is ``(B, >= d_in_proj)`` with a unit last stride, in bf16 or
    f32; BCNorm, dt / lambda / a, and the state update + readout of `siso_decode` run in
    one ``m3s_decode_layer`` launch. ``q_bias`` / ``k_bias`` are the layer's c_bias /
    b_bias. Returns ``(y (B, H, P), next_state)``; the state is updated in place."""
    from .scan_prep import SISOState

    batch = proj.shape[0]
    dev = _device_of(proj, b_norm_weight, c_norm_weight, dt_bias, q_bias, k_bias, d_skip, *state)
    mt = proj.dtype
    dcode = _lib.dtype_code(mt)
    if proj.dim() != 2 or proj.stride(1) != 1:
        raise ValueError("proj must be (B, d_in_proj) with a unit last stride")
    if not _lib.supported(2, dcode, 0, state_dim, headdim):
        raise ValueError(f"no decode kernel for {mt} d_state={state_dim} headdim={headdim}")
    ssm = _state_buf(state.ssm, (batch, nheads, headdim, state_dim), dev)
    kst = _state_buf(state.k, (batch, nheads, state_dim), dev)
    vst = _state_buf(state.v, (batch, nheads, headdim), dev)
    phist = _state_buf(state.phi, (batch, nheads, n_angles), dev)
    wb, wc, bias = _f32c(b_norm_weight), _f32c(c_norm_weight), _f32c(dt_bias)
    qb_c, kb_c, d_c = _f32c(q_bias), _f32c(k_bias), _f32c(d_skip)
    y = empty(batch, nheads, headdim, device=dev, dtype=mt)
    a = _lib.DecodeLayerArgs()
    a.struct_size = ctypes.sizeof(_lib.DecodeLayerArgs)
    a.batch, a.nheads, a.headdim, a.state_dim, a.n_angles = batch, nheads, headdim, state_dim, n_angles
    a.dtype, a.a_floor, a.norm_eps = dcode, float(a_floor), float(norm_eps)
    a.proj, a.proj_stride = proj.data_ptr(), proj.stride(0)
    a.b_norm_weight, a.c_norm_weight, a.dt_bias = wb.data_ptr(), wc.data_ptr(), bias.data_ptr()
    a.q_bias, a.k_bias, a.d_skip = qb_c.data_ptr(), kb_c.data_ptr(), _lib.ptr(d_c)
    a.ssm, a.k_state, a.v_state, a.phi_state = (t.data_ptr() for t in (ssm, kst, vst, phist))
    a.y = y.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.load().m3s_decode_layer(ctypes.byref(a), _lib.stream_handle(dev)),
                   "m3s_decode_layer")
    return y, SISOState(ssm=ssm, k=kst, v=vst, phi=phist)


def siso_decode_folded(*args, **kw):
    """``kernel_decode.py:363-464``. Same kernel as `siso_decode`: on MI355X one
    workgroup per (b, h) state serves both of the reference's grids."""
    return siso_decode(*args, **kw)


def decode_step(*args, folded: bool = True, **kw):
    """``kernel_decode.py:467-471``."""
    return siso_decode(*args, **kw)


def decode_loop(q, k, v, adt, dt, lam, angles, q_bias, k_bias, state, d_skip=None, z=None,
                dtype_policy: LY.DtypePolicy | str = LY.BF16, interpret: Any = False,
                folded: bool = False):
    """``kernel_decode.py:536-573``: ``L`` decode steps in a Python loop; inputs have a
    time axis (q, k ``(B, L, N)``; v, z ``(B, H, L, P)``; adt/dt/lam ``(B, H, L)``;
    angles ``(B, L, Nr)``). Returns ``(y (B, H, L, P), state)``."""
    outs = []
    for t in range(q.shape[1]):
        y, state = decode_step(
            q[:, t], k[:, t], v[:, :, t], adt[:, :, t], dt[:, :, t], lam[:, :, t], angles[:, t],
            q_bias, k_bias, state, d_skip=d_skip, z=None if z is None else z[:, :, t],
            dtype_policy=dtype_policy)
        outs.append(y)
    return torch.stack(outs, dim=2), state


def decode_scan(q, k, v, adt, dt, lam, angles, q_bias, k_bias, state, d_skip=None, z=None,
                dtype_policy: LY.DtypePolicy | str = LY.BF16, interpret: Any = False,
                folded: bool = True):
    """``kernel_decode.py:474-533``: a known-length run of ``L`` decode steps (the
    reference's ``lax.scan`` of ``decode_step``) as ONE ``m3s_decode_scan`` launch: each
    (b, h) state is read once, stepped ``L`` times on chip and written once. Inputs as
    `decode_loop` (q, k ``(B, L, N)``; v, z ``(B, H, L, P)``; adt/dt/lam ``(B, H, L)``;
    angles ``(B, L, Nr)``); every step is `siso_decode`'s arithmetic, so the results are
    `decode_loop`'s. Returns ``(y (B, H, L, P), state)``; the state is updated in place."""
    from .scan_prep import SISOState

    pol = LY.policy(dtype_policy)
    batch, steps, state_dim = q.shape
    nheads, headdim = v.shape[1], v.shape[3]
    n_angles = angles.shape[-1]
    if tuple(k.shape) != (batch, steps, state_dim):
        raise ValueError(f"k shape {tuple(k.shape)} must match q {tuple(q.shape)}")
    if tuple(v.shape[:3]) != (batch, nheads, steps):
        raise ValueError(f"v must be (B, H, L, P) with B={batch}, L={steps}, got {tuple(v.shape)}")
    for name, t in (("adt", adt), ("dt", dt), ("lam", lam)):
        if tuple(t.shape) != (batch, nheads, steps):
            raise ValueError(f"{name} must be (B, H, L) = {(batch, nheads, steps)}, "
                             f"got {tuple(t.shape)}")
    if tuple(angles.shape[:2]) != (batch, steps):
        raise ValueError(f"angles must be (B, L, Nr), got {tuple(angles.shape)}")
    if z is not None and tuple(z.shape) != tuple(v.shape):
        raise ValueError("z must match v")
    dev = _device_of(q, k, v, adt, dt, lam, angles, q_bias, k_bias, d_skip, z, *state)
    mt = pol.matmul
    width = LY.decode_headdim(pol.name, state_dim, headdim)
    if width is None:
        raise ValueError(f"no decode kernel for policy={pol.name} d_state={state_dim} headdim={headdim}")
    ssm = _state_buf(state.ssm, (batch, nheads, headdim, state_dim), dev)
    kst = _state_buf(state.k, (batch, nheads, state_dim), dev)
    vst = _state_buf(state.v, (batch, nheads, headdim), dev)
    phist = _state_buf(state.phi, (batch, nheads, n_angles), dev)
    if steps == 0:   # a scan of length 0: no output rows, the state as it was
        y_dtype = v.dtype if v.dtype in (torch.bfloat16, torch.float32) else mt
        return (torch.empty(batch, nheads, 0, headdim, device=dev, dtype=y_dtype),
                SISOState(ssm=ssm, k=kst, v=vst, phi=phist))
    r = headdim // width
    if r > 1:   # sub-heads of `width` columns, as siso_decode
        ssm_k, vst_k = ssm.view(batch, nheads * r, width, state_dim), vst.view(batch, nheads * r, width)
        kst_k, phist_k = _rep(kst, r), _rep(phist, r)
        v, z = _split_cols(v, r), _split_cols(z, r)
        adt, dt, lam = _rep(adt, r), _rep(dt, r), _rep(lam, r)
        q_bias, k_bias, d_skip = _rep(q_bias, r, 0), _rep(k_bias, r, 0), _rep(d_skip, r, 0)
    else:
        ssm_k, vst_k, kst_k, phist_k = ssm, vst, kst, phist
    qc, kc, vc, zc = _mt(q, mt), _mt(k, mt), _mt(v, mt), _mt(z, mt)
    adt_c, dt_c, lam_c, ang_c = _f32c(adt), _f32c(dt), _f32c(lam), _f32c(angles)
    qb_c, kb_c, d_c = _f32c(q_bias), _f32c(k_bias), _f32c(d_skip)
    y = empty(batch, nheads * r, steps, width, device=dev, dtype=mt)

    a = _lib.DecodeScanArgs()
    a.struct_size = ctypes.sizeof(_lib.DecodeScanArgs)
    a.batch, a.steps, a.nheads, a.headdim = batch, steps, nheads * r, width
    a.state_dim, a.n_angles = state_dim, n_angles
    a.dtype = _lib.dtype_code(mt)
    a.has_d, a.has_z = int(d_c is not None), int(zc is not None)
    a.q, a.k, a.v, a.z = qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), _lib.ptr(zc)
    a.adt, a.dt, a.lam, a.angles = adt_c.data_ptr(), dt_c.data_ptr(), lam_c.data_ptr(), ang_c.data_ptr()
    a.q_bias, a.k_bias, a.d_skip = qb_c.data_ptr(), kb_c.data_ptr(), _lib.ptr(d_c)
    a.ssm, a.k_state, a.v_state, a.phi_state = (t.data_ptr() for t in (ssm_k, kst_k, vst_k, phist_k))
    a.y = y.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.load().m3s_decode_scan(ctypes.byref(a), _lib.stream_handle(dev)),
                   "m3s_decode_scan")
    if r > 1:
        kst.copy_(kst_k[:, ::r])
        phist.copy_(phist_k[:, ::r])
        y = _merge_cols(y, r)
    y_dtype = v.dtype if v.dtype in (torch.bfloat16, torch.float32) else mt
    if y.dtype != y_dtype:
        y = y.to(y_dtype)
    return y, SISOState(ssm=ssm, k=kst, v=vst, phi=phist)


# ======================================================================================
# Backward (kernel_bwd.py:358-669)
# ======================================================================================


class KernelGrads(NamedTuple):
    """``kernel_bwd.py:63-100``. ``dq``/``dk`` are summed over heads (``(B, L, N)``,
    f32); ``dv``/``dz`` come back in the dtype policy's operand type (f32 or bf16);
    ``dq_bias``/``dk_bias`` are already reduced over batch and time."""

    dq: Tensor
    dk: Tensor
    dv: Tensor
    dadt: Tensor
    dqk_diag: Tensor
    dscale: Tensor
    dphi: Tensor
    dz: Optional[Tensor]
    uw: Tensor
    dq_bias: Tensor
    dk_bias: Tensor
    k_final: Tensor
    dseed_ssm: Tensor


def _out_buffer(out: Optional[Tensor], like: Tensor, mt: torch.dtype, name: str) -> Tensor:
    """``out`` checked as a (B, H, L, P) destination the kernel writes in place, or a new
    tensor laid out like ``like``."""
    if out is None:
        return _empty_like_layout(like, mt)
    vec = 16 // out.element_size()
    if (tuple(out.shape) != tuple(like.shape) or out.dtype != mt or out.device != like.device
            or out.stride(3) != 1 or out.data_ptr() % 16
            or any(out.stride(i) % vec for i in range(3))):
        raise ValueError(f"{name} must be a {tuple(like.shape)} {mt} tensor on {like.device} "
                         "with 16-byte aligned rows and a unit last stride")
    return out


def _nmajor_states(chunk_states: Tensor, mt: torch.dtype) -> Tensor:
    """The kernel reads chunk states N-major, ``(B, H, nc, N, P)`` contiguous. The
    forward's residual is a transposed view of exactly that; anything else is copied."""
    t = chunk_states.transpose(-1, -2)
    if t.dtype != mt:
        t = t.to(mt)
    return t if t.is_contiguous() else t.contiguous()


def siso_backward_kernel(
    dy: Tensor, ybar: Tensor, z: Optional[Tensor], q: Tensor, k: Tensor, v: Tensor,
    adt: Tensor, gamma: Tensor, scale: Tensor, phi: Tensor, q_bias: Tensor, k_bias: Tensor,
    chunk_states: Tensor, d_skip: Optional[Tensor] = None,
    dfinal_ssm: Optional[Tensor] = None, chunk: int = 128,
    dtype_policy: LY.DtypePolicy | str = LY.BF16, interpret: Any = False,
    device_kind: str | None = None, *, dfinal_v: Optional[Tensor] = None,
    dv_out: Optional[Tensor] = None, dz_out: Optional[Tensor] = None,
) -> KernelGrads:
    """Reverse chunk scan (``kernel_bwd.py:358-395``). ``dfinal_v`` (keyword-only) is
    added to ``dv``'s last row inside the kernel, before the cast to the operand type
    (the reference does it in its epilogue, ``kernel_bwd.py:632-637``). ``dv_out`` /
    ``dz_out`` (keyword-only) are ``(B, H, L, P)`` buffers of the operand type, any
    strides with a unit P stride (e.g. slices of the projection's gradient), that
    receive ``dv`` / ``dz`` in place of fresh tensors."""
    pol = LY.policy(dtype_policy)
    LY.validate_chunk(chunk)
    batch, seqlen, state_dim = q.shape
    nheads, headdim = v.shape[1], v.shape[3]
    n_angles = phi.shape[-1]
    LY.num_chunks(seqlen, chunk)
    width = _width(pol, chunk, state_dim, headdim, "backward")
    if width != headdim and tuple(v.shape) == (batch, nheads, seqlen, headdim):
        return _backward_split(dy, ybar, z, q, k, v, adt, gamma, scale, phi, q_bias, k_bias,
                               chunk_states, d_skip, dfinal_ssm, chunk, pol, dfinal_v, dv_out,
                               dz_out, headdim // width)
    chunk = _tile(pol, chunk, state_dim, headdim, "backward")
    nc = seqlen // chunk
    if tuple(dy.shape) != tuple(v.shape) or tuple(ybar.shape) != tuple(v.shape):
        raise ValueError("dy and ybar must be (B, H, L, P) like v")
    if tuple(chunk_states.shape) != (batch, nheads, nc, headdim, state_dim):
        raise ValueError(f"chunk_states must be (B, H, nc, P, N) = "
                         f"{(batch, nheads, nc, headdim, state_dim)}, got {tuple(chunk_states.shape)}")
    dev = _device_of(dy, ybar, z, q, k, v, adt, gamma, scale, q_bias, k_bias,
                     *(phi if isinstance(phi, PhiStrips) else (phi,)),
                     chunk_states, d_skip, dfinal_ssm, dfinal_v)
    mt = pol.matmul
    dcode = _lib.dtype_code(mt)
    if not _lib.supported(1, dcode, chunk, state_dim, headdim):
        raise ValueError(
            f"no backward kernel for policy={pol.name} chunk={chunk} d_state={state_dim} "
            f"headdim={headdim}")
    dyc, zc, vc = _bhlp_operand(dy, mt), _bhlp_operand(z, mt), _bhlp_operand(v, mt)
    qc, kc = _mt(q, mt), _mt(k, mt)
    ybc = _mt(ybar, mt)
    adt_c, gam_c, scl_c = _f32c(adt), _f32c(gamma), _f32c(scale)
    qb_c, kb_c, d_c = _f32c(q_bias), _f32c(k_bias), _f32c(d_skip)
    cs = _nmajor_states(chunk_states, mt)
    dfs, dfv = _f32c(dfinal_ssm), _f32c(dfinal_v)

    f32 = dict(device=dev, dtype=torch.float32)
    dq = empty(batch, seqlen, state_dim, **f32)
    dk = empty(batch, seqlen, state_dim, **f32)
    dv = _out_buffer(dv_out, vc, mt, "dv_out")
    dz = _out_buffer(dz_out, zc, mt, "dz_out") if zc is not None else None
    dadt = empty(batch, nheads, seqlen, **f32)
    dqk = empty(batch, nheads, seqlen, **f32)
    dscale = empty(batch, nheads, seqlen, **f32)
    uw = empty(batch, nheads, seqlen, **f32)
    dphi = empty(batch, nheads, seqlen, n_angles, **f32)
    dqb = empty(batch, nheads, state_dim, **f32)
    dkb = empty(batch, nheads, state_dim, **f32)
    kfin = empty(batch, nheads, state_dim, **f32)
    dseed = empty(batch, nheads, headdim, state_dim, **f32)
    ws_bytes = _lib.load().m3s_bwd_workspace_bytes(dcode, batch, seqlen, nheads, state_dim)
    workspace = empty(ws_bytes, device=dev, dtype=torch.uint8)

    a = _lib.BwdArgs()
    a.struct_size = ctypes.sizeof(_lib.BwdArgs)
    a.batch, a.seqlen, a.nheads, a.headdim = batch, seqlen, nheads, headdim
    a.state_dim, a.n_angles, a.chunk = state_dim, n_angles, chunk
    a.dtype = dcode
    a.has_d, a.has_z = int(d_c is not None), int(zc is not None)
    a.dy, a.ybar, a.z = _lib.bhlp(dyc), ybc.data_ptr(), _lib.bhlp(zc)
    a.q, a.k, a.v = qc.data_ptr(), kc.data_ptr(), _lib.bhlp(vc)
    a.adt, a.gamma, a.scale = (t.data_ptr() for t in (adt_c, gam_c, scl_c))
    keep = _phi_fields(a, phi, dev)  # noqa: F841  (alive until the launch)
    a.q_bias, a.k_bias, a.d_skip = qb_c.data_ptr(), kb_c.data_ptr(), _lib.ptr(d_c)
    a.chunk_states, a.dfinal_ssm, a.dfinal_v = cs.data_ptr(), _lib.ptr(dfs), _lib.ptr(dfv)
    a.dq, a.dk, a.dv, a.dz = dq.data_ptr(), dk.data_ptr(), _lib.bhlp(dv), _lib.bhlp(dz)
    a.dadt, a.dqk_diag, a.dscale, a.uw = (t.data_ptr() for t in (dadt, dqk, dscale, uw))
    a.dphi, a.dq_bias, a.dk_bias = dphi.data_ptr(), dqb.data_ptr(), dkb.data_ptr()
    a.k_final, a.dseed_ssm = kfin.data_ptr(), dseed.data_ptr()
    a.workspace = workspace.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.load().m3s_bwd(ctypes.byref(a), _lib.stream_handle(dev)), "m3s_bwd")
    return KernelGrads(dq=dq, dk=dk, dv=dv, dadt=dadt, dqk_diag=dqk, dscale=dscale, dphi=dphi,
                       dz=dz, uw=uw, dq_bias=dqb.sum(0), dk_bias=dkb.sum(0), k_final=kfin,
                       dseed_ssm=dseed)


def _backward_split(dy, ybar, z, q, k, v, adt, gamma, scale, phi, q_bias, k_bias, chunk_states,
                    d_skip, dfinal_ssm, chunk, pol, dfinal_v, dv_out, dz_out, r):
    """`siso_backward_kernel` for heads run as r sub-heads (see `_split_cols`): the
    sub-heads' gradients of the inputs they share are summed per head."""
    batch, nheads, seqlen, headdim = v.shape
    state_dim = q.shape[-1]
    width = headdim // r
    cs = chunk_states.unflatten(3, (r, width)).permute(0, 1, 3, 2, 4, 5).reshape(
        batch, nheads * r, chunk_states.shape[2], width, state_dim)

    def in_place(out):   # a sub-head view of the caller's buffer, or None (reshape copied)
        if out is None:
            return None
        sv = _split_cols(out, r)
        same = sv.untyped_storage().data_ptr() == out.untyped_storage().data_ptr()
        return sv if same else None

    dv_v, dz_v = in_place(dv_out), in_place(dz_out)
    kg = siso_backward_kernel(
        _split_cols(dy, r), _split_cols(ybar, r), _split_cols(z, r), q, k, _split_cols(v, r),
        _rep(adt, r), _rep(gamma, r), _rep(scale, r), _rep_phi(phi, r), _rep(q_bias, r, 0),
        _rep(k_bias, r, 0), cs, d_skip=_rep(d_skip, r, 0),
        dfinal_ssm=None if dfinal_ssm is None else dfinal_ssm.reshape(batch, nheads * r, width, state_dim),
        chunk=chunk, dtype_policy=pol,
        dfinal_v=None if dfinal_v is None else dfinal_v.reshape(batch, nheads * r, width),
        dv_out=dv_v, dz_out=dz_v)

    def merged(g, out, out_v):
        if g is None:
            return None
        if out_v is not None:
            return out
        m = _merge_cols(g, r)
        if out is not None:
            out.copy_(m)
            return out
        return m

    return KernelGrads(
        dq=kg.dq, dk=kg.dk, dv=merged(kg.dv, dv_out, dv_v), dadt=_head_sum(kg.dadt, r),
        dqk_diag=_head_sum(kg.dqk_diag, r), dscale=_head_sum(kg.dscale, r),
        dphi=_head_sum(kg.dphi, r), dz=merged(kg.dz, dz_out, dz_v),
        uw=kg.uw[:, ::r].contiguous(), dq_bias=_head_sum(kg.dq_bias, r, 0),
        dk_bias=_head_sum(kg.dk_bias, r, 0), k_final=kg.k_final[:, ::r].contiguous(),
        dseed_ssm=kg.dseed_ssm.reshape(batch, nheads, headdim, state_dim))


class SISOGrads(NamedTuple):
    """``kernel_bwd.py:514-531``: gradients w.r.t. everything `siso_forward` takes."""

    dq: Tensor
    dk: Tensor
    dv: Tensor
    dadt: Tensor
    dgamma: Tensor
    dscale: Tensor
    dphi: Tensor
    dq_bias: Tensor
    dk_bias: Tensor
    dd_skip: Optional[Tensor]
    dz: Optional[Tensor]
    dseed_ssm: Optional[Tensor]
    dseed_k: Optional[Tensor]
    dseed_v: Optional[Tensor]
    dseed_coef: Optional[Tensor]


def siso_backward(
    dy: Tensor, q: Tensor, k: Tensor, v: Tensor, adt: Tensor, gamma: Tensor, scale: Tensor,
    phi: Tensor, q_bias: Tensor, k_bias: Tensor, ybar: Tensor, chunk_states: Tensor,
    d_skip: Optional[Tensor] = None, z: Optional[Tensor] = None,
    seed_ssm: Optional[Tensor] = None, seed_k: Optional[Tensor] = None,
    seed_v: Optional[Tensor] = None, seed_coef: Optional[Tensor] = None,
    dfinal_ssm: Optional[Tensor] = None, dfinal_k: Optional[Tensor] = None,
    dfinal_v: Optional[Tensor] = None, chunk: int = 128,
    dtype_policy: LY.DtypePolicy | str = LY.BF16, interpret: Any = False,
    device_kind: str | None = None, *, dv_out: Optional[Tensor] = None,
    dz_out: Optional[Tensor] = None,
) -> SISOGrads:
    """The HIP reverse scan plus the small epilogue of ``kernel_bwd.py:534-669``
    (dgamma, dD, the dfinal_k rotation pullback, seed gradients), in device torch ops
    on ``(B, H, L)``-sized tensors or smaller."""
    batch, seqlen, state_dim = q.shape
    nheads, headdim = v.shape[1], v.shape[3]
    n_angles = phi.shape[-1]
    kg = siso_backward_kernel(dy, ybar, z, q, k, v, adt, gamma, scale, phi, q_bias, k_bias,
                              chunk_states, d_skip=d_skip, dfinal_ssm=dfinal_ssm, chunk=chunk,
                              dtype_policy=dtype_policy, dfinal_v=dfinal_v,
                              dv_out=dv_out, dz_out=dz_out)
    dq, dk, dphi = kg.dq, kg.dk, kg.dphi
    dq_bias, dk_bias = kg.dq_bias, kg.dk_bias
    dgamma = kg.dqk_diag * kg.uw
    # over L (contiguous) first, then over B: one fast row reduction instead of a strided one
    dd_skip = kg.dqk_diag.sum(dim=2).sum(dim=0) if d_skip is not None else None
    if dfinal_k is not None:
        phi_last = phi.last() if isinstance(phi, PhiStrips) else phi[:, :, -1, :].float()
        cos_l, sin_l = LY.rope_cos_sin(phi_last, state_dim)
        dk_rot = LY.rope_apply(dfinal_k.float(), cos_l, -sin_l)     # (B, H, N)
        dk = dk.clone()
        dk[:, -1, :] += dk_rot.sum(dim=1)
        dk_bias = dk_bias + dk_rot.sum(dim=0)
        dphi = dphi.clone()
        dphi[:, :, -1, :] += LY.rope_dphi(kg.k_final, dfinal_k.float(), n_angles)
    if seed_ssm is not None:
        adj = kg.dseed_ssm
        coef = seed_coef.float()[..., None, None]
        dseed_k = (adj * coef * seed_v.float()[..., :, None]).sum(dim=2)
        dseed_v = (adj * coef * seed_k.float()[..., None, :]).sum(dim=3)
        dseed_coef = (adj * (seed_v.float()[..., :, None] * seed_k.float()[..., None, :])).sum(dim=(2, 3))
        dseed_ssm = adj
    else:
        dseed_ssm = dseed_k = dseed_v = dseed_coef = None
    return SISOGrads(dq=dq, dk=dk, dv=kg.dv, dadt=kg.dadt, dgamma=dgamma, dscale=kg.dscale,
                     dphi=dphi, dq_bias=dq_bias, dk_bias=dk_bias, dd_skip=dd_skip, dz=kg.dz,
                     dseed_ssm=dseed_ssm, dseed_k=dseed_k, dseed_v=dseed_v,
                     dseed_coef=dseed_coef)


# ======================================================================================
# BCNorm (layer.py:190-198 applied to B and C, layer.py:235-236)
# ======================================================================================


def _norm_rows_ok(t: Tensor) -> bool:
    vec = 16 // t.element_size()
    return (t.dim() == 3 and t.stride(2) == 1 and t.data_ptr() % 16 == 0
            and t.stride(0) % vec == 0 and t.stride(1) % vec == 0)


def bcnorm_supported(x: Tensor) -> bool:
    """True if `bcnorm_forward` / `bcnorm_backward` take ``x`` (a (B, L, N) view) in place:
    bf16 or f32, 16-byte aligned rows, N a multiple of 16 bytes and at most 64 of them."""
    if x.dtype not in (torch.bfloat16, torch.float32) or not x.is_cuda:
        return False
    vec = 16 // x.element_size()
    n = x.shape[-1]
    return n % vec == 0 and n // vec <= 64 and _norm_rows_ok(x)


def bcnorm_forward(xs, weights, eps: float, theta=None):
    """RMSNorm of each (B, L, N) view in ``xs`` (one or two, same shape and dtype) with its
    gain; one ``m3s_norm_fwd`` launch. Returns ``(ys, rstds)``: dense (B, L, N) outputs in
    the input dtype and the (B, L) f32 reciprocal RMS values the backward reuses.

    ``theta = (angles (B, L, Nr), dt_raw (B, L, H), dt_bias (H,), chunk)`` (raw projection
    slices in the inputs' dtype; ``chunk`` the tile the scan runs at, `layout.kernel_chunk`)
    also computes, in the same launch, the `RawAngles` that `siso_forward_raw` reads; the
    result is then ``(ys, rstds, RawAngles)``."""
    x0 = xs[0]
    dev = _device_of(*xs, *weights)
    batch, seqlen, width = x0.shape
    for x in xs:
        if tuple(x.shape) != tuple(x0.shape) or x.dtype != x0.dtype or not _norm_rows_ok(x):
            raise ValueError("bcnorm inputs must share shape and dtype, with 16-byte aligned rows")
    ys = [empty(batch, seqlen, width, device=dev, dtype=x0.dtype) for _ in xs]
    rstds = [empty(batch, seqlen, device=dev, dtype=torch.float32) for _ in xs]
    ws = [_f32c(w) for w in weights]
    a = _lib.NormFwdArgs()
    a.struct_size = ctypes.sizeof(_lib.NormFwdArgs)
    a.batch, a.seqlen, a.width = batch, seqlen, width
    a.dtype, a.count, a.eps = _lib.dtype_code(x0.dtype), len(xs), float(eps)
    for i, x in enumerate(xs):
        a.x[i] = _lib.blx(x)
        a.weight[i], a.y[i], a.rstd[i] = ws[i].data_ptr(), ys[i].data_ptr(), rstds[i].data_ptr()
    keep = None
    if theta is not None:
        angles, dt_raw, dt_bias, chunk = theta
        nr, nh = angles.shape[-1], dt_raw.shape[-1]
        if (tuple(angles.shape[:2]) != (batch, seqlen) or tuple(dt_raw.shape[:2]) != (batch, seqlen)
                or angles.dtype != x0.dtype or dt_raw.dtype != x0.dtype or chunk % 16
                or seqlen % chunk or nr % 4):
            raise ValueError("bcnorm theta: angles (B, L, Nr) and dt_raw (B, L, H) in the inputs' "
                             "dtype, a chunk that is a multiple of 16 dividing L, Nr % 4 == 0")
        _device_of(angles, dt_raw, dt_bias)
        bias = _f32c(dt_bias)
        table = empty(batch, seqlen, nr, device=dev, dtype=torch.float32)
        prefix = empty(batch, nh, seqlen // 16, nr, device=dev, dtype=torch.float32)
        ctot = empty(batch, nh, seqlen // chunk, nr, device=dev, dtype=torch.float32)
        a.nheads, a.n_angles, a.theta_chunk = nh, nr, chunk
        a.angles, a.dt_raw = _lib.blx(angles), _lib.blx(dt_raw)
        a.dt_bias, a.theta_table = bias.data_ptr(), table.data_ptr()
        a.theta_prefix, a.theta_chunk_totals = prefix.data_ptr(), ctot.data_ptr()
        keep = (bias, RawAngles(table, prefix, ctot, chunk))
    with torch.cuda.device(dev):
        _lib.check(_lib.load().m3s_norm_fwd(ctypes.byref(a), _lib.stream_handle(dev)),
                   "m3s_norm_fwd")
    if keep is not None:
        return ys, rstds, keep[1]
    return ys, rstds


def bcnorm_backward(xs, weights, rstds, dys, dxs):
    """Backward of `bcnorm_forward`: ``dys`` are f32 (B, L, N) cotangents (cast to the
    input dtype first, as the scan's q/k gradients are, ``siso.py:140-148``); the input
    gradients are written into ``dxs`` ((B, L, N) views of the input dtype, e.g. slices
    of the projection's gradient). Returns the f32 gain gradients."""
    x0 = xs[0]
    dev = _device_of(*xs, *weights, *rstds, *dys, *dxs)
    batch, seqlen, width = x0.shape
    for dx in dxs:
        if tuple(dx.shape) != tuple(x0.shape) or dx.dtype != x0.dtype or not _norm_rows_ok(dx):
            raise ValueError("bcnorm gradient buffers must match the inputs, with 16-byte aligned rows")
    ws = [_f32c(w) for w in weights]
    dyc = [_f32c(d) for d in dys]
    dws = [empty(width, device=dev, dtype=torch.float32) for _ in xs]
    lib = _lib.load()
    work = empty(lib.m3s_norm_bwd_workspace_bytes(width), device=dev, dtype=torch.uint8)
    a = _lib.NormBwdArgs()
    a.struct_size = ctypes.sizeof(_lib.NormBwdArgs)
    a.batch, a.seqlen, a.width = batch, seqlen, width
    a.dtype, a.count = _lib.dtype_code(x0.dtype), len(xs)
    for i, x in enumerate(xs):
        a.x[i], a.dx[i] = _lib.blx(x), _lib.blx(dxs[i])
        a.weight[i], a.rstd[i] = ws[i].data_ptr(), rstds[i].data_ptr()
        a.dy[i], a.dweight[i] = dyc[i].data_ptr(), dws[i].data_ptr()
    a.workspace = work.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(lib.m3s_norm_bwd(ctypes.byref(a), _lib.stream_handle(dev)), "m3s_norm_bwd")
    return dws


def adamw_update(params, grads, exp_avg, exp_avg_sq, lr: float, beta1: float, beta2: float,
                 eps: float, weight_decay: float, count: int,
                 grad_scale: Optional[Tensor] = None) -> None:
    """Update number ``count`` (>= 1) of clip-then-AdamW over lists of dense float32
    device tensors, in place, one ``m3s_adamw`` pass (optax ``chain(clip_by_global_norm,
    adamw)``, ``train.py:799-805``, after the global norm). ``grad_scale``: a float32
    device scalar multiplying every gradient (the clip factor), or None."""
    n = len(params)
    if not (len(grads) == len(exp_avg) == len(exp_avg_sq) == n):
        raise ValueError("adamw_update: the four tensor lists must have equal length")
    if count < 1:
        raise ValueError("adamw_update: the update count starts at 1")
    dev = None
    for group in (params, grads, exp_avg, exp_avg_sq):
        for t in group:
            if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
                raise ValueError("adamw_update: every tensor must be a dense float32 device tensor")
            if dev is None:
                dev = t.device
            if t.device != dev:
                raise ValueError("adamw_update: tensors on different devices")
    for p, g, m, v in zip(params, grads, exp_avg, exp_avg_sq):
        if not (p.shape == g.shape == m.shape == v.shape):
            raise ValueError("adamw_update: a parameter, its gradient and moments differ in shape")
    if grad_scale is not None and (not grad_scale.is_cuda or grad_scale.dtype != torch.float32
                                   or grad_scale.numel() != 1 or grad_scale.device != dev):
        raise ValueError("adamw_update: grad_scale must be a float32 device scalar")
    if n == 0:
        return
    ptrs = ctypes.c_void_p * n
    a = _lib.AdamwArgs()
    a.struct_size = ctypes.sizeof(_lib.AdamwArgs)
    a.count = n
    arrays = [ptrs(*[t.data_ptr() for t in group])
              for group in (params, grads, exp_avg, exp_avg_sq)]
    numel = (ctypes.c_int64 * n)(*[t.numel() for t in params])
    a.params, a.grads, a.exp_avg, a.exp_avg_sq = [ctypes.cast(x, ctypes.c_void_p) for x in arrays]
    a.numel = ctypes.cast(numel, ctypes.c_void_p)
    a.grad_scale = grad_scale.data_ptr() if grad_scale is not None else None
    # every scalar formed in double precision (as a framework passes Python scalars)
    a.one_minus_beta1, a.beta2, a.one_minus_beta2 = 1.0 - beta1, beta2, 1.0 - beta2
    a.eps, a.param_decay = eps, 1.0 - lr * weight_decay
    a.step_size = lr / (1.0 - beta1 ** count)
    a.bias_correction2_sqrt = math.sqrt(1.0 - beta2 ** count)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().m3s_adamw(ctypes.byref(a), _lib.stream_handle(dev)), "m3s_adamw")


def wgrad_supported(a: Tensor, b: Tensor) -> bool:
    """Whether `wgrad` takes these operands: bf16 device matrices of one device with unit
    column stride, 16-byte aligned rows, a token count that is a multiple of 32 and
    operands under 2 GiB."""
    if not (a.is_cuda and b.is_cuda and a.dtype == b.dtype == torch.bfloat16
            and a.dim() == b.dim() == 2 and a.device == b.device and a.shape[0] == b.shape[0]):
        return False
    m = a.shape[0]
    if m == 0 or m % 32 or a.shape[1] == 0 or b.shape[1] == 0:
        return False
    for t in (a, b):
        if t.stride(1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16 or t.stride(0) < t.shape[1]:
            return False
        if ((m - 1) * t.stride(0) + t.shape[1]) * 2 >= 1 << 31:
            return False
    return True


def wgrad(a: Tensor, b: Tensor) -> Tensor:
    """``a^T b`` in float32 for token-major bf16 ``a (M, P)`` and ``b (M, Q)``: a
    projection's weight gradient (one ``m3s_wgrad`` call: MFMA tiles over token splits,
    the split partials added in a fixed order). Operands must pass `wgrad_supported`."""
    if not wgrad_supported(a, b):
        raise ValueError("wgrad: a (M, P) and b (M, Q) must be bf16 device matrices with unit "
                         "column stride, 16-byte aligned rows and M a multiple of 32")
    lib = _lib.load()
    m, p, q = a.shape[0], a.shape[1], b.shape[1]
    c = empty(p, q, device=a.device, dtype=torch.float32)
    nbytes = lib.m3s_wgrad_workspace_bytes(m, p, q)
    if nbytes < 0:
        raise ValueError(f"wgrad: bad shape {(m, p, q)}")
    ws = empty(max(nbytes // 4, 1), device=a.device, dtype=torch.float32)
    w = _lib.WgradArgs()
    w.struct_size = ctypes.sizeof(_lib.WgradArgs)
    w.tokens, w.rows, w.cols = m, p, q
    w.a, w.lda = a.data_ptr(), a.stride(0)
    w.b, w.ldb = b.data_ptr(), b.stride(0)
    w.c, w.ldc = c.data_ptr(), q
    w.workspace = ws.data_ptr() if nbytes > 0 else None
    with torch.cuda.device(a.device):
        _lib.check(lib.m3s_wgrad(ctypes.byref(w), _lib.stream_handle(a.device)), "m3s_wgrad")
    return c


#: Rows that ``m3s_gemv``'s MFMA tiles take (5 to this many; 1-4 rows stream).
GEMM_ROWS_MAX = 1024
#: Row counts for which `matmul` prefers those tiles over the library product: measured
#: on the LM's and the layer's projection widths (K 768-2048, N 768-4480), the tiles were
#: faster from 32 to 256 rows (256 rows of the LM's in_proj 8.0 against 12.7 us, fc1 7.8
#: against 12.2 us) and the library at 8 rows and from 512.
MATMUL_TILE_ROWS = (32, 256)


def gemv_supported(x: Tensor, w: Tensor) -> bool:
    """Whether `gemv` takes ``x @ w``: bf16 device operands on one device with unit
    column strides, ``w`` ``(K, N)`` row-major with N a multiple of 8 and 16-byte aligned
    rows; 1 to 4 rows with K at most 4096 (the streaming pass), or 5 to `GEMM_ROWS_MAX`
    rows with K a multiple of 64 and 16-byte aligned x rows (the MFMA tiles)."""
    if not (x.is_cuda and w.is_cuda and x.dtype == w.dtype == torch.bfloat16
            and x.dim() == 2 and w.dim() == 2 and x.device == w.device):
        return False
    m, k = x.shape
    kw, n = w.shape
    if not (k == kw and k > 0 and n > 0 and n % 8 == 0 and x.stride(1) == 1
            and w.stride(1) == 1 and w.stride(0) % 8 == 0 and w.data_ptr() % 16 == 0):
        return False
    if 1 <= m <= 4:
        return k <= 4096
    return (m <= GEMM_ROWS_MAX and k % 64 == 0 and x.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0)


def gemv(x: Tensor, w: Tensor) -> Tensor:
    """``x @ w`` for a decode step's few rows (one ``m3s_gemv`` launch: a single streaming
    pass over the weight, float32 accumulation, bf16 out). Operands must pass
    `gemv_supported`."""
    if not gemv_supported(x, w):
        raise ValueError("gemv: x (M, K) and w (K, N) must be bf16 device matrices with unit "
                         "column stride, N % 8 == 0 and 16-byte aligned w rows; M <= 4 needs "
                         f"K <= 4096, 5 <= M <= {GEMM_ROWS_MAX} K % 64 == 0 and aligned x rows")
    m, k = x.shape
    n = w.shape[1]
    y = empty(m, n, device=x.device, dtype=torch.bfloat16)
    a = _lib.GemvArgs()
    a.struct_size = ctypes.sizeof(_lib.GemvArgs)
    a.rows, a.k, a.n = m, k, n
    a.x, a.ldx = x.data_ptr(), x.stride(0) if m > 1 else k
    a.w, a.ldw = w.data_ptr(), w.stride(0)
    a.y, a.ldy = y.data_ptr(), n
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().m3s_gemv(ctypes.byref(a), _lib.stream_handle(x.device)),
                   "m3s_gemv")
    return y


def matmul(x: Tensor, w: Tensor) -> Tensor:
    """``x @ w``: through `gemv` for one or two rows (a decode step's projections: inside a
    recorded decode step 3.6-4 us against the library's 5.8-8.5 us at the LM's widths) and
    for `MATMUL_TILE_ROWS` rows (a batch of decode tokens) when it takes them, else the
    library product (three and four rows are faster there)."""
    if x.dim() == 2 and gemv_supported(x, w):
        m = x.shape[0]
        if m <= 2 or MATMUL_TILE_ROWS[0] <= m <= MATMUL_TILE_ROWS[1]:
            return gemv(x, w)
    return x @ w


def rms_forward(x: Tensor, weight: Tensor, eps: float, out_dtype: torch.dtype,
                add: Optional[Tensor] = None):
    """LM block norm: ``x`` (..., D) in f32 or bf16 -> ``(y (..., D) in out_dtype, rstd
    (...,) f32)`` with ``y = x rstd w``, ``rstd = 1/sqrt(mean(x^2) + eps)`` in f32 (one
    ``m3s_rms_fwd`` launch; ``layer.py:190-198`` as ``model.py:194-232`` applies it).

    With ``add`` (same shape, in ``out_dtype``: a block's output) the launch first forms
    the residual sum ``s = x + add`` in x's dtype and normalises ``s``; it then returns
    ``(y, rstd, s)``."""
    if not x.is_cuda:
        raise ValueError("rms_forward: x must be a ROCm device tensor")
    x = x.contiguous()
    w = weight.float().contiguous()
    d = x.shape[-1]
    y = empty(x.shape, device=x.device, dtype=out_dtype)
    rstd = empty(x.shape[:-1], device=x.device, dtype=torch.float32)
    a = _lib.RmsArgs()
    a.struct_size = ctypes.sizeof(_lib.RmsArgs)
    a.x_dtype, a.y_dtype = _lib.dtype_code(x.dtype), _lib.dtype_code(out_dtype)
    a.width, a.rows, a.eps = d, x.numel() // d, float(eps)
    a.x, a.weight, a.y, a.rstd = x.data_ptr(), w.data_ptr(), y.data_ptr(), rstd.data_ptr()
    s = None
    if add is not None:
        if add.shape != x.shape or add.dtype != out_dtype or add.device != x.device:
            raise ValueError("rms_forward: add must match x's shape, in out_dtype, on x's device")
        add = add.contiguous()
        s = empty_like(x)
        a.add, a.sum = add.data_ptr(), s.data_ptr()
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().m3s_rms_fwd(ctypes.byref(a), _lib.stream_handle(x.device)),
                   "m3s_rms_fwd")
    return (y, rstd) if add is None else (y, rstd, s)


def rms_backward(x: Tensor, weight: Tensor, rstd: Tensor, dy: Tensor,
                 dsum: Optional[Tensor] = None, add_dtype: Optional[torch.dtype] = None):
    """Cotangents of `rms_forward`: ``dy`` (..., D) in y's dtype -> ``(dx in x's dtype,
    dweight (D,) f32)``, dweight summed in a fixed order (one ``m3s_rms_bwd`` call).

    Residual form: ``x`` is the sum the forward normalised; ``dsum`` (x's dtype, or None
    for zero) is the cotangent the rest of the network gives that sum, and ``dx`` becomes
    ``dsum`` plus the norm's pullback. With ``add_dtype`` the same ``dx`` comes back a
    second time in that dtype (the cotangent of the added block output):
    ``(dx, dweight, dadd)``."""
    x = x.contiguous()
    dy = dy.contiguous()
    w = weight.float().contiguous()
    d = x.shape[-1]
    dx = empty_like(x)
    dw = empty(d, device=x.device, dtype=torch.float32)
    ws = empty(max(_lib.load().m3s_rms_bwd_workspace_bytes(d), 0) // 4 + 1,
                     device=x.device, dtype=torch.float32)
    a = _lib.RmsArgs()
    a.struct_size = ctypes.sizeof(_lib.RmsArgs)
    a.x_dtype, a.y_dtype = _lib.dtype_code(x.dtype), _lib.dtype_code(dy.dtype)
    a.width, a.rows = d, x.numel() // d
    a.x, a.weight, a.rstd, a.dy = x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr()
    a.dx, a.dweight, a.workspace = dx.data_ptr(), dw.data_ptr(), ws.data_ptr()
    if dsum is not None:
        if dsum.shape != x.shape or dsum.device != x.device:
            raise ValueError("rms_backward: dsum must match x's shape and device")
        dsum = dsum.to(x.dtype).contiguous()
        a.dsum = dsum.data_ptr()
    dadd = None
    if add_dtype is not None:
        if add_dtype != dy.dtype:
            raise ValueError("rms_backward: the added tensor's dtype must be dy's")
        dadd = empty(x.shape, device=x.device, dtype=add_dtype)
        a.dadd = dadd.data_ptr()
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().m3s_rms_bwd(ctypes.byref(a), _lib.stream_handle(x.device)),
                   "m3s_rms_bwd")
    return (dx, dw) if add_dtype is None else (dx, dw, dadd)


def _swiglu_args(h: Tensor, width: int) -> "_lib.SwigluArgs":
    if not h.is_cuda:
        raise ValueError("swiglu: h must be a ROCm device tensor")
    if h.shape[-1] != 2 * width or not h.is_contiguous():
        raise ValueError(f"swiglu: h must be a dense (..., {2 * width}) tensor")
    a = _lib.SwigluArgs()
    a.struct_size = ctypes.sizeof(_lib.SwigluArgs)
    a.dtype = _lib.dtype_code(h.dtype)
    a.rows, a.width = h.numel() // (2 * width), width
    a.h = h.data_ptr()
    return a


def swiglu_forward(h: Tensor, width: int) -> Tensor:
    """``h`` (..., 2 width) = value | gate -> ``value * silu(gate)`` (..., width) in h's
    dtype (one ``m3s_swiglu_fwd`` launch; ``model.py:125-140``'s elementwise middle)."""
    a = _swiglu_args(h, width)
    out = empty(*h.shape[:-1], width, device=h.device, dtype=h.dtype)
    a.a = out.data_ptr()
    with torch.cuda.device(h.device):
        _lib.check(_lib.load().m3s_swiglu_fwd(ctypes.byref(a), _lib.stream_handle(h.device)),
                   "m3s_swiglu_fwd")
    return out


def swiglu_backward(h: Tensor, da: Tensor, width: int) -> Tensor:
    """Cotangent of `swiglu_forward`: ``da`` (..., width) -> ``dh`` (..., 2 width) =
    [d value | d gate] (one ``m3s_swiglu_bwd`` launch)."""
    a = _swiglu_args(h, width)
    da = da.to(h.dtype).contiguous()
    if tuple(da.shape) != (*h.shape[:-1], width):
        raise ValueError("swiglu: da must be (..., width)")
    dh = empty_like(h)
    a.da, a.dh = da.data_ptr(), dh.data_ptr()
    with torch.cuda.device(h.device):
        _lib.check(_lib.load().m3s_swiglu_bwd(ctypes.byref(a), _lib.stream_handle(h.device)),
                   "m3s_swiglu_bwd")
    return dh


def transpose_pad(w: Tensor, dtype: torch.dtype, out_rows: int) -> Tensor:
    """``w`` (R, C) -> a dense (out_rows, R) tensor of ``dtype`` holding ``w.T`` in its
    first C rows and zeros below (one ``m3s_transpose`` launch): the projection weights'
    GEMM layout."""
    dev = _device_of(w)
    if w.dim() != 2 or w.stride(1) != 1:
        w = w.contiguous()
    rows, cols = w.shape
    out = empty(out_rows, rows, device=dev, dtype=dtype)
    a = _lib.TransposeArgs()
    a.struct_size = ctypes.sizeof(_lib.TransposeArgs)
    a.rows, a.cols, a.out_rows = rows, cols, out_rows
    a.in_dtype, a.out_dtype = _lib.dtype_code(w.dtype), _lib.dtype_code(dtype)
    a.inp, a.in_stride, a.out = w.data_ptr(), w.stride(0), out.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.load().m3s_transpose(ctypes.byref(a), _lib.stream_handle(dev)),
                   "m3s_transpose")
    return out
