"""Dtype policy, the rotary permutation and the rope helpers (``layout.py`` surface).

Only the maths helpers of the reference's ``layout.py`` carry over (``layout.py:243-506``).
Its TPU machinery -- Mosaic BlockSpecs, VMEM limits, scalar-stream reshapes, layout
pinning, AOT lowering -- has no counterpart here: the HIP kernels own their
addressing and launch shapes.
"""

from __future__ import annotations

import dataclasses
import functools

import torch


@dataclasses.dataclass(frozen=True)
class DtypePolicy:
    """Which dtype each role uses (``layout.py:243-291``).

    ``matmul`` is the MFMA operand type: bf16 runs ``v_mfma_f32_16x16x32_bf16``, f32
    runs ``v_mfma_f32_16x16x4_f32``. Accumulation, state, decay and angles are always
    f32; ``saved_state`` is the dtype of the per-chunk state residual.
    """

    name: str
    matmul: torch.dtype
    accum: torch.dtype = torch.float32
    state: torch.dtype = torch.float32
    saved_state: torch.dtype = torch.bfloat16

    @property
    def highest(self) -> bool:
        return self.matmul == torch.float32


#: Production setting: bf16 MFMA operands, f32 accumulate (``layout.py:281``).
BF16 = DtypePolicy("bf16", torch.bfloat16)
#: Validation setting: everything f32 (``layout.py:285``).
F32 = DtypePolicy("f32", torch.float32, saved_state=torch.float32)


def policy(name) -> DtypePolicy:
    """``layout.py:288-294``: ``"bf16"`` or ``"f32"`` (and their aliases)."""
    if isinstance(name, DtypePolicy):
        return name
    key = str(name).strip().lower()
    if key in ("bf16", "bfloat16", "default"):
        return BF16
    if key in ("f32", "fp32", "float32", "highest"):
        return F32
    raise ValueError(f"Unknown dtype policy {name!r}; want 'bf16' or 'f32'")


@functools.lru_cache(maxsize=None)
def _perm_list(n: int) -> tuple:
    if n % 2 != 0:
        raise ValueError(f"state dim must be even for rotary pairing, got {n}")
    return tuple(list(range(0, n, 2)) + list(range(1, n, 2)))


def deinterleave_perm(n: int) -> torch.Tensor:
    """``layout.py:299-320``: ``new[j] = old[2j]``, ``new[n/2 + j] = old[2j + 1]``."""
    return torch.tensor(_perm_list(n), dtype=torch.long)


def interleave_perm(n: int) -> torch.Tensor:
    """``layout.py:323-326``: inverse of `deinterleave_perm`."""
    return torch.argsort(deinterleave_perm(n))


def apply_perm(x: torch.Tensor, axis: int = -1) -> torch.Tensor:
    """``layout.py:329-331``."""
    return torch.index_select(x, axis, deinterleave_perm(x.shape[axis]).to(x.device))


def unapply_perm(x: torch.Tensor, axis: int = -1) -> torch.Tensor:
    """``layout.py:334-337``."""
    return torch.index_select(x, axis, interleave_perm(x.shape[axis]).to(x.device))


def rope_cos_sin(phi: torch.Tensor, state_dim: int):
    """``layout.py:345-372``: ``cos``/``sin`` of ``[phi, 0-pad to N/2]`` doubled to N."""
    half = state_dim // 2
    nr = phi.shape[-1]
    if nr > half:
        raise ValueError(f"n_angles ({nr}) exceeds state_dim // 2 ({half})")
    if nr < half:
        phi = torch.cat([phi, phi.new_zeros(*phi.shape[:-1], half - nr)], dim=-1)
    full = torch.cat([phi, phi], dim=-1)
    return torch.cos(full), torch.sin(full)


def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``layout.py:375-398``: ``x*cos + [-x_hi, x_lo]*sin`` (half-split layout)."""
    half = x.shape[-1] // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * cos + rot * sin


def rope_dphi(x_rot: torch.Tensor, dx_rot: torch.Tensor, n_angles: int) -> torch.Tensor:
    """``layout.py:414-428``: ``dphi_j = dx_hi_j*x_lo_j - dx_lo_j*x_hi_j``, j < Nr."""
    half = x_rot.shape[-1] // 2
    lo, hi = x_rot[..., :half], x_rot[..., half:]
    dlo, dhi = dx_rot[..., :half], dx_rot[..., half:]
    return (dhi * lo - dlo * hi)[..., :n_angles]


def num_chunks(seqlen: int, chunk: int) -> int:
    """``layout.py:500-506``."""
    if seqlen % chunk != 0:
        raise ValueError(
            f"seqlen ({seqlen}) must be a multiple of chunk ({chunk}); "
            "pad the sequence before calling."
        )
    return seqlen // chunk


#: Chunk lengths the HIP kernels are instantiated for.
SUPPORTED_CHUNKS = (32, 64, 128, 256)


def validate_chunk(chunk: int) -> None:
    """GPU chunk rule, replacing the reference's Mosaic rule ``chunk % 128 == 0``
    (``layout.py:225-236``): any of `SUPPORTED_CHUNKS`. The reference's chunked maths
    (``reference.siso_chunked``) accepts any divisor of L; 32..256 are the tile sizes
    the MFMA kernels are built for."""
    if chunk not in SUPPORTED_CHUNKS:
        raise ValueError(f"chunk must be one of {SUPPORTED_CHUNKS}, got {chunk}")
