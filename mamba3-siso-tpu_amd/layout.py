"""Dtype policy, the rotary permutation and the rope helpers (``layout.py`` surface).

Only the maths helpers of the reference's ``layout.py`` carry over (``layout.py:243-506``).
Its TPU machinery -- Mosaic BlockSpecs, VMEM limits, scalar-stream reshapes, layout
pinning, AOT lowering -- has no counterpart here: the HIP kernels own their
addressing and launch shapes.
"""

from __future__ import annotations

import dataclasses
import functools
from typing import Optional

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


#: Chunk lengths the HIP kernels are instantiated for (the union over shapes; which
#: (chunk, d_state, headdim) exist per policy is `KERNELS`). A longer chunk is scanned
#: in tiles of one of these (`kernel_chunk`).
SUPPORTED_CHUNKS = (32, 64, 128)

#: The compiled kernel instantiations: role -> {(policy, chunk, d_state, headdim)}; decode
#: has no chunk (0). Mirrors the instantiation tables of ``csrc/m3s_fwd.hip``,
#: ``m3s_bwd.hip`` and ``m3s_decode.hip``; ``tests/test_abi_cpu.py`` checks this mirror
#: against the library's ``m3s_supported`` entry by entry, so `SISOConfig` can reject an
#: unsupported shape at construction without loading the library.
KERNELS = {
    "forward": frozenset({
        ("bf16", 128, 128, 64), ("bf16", 64, 128, 64), ("bf16", 32, 128, 64),
        ("bf16", 128, 64, 64), ("bf16", 64, 64, 64), ("bf16", 32, 64, 64),
        ("bf16", 128, 32, 16), ("bf16", 64, 32, 16), ("bf16", 32, 32, 16),
        ("bf16", 128, 16, 16), ("bf16", 64, 16, 16), ("bf16", 32, 16, 16),
        ("bf16", 32, 256, 64),
        ("f32", 64, 128, 64), ("f32", 32, 128, 64),
        ("f32", 64, 64, 64), ("f32", 32, 64, 64),
        ("f32", 128, 32, 16), ("f32", 64, 32, 16), ("f32", 32, 32, 16),
        ("f32", 128, 16, 16), ("f32", 64, 16, 16), ("f32", 32, 16, 16),
    }),
    "backward": frozenset({
        ("bf16", 128, 128, 64), ("bf16", 64, 128, 64), ("bf16", 32, 128, 64),
        ("bf16", 128, 64, 64), ("bf16", 64, 64, 64), ("bf16", 32, 64, 64),
        ("bf16", 128, 32, 16), ("bf16", 64, 32, 16), ("bf16", 32, 32, 16),
        ("bf16", 128, 16, 16), ("bf16", 64, 16, 16), ("bf16", 32, 16, 16),
        ("bf16", 32, 256, 64),
        ("f32", 32, 128, 64),
        ("f32", 64, 64, 64), ("f32", 32, 64, 64),
        ("f32", 128, 32, 16), ("f32", 64, 32, 16), ("f32", 32, 32, 16),
        ("f32", 128, 16, 16), ("f32", 64, 16, 16), ("f32", 32, 16, 16),
    }),
    "decode": frozenset({
        (pol, 0, n, p) for pol in ("bf16", "f32") for n, p in ((128, 64), (64, 64), (32, 16), (16, 16))
    } | {("bf16", 0, 256, 64)}),
}


def kernel_chunk(policy_name: str, chunk: int, d_state: int, headdim: int) -> Optional[int]:
    """The chunk the scan kernels run for a requested ``chunk``: the largest compiled
    chunk (forward and backward both, so the forward's per-chunk states are the ones the
    backward reads) that divides ``chunk``; None if there is none.

    The chunked form is exact for any chunk length -- the intra-chunk quadratic form plus
    the carried state reproduce the recurrence (``reference.py:217-330``) -- so a chunk of
    512 scanned as four 128-token tiles gives the same results to float rounding. The
    caller's chunk still has to divide the sequence (``layout.py:500-506``)."""
    pol = policy(policy_name).name
    for c in sorted(SUPPORTED_CHUNKS, reverse=True):
        if (chunk % c == 0 and (pol, c, d_state, headdim) in KERNELS["forward"]
                and (pol, c, d_state, headdim) in KERNELS["backward"]):
            return c
    return None


def kernel_headdim(policy_name: str, chunk: int, d_state: int, headdim: int) -> Optional[int]:
    """The head width the kernels run for ``headdim``: ``headdim`` itself when it has
    scan (`kernel_chunk`) and decode kernels, else the largest compiled width dividing
    it; None if there is none.

    Given a head's scores ``q~ . k^`` and decays, its output and state are independent
    across the P columns of v (``reference.py:217-330``): a head of width P runs exactly
    as P / P' heads of width P' that share its q, k, scalars, phi and biases, with the
    shared inputs' gradients summed over them."""
    pol = policy(policy_name).name

    def ok(p):
        return (kernel_chunk(pol, chunk, d_state, p) is not None
                and (pol, 0, d_state, p) in KERNELS["decode"])

    if ok(headdim):
        return headdim
    widths = sorted({p for (q, _, n, p) in KERNELS["forward"] if q == pol and n == d_state},
                    reverse=True)
    for p in widths:
        if p < headdim and headdim % p == 0 and ok(p):
            return p
    return None


def decode_headdim(policy_name: str, d_state: int, headdim: int) -> Optional[int]:
    """`kernel_headdim` for the decode kernels alone (no chunk)."""
    pol = policy(policy_name).name
    widths = sorted({p for (q, _, n, p) in KERNELS["decode"] if q == pol and n == d_state},
                    reverse=True)
    if headdim in widths:
        return headdim
    for p in widths:
        if p < headdim and headdim % p == 0:
            return p
    return None


def missing_kernels(policy_name: str, chunk: int, d_state: int, headdim: int) -> list:
    """The roles (forward, backward, decode) with no compiled kernel to run this shape
    (for the scans at `kernel_chunk`, as heads of `kernel_headdim`)."""
    pol = policy(policy_name).name
    width = kernel_headdim(pol, chunk, d_state, headdim)
    if width is not None:
        return []
    out = []
    if kernel_chunk(pol, chunk, d_state, headdim) is None:
        out += ["forward", "backward"]
    if (pol, 0, d_state, headdim) not in KERNELS["decode"]:
        out.append("decode")
    return out


def compiled_chunks(policy_name: str, d_state: int, headdim: int) -> tuple:
    """Chunks with both a forward and a backward kernel for (policy, d_state, headdim)."""
    pol = policy(policy_name).name
    return tuple(c for c in SUPPORTED_CHUNKS
                 if (pol, c, d_state, headdim) in KERNELS["forward"]
                 and (pol, c, d_state, headdim) in KERNELS["backward"])


def validate_chunk(chunk: int) -> None:
    """The reference's rule, a positive multiple of 128 (``layout.py:225-236``), widened
    to the shorter kernel tiles 32 and 64. A multiple of 128 above 128 runs as 128-token
    (or shorter) tiles (`kernel_chunk`)."""
    if not isinstance(chunk, int) or chunk <= 0 or (chunk % 128 and chunk not in SUPPORTED_CHUNKS):
        raise ValueError(f"chunk must be 32, 64 or a positive multiple of 128, got {chunk}")


def validate_kernel_shape(policy_name: str, chunk: int, d_state: int, headdim: int) -> None:
    """Raise ``ValueError`` unless forward, backward and decode kernels are all compiled
    to run this (policy, chunk, d_state, headdim) -- the check the reference makes on its
    chunk when the config is built (``layer.py:97-99``), widened to the whole shape
    because the HIP kernels are compiled per shape."""
    validate_chunk(chunk)
    missing = missing_kernels(policy_name, chunk, d_state, headdim)
    if missing:
        ok = compiled_chunks(policy_name, d_state, headdim)
        hint = (f"chunks compiled for this policy and shape: {list(ok)}" if ok else
                "no chunk is compiled for this policy and shape")
        raise ValueError(
            f"no {'/'.join(missing)} kernel for policy={policy(policy_name).name} "
            f"chunk={chunk} d_state={d_state} headdim={headdim}; {hint}")
