"""Weight layout conversion between an upstream torch ``state_dict`` and `SISOParams`.

Restates ``convert.py:58-176`` of the reference (host-side format conversion, not a
compute path): transpose the two linears from torch's ``(out, in)`` to ``(in, out)``;
apply the de-interleave permutation to every tensor on the state axis (the B and C
column blocks of ``in_proj``, the two norm gains, the two biases); squeeze the MIMO
rank of the biases (``(H, 1, N)`` -> ``(H, N)``). ``dt_bias``, ``D`` and ``out_proj``
pass through. The names ``torch_to_jax`` / ``jax_to_torch`` are kept so code written
against the reference runs unchanged; ``params_from_state_dict`` /
``state_dict_from_params`` are the descriptive aliases.
"""

from __future__ import annotations

from typing import Any, Mapping

import numpy as np
import torch

from . import layout as LY
from .layer import SISOConfig, SISOParams


def _to_numpy(x: Any) -> np.ndarray:
    """``convert.py:39-51``: torch tensors (bf16 included) widen on the torch side."""
    if hasattr(x, "detach"):
        x = x.detach().cpu()
        if hasattr(x, "float"):
            x = x.float()
    return np.asarray(x, dtype=np.float32)


def _perm(n: int) -> np.ndarray:
    return LY.deinterleave_perm(n).numpy()


def config_from_state_dict(sd: Mapping[str, Any], headdim: int = 64, **overrides) -> SISOConfig:
    """``convert.py:58-89``: ``d_model``/``d_in_proj`` from ``in_proj.weight``,
    ``d_state``/``nheads`` from ``B_bias``; ``headdim`` must be supplied."""
    in_proj = _to_numpy(sd["in_proj.weight"])
    d_in_proj, d_model = in_proj.shape
    b_bias = _to_numpy(sd["B_bias"])
    nheads, d_state = b_bias.shape[0], b_bias.shape[-1]
    d_inner = nheads * headdim
    if d_inner % d_model != 0:
        raise ValueError(
            f"nheads*headdim = {d_inner} is not a multiple of d_model = {d_model}; "
            f"headdim={headdim} is probably wrong for this checkpoint")
    cfg = SISOConfig(d_model=d_model, d_state=d_state, headdim=headdim,
                     expand=d_inner // d_model, **overrides)
    if cfg.d_in_proj != d_in_proj:
        raise ValueError(
            f"in_proj width {d_in_proj} does not match the config's {cfg.d_in_proj}. "
            f"This checkpoint may be MIMO (mimo_rank > 1), which is out of scope, or "
            f"headdim is not {headdim}.")
    return cfg


def torch_to_jax(sd: Mapping[str, Any], cfg: SISOConfig, dtype=torch.float32,
                 device=None) -> SISOParams:
    """``convert.py:92-149``: a torch ``state_dict`` -> `SISOParams` (permuted layout).

    Norm gains are accepted as ``B_norm.weight`` (upstream) or ``B_norm_weight``.
    """
    n = cfg.d_state
    perm = _perm(n)
    in_proj = _to_numpy(sd["in_proj.weight"]).T.copy()
    out_proj = _to_numpy(sd["out_proj.weight"]).T.copy()
    b_start = 2 * cfg.d_inner
    for start in (b_start, b_start + n):
        in_proj[:, start:start + n] = in_proj[:, start:start + n][:, perm]

    def norm_gain(prefix: str) -> np.ndarray:
        for key in (f"{prefix}_norm.weight", f"{prefix}_norm_weight"):
            if key in sd:
                return _to_numpy(sd[key])
        raise KeyError(f"missing {prefix} norm weight ({prefix}_norm.weight)")

    def bias(prefix: str) -> np.ndarray:
        arr = _to_numpy(sd[f"{prefix}_bias"])
        if arr.ndim == 3:
            if arr.shape[1] != 1:
                raise ValueError(f"{prefix}_bias has mimo_rank {arr.shape[1]}; MIMO is out of scope")
            arr = arr[:, 0]
        return arr

    def t(a):
        return torch.as_tensor(np.ascontiguousarray(a), dtype=dtype, device=device)

    return SISOParams(
        in_proj=t(in_proj), out_proj=t(out_proj),
        dt_bias=t(_to_numpy(sd["dt_bias"])),
        b_norm_weight=t(norm_gain("B")[perm]), c_norm_weight=t(norm_gain("C")[perm]),
        b_bias=t(bias("B")[:, perm]), c_bias=t(bias("C")[:, perm]),
        d_skip=t(_to_numpy(sd["D"])),
    )


def jax_to_torch(params: SISOParams, cfg: SISOConfig) -> dict:
    """``convert.py:152-176``: inverse of `torch_to_jax`, as float32 numpy arrays in
    torch's shapes and order."""
    n = cfg.d_state
    inv = LY.interleave_perm(n).numpy()
    in_proj = _to_numpy(params.in_proj).copy()
    b_start = 2 * cfg.d_inner
    for start in (b_start, b_start + n):
        in_proj[:, start:start + n] = in_proj[:, start:start + n][:, inv]
    return {
        "in_proj.weight": in_proj.T.copy(),
        "out_proj.weight": _to_numpy(params.out_proj).T.copy(),
        "dt_bias": _to_numpy(params.dt_bias),
        "B_norm.weight": _to_numpy(params.b_norm_weight)[inv],
        "C_norm.weight": _to_numpy(params.c_norm_weight)[inv],
        "B_bias": _to_numpy(params.b_bias)[:, inv][:, None, :],
        "C_bias": _to_numpy(params.c_bias)[:, inv][:, None, :],
        "D": _to_numpy(params.d_skip),
    }


params_from_state_dict = torch_to_jax
state_dict_from_params = jax_to_torch
