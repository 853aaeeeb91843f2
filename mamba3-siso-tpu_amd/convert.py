"""Upstream torch checkpoints <-> this package's parameter trees.

The on-disk format is upstream's (``convert.py:58-356`` of the reference reads and
writes the same one): the two linears are stored torch-style ``(out, in)``, the
state-axis tensors in the interleaved rotary layout, the B/C biases with a MIMO rank
axis of 1. The kernels want ``(in, out)`` linears and the permuted half-split rotary
layout (``layout.py:299-337``).

Design: every difference between the two sides is data, not code. `MIXER_LEAVES` lists,
per `SISOParams` field, its torch key(s) and the three things that can happen to it --
a transpose, the state-axis permutation (on the last axis, or on the B and C column
blocks of the projection), and the rank axis. One pair of functions (`_leaf_in`,
`_leaf_out`) applies a table row in either direction, and the whole-model mapping is a
second table (`BLOCK_LEAVES`, `TOP_LEAVES`) of `LMParams` paths to released key names,
walked by the same loop for import and export. Released ``config.json`` files are read
through a field table and a list of refusal rules.

The reference's names are kept (``torch_to_jax`` / ``jax_to_torch`` /
``config_from_state_dict`` / ``config_from_hf`` / ``load_lm_state_dict`` /
``load_pretrained``) so code written against it runs unchanged.
``params_from_state_dict`` / ``state_dict_from_params`` are descriptive aliases.
`load_pretrained` reads a LOCAL directory only; there is no network download.
"""

from __future__ import annotations

import dataclasses
import json
import os
from typing import Any, Mapping, Optional

import numpy as np
import torch

from . import layout as LY
from .layer import SISOConfig, SISOParams


# ------------------------------------------------------------------------------------
# one layer (the "mixer")
# ------------------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class Leaf:
    """How one `SISOParams` field is stored in an upstream state dict.

    ``keys``: accepted torch names, the first one written on export. ``transpose``:
    torch keeps ``(out, in)``. ``perm``: where the state-axis permutation applies --
    ``"last"`` (the trailing N axis) or ``"bc_blocks"`` (the B and C column blocks of the
    projection). ``rank_axis``: stored as ``(H, rank, N)`` with rank 1 (SISO)."""

    field: str
    keys: tuple
    transpose: bool = False
    perm: Optional[str] = None
    rank_axis: bool = False


MIXER_LEAVES = (
    Leaf("in_proj", ("in_proj.weight",), transpose=True, perm="bc_blocks"),
    Leaf("out_proj", ("out_proj.weight",), transpose=True),
    Leaf("dt_bias", ("dt_bias",)),
    Leaf("b_norm_weight", ("B_norm.weight", "B_norm_weight"), perm="last"),
    Leaf("c_norm_weight", ("C_norm.weight", "C_norm_weight"), perm="last"),
    Leaf("b_bias", ("B_bias",), perm="last", rank_axis=True),
    Leaf("c_bias", ("C_bias",), perm="last", rank_axis=True),
    Leaf("d_skip", ("D",)),
)
assert tuple(leaf.field for leaf in MIXER_LEAVES) == SISOParams._fields


def _f32(x: Any) -> np.ndarray:
    """A float32 numpy copy of a tensor or array. Torch tensors are widened by torch
    first, so bf16 checkpoints (which numpy cannot represent) convert too."""
    if isinstance(x, torch.Tensor):
        x = x.detach().to("cpu", torch.float32).numpy()
    return np.array(x, dtype=np.float32, copy=True)


def _state_index(leaf: Leaf, cfg: SISOConfig, width: int) -> np.ndarray:
    """Index array over the permuted axis: position i of our layout reads position
    ``idx[i]`` of upstream's. Only the B and C blocks move for ``bc_blocks``."""
    n = cfg.d_state
    perm = LY.deinterleave_perm(n).numpy()
    if leaf.perm == "last":
        return perm
    idx = np.arange(width)
    for start in (2 * cfg.d_inner, 2 * cfg.d_inner + n):
        idx[start:start + n] = start + perm
    return idx


def _leaf_in(leaf: Leaf, raw: np.ndarray, cfg: SISOConfig) -> np.ndarray:
    """Upstream array -> ours, per the table row."""
    a = raw
    if leaf.rank_axis and a.ndim == 3:
        if a.shape[1] != 1:
            raise ValueError(f"{leaf.keys[0]} has shape {a.shape}: mimo_rank={a.shape[1]}, "
                             "but only rank-1 (SISO) layers convert")
        a = a[:, 0, :]
    if leaf.transpose:
        a = a.T
    if leaf.perm is not None:
        a = a[..., _state_index(leaf, cfg, a.shape[-1])]
    return np.ascontiguousarray(a)


def _leaf_out(leaf: Leaf, ours: np.ndarray, cfg: SISOConfig) -> np.ndarray:
    """Ours -> upstream array: the inverse of `_leaf_in`."""
    a = ours
    if leaf.perm is not None:
        a = a[..., np.argsort(_state_index(leaf, cfg, a.shape[-1]))]
    if leaf.transpose:
        a = a.T
    if leaf.rank_axis:
        a = a[:, None, :]
    return np.ascontiguousarray(a)


def _lookup(sd: Mapping[str, Any], names, where: str = ""):
    for name in names:
        if name in sd:
            return sd[name]
    raise KeyError(f"state dict{where} has none of {list(names)}")


def config_from_state_dict(sd: Mapping[str, Any], headdim: int = 64, **overrides) -> SISOConfig:
    """Infer a `SISOConfig` from a layer's torch state dict (``convert.py:58-89``).

    ``in_proj.weight`` gives ``d_model`` and the projection width, ``B_bias`` gives
    ``nheads`` and ``d_state``; ``headdim`` cannot be read off the weights and must be
    supplied. The projection width is then checked against the config, which catches a
    wrong ``headdim`` and MIMO checkpoints (whose B/C blocks are rank times wider)."""
    rows, d_model = tuple(_lookup(sd, ("in_proj.weight",)).shape)
    bias_shape = tuple(_lookup(sd, ("B_bias",)).shape)
    nheads, d_state = bias_shape[0], bias_shape[-1]
    expand, rem = divmod(nheads * headdim, d_model)
    if rem or expand == 0:
        raise ValueError(f"{nheads} heads of headdim {headdim} give d_inner={nheads * headdim}, "
                         f"not a whole multiple of d_model={d_model}: wrong headdim?")
    cfg = SISOConfig(d_model=d_model, d_state=d_state, headdim=headdim, expand=expand, **overrides)
    if cfg.d_in_proj != rows:
        raise ValueError(f"in_proj.weight has {rows} output rows; a SISO layer with this "
                         f"config has {cfg.d_in_proj}. MIMO layers (rank > 1) are not "
                         f"supported, and a wrong headdim (here {headdim}) also shows up this way")
    return cfg


def torch_to_jax(sd: Mapping[str, Any], cfg: SISOConfig, dtype=torch.float32,
                 device=None) -> SISOParams:
    """A layer's torch state dict -> `SISOParams` in the kernels' layout
    (``convert.py:92-149``). Norm gains are found as ``B_norm.weight`` (upstream) or
    ``B_norm_weight``."""
    out = {}
    for leaf in MIXER_LEAVES:
        arr = _leaf_in(leaf, _f32(_lookup(sd, leaf.keys)), cfg)
        out[leaf.field] = torch.as_tensor(arr, dtype=dtype, device=device)
    return SISOParams(**out)


def jax_to_torch(params: SISOParams, cfg: SISOConfig) -> dict:
    """`SISOParams` -> a torch-format state dict of float32 numpy arrays
    (``convert.py:152-176``); the exact inverse of `torch_to_jax`."""
    return {leaf.keys[0]: _leaf_out(leaf, _f32(getattr(params, leaf.field)), cfg)
            for leaf in MIXER_LEAVES}


params_from_state_dict = torch_to_jax
state_dict_from_params = jax_to_torch


# ------------------------------------------------------------------------------------
# whole released checkpoints
# ------------------------------------------------------------------------------------

#: Per-block leaves of a released ``MambaLMHeadModel``: (path in `model.BlockParams`,
#: key template, transposed, present only with an MLP). The mixer itself is the
#: `MIXER_LEAVES` table under ``MIXER_PREFIX``.
BLOCK_LEAVES = (
    ("norm_gain", "backbone.layers.{i}.norm.weight", False, False),
    ("mlp_norm_gain", "backbone.layers.{i}.norm2.weight", False, True),
    ("mlp.fc1", "backbone.layers.{i}.mlp.fc1.weight", True, True),
    ("mlp.fc2", "backbone.layers.{i}.mlp.fc2.weight", True, True),
)
#: Model-level leaves: (path in `model.LMParams`, key, transposed).
TOP_LEAVES = (
    ("embed", "backbone.embedding.weight", False),
    ("final_norm", "backbone.norm_f.weight", False),
    ("head", "lm_head.weight", True),
)
MIXER_PREFIX = "backbone.layers.{i}.mixer."

#: ``config.json`` fields read into `SISOConfig`: (key under ``ssm_cfg``, field, type).
#: Fields absent from the file keep `SISOConfig`'s defaults.
HF_SSM_FIELDS = (
    ("d_state", "d_state", int),
    ("headdim", "headdim", int),
    ("expand", "expand", int),
    ("rope_fraction", "rope_fraction", float),
    ("A_floor", "a_floor", float),
    ("dt_min", "dt_min", float),
    ("dt_max", "dt_max", float),
    ("dt_init_floor", "dt_init_floor", float),
)

#: Released configurations this package does not implement: (test on (config.json,
#: ssm_cfg), message). Each names what the checkpoint has that a SISO stack lacks.
HF_REFUSALS: tuple = (
    (lambda top, ssm: ssm.get("layer", "Mamba3") != "Mamba3",
     lambda top, ssm: f"ssm_cfg.layer={ssm.get('layer')!r}: only Mamba3 layers load"),
    (lambda top, ssm: bool(ssm.get("mimo")) or (ssm.get("mimo_rank") or 1) != 1,
     lambda top, ssm: "a MIMO checkpoint (mimo / mimo_rank > 1); only SISO layers load"),
    (lambda top, ssm: bool(top.get("attn_layer_idx")),
     lambda top, ssm: f"attention layers at {top['attn_layer_idx']}: hybrid attention "
                      "stacks do not load"),
    (lambda top, ssm: ssm.get("ngroups", 1) != 1,
     lambda top, ssm: f"ngroups={ssm['ngroups']}: only the SISO grouping (1) loads"),
)


def config_from_hf(cfg_json: Mapping[str, Any], **overrides):
    """A released ``config.json`` -> `model.LMConfig` (``convert.py:202-267``).

    The vocabulary is rounded up to ``pad_vocab_size_multiple``, the width the released
    embedding has. The chunk is 128 unless overridden: the file's ``chunk_size`` is the
    upstream kernel's tiling, not a property of the weights. ``overrides`` replace any
    `SISOConfig` field. Refused with ``ValueError``: see `HF_REFUSALS`."""
    from . import model as M

    ssm = dict(cfg_json.get("ssm_cfg") or {})
    for test, message in HF_REFUSALS:
        if test(cfg_json, ssm):
            raise ValueError(f"cannot load this checkpoint: {message(cfg_json, ssm)}")
    fields: dict = {"d_model": int(cfg_json["d_model"]), "chunk": 128}
    fields.update({dst: kind(ssm[src]) for src, dst, kind in HF_SSM_FIELDS if src in ssm})
    fields.update({k: v for k, v in overrides.items() if k != "d_intermediate"})
    multiple = max(1, int(cfg_json.get("pad_vocab_size_multiple") or 1))
    vocab = -(-int(cfg_json["vocab_size"]) // multiple) * multiple
    return M.LMConfig(vocab_size=vocab, n_layers=int(cfg_json["n_layer"]),
                      siso=SISOConfig(**fields),
                      tie_head=bool(cfg_json.get("tie_embeddings", True)),
                      d_intermediate=int(cfg_json.get("d_intermediate", 0)))


def _get_path(obj, path: str):
    for part in path.split("."):
        obj = None if obj is None else getattr(obj, part)
    return obj


def _model_leaves(cfg):
    """(path, key, transposed) of every non-mixer tensor the config implies, in a fixed
    order; block paths are prefixed ``blocks.{i}.``."""
    out = []
    for i in range(cfg.n_layers):
        for path, key, tr, mlp_only in BLOCK_LEAVES:
            if cfg.d_intermediate or not mlp_only:
                out.append((f"blocks.{i}.{path}", key.format(i=i), tr))
    for path, key, tr in TOP_LEAVES:
        if path != "head" or not cfg.tie_head:
            out.append((path, key, tr))
    return out


def load_lm_state_dict(sd: Mapping[str, Any], cfg, dtype=torch.float32, device=None):
    """A released ``MambaLMHeadModel`` state dict -> `model.LMParams`
    (``convert.py:270-330``). Strict: a tensor the config implies but the dict lacks
    raises ``KeyError`` with its name, and an embedding whose width is not the padded
    vocabulary raises ``ValueError``."""
    from . import model as M

    def tensor(arr):
        return torch.as_tensor(np.ascontiguousarray(arr), dtype=dtype, device=device)

    flat = {}
    for path, key, tr in _model_leaves(cfg):
        if key not in sd:
            raise KeyError(f"released state dict lacks {key!r}, which the config implies")
        arr = _f32(sd[key])
        flat[path] = tensor(arr.T if tr else arr)
    want = (cfg.vocab_size, cfg.d_model)
    if tuple(flat["embed"].shape) != want:
        raise ValueError(f"backbone.embedding.weight is {tuple(flat['embed'].shape)} but the "
                         f"config needs {want} (vocab_size rounded up to "
                         "pad_vocab_size_multiple)")
    blocks = []
    for i in range(cfg.n_layers):
        prefix = MIXER_PREFIX.format(i=i)
        mixer = {k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)}
        if not mixer:
            raise KeyError(f"released state dict has no {prefix}* tensors (layer {i} of "
                           f"{cfg.n_layers})")
        mlp = None
        if cfg.d_intermediate:
            mlp = M.MLPParams(fc1=flat[f"blocks.{i}.mlp.fc1"], fc2=flat[f"blocks.{i}.mlp.fc2"])
        blocks.append(M.BlockParams(
            norm_gain=flat[f"blocks.{i}.norm_gain"],
            siso=torch_to_jax(mixer, cfg.siso, dtype, device),
            mlp_norm_gain=flat.get(f"blocks.{i}.mlp_norm_gain"), mlp=mlp))
    return M.LMParams(embed=flat["embed"], blocks=blocks, final_norm=flat["final_norm"],
                      head=flat.get("head"))


def lm_state_dict(params, cfg) -> dict:
    """`model.LMParams` -> a released-format state dict of float32 numpy arrays; the
    inverse of `load_lm_state_dict`. With a tied head ``lm_head.weight`` is the
    embedding, as upstream stores one shared tensor under both names."""
    sd: dict = {}
    for path, key, tr in _model_leaves(cfg):
        arr = _f32(_get_path_indexed(params, path))
        sd[key] = np.ascontiguousarray(arr.T) if tr else arr
    for i, blk in enumerate(params.blocks):
        prefix = MIXER_PREFIX.format(i=i)
        sd.update({prefix + k: v for k, v in jax_to_torch(blk.siso, cfg.siso).items()})
    if cfg.tie_head:
        sd["lm_head.weight"] = sd["backbone.embedding.weight"]
    return sd


def _get_path_indexed(params, path: str):
    if path.startswith("blocks."):
        _, i, rest = path.split(".", 2)
        return _get_path(params.blocks[int(i)], rest)
    return _get_path(params, path)


def _read_weights(path: str) -> Mapping[str, Any]:
    st = os.path.join(path, "model.safetensors")
    if os.path.exists(st):
        from safetensors.torch import load_file
        return load_file(st, device="cpu")
    # weights_only: tensors and containers only, no code in the file runs
    return torch.load(os.path.join(path, "pytorch_model.bin"), map_location="cpu",
                      weights_only=True)


def load_pretrained(path: str, dtype=torch.float32, device=None, **cfg_overrides):
    """A released checkpoint in a LOCAL directory -> ``(params, cfg)``
    (``convert.py:333-356``, without the Hub download): ``config.json`` plus
    ``model.safetensors`` (preferred) or ``pytorch_model.bin``."""
    if not os.path.isdir(path):
        raise ValueError(f"{path!r}: expected a local checkpoint directory (config.json + "
                         "weights); hub names are not fetched")
    with open(os.path.join(path, "config.json")) as fh:
        cfg = config_from_hf(json.load(fh), **cfg_overrides)
    return load_lm_state_dict(_read_weights(path), cfg, dtype, device), cfg
