"""Weight layout conversion between an upstream torch ``state_dict`` and `SISOParams`.

Restates ``convert.py:58-176`` of the reference (host-side format conversion, not a
compute path): transpose the two linears from torch's ``(out, in)`` to ``(in, out)``;
apply the de-interleave permutation to every tensor on the state axis (the B and C
column blocks of ``in_proj``, the two norm gains, the two biases); squeeze the MIMO
rank of the biases (``(H, 1, N)`` -> ``(H, N)``). ``dt_bias``, ``D`` and ``out_proj``
pass through. The names ``torch_to_jax`` / ``jax_to_torch`` are kept so code written
against the reference runs unchanged; ``params_from_state_dict`` /
``state_dict_from_params`` are the descriptive aliases.

Whole released checkpoints (``convert.py:179-356``): `config_from_hf` reads a released
``config.json`` (vocab padding, chunk override, MIMO / hybrid / ngroups refusal) and
`load_lm_state_dict` maps a ``MambaLMHeadModel`` state dict (``backbone.``-prefixed keys)
onto `model.LMParams`, widening bf16 tensors on the torch side. `load_pretrained` reads a
LOCAL checkpoint directory (``config.json`` plus ``model.safetensors`` or
``pytorch_model.bin``); there is no network download.
"""

from __future__ import annotations

from typing import Any, Mapping

import json
import os

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


# ------------------------------------------------------------------------------------
# whole released checkpoints (convert.py:179-356)
# ------------------------------------------------------------------------------------
#
# A released ``MambaLMHeadModel`` state dict, per block i:
#   backbone.layers.{i}.norm.weight (d_model,); backbone.layers.{i}.mixer.* (the layer's
#   torch state dict); with an MLP: backbone.layers.{i}.norm2.weight (d_model,),
#   backbone.layers.{i}.mlp.fc1.weight (2*d_int, d_model), .mlp.fc2.weight (d_model, d_int)
# plus backbone.embedding.weight (vocab_padded, d_model), backbone.norm_f.weight and
# lm_head.weight (vocab_padded, d_model; the embedding itself when tied).

MIXER_PREFIX = "backbone.layers.{i}.mixer."


def config_from_hf(cfg_json: Mapping[str, Any], **overrides):
    """A released ``config.json`` -> `model.LMConfig` (``convert.py:202-267``).

    ``vocab_size`` is padded up to ``pad_vocab_size_multiple`` (upstream pads inside the
    model, so the checkpoint's embedding has the padded width). ``chunk`` defaults to
    128, as in the reference, whatever the file says; ``overrides`` replace any
    `SISOConfig` field. Raises ``ValueError`` for a non-Mamba3 layer, MIMO, attention
    layers or ``ngroups != 1``."""
    from . import model as M

    ssm = dict(cfg_json.get("ssm_cfg", {}))
    layer_name = ssm.pop("layer", "Mamba3")
    if layer_name != "Mamba3":
        raise ValueError(f"ssm_cfg.layer is {layer_name!r}, expected 'Mamba3'")
    if ssm.get("mimo", False) or ssm.get("mimo_rank", 1) not in (1, None):
        raise ValueError("this checkpoint is MIMO; only SISO is implemented")
    if cfg_json.get("attn_layer_idx"):
        raise ValueError(f"checkpoint has attention layers at {cfg_json['attn_layer_idx']}; "
                         "hybrid attention/SSM stacks are not implemented")
    if ssm.get("ngroups", 1) != 1:
        raise ValueError(f"ngroups={ssm['ngroups']}, only ngroups=1 (SISO) is implemented")
    vocab = int(cfg_json["vocab_size"])
    mult = int(cfg_json.get("pad_vocab_size_multiple", 1) or 1)
    vocab += (-vocab) % mult
    kw: dict[str, Any] = {
        "d_model": int(cfg_json["d_model"]),
        "d_state": int(ssm.get("d_state", 128)),
        "headdim": int(ssm.get("headdim", 64)),
        "expand": int(ssm.get("expand", 2)),
        "rope_fraction": float(ssm.get("rope_fraction", 0.5)),
        "chunk": 128,
    }
    for src, dst in (("A_floor", "a_floor"), ("dt_min", "dt_min"), ("dt_max", "dt_max"),
                     ("dt_init_floor", "dt_init_floor")):
        if src in ssm:
            kw[dst] = float(ssm[src])
    kw.update({k: v for k, v in overrides.items() if k != "d_intermediate"})
    return M.LMConfig(vocab_size=vocab, n_layers=int(cfg_json["n_layer"]),
                      siso=SISOConfig(**kw), tie_head=bool(cfg_json.get("tie_embeddings", True)),
                      d_intermediate=int(cfg_json.get("d_intermediate", 0)))


def load_lm_state_dict(sd: Mapping[str, Any], cfg, dtype=torch.float32, device=None):
    """A released ``MambaLMHeadModel`` state dict -> `model.LMParams`
    (``convert.py:270-330``). Linear weights are transposed to ``(in, out)``; each mixer
    goes through `torch_to_jax`; bf16 tensors are widened on the torch side. Strict: a
    key the config implies but the dict lacks raises ``KeyError`` naming it, and an
    embedding whose width disagrees with the (padded) vocabulary raises ``ValueError``."""
    from . import model as M

    def get(key: str) -> np.ndarray:
        if key not in sd:
            raise KeyError(f"checkpoint is missing {key!r}")
        return _to_numpy(sd[key])

    def t(a):
        return torch.as_tensor(np.ascontiguousarray(a), dtype=dtype, device=device)

    embed = get("backbone.embedding.weight")
    if embed.shape != (cfg.vocab_size, cfg.d_model):
        raise ValueError(f"embedding is {embed.shape}, config implies "
                         f"{(cfg.vocab_size, cfg.d_model)}; check pad_vocab_size_multiple")
    blocks = []
    for i in range(cfg.n_layers):
        pre = MIXER_PREFIX.format(i=i)
        mixer = {k[len(pre):]: sd[k] for k in sd if k.startswith(pre)}
        if not mixer:
            raise KeyError(f"no keys under {pre!r}; is this a Mamba-3 checkpoint?")
        siso = torch_to_jax(mixer, cfg.siso, dtype, device)
        mlp = mlp_norm = None
        if cfg.d_intermediate:
            mlp = M.MLPParams(fc1=t(get(f"backbone.layers.{i}.mlp.fc1.weight").T),
                              fc2=t(get(f"backbone.layers.{i}.mlp.fc2.weight").T))
            mlp_norm = t(get(f"backbone.layers.{i}.norm2.weight"))
        blocks.append(M.BlockParams(norm_gain=t(get(f"backbone.layers.{i}.norm.weight")),
                                    siso=siso, mlp_norm_gain=mlp_norm, mlp=mlp))
    head = None if cfg.tie_head else t(get("lm_head.weight").T)
    return M.LMParams(embed=t(embed), blocks=blocks, final_norm=t(get("backbone.norm_f.weight")),
                      head=head)


def lm_state_dict(params, cfg) -> dict:
    """Inverse of `load_lm_state_dict`: `model.LMParams` -> a released-format state dict
    of float32 numpy arrays (``lm_head.weight`` is the embedding when the head is tied,
    as upstream's shared tensor is)."""
    sd: dict[str, np.ndarray] = {"backbone.embedding.weight": _to_numpy(params.embed)}
    for i, b in enumerate(params.blocks):
        pre = MIXER_PREFIX.format(i=i)
        for k, v in jax_to_torch(b.siso, cfg.siso).items():
            sd[pre + k] = v
        sd[f"backbone.layers.{i}.norm.weight"] = _to_numpy(b.norm_gain)
        if b.mlp is not None:
            sd[f"backbone.layers.{i}.norm2.weight"] = _to_numpy(b.mlp_norm_gain)
            sd[f"backbone.layers.{i}.mlp.fc1.weight"] = _to_numpy(b.mlp.fc1).T.copy()
            sd[f"backbone.layers.{i}.mlp.fc2.weight"] = _to_numpy(b.mlp.fc2).T.copy()
    sd["backbone.norm_f.weight"] = _to_numpy(params.final_norm)
    sd["lm_head.weight"] = (sd["backbone.embedding.weight"] if params.head is None
                            else _to_numpy(params.head).T.copy())
    return sd


def load_pretrained(path: str, dtype=torch.float32, device=None, **cfg_overrides):
    """A released checkpoint from a LOCAL directory -> ``(params, cfg)``
    (``convert.py:333-356`` without the Hub download). Reads ``config.json`` and
    ``model.safetensors`` (preferred) or ``pytorch_model.bin`` (loaded with
    ``weights_only=True``: no code in the file runs)."""
    if not os.path.isdir(path):
        raise ValueError(f"{path!r} is not a local checkpoint directory (no network here)")
    with open(os.path.join(path, "config.json")) as fh:
        cfg = config_from_hf(json.load(fh), **cfg_overrides)
    st = os.path.join(path, "model.safetensors")
    if os.path.exists(st):
        from safetensors.torch import load_file
        sd = load_file(st, device="cpu")
    else:
        sd = torch.load(os.path.join(path, "pytorch_model.bin"), map_location="cpu",
                        weights_only=True)
    return load_lm_state_dict(sd, cfg, dtype, device), cfg
