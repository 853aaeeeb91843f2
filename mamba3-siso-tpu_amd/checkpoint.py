"""Save and load LM weights as a self-describing ``.npz`` (``checkpoint.py`` surface).

One npz entry per tensor under a readable name (``embed``, ``blocks.0.norm_gain``,
``blocks.0.siso.in_proj``, ``blocks.0.mlp.fc1``, ``final_norm``, ``head``; absent leaves
are skipped) plus ``__config__``: the UTF-8 JSON of the `model.LMConfig` and each
array's dtype name. No pickle: loading never runs code from the file. Arrays are in the
tree's own layout (linears ``(in, out)``, state-axis tensors permuted), so files are
interchangeable with the reference's format (``checkpoint.py:38-204``).

bfloat16 has no numpy dtype: such arrays are written as 2-byte void (``|V2``) holding the
raw bf16 bits, with ``"bfloat16"`` recorded in the JSON, and `load` reinterprets them --
the same on-disk representation the reference's writer produces.
"""

from __future__ import annotations

import dataclasses
import json
from typing import Any

import numpy as np
import torch

from . import layer as LY
from . import model as M

#: Bumped if the on-disk layout changes in a way old readers cannot handle.
FORMAT_VERSION = 1

#: The npz entry holding the JSON config (not a valid leaf name, so it cannot collide).
CONFIG_KEY = "__config__"

_NP_FLOAT = {torch.float32: np.float32, torch.float64: np.float64, torch.float16: np.float16}


def _named_leaves(params: M.LMParams) -> list:
    """``(name, tensor)`` for every present leaf, in tree order (``checkpoint.py:44-66``
    names: attribute names and list indices joined by dots)."""
    out = [("embed", params.embed)]
    for i, b in enumerate(params.blocks):
        out.append((f"blocks.{i}.norm_gain", b.norm_gain))
        out.extend((f"blocks.{i}.siso.{f}", getattr(b.siso, f)) for f in LY.SISOParams._fields)
        if b.mlp_norm_gain is not None:
            out.append((f"blocks.{i}.mlp_norm_gain", b.mlp_norm_gain))
        if b.mlp is not None:
            out.extend(((f"blocks.{i}.mlp.fc1", b.mlp.fc1), (f"blocks.{i}.mlp.fc2", b.mlp.fc2)))
    out.append(("final_norm", params.final_norm))
    if params.head is not None:
        out.append(("head", params.head))
    return out


def config_to_dict(cfg: M.LMConfig) -> dict:
    """`model.LMConfig` -> JSON-safe dict (``checkpoint.py:68-91``)."""
    return {"format_version": FORMAT_VERSION, "vocab_size": cfg.vocab_size,
            "n_layers": cfg.n_layers, "tie_head": cfg.tie_head,
            "d_intermediate": cfg.d_intermediate,
            "siso": {f.name: getattr(cfg.siso, f.name) for f in dataclasses.fields(LY.SISOConfig)}}


def config_from_dict(d: dict) -> M.LMConfig:
    """Inverse of `config_to_dict` (``checkpoint.py:94-116``). ``siso`` entries that
    `SISOConfig` does not define are ignored and absent ones keep its defaults, so files
    from a writer with more (or fewer) config fields still load. A file whose layout
    version is above `FORMAT_VERSION` is refused."""
    version = int(d.get("format_version", 0))
    if version > FORMAT_VERSION:
        raise ValueError(f"unsupported checkpoint layout v{version} (this reader handles "
                         f"layouts up to v{FORMAT_VERSION})")
    defined = LY.SISOConfig.__dataclass_fields__
    siso = LY.SISOConfig(**{k: d["siso"][k] for k in defined if k in d["siso"]})
    top = dict(vocab_size=int(d["vocab_size"]), n_layers=int(d["n_layers"]),
               tie_head=bool(d["tie_head"]), d_intermediate=int(d.get("d_intermediate", 0)))
    return M.LMConfig(siso=siso, **top)


def _to_array(t: torch.Tensor, dtype) -> tuple[np.ndarray, str]:
    t = t.detach().to("cpu")
    if dtype is not None:
        t = t.to(dtype)
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.dtype("V2")), "bfloat16"
    if t.dtype not in _NP_FLOAT:
        raise ValueError(f"cannot store dtype {t.dtype}")
    a = t.contiguous().numpy()
    return a, str(a.dtype)


def _from_array(a: np.ndarray, stored: str) -> torch.Tensor:
    if a.dtype.kind == "V" or stored == "bfloat16":
        if stored != "bfloat16" or a.dtype.itemsize != 2:
            raise ValueError(f"opaque array of {a.dtype} recorded as {stored!r}")
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a).copy())


def save(path: str, params: M.LMParams, cfg: M.LMConfig, dtype: Any = None) -> str:
    """Write ``params`` and ``cfg`` to ``path`` (``checkpoint.py:130-163``). ``dtype``
    (e.g. ``torch.bfloat16``, which halves the file) casts every array first. Returns the
    path written (numpy appends ``.npz`` when missing)."""
    arrays: dict[str, np.ndarray] = {}
    dtypes: dict[str, str] = {}
    for name, leaf in _named_leaves(params):
        arrays[name], dtypes[name] = _to_array(leaf, dtype)
    meta = {**config_to_dict(cfg), "dtypes": dtypes}
    arrays[CONFIG_KEY] = np.frombuffer(json.dumps(meta).encode("utf-8"), dtype=np.uint8)
    np.savez(path, **arrays)
    return path if path.endswith(".npz") else path + ".npz"


def _manifest_problems(files: set, expected: dict) -> list:
    """What keeps an npz's arrays from matching the tree its config implies: expected
    names it lacks, then names it has beyond those, as readable strings."""
    lacking = [n for n in expected if n not in files]
    surplus = sorted(files - set(expected) - {CONFIG_KEY})
    out = [f"is missing array {n!r}" for n in lacking]
    if surplus:
        out.append(f"holds arrays the config does not define (unexpected arrays): {surplus}")
    return out


def load(path: str, dtype: Any = None, device=None) -> tuple:
    """Read a checkpoint written by `save` -> ``(params, cfg)`` (``checkpoint.py:166-204``).
    The file's own config rebuilds the tree (`model.lm_template`); the arrays must be
    exactly that tree's leaves, each of its leaf's shape, else ``ValueError``. ``dtype``
    casts on load (``torch.float32`` widens a bf16 file)."""
    with np.load(path, allow_pickle=False) as z:
        files = set(z.files)
        if CONFIG_KEY not in files:
            raise ValueError(f"{path}: no {CONFIG_KEY} record, so this npz is not a "
                             f"Mamba-3 SISO checkpoint")
        meta = json.loads(bytes(z[CONFIG_KEY]).decode("utf-8"))
        cfg = config_from_dict(meta)
        template = M.lm_template(cfg)
        expected = dict(_named_leaves(template))
        problems = _manifest_problems(files, expected)
        if problems:
            raise ValueError(f"{path} " + "; ".join(problems))
        recorded = meta.get("dtypes", {})
        tensors: dict[str, torch.Tensor] = {}
        for name, leaf in expected.items():
            arr = z[name]
            if arr.shape != tuple(leaf.shape):
                raise ValueError(f"array {name!r} is {arr.shape} on disk but {tuple(leaf.shape)} "
                                 f"under the stored config (shape mismatch)")
            t = _from_array(arr, recorded.get(name, str(arr.dtype)))
            tensors[name] = t.to(device=device, dtype=dtype) if (dtype or device) else t
    by_id = {id(leaf): name for name, leaf in expected.items()}
    return M.lm_map(lambda leaf: tensors[by_id[id(leaf)]], template), cfg
