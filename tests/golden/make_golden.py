"""Write the golden fixtures under tests/golden/ from the reference's torch code.

Run in the build container only (the reference tree does not exist on the GPU box):

    python tests/golden/make_golden.py [/root/reference]

The reference's ``mamba3_pallas/torch_ref.py`` needs only torch, so it is loaded by
file path (its package ``__init__`` imports JAX, which is absent). Two upstream
functions are exercised on small seeded inputs and their inputs/outputs saved as
``.npz`` data:

* ``mamba3_siso_ref`` (``torch_ref.py:64-138``) -- upstream's three-term recurrent
  step reference at the kernel boundary, interleaved rotary layout;
* ``Mamba3SISOTorch.forward`` (``torch_ref.py:141-237``) -- the layer (in_proj split
  order, BCNorm, C-is-query / B-is-key, biases, D skip, gate, out_proj), with its
  ``state_dict``.

Only data is written; no reference source is copied.
"""

from __future__ import annotations

import importlib.util
import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def load_torch_ref(ref_root: Path):
    path = ref_root / "mamba3_pallas" / "torch_ref.py"
    spec = importlib.util.spec_from_file_location("_m3_torch_ref", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def kernel_case(tr, name, b, seqlen, h, n, p, nr, seed, with_dz=True):
    rng = np.random.default_rng(seed)

    def rn(*s):
        return rng.standard_normal(s).astype(np.float32)

    def norm_rows(x):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)

    q = norm_rows(rn(b, seqlen, n))
    k = norm_rows(rn(b, seqlen, n))
    v = rn(b, seqlen, h, p)
    z = rn(b, seqlen, h, p)
    # Larger dt than at init so decay and rotation both act within a few dozen steps.
    dt = np.exp(rng.uniform(math.log(0.01), math.log(0.5), (b, h, seqlen))).astype(np.float32)
    a_raw = rn(b, h, seqlen)
    a = -(np.maximum(a_raw, 0) + 1.0 / (1.0 - np.minimum(a_raw, 0)))
    a = np.minimum(a, -1e-4).astype(np.float32)
    adt = (a * dt).astype(np.float32)
    trap = rn(b, h, seqlen)
    angles = rn(b, seqlen, nr)
    q_bias = rn(h, n) * 0.1
    k_bias = rn(h, n) * 0.1
    d = rn(h)

    T = torch.from_numpy
    Q = T(q)[:, :, None, :].expand(b, seqlen, h, n).contiguous()
    K = T(k)[:, :, None, :].expand(b, seqlen, h, n).contiguous()
    Ang = T(angles)[:, :, None, :].expand(b, seqlen, h, nr).contiguous()
    out, (ang_s, ssm_s, k_s, v_s) = tr.mamba3_siso_ref(
        Q, K, T(v), T(adt), T(dt), T(trap), T(q_bias), T(k_bias), Ang,
        D=T(d) if with_dz else None, Z=T(z) if with_dz else None,
    )
    np.savez_compressed(
        HERE / f"{name}.npz",
        q=q, k=k, v=v, z=z, adt=adt, dt=dt, trap=trap, angles=angles,
        q_bias=q_bias, k_bias=k_bias, d=d, with_dz=np.array(with_dz),
        out=out.numpy(), angle_state=ang_s.numpy(), ssm_state=ssm_s.numpy(),
        k_state=k_s.numpy(), v_state=v_s.numpy(),
    )


def layer_case(tr, name, d_model, d_state, headdim, expand, rope_fraction, b, seqlen, seed):
    torch.manual_seed(seed)
    m = tr.Mamba3SISOTorch(d_model=d_model, d_state=d_state, headdim=headdim,
                           expand=expand, rope_fraction=rope_fraction)
    # The module initialises biases, norm gains and D to 1; perturb them so the
    # fixture exercises their placement and the rotary permutation of each.
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for pname in ("B_bias", "C_bias", "B_norm_weight", "C_norm_weight", "D"):
            prm = getattr(m, pname)
            prm.add_(0.3 * torch.randn(prm.shape, generator=g))
        m.dt_bias.add_(0.5)  # larger dt so the recurrence moves within 64 tokens
    u = (torch.randn(b, seqlen, d_model, generator=g) * 0.5).float()
    with torch.no_grad():
        y = m(u)
    sd = {k_: v_.detach().numpy() for k_, v_ in m.state_dict().items()}
    np.savez_compressed(
        HERE / f"{name}.npz", u=u.numpy(), y=y.numpy(),
        cfg=np.array([d_model, d_state, headdim, expand], np.int64),
        rope_fraction=np.array(rope_fraction),
        **{"sd__" + k_.replace(".", "__"): v_ for k_, v_ in sd.items()},
    )


def main(argv):
    ref_root = Path(argv[1] if len(argv) > 1 else "/root/reference")
    tr = load_torch_ref(ref_root)
    kernel_case(tr, "torch_ref_kernel_gated", b=2, seqlen=96, h=3, n=16, p=16, nr=4, seed=7)
    kernel_case(tr, "torch_ref_kernel_plain", b=1, seqlen=64, h=2, n=32, p=16, nr=16, seed=8,
                with_dz=False)
    layer_case(tr, "torch_ref_layer_half", d_model=32, d_state=16, headdim=16, expand=2,
               rope_fraction=0.5, b=2, seqlen=64, seed=11)
    layer_case(tr, "torch_ref_layer_full", d_model=32, d_state=16, headdim=16, expand=1,
               rope_fraction=1.0, b=1, seqlen=64, seed=12)
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main(sys.argv)
