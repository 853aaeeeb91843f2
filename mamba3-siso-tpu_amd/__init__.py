"""MI355X-native Mamba-3 SISO selective-scan layer.

A drop-in for the reference's layer path (``mamba3_pallas``): the same
``SISOConfig`` / ``SISOParams`` / ``init_params`` / ``mamba3_siso_layer`` /
``SISOState`` / ``decode_step`` / ``convert`` surface, with the three hot kernels
(chunked forward, reverse-scan backward, single-token decode) hand-written in HIP
for gfx950 and loaded from ``csrc/libm3s.so`` through a C ABI.

torch is imported before the library so the library binds to the HIP runtime torch
already loaded (both carry the soname ``libamdhip64.so.7``).
"""

from __future__ import annotations

import torch  # noqa: F401  (must precede the C-ABI library load)

from . import layout  # noqa: F401
from .layout import BF16, F32, DtypePolicy, deinterleave_perm, interleave_perm, policy  # noqa: F401
