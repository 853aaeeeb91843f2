"""MI355X-native Mamba-3 SISO selective-scan layer.

A drop-in for the reference's layer path (``mamba3_pallas``): the same
``SISOConfig`` / ``SISOParams`` / ``init_params`` / ``mamba3_siso_layer`` /
``SISOState`` / ``decode_step`` / ``convert`` surface, with the three hot kernels
(chunked forward, reverse-scan backward, single-token decode) hand-written in HIP
for gfx950 and loaded from ``csrc/libm3s.so`` through the C ABI of ``include/m3s.h``.

torch is imported before the library so the library binds to the HIP runtime torch
already loaded (both carry the soname ``libamdhip64.so.7``).
"""

from __future__ import annotations

import torch  # noqa: F401  (must precede the C-ABI library load)

from . import convert, kernels, layout  # noqa: F401
from . import kernel_bwd, kernel_decode, kernel_fwd  # noqa: F401
from . import checkpoint, model, train  # noqa: F401
from .kernels import (  # noqa: F401
    ForwardResiduals, KernelGrads, SISOGrads, decode_loop, decode_scan, decode_step,
    siso_backward, siso_backward_kernel, siso_decode, siso_decode_folded, siso_forward,
)
from .layer import (  # noqa: F401
    SISOConfig, SISOParams, init_params, mamba3_siso_decode_step, mamba3_siso_layer,
    rms_norm, split_in_proj,
)
from .layout import BF16, F32, DtypePolicy, deinterleave_perm, interleave_perm, policy  # noqa: F401
from .scan_prep import (  # noqa: F401
    Preprocessed, SISOState, cumulative_angles, heavy_tail, preprocess, trapezoid_coeffs,
    zero_state,
)
from .siso import SISOOutput, siso, siso_segment  # noqa: F401
