"""Module-name alias of ``mamba3_pallas.kernel_decode``: the single-token decode."""
from .kernels import (  # noqa: F401
    decode_loop, decode_scan, decode_step, siso_decode, siso_decode_folded,
)
