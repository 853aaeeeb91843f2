"""Module-name alias of ``mamba3_pallas.kernel_fwd``: the chunked forward."""
from .kernels import ForwardResiduals, siso_forward  # noqa: F401
