"""Module-name alias of ``mamba3_pallas.kernel_bwd``: the reverse-scan backward."""
from .kernels import KernelGrads, SISOGrads, siso_backward, siso_backward_kernel  # noqa: F401
