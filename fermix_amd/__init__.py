"""fermix_amd: batched fp32 slogdet / slogpf / det / pf on AMD Instinct MI355X
(gfx950) with hand-written HIP kernels behind a C ABI (include/fermix.h), keeping the
Python interface of ChenAo-Phys/fermix."""

from .api import FermixDeviceError, FermixFallbackWarning, FermixTuneWarning, det, pf, slogdet, slogpf

__all__ = [
    "slogdet",
    "slogpf",
    "det",
    "pf",
    "FermixFallbackWarning",
    "FermixDeviceError",
    "FermixTuneWarning",
]
