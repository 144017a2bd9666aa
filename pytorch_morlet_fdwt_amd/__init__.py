"""MI355X-native wavelet transforms for PyTorch-ROCm (drop-in for pytorch_morlet_fdwt).

* :func:`dwt`, :func:`idwt`, :func:`wavedec`, :func:`waverec`, :class:`DWT1D`,
  :class:`IDWT1D` -- Mallat fast wavelet transform (O(N)), PyWavelets-compatible.

Every operator runs hand-written HIP kernels for gfx950 (``libfdwt_hip.so``, C ABI in
``include/fdwt_hip.h``) on ROCm tensors; there is no CPU fallback.  Use
``import pytorch_morlet_fdwt_amd as fdwt`` in code written for the reference.
"""

from . import config
from .dwt import DWT1D, IDWT1D, dwt, dwt_max_level, idwt, wavedec, waverec
from .wavelets import FilterBank, get_filter_bank

__version__ = "0.1.0"

__all__ = [
    "config", "DWT1D", "IDWT1D", "dwt", "dwt_max_level", "idwt", "wavedec", "waverec",
    "FilterBank", "get_filter_bank",
]
