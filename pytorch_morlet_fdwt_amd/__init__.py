"""``pytorch_morlet_fdwt_amd`` -- the fdwt filter-bank transforms as hand-written HIP
kernels for MI355X (gfx950), behind the same Python names as ``pytorch_morlet_fdwt``.

What it provides:

* discrete wavelet transforms with PyWavelets semantics -- single level (``dwt`` /
  ``idwt``), multilevel (``wavedec`` / ``waverec``, every level fused into one kernel
  launch per direction) and their modules ``DWT1D`` / ``IDWT1D``;
* the Morlet continuous wavelet transform (``cwt``, ``CWT1D``; plans through
  ``MorletPlan``, frequency/scale conversion helpers), computed octave by octave;
* sequence layers built on both: ``MorletTokenMixer`` and ``WaveletTokenMixer`` for
  (batch, length, dim) tokens, ``MorletAttention`` and ``MorletChannelMixAttention`` for
  (B, H, C, T, D) patch tokens, where the scalogram is reduced on chip and never stored.

Tensors must live on a ROCm device: the kernels in ``libfdwt_hip.so`` (C ABI in
``include/fdwt_hip.h``) are the only implementation, and a missing library or a CPU tensor
raises instead of falling back.  Existing code switches with
``import pytorch_morlet_fdwt_amd as fdwt``.
"""

from . import config
from .cwt import CWT1D, MorletPlan, cwt, freqs_to_scales, scales_to_freqs
from .dwt import DWT1D, IDWT1D, dwt, dwt_max_level, idwt, wavedec, waverec
from .layers import (MorletAttention, MorletChannelMixAttention, MorletTokenMixer,
                     WaveletTokenMixer)
from .wavelets import FilterBank, get_filter_bank

__version__ = "0.1.0"

__all__ = [
    "config", "CWT1D", "MorletPlan", "cwt", "freqs_to_scales", "scales_to_freqs",
    "DWT1D", "IDWT1D", "dwt", "dwt_max_level", "idwt", "wavedec", "waverec",
    "MorletAttention", "MorletChannelMixAttention", "MorletTokenMixer", "WaveletTokenMixer",
    "FilterBank", "get_filter_bank",
]
