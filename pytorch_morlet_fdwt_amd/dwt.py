"""Fast (Mallat) discrete wavelet transform on MI355X (reference: src/fdwt/dwt.py).

The functional API mirrors PyWavelets (``dwt``, ``idwt``, ``wavedec``, ``waverec``) and the
reference package: the transform runs along the last dimension, every leading dimension is
a batch dimension, and coefficients are identical to ``pywt`` up to floating point rounding.

Every forward and backward is a hand-written HIP kernel (``csrc/dwt.hip``):

* one level: ``_Analysis`` / ``_Synthesis`` -- each is the other's backward (exact
  transposes), so double backward works like in the reference (dwt.py:36-82);
* several levels: ``_AnalysisChain`` / ``_SynthesisChain`` run all levels of ``wavedec`` /
  ``waverec`` in one launch with each row held in LDS; again each is the other's backward.
"""

from __future__ import annotations

import functools

from typing import List, Optional, Sequence, Tuple

import torch
from torch import nn

from . import _lib
from .wavelets import WaveletLike, get_filter_bank

__all__ = ["dwt", "idwt", "wavedec", "waverec", "dwt_max_level", "dwt_coeff_len", "DWT1D",
           "IDWT1D", "MODES"]

MODES = {"zero": 0, "periodic": 1, "symmetric": 2, "reflect": 3, "periodization": 4}
_PERIODIZATION = MODES["periodization"]
_SYN_MAX_LEVELS = 16  # FDWT_SYN_MAX_LEVELS: levels per fdwt_synthesis_chain launch
_ZERO = MODES["zero"]


def _compute_dtype(dtype: torch.dtype) -> torch.dtype:
    return torch.float64 if dtype == torch.float64 else torch.float32


def _check_dtype(x: torch.Tensor):
    if not x.is_floating_point():
        raise TypeError(f"expected a floating point tensor, got {x.dtype}")


def _rows(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(-1, t.shape[-1]).contiguous()


def _contig(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """The entry points take a data pointer and a row count: any contiguous layout of the rows
    will do, so only a non-contiguous tensor is copied (no reshape on the hot path)."""
    return t if t is None or t.is_contiguous() else t.contiguous()


# ----------------------------------------------------------------------------- launches
def _analysis(x2, h0, h1, mode, off, n_out):
    R, n = x2.shape
    y0 = torch.empty((R, n_out), device=x2.device, dtype=x2.dtype)
    y1 = torch.empty_like(y0)
    if R:
        _lib.launch("fdwt_dwt_analysis", x2.device,
                    _lib.ptr(x2), _lib.ptr(y0), _lib.ptr(y1), _lib.ptr(h0), _lib.ptr(h1), R, n,
                    n_out, h0.numel(), mode, off, _lib.dtype_code(x2.dtype),
                    _lib.stream(x2.device))
    return y0, y1


def _synthesis(a2, d2, h0, h1, mode, off, n, R, dtype, device):
    y = torch.empty((R, n), device=device, dtype=dtype)
    if R:
        nc = (a2 if a2 is not None else d2).shape[-1]
        _lib.launch("fdwt_dwt_synthesis", device,
                    _lib.ptr(a2), _lib.ptr(d2), _lib.ptr(y), _lib.ptr(h0), _lib.ptr(h1), R, nc, n,
                    h0.numel(), mode, off, _lib.dtype_code(dtype), _lib.stream(device))
    return y


@functools.lru_cache(maxsize=None)
@functools.lru_cache(maxsize=None)
def _chain_max(taps: int, dtype) -> int:
    return _lib.lib().fdwt_chain_max_length(taps, _lib.dtype_code(dtype))


def _chain_fits(n: int, taps: int, dtype) -> bool:
    return n <= _chain_max(taps, dtype)


def _one_launch(levels: int, n: int, taps: int, dtype):
    """The C++ autograd nodes when a chain of ``levels`` over rows of ``n`` samples and its
    transpose both run as one launch (the common case), else None (dwt.py's Functions, which
    split long rows and deep chains into several launches)."""
    if levels > _SYN_MAX_LEVELS or (levels > 1 and not _chain_fits(n, taps, dtype)):
        return None
    return _lib.ext()


def _analysis_chain(x2, h0, h1, mode, off, n_in, n_out, lead=None):
    """Levels l = 0..J-1 of an analysis chain on the contiguous rows of x2 (any shape
    (*lead, n_in[0])).  Returns (details, approx), shaped (*lead, n) when the whole chain is one
    launch (2-D (R, n) otherwise).  Rows too long for LDS run their first levels one at a time."""
    lead = tuple(x2.shape[:-1]) if lead is None else lead
    R = x2.numel() // x2.shape[-1] if x2.shape[-1] else 0
    J = len(n_in)
    taps = h0.numel()
    details = [None] * J
    l = 0
    cur = x2
    while l < J and J - l > 1 and not _chain_fits(n_in[l], taps, x2.dtype):
        cur = cur.reshape(R, cur.shape[-1])
        if cur.shape[-1] < n_in[l]:
            cur = torch.nn.functional.pad(cur, (0, n_in[l] - cur.shape[-1]))
        cur, details[l] = _analysis(cur, h0, h1, mode, off, n_out[l])
        l += 1
    if l < J:
        if cur.shape[-1] < n_in[l]:
            cur = torch.nn.functional.pad(cur, (0, n_in[l] - cur.shape[-1]))
        shp = lead if l == 0 else (R,)
        outs = [torch.empty((*shp, n_out[k]), device=x2.device, dtype=x2.dtype)
                for k in range(l, J)]
        approx = torch.empty((*shp, n_out[J - 1]), device=x2.device, dtype=x2.dtype)
        if R:
            _lib.launch("fdwt_analysis_chain", x2.device,
                        _lib.ptr(cur), _lib.ptr_array(outs), _lib.ptr(approx), _lib.ptr(h0),
                        _lib.ptr(h1), R, _lib.i64_array(n_in[l:]), _lib.i64_array(n_out[l:]),
                        J - l, taps, mode, off, _lib.dtype_code(x2.dtype),
                        _lib.stream(x2.device))
        details[l:] = outs
        cur = approx
    return details, cur


def _synthesis_chain(a2, ds, h0, h1, mode, off, nc, n_out, R, dtype, device, lead=None):
    """Levels k = 0..K-1 (coarsest first) of a synthesis chain on contiguous bands (any shape
    with R rows).  a2 / ds[k] may be None.  The output is shaped (*lead, n_out[-1]) when the
    last level runs in the chain (2-D (R, n) otherwise, or when lead is None)."""
    K = len(nc)
    taps = h0.numel()
    # the chain keeps every output but the last on chip: run it while that fits, then the
    # remaining (long) levels one at a time
    k_end = K
    while k_end > 1 and not _chain_fits(n_out[k_end - 1], taps, dtype):
        k_end -= 1
    cur = None
    # at most _SYN_MAX_LEVELS levels per launch; a later group starts from the first nc[g0]
    # samples of the previous group's output
    for g0 in range(0, k_end, _SYN_MAX_LEVELS):
        g1 = min(k_end, g0 + _SYN_MAX_LEVELS)
        a_in = a2 if g0 == 0 else cur[:, :nc[g0]].contiguous()
        shp = lead if (lead is not None and g1 == K) else (R,)
        cur = torch.empty((*shp, n_out[g1 - 1]), device=device, dtype=dtype)
        if R:
            _lib.launch("fdwt_synthesis_chain", device,
                        _lib.ptr(a_in), _lib.ptr_array(ds[g0:g1]), _lib.ptr(cur), _lib.ptr(h0),
                        _lib.ptr(h1), R, _lib.i64_array(nc[g0:g1]),
                        _lib.i64_array(n_out[g0:g1]), g1 - g0, taps, mode, off,
                        _lib.dtype_code(dtype), _lib.stream(device))
    for k in range(k_end, K):
        a = cur[:, :nc[k]].contiguous()
        cur = _synthesis(a, ds[k], h0, h1, mode, off, n_out[k], R, dtype, device)
    return cur


# ----------------------------------------------------------------------------- autograd
class _Analysis(torch.autograd.Function):
    """(y0, y1) = A x ; backward = A^T, implemented by :class:`_Synthesis` (dwt.py:36-56)."""

    @staticmethod
    def forward(ctx, x, h0, h1, mode: int, off: int, n_out: int):
        _lib.require_gpu(x)
        ctx.save_for_backward(h0, h1)
        ctx.cfg = (mode, off, x.shape[-1])
        lead = x.shape[:-1]
        y0, y1 = _analysis(_rows(x), h0, h1, mode, off, n_out)
        return y0.reshape(*lead, n_out), y1.reshape(*lead, n_out)

    @staticmethod
    def backward(ctx, g0, g1):
        h0, h1 = ctx.saved_tensors
        mode, off, n = ctx.cfg
        gx = None
        if ctx.needs_input_grad[0]:
            if g0 is None:
                g0 = torch.zeros_like(g1)
            if g1 is None:
                g1 = torch.zeros_like(g0)
            gx = _Synthesis.apply(g0, g1, h0, h1, mode, off, n)
        return gx, None, None, None, None, None


class _Synthesis(torch.autograd.Function):
    """y = A^T (a, d) ; backward = A, implemented by :class:`_Analysis` (dwt.py:59-82)."""

    @staticmethod
    def forward(ctx, a, d, h0, h1, mode: int, off: int, n: int):
        _lib.require_gpu(a, d)
        ctx.save_for_backward(h0, h1)
        ctx.cfg = (mode, off, a.shape[-1])
        lead = a.shape[:-1]
        a2, d2 = _rows(a), _rows(d)
        y = _synthesis(a2, d2, h0, h1, mode, off, n, a2.shape[0], a.dtype, a.device)
        return y.reshape(*lead, n)

    @staticmethod
    def backward(ctx, gy):
        h0, h1 = ctx.saved_tensors
        mode, off, nc = ctx.cfg
        ga, gd = None, None
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
            ga, gd = _Analysis.apply(gy, h0, h1, mode, off, nc)
        return ga, gd, None, None, None, None, None


class _AnalysisChain(torch.autograd.Function):
    """All levels of an analysis chain in one node: returns (d_0, ..., d_{J-1}, a_J).
    Backward is :class:`_SynthesisChain` with the transposed level parameters."""

    @staticmethod
    def run(x, h0, h1, mode: int, off: int, n_in: tuple, n_out: tuple):
        """The transform itself (no autograd node)."""
        _lib.require_gpu(x)
        lead = tuple(x.shape[:-1])
        details, approx = _analysis_chain(_contig(x), h0, h1, mode, off, n_in, n_out, lead)
        nd = len(lead) + 1
        outs = [d if d.dim() == nd else d.reshape(*lead, d.shape[-1]) for d in details]
        outs.append(approx if approx.dim() == nd else approx.reshape(*lead, approx.shape[-1]))
        return tuple(outs)

    @staticmethod
    def forward(ctx, x, h0, h1, mode: int, off: int, n_in: tuple, n_out: tuple):
        ctx.save_for_backward(h0, h1)
        ctx.cfg = (mode, off, n_in, n_out)
        return _AnalysisChain.run(x, h0, h1, mode, off, n_in, n_out)

    @staticmethod
    def backward(ctx, *grads):
        h0, h1 = ctx.saved_tensors
        mode, off, n_in, n_out = ctx.cfg
        if not ctx.needs_input_grad[0]:
            return (None,) * 7
        gd, ga = list(grads[:-1]), grads[-1]
        # transpose: coarsest level first; nc = n_out[l], output length = n_in[l].  A graph
        # node only when the backward itself is differentiated (create_graph=True)
        args = (h0, h1, mode, off, tuple(n_out[::-1]), tuple(n_in[::-1]), ga, *gd[::-1])
        gx = (_SynthesisChain.apply(*args) if torch.is_grad_enabled()
              else _SynthesisChain.run(*args))
        return gx, None, None, None, None, None, None


class _SynthesisChain(torch.autograd.Function):
    """All levels of a synthesis chain in one node (coarsest first).  Inputs: the coarsest
    low band ``a`` and the high bands ``ds`` (any may be None = zeros).  Backward is
    :class:`_AnalysisChain` with the transposed level parameters."""

    @staticmethod
    def forward(ctx, h0, h1, mode: int, off: int, nc: tuple, n_out: tuple, a, *ds):
        ctx.save_for_backward(h0, h1)
        ctx.cfg = (mode, off, nc, n_out)
        ctx.n_ds = len(ds)
        return _SynthesisChain.run(h0, h1, mode, off, nc, n_out, a, *ds)

    @staticmethod
    def run(h0, h1, mode: int, off: int, nc: tuple, n_out: tuple, a, *ds):
        """The transform itself (no autograd node)."""
        ref = a if a is not None else next(d for d in ds if d is not None)
        _lib.require_gpu(a, *ds)
        lead = ref.shape[:-1]
        R = 1
        for s in lead:
            R *= s
        y = _synthesis_chain(_contig(a), [_contig(d) for d in ds], h0, h1, mode, off, nc, n_out,
                             R, ref.dtype, ref.device, tuple(lead))
        return y if y.dim() == len(lead) + 1 else y.reshape(*lead, n_out[-1])

    @staticmethod
    def backward(ctx, gy):
        h0, h1 = ctx.saved_tensors
        mode, off, nc, n_out = ctx.cfg
        if not any(ctx.needs_input_grad[6:]):
            return (None,) * (7 + ctx.n_ds)
        args = (gy, h0, h1, mode, off, tuple(n_out[::-1]), tuple(nc[::-1]))
        outs = (_AnalysisChain.apply(*args) if torch.is_grad_enabled()
                else _AnalysisChain.run(*args))
        gds = list(outs[:-1])[::-1]  # coarsest first
        return (None,) * 6 + (outs[-1],) + tuple(gds)


# ----------------------------------------------------------------------------- API
def _mode_id(mode: str) -> int:
    try:
        return MODES[mode]
    except (KeyError, TypeError):
        raise ValueError(f"unsupported mode '{mode}', expected one of {sorted(MODES)}") from None


def _bank(wavelet, x: torch.Tensor):
    bank = get_filter_bank(wavelet)
    return bank, bank.tensors(x.device, _compute_dtype(x.dtype))


def dwt_coeff_len(n: int, filter_len: int, mode: str) -> int:
    """dwt.py:97-100."""
    if mode == "periodization":
        return (n + 1) // 2
    return (n + filter_len - 1) // 2


def _check_length(n: int):
    if n < 1:
        raise ValueError("the signal must have at least one sample along the last dimension")


def dwt(x: torch.Tensor, wavelet: WaveletLike = "db4", mode: str = "symmetric"
        ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Single level DWT along the last dimension. Returns ``(cA, cD)`` like ``pywt.dwt``."""
    _check_dtype(x)
    m = _mode_id(mode)
    bank, f = _bank(wavelet, x)
    L = bank.length
    _check_length(x.shape[-1])
    off = L // 2 if m == _PERIODIZATION else 1
    return _Analysis.apply(x, f["dec_lo"], f["dec_hi"], m, off, dwt_coeff_len(x.shape[-1], L, mode))


def _idwt_geometry(m: int, L: int, nc: int):
    """dwt.py:127-134: idwt is the transpose of a periodized analysis, or of a zero-padded
    one cropped to 2 nc - L + 2."""
    if m == _PERIODIZATION:
        return _PERIODIZATION, 2 * nc, L // 2
    n = 2 * nc - L + 2
    if n <= 0:
        raise ValueError(f"coefficients of length {nc} are too short for a filter of length {L}")
    return _ZERO, n, 1


def idwt(cA: Optional[torch.Tensor], cD: Optional[torch.Tensor], wavelet: WaveletLike = "db4",
         mode: str = "symmetric") -> torch.Tensor:
    """Single level inverse DWT, identical to ``pywt.idwt``."""
    if cA is None and cD is None:
        raise ValueError("at least one of cA, cD must be given")
    cA = torch.zeros_like(cD) if cA is None else cA
    cD = torch.zeros_like(cA) if cD is None else cD
    if cA.shape != cD.shape:
        raise ValueError(f"cA and cD shapes differ: {tuple(cA.shape)} vs {tuple(cD.shape)}")
    _check_dtype(cA)
    m = _mode_id(mode)
    bank, f = _bank(wavelet, cA)
    L, nc = bank.length, cA.shape[-1]
    _check_length(nc)
    m, n, off = _idwt_geometry(m, L, nc)
    return _Synthesis.apply(cA, cD.to(cA.dtype), f["rec_lo_rev"], f["rec_hi_rev"], m, off, n)


def dwt_max_level(n: int, wavelet: WaveletLike = "db4") -> int:
    """Same as ``pywt.dwt_max_level`` (dwt.py:138-143)."""
    L = get_filter_bank(wavelet).length
    if L < 2 or n < L - 1:
        return 0
    return (n // (L - 1)).bit_length() - 1


def wavedec(x: torch.Tensor, wavelet: WaveletLike = "db4", mode: str = "symmetric",
            level: Optional[int] = None) -> List[torch.Tensor]:
    """Multilevel DWT: ``[cA_n, cD_n, ..., cD_1]`` exactly like ``pywt.wavedec``.
    All levels run in one fused launch (``_AnalysisChain``)."""
    if level is None:
        level = dwt_max_level(x.shape[-1], wavelet)
    if level < 0:
        raise ValueError("level must be >= 0")
    _check_dtype(x)
    m = _mode_id(mode)
    if level == 0:
        return [x]
    bank, f = _bank(wavelet, x)
    L = bank.length
    _check_length(x.shape[-1])
    off = L // 2 if m == _PERIODIZATION else 1
    n_in, n_out = [], []
    n = x.shape[-1]
    for _ in range(level):
        n_in.append(n)
        n = dwt_coeff_len(n, L, mode)
        n_out.append(n)
    fast = _one_launch(level, x.shape[-1], L, x.dtype)
    if fast is not None:
        outs = fast.analysis_chain(x, f["dec_lo"], f["dec_hi"], m, off, n_in, n_out)
    else:
        outs = _AnalysisChain.apply(x, f["dec_lo"], f["dec_hi"], m, off, tuple(n_in),
                                    tuple(n_out))
    return [outs[-1]] + list(outs[:-1])[::-1]


def waverec(coeffs: Sequence[torch.Tensor], wavelet: WaveletLike = "db4",
            mode: str = "symmetric") -> torch.Tensor:
    """Inverse of :func:`wavedec`, like ``pywt.waverec`` (same trimming rule, dwt.py:161-171).
    All levels run in one fused launch (``_SynthesisChain``)."""
    if len(coeffs) == 0:
        raise ValueError("coeffs must not be empty")
    a = coeffs[0]
    if len(coeffs) == 1:
        return a
    m = _mode_id(mode)
    ref = a if a is not None else next(c for c in coeffs[1:] if c is not None)
    _check_dtype(ref)
    bank, f = _bank(wavelet, ref)
    L = bank.length
    nc, n_out = [], []
    cur = a.shape[-1] if a is not None else coeffs[1].shape[-1]
    for d in coeffs[1:]:
        dn = d.shape[-1]
        if cur == dn + 1:
            cur = dn
        if cur != dn:
            raise ValueError(f"cA and cD shapes differ: {cur} vs {dn}")
        if d.shape[:-1] != ref.shape[:-1]:
            raise ValueError("all coefficient arrays must share their leading dimensions")
        mm, n, off = _idwt_geometry(m, L, dn)
        nc.append(dn)
        n_out.append(n)
        cur = n
    mm = _PERIODIZATION if m == _PERIODIZATION else _ZERO
    off = L // 2 if m == _PERIODIZATION else 1
    # a low band one sample longer than its detail is trimmed (its gradient gets a zero)
    if a is not None and a.shape[-1] == nc[0] + 1:
        a = a[..., :-1]
    ds = [d.to(ref.dtype) if d is not None else None for d in coeffs[1:]]
    fast = _one_launch(len(nc), n_out[-1], L, ref.dtype)
    if fast is not None:
        return fast.synthesis_chain(f["rec_lo_rev"], f["rec_hi_rev"], mm, off, nc, n_out, a, ds)
    return _SynthesisChain.apply(f["rec_lo_rev"], f["rec_hi_rev"], mm, off, tuple(nc),
                                 tuple(n_out), a, *ds)


class DWT1D(nn.Module):
    """Multilevel 1D DWT along the last dimension (dwt.py:174-192).

    ``forward(x)`` returns ``[cA_J, cD_J, ..., cD_1]`` (PyWavelets ordering).
    """

    def __init__(self, wavelet: WaveletLike = "db4", level: Optional[int] = None,
                 mode: str = "symmetric"):
        super().__init__()
        _mode_id(mode)
        self.bank = get_filter_bank(wavelet)
        self.level = level
        self.mode = mode

    def forward(self, x: torch.Tensor) -> List[torch.Tensor]:
        return wavedec(x, self.bank, self.mode, self.level)

    def extra_repr(self) -> str:
        return f"wavelet={self.bank.name}, level={self.level}, mode={self.mode}"


class IDWT1D(nn.Module):
    """Inverse of :class:`DWT1D` (dwt.py:195-208)."""

    def __init__(self, wavelet: WaveletLike = "db4", mode: str = "symmetric"):
        super().__init__()
        _mode_id(mode)
        self.bank = get_filter_bank(wavelet)
        self.mode = mode

    def forward(self, coeffs: Sequence[torch.Tensor]) -> torch.Tensor:
        return waverec(coeffs, self.bank, self.mode)

    def extra_repr(self) -> str:
        return f"wavelet={self.bank.name}, mode={self.mode}"
