"""Continuous wavelet transform with the (complex) Morlet wavelet on MI355X
(reference: src/fdwt/cwt.py).

    W[s, n] = sum_m x[m] * conj(psi((m - n) / s)) / norm(s)
    psi(t)  = pi^(-1/4) * (exp(i*w0*t) - exp(-w0^2/2)) * exp(-t^2/2)

``norm(s)`` is ``sqrt(s)`` (``norm="l2"``) or ``s`` (``norm="l1"``).  The signal is zero
padded and the Gaussian envelope is truncated at ``truncate`` standard deviations.

``method="fast"`` (default) is the octave pyramid ("algorithme a trous"): octave j
convolves a half-band low-passed copy x_j of the signal with Morlet filters dilated by 2^j,
so every filter keeps O(1) taps.  ``method="direct"`` is the exact sampled convolution (a
single octave) and ``method="fft"`` applies the direct filters through torch.fft.

``fast`` and ``direct`` run hand-written HIP kernels (``csrc/cwt.hip``) for the forward,
the input gradient and the filter gradient; the fused ``morlet_mix`` (MorletTokenMixer) and
``spectral_softmax`` (MorletAttention) never store the scalogram.  The octave plan, the
half-band design and the filter synthesis follow the reference exactly (cwt.py:54-203), so
results agree with it to floating point rounding.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from functools import lru_cache
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch
from torch import nn

from . import _lib
from .config import resolve_precision

__all__ = ["cwt", "CWT1D", "MorletPlan", "freqs_to_scales", "scales_to_freqs", "morlet_mix",
           "spectral_softmax"]

_PI_M14 = math.pi ** -0.25
_MAX_FILTERS = 256  # FDWT_MORLET_MAX_FILTERS
_MAX_STAGE_SCALES = 64  # FDWT_CWT_MAX_SCALES


def freqs_to_scales(freqs, fs: float = 1.0, w0: float = 6.0) -> torch.Tensor:
    """Scale (in samples) whose Morlet centre frequency is ``freqs`` (cwt.py:54-57)."""
    f = torch.as_tensor(freqs, dtype=torch.float64)
    return w0 * fs / (2 * math.pi * f)


def scales_to_freqs(scales, fs: float = 1.0, w0: float = 6.0) -> torch.Tensor:
    s = torch.as_tensor(scales, dtype=torch.float64)
    return w0 * fs / (2 * math.pi * s)


def _halfband(c: int, beta: float) -> torch.Tensor:
    """Kaiser-windowed half-band low-pass, unit DC gain (cwt.py:65-68)."""
    n = torch.arange(-c, c + 1, dtype=torch.float64)
    h = 0.5 * torch.sinc(n / 2) * torch.from_numpy(np.kaiser(2 * c + 1, beta))
    return h / h.sum()


@dataclass
class _Stage:
    octave: int
    dil: int                # filter dilation 2**octave
    scale_idx: List[int]    # global scale indices, sorted by support
    half: int               # filters have 2*half+1 taps (at spacing `dil`)
    support: List[int]      # per scale half-support (taps)


class MorletPlan:
    """Static description of a Morlet CWT: scale grouping, filter sizes and margins
    (reference cwt.py:80-139).  Depends only on the initial scales, so it is built once and
    reused while learnable scales evolve."""

    def __init__(self, scales: Sequence[float], w0: float = 6.0, truncate: float = 4.0,
                 norm: str = "l2", complex: bool = True, method: str = "fast",
                 support_margin: float = 1.0):
        if method not in ("fast", "direct", "fft"):
            raise ValueError(f"unknown method '{method}' (expected 'fast', 'direct' or 'fft')")
        if norm not in ("l1", "l2"):
            raise ValueError("norm must be 'l1' or 'l2'")
        scales = [float(s) for s in scales]
        if not scales or min(scales) <= 0:
            raise ValueError("scales must be a non-empty sequence of positive numbers")
        self.scales, self.w0, self.truncate, self.norm = scales, float(w0), float(truncate), norm
        self.complex, self.method = bool(complex), method
        self.channels = 2 if complex else 1
        reach = truncate * support_margin

        # octave j holds the scales in [2^j s_th, 2^(j+1) s_th)
        self.s_th = (w0 + truncate) / (0.8 * math.pi)
        groups: Dict[int, List[int]] = {}
        for i, s in enumerate(scales):
            j = 0 if method != "fast" else max(0, math.floor(math.log2(s / self.s_th)))
            groups.setdefault(j, []).append(i)
        self.stages: List[_Stage] = []
        for j in sorted(groups):
            dil = 2 ** j
            sup = {i: max(1, math.ceil(reach * scales[i] / dil)) for i in groups[j]}
            idx = sorted(groups[j], key=lambda i: sup[i])
            self.stages.append(_Stage(j, dil, idx, max(sup.values()), [sup[i] for i in idx]))
        self.n_octaves = self.stages[-1].octave + 1
        self.center = max(st.half for st in self.stages)
        self._dil = [0.0] * len(scales)
        self._sup = [0.0] * len(scales)
        for st in self.stages:
            for i, c in zip(st.scale_idx, st.support):
                self._dil[i], self._sup[i] = float(st.dil), float(c)

        c_lp, beta = (16, 8.0) if truncate <= 4.5 else (24, 10.0)
        self.lowpass = _halfband(c_lp, beta) if self.n_octaves > 1 else torch.zeros(1, dtype=torch.float64)
        self.c_lp = c_lp if self.n_octaves > 1 else 0

        # x_j (j >= 1) lives on [-M_j, N + M_j) so that coarse octaves see the zero padded
        # signal exactly; x_0 is the input itself
        J = self.n_octaves - 1
        by_oct = {st.octave: st for st in self.stages}
        self.margins = [0] * (J + 1)
        for j in range(J, 0, -1):
            own = by_oct[j].half * 2 ** j if j in by_oct else 0
            nxt = self.margins[j + 1] + self.c_lp * 2 ** j if j < J else 0
            self.margins[j] = max(own, nxt)
        self._cache: Dict = {}

    @property
    def num_scales(self) -> int:
        return len(self.scales)

    def stage_rows(self, k: int) -> List[int]:
        """Rows of stage k in the filter tensor (row i*C + c in user scale order)."""
        st = self.stages[k]
        return [i * self.channels + c for i in st.scale_idx for c in range(self.channels)]

    def filter_geometry(self):
        """Per-scale dilation and half support as ctypes int32 arrays (filter kernels), one
        pair per chunk of at most FDWT_MORLET_MAX_FILTERS scales: [(i0, i1, dil, sup)]."""
        if "geom" not in self._cache:
            S = self.num_scales
            self._cache["geom"] = [
                (i0, min(S, i0 + _MAX_FILTERS),
                 _i32([int(d) for d in self._dil[i0:i0 + _MAX_FILTERS]]),
                 _i32([int(c) for c in self._sup[i0:i0 + _MAX_FILTERS]]))
                for i0 in range(0, S, _MAX_FILTERS)]
        return self._cache["geom"]

    def w0_device(self, w0, device: torch.device) -> torch.Tensor:
        """w0 as a float64 device scalar (a tensor is converted on the device, no sync)."""
        if isinstance(w0, torch.Tensor):
            return w0.detach().to(device=device, dtype=torch.float64).reshape(1).contiguous()
        key = ("w0", float(w0), device)
        if key not in self._cache:
            self._cache[key] = torch.tensor([float(w0)], dtype=torch.float64, device=device)
        return self._cache[key]

    def halfband_taps(self, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
        """``taps[t] = lowpass[c_lp + t]`` (t = 0..c_lp), as used by the half-band kernel."""
        key = ("hb", device, dtype)
        if key not in self._cache:
            self._cache[key] = self.lowpass[self.c_lp:].to(device=device, dtype=dtype).contiguous()
        return self._cache[key]

    def _index(self, k: int, device) -> torch.Tensor:
        key = ("idx", k, device)
        if key not in self._cache:
            self._cache[key] = torch.tensor(self.stages[k].scale_idx, device=device, dtype=torch.long)
        return self._cache[key]

    def stage_taps(self, H: torch.Tensor, k: int) -> torch.Tensor:
        """Compact tap table of stage k: taps[s][t][ch] = H[i_s * C + ch, center + t]."""
        st = self.stages[k]
        C = self.channels
        h = H.view(self.num_scales, C, -1).index_select(0, self._index(k, H.device))
        return h[:, :, self.center:self.center + st.half + 1].transpose(1, 2).contiguous()

    def filters(self, scales: torch.Tensor, w0, dtype: torch.dtype) -> torch.Tensor:
        """All sampled Morlet filters as one ``(S*C, 2*center+1)`` tensor (row ``i*C + c``),
        reference cwt.py:181-203.  Built on k >= 0 and mirrored, so the real rows are exactly
        even and the imaginary rows exactly odd (the HIP kernels rely on that symmetry).
        Differentiable w.r.t. ``scales`` and ``w0`` (when it is a tensor).  On a ROCm device
        one HIP kernel builds the bank and one computes its gradient; on the CPU (host-side
        planning and inspection) it is the torch expression below."""
        if scales.is_cuda:
            return _MorletFiltersFunction.apply(scales, w0, self, dtype)
        dev = scales.device
        f64 = torch.float64
        s = scales.to(f64)[:, None]
        dil = torch.tensor(self._dil, dtype=f64, device=dev)[:, None]
        sup = torch.tensor(self._sup, dtype=f64, device=dev)[:, None]
        k = torch.arange(0, self.center + 1, device=dev, dtype=f64)[None, :]
        t = k * dil / s
        env = torch.exp(-0.5 * t * t) * (k <= sup)
        amp = _PI_M14 * dil / (s.sqrt() if self.norm == "l2" else s)
        w0_ = torch.as_tensor(w0, dtype=f64, device=dev)
        w0t = w0_ * t
        re = (torch.cos(w0t) - torch.exp(-0.5 * w0_ * w0_)) * env * amp
        re = torch.cat([re[:, 1:].flip(-1), re], 1)
        if not self.complex:
            return re.to(dtype)
        im = torch.sin(w0t) * env * amp
        im = torch.cat([-im[:, 1:].flip(-1), im], 1)
        return torch.stack([re, im], 1).reshape(-1, re.shape[1]).to(dtype)


class _MorletFiltersFunction(torch.autograd.Function):
    """Device filter bank: ``fdwt_morlet_filters`` (forward) and
    ``fdwt_morlet_filters_backward`` (gradient w.r.t. scales and w0), reference
    cwt.py:181-203.  ``w0`` is a float or a tensor; its gradient is returned in the latter
    case."""

    @staticmethod
    def forward(ctx, scales, w0, plan: "MorletPlan", dtype):
        dev = scales.device
        s = scales.detach().to(torch.float64).contiguous()
        w = plan.w0_device(w0, dev)
        H = torch.empty((plan.num_scales * plan.channels, 2 * plan.center + 1), device=dev,
                        dtype=_out_dtype(dtype))
        for i0, i1, dil, sup in plan.filter_geometry():
            _lib.launch("fdwt_morlet_filters", dev, _lib.ptr(s[i0:]), _lib.ptr(w), dil, sup,
                        i1 - i0, plan.center, plan.channels, int(plan.norm == "l2"),
                        _lib.ptr(H[i0 * plan.channels:]), _lib.dtype_code(H.dtype),
                        _lib.stream(dev))
        ctx.plan, ctx.w0_tensor = plan, isinstance(w0, torch.Tensor)
        ctx.scales_dtype = scales.dtype
        ctx.w0_meta = (w0.dtype, w0.shape) if ctx.w0_tensor else None
        ctx.save_for_backward(s, w)
        return H if H.dtype == dtype else H.to(dtype)

    @staticmethod
    def backward(ctx, gH):
        plan: MorletPlan = ctx.plan
        s, w = ctx.saved_tensors
        dev = s.device
        gH = gH.contiguous()
        if gH.dtype not in (torch.float32, torch.float64):
            gH = gH.float()
        geom = plan.filter_geometry()
        S = plan.num_scales
        # g[:S] = d/ds per scale; g[S + c] = chunk c's share of d/dw0, summed in chunk order
        g = torch.empty(S + len(geom), device=dev, dtype=torch.float64)
        for c, (i0, i1, dil, sup) in enumerate(geom):
            _lib.launch("fdwt_morlet_filters_backward", dev, _lib.ptr(s[i0:]), _lib.ptr(w), dil,
                        sup, i1 - i0, plan.center, plan.channels, int(plan.norm == "l2"),
                        _lib.ptr(gH[i0 * plan.channels:]), _lib.dtype_code(gH.dtype),
                        _lib.ptr(g[i0:]), _lib.ptr(g[S + c:]), _lib.stream(dev))
        g_s = g[:plan.num_scales].to(ctx.scales_dtype)
        g_w0 = None
        if ctx.w0_tensor:
            g_w0 = (g[S] if len(geom) == 1 else g[S:].sum()).to(ctx.w0_meta[0]).reshape(ctx.w0_meta[1])
        return g_s, g_w0, None, None


# --------------------------------------------------------------------------- stage launches
def _out_dtype(dtype: torch.dtype) -> torch.dtype:
    return torch.float64 if dtype == torch.float64 else torch.float32


def _i32(values):
    import ctypes
    return (ctypes.c_int32 * max(1, len(values)))(*[int(v) for v in values])


@dataclass
class _Group:
    """One launch of a stage: its scales g0 .. g1 - 1 (in the stage's support order; each
    stage kernel takes at most FDWT_CWT_MAX_SCALES of them, so an octave with more scales is
    launched in consecutive groups with the octave's dilation and tap table)."""
    g0: int
    g1: int
    sup: object    # ctypes int32 supports of the group (non-decreasing)
    chan: object   # ctypes int32 global scale indices (output channels of the scalogram)
    local: object  # ctypes int32 0 .. g1 - g0 - 1 (channels of a per-group dL/dW)

    @property
    def n(self) -> int:
        return self.g1 - self.g0


def _stage_groups(plan: MorletPlan, k: int) -> List[_Group]:
    key = ("groups", k)
    if key not in plan._cache:
        st = plan.stages[k]
        n = len(st.scale_idx)
        plan._cache[key] = [
            _Group(g0, min(n, g0 + _MAX_STAGE_SCALES), _i32(st.support[g0:g0 + _MAX_STAGE_SCALES]),
                   _i32(st.scale_idx[g0:g0 + _MAX_STAGE_SCALES]),
                   _i32(range(min(n, g0 + _MAX_STAGE_SCALES) - g0)))
            for g0 in range(0, n, _MAX_STAGE_SCALES)]
    return plan._cache[key]


def _lowpass_step(plan: MorletPlan, xj: torch.Tensor, j: int, N: int) -> torch.Tensor:
    """x_{j+1} = dilated half-band low-pass of x_j with the plan's margins (cwt.py:512-519)."""
    R = xj.shape[0]
    m0, m1 = plan.margins[j], plan.margins[j + 1]
    y = torch.empty((R, N + 2 * m1), device=xj.device, dtype=xj.dtype)
    off = m0 - m1 + plan.c_lp * 2 ** j
    dil = 2 ** j
    _lib.launch("fdwt_halfband", xj.device, _lib.ptr(xj), _lib.ptr(plan.halfband_taps(xj.device, xj.dtype)),
                _lib.ptr(y), R, xj.shape[1], y.shape[1], plan.c_lp, off - dil * plan.c_lp, dil, 0,
                _lib.dtype_code(xj.dtype), _lib.stream(xj.device))
    return y


def _lowpass_transpose(plan: MorletPlan, g_next: torch.Tensor, j: int, N: int) -> torch.Tensor:
    """Adjoint of :func:`_lowpass_step`: gradient of x_j from the gradient of x_{j+1}."""
    R = g_next.shape[0]
    m0, m1 = plan.margins[j], plan.margins[j + 1]
    gx = torch.empty((R, N + 2 * m0), device=g_next.device, dtype=g_next.dtype)
    off = m0 - m1 + plan.c_lp * 2 ** j
    dil = 2 ** j
    _lib.launch("fdwt_halfband", g_next.device, _lib.ptr(g_next),
                _lib.ptr(plan.halfband_taps(g_next.device, g_next.dtype)), _lib.ptr(gx), R,
                g_next.shape[1], gx.shape[1], plan.c_lp, dil * plan.c_lp - off, dil, 0,
                _lib.dtype_code(g_next.dtype), _lib.stream(g_next.device))
    return gx


def _lowpass_chain(plan: MorletPlan, x: torch.Tensor) -> List[torch.Tensor]:
    xs = [x]
    N = x.shape[1]
    for j in range(plan.n_octaves - 1):
        xs.append(_lowpass_step(plan, xs[j], j, N))
    return xs


def _operand_code(dt, precision: str) -> int:
    """C-ABI dtype code of the bank's backward entry points: fp32 storage with bf16 matrix
    operands for the reference's "bf16" precision (conv.py:192-196), else the storage dtype.
    ("tf32" computes in fp32: CDNA4 has no TF32 matrix format.)"""
    if precision == "bf16" and dt == torch.float32:
        return _lib.F32_BF16
    return _lib.dtype_code(dt)


def _stage_backward(plan, k, grp: _Group, xj, g, g_scales, chan, taps, gx, accumulate,
                    need_h, precision: str = "ieee"):
    """grad-x of one launch group (accumulated into gx) and, if asked, the group's tap
    gradient (g1 - g0, 2 half + 1, C).  ``chan`` gives the group's channels in g, ``taps``
    is the stage's whole tap table; ``precision`` as ``resolve_precision`` returns it."""
    st = plan.stages[k]
    R, n_out = g.shape[0], g.shape[2]
    C = plan.channels
    mj = plan.margins[st.octave]
    dev, dt = g.device, g.dtype
    tg = taps[grp.g0:grp.g1]
    code = _operand_code(dt, precision)
    _lib.launch("fdwt_morlet_backward_x", dev, _lib.ptr(g), _lib.ptr(tg), _lib.ptr(gx), R,
                gx.shape[1], n_out, mj, grp.n, st.half, grp.sup, chan, st.dil, C,
                g_scales, int(accumulate), code, _lib.stream(dev))
    if not need_h:
        return None
    L = _lib.lib()
    ws_n = L.fdwt_morlet_backward_h_workspace(R, n_out, grp.n, st.half, C)
    ws = torch.empty(max(1, ws_n), device=dev, dtype=dt)
    gh = torch.empty((grp.n, 2 * st.half + 1, C), device=dev, dtype=dt)
    _lib.launch("fdwt_morlet_backward_h", dev, _lib.ptr(xj), _lib.ptr(g), _lib.ptr(ws), ws_n,
                _lib.ptr(gh), R, xj.shape[1], n_out, mj, grp.n, st.half, grp.sup, chan,
                st.dil, C, g_scales, 0, code, _lib.stream(dev))
    return gh


def _scatter_gh(plan: MorletPlan, gH: torch.Tensor, k: int, gh: torch.Tensor):
    """gH[rows of stage k, centre - half .. centre + half] = gh (S_j, 2 half + 1, C)."""
    st = plan.stages[k]
    C = plan.channels
    view = gH.view(plan.num_scales, C, -1)
    cols = slice(plan.center - st.half, plan.center + st.half + 1)
    idx = plan._index(k, gH.device)
    view[idx, :, cols] = gh.transpose(1, 2).to(gH.dtype)


# --------------------------------------------------------------------------- autograd
class _MorletCWTFunction(torch.autograd.Function):
    """All octaves of the transform in one autograd node (reference cwt.py:213-281)."""

    @staticmethod
    def forward(ctx, x, plan: MorletPlan, H):
        _lib.require_gpu(x, H)
        R, N = x.shape
        C = plan.channels
        y = torch.empty((R, plan.num_scales, N, C), device=x.device, dtype=_out_dtype(x.dtype))
        need_h = ctx.needs_input_grad[2]
        H = H.to(x.dtype)
        xs = [x]
        by_oct = {st.octave: k for k, st in enumerate(plan.stages)}
        tables = {}
        for j in range(plan.n_octaves):
            if j in by_oct:
                k = by_oct[j]
                st = plan.stages[k]
                taps = tables[k] = plan.stage_taps(H, k)
                for grp in _stage_groups(plan, k):
                    _lib.launch("fdwt_morlet_forward", x.device, _lib.ptr(xs[j]),
                                _lib.ptr(taps[grp.g0:grp.g1]), _lib.ptr(y), R, xs[j].shape[1], N,
                                plan.margins[j], grp.n, st.half, grp.sup, grp.chan, st.dil, C,
                                plan.num_scales, _lib.dtype_code(x.dtype), _lib.stream(x.device))
            if j + 1 < plan.n_octaves:
                xs.append(_lowpass_step(plan, xs[j], j, N))
        ctx.plan = plan
        ctx.x_dtype = x.dtype
        ctx.need_h = need_h
        ctx.n_x = len(xs) if need_h else 0
        ctx.tables = tables
        ctx.save_for_backward(*(xs if need_h else []), H)
        return y

    @staticmethod
    def backward(ctx, g):
        plan: MorletPlan = ctx.plan
        saved = ctx.saved_tensors
        xs, H = saved[:ctx.n_x], saved[-1]
        g = g.contiguous().to(H.dtype)
        R, _, N, _ = g.shape
        by_oct = {st.octave: k for k, st in enumerate(plan.stages)}
        gH = torch.zeros_like(H) if ctx.need_h else None
        g_next = None
        for j in range(plan.n_octaves - 1, -1, -1):
            mj = plan.margins[j]
            if g_next is not None:
                gx = _lowpass_transpose(plan, g_next, j, N)
                filled = True
            else:
                gx = torch.empty((R, N + 2 * mj), device=g.device, dtype=g.dtype)
                filled = False
            if j in by_oct:
                k = by_oct[j]
                taps = ctx.tables[k]  # the forward's compact tap tables
                ghs = []
                for grp in _stage_groups(plan, k):
                    gh = _stage_backward(plan, k, grp, xs[j] if ctx.need_h else None, g,
                                         plan.num_scales, grp.chan, taps, gx, filled, ctx.need_h,
                                         resolve_precision(g.dtype))
                    filled = True
                    if gh is not None:
                        ghs.append(gh)
                if ghs:
                    _scatter_gh(plan, gH, k, ghs[0] if len(ghs) == 1 else torch.cat(ghs))
            if not filled:
                gx.zero_()
            g_next = gx
        gx = g_next.to(ctx.x_dtype) if ctx.needs_input_grad[0] else None
        return gx, None, gH


def _stage_chunks(R: int, chunk: int, unit: int):
    """Row chunks of about `chunk` rows, each a whole multiple of `unit` rows."""
    step = max(unit, (max(1, chunk) // unit) * unit)
    return [(r0, min(R, r0 + step)) for r0 in range(0, R, step)]


class _MorletMixFunction(torch.autograd.Function):
    """y[r, n] = sum_s a[d, s] |W_s[r, n]| + b[d, s] Re W_s[r, n] without materialising W
    (reference cwt.py:284-376).  Forward: one fused HIP launch per octave accumulating y.
    Backward: per octave, in row chunks of at most MIX_CHUNK_BYTES of dL/dW, the fused kernel
    writes dL/dW and partial (ga, gb) sums, then the grad-x / grad-h kernels consume it."""

    # Row chunks of dL/dW: 2 GiB (the reference uses 256 MiB); on a 288 GB MI355X the larger
    # chunk costs little memory and cuts the backward's launches 8x at large batch sizes.
    MIX_CHUNK_BYTES = 2 * 2**30

    @staticmethod
    def forward(ctx, x, plan: MorletPlan, H, a, b):
        _lib.require_gpu(x, H, a, b)
        R, N = x.shape
        D = a.shape[0]
        dt = _out_dtype(x.dtype)
        a_, b_ = a.to(dt).contiguous(), b.to(dt).contiguous()
        H = H.to(dt)
        y = torch.empty((R, N), device=x.device, dtype=dt)
        xs = [x]
        by_oct = {st.octave: k for k, st in enumerate(plan.stages)}
        tables = {}
        first = True
        for j in range(plan.n_octaves):
            if j in by_oct:
                k = by_oct[j]
                st = plan.stages[k]
                taps = tables[k] = plan.stage_taps(H, k)
                for grp in _stage_groups(plan, k):
                    _lib.launch("fdwt_mix_forward", x.device, _lib.ptr(xs[j]),
                                _lib.ptr(taps[grp.g0:grp.g1]), _lib.ptr(a_), _lib.ptr(b_),
                                _lib.ptr(y), R, xs[j].shape[1], N, plan.margins[j], grp.n,
                                st.half, grp.sup, grp.chan, st.dil, plan.channels, a_.shape[1],
                                D, 0, 0 if first else 1, _lib.dtype_code(dt),
                                _lib.stream(x.device))
                    first = False
            if j + 1 < plan.n_octaves:
                xs.append(_lowpass_step(plan, xs[j], j, N))
        if first:
            y.zero_()
        ctx.plan = plan
        ctx.x_dtype = x.dtype
        ctx.tables = tables
        ctx.save_for_backward(*xs, H, a_, b_)
        ctx.n_x = len(xs)
        return y

    @staticmethod
    def backward(ctx, gy):
        plan: MorletPlan = ctx.plan
        saved = ctx.saved_tensors
        nx = ctx.n_x
        xs = saved[:nx]
        H, a, b = saved[nx:nx + 3]
        gy = gy.contiguous().to(a.dtype)
        prec = resolve_precision(gy.dtype)  # the compute dtype, as the reference's launchers
        R, N = gy.shape
        D = a.shape[0]
        C = plan.channels
        dev, dt = gy.device, gy.dtype
        need_h = ctx.needs_input_grad[2]
        gH = torch.zeros_like(H) if need_h else None
        gab = torch.zeros((D, a.shape[1], 2), device=dev, dtype=a.dtype)  # (ga, gb) per scale
        by_oct = {st.octave: k for k, st in enumerate(plan.stages)}
        L = _lib.lib()
        g_next = None
        for j in range(plan.n_octaves - 1, -1, -1):
            mj = plan.margins[j]
            if g_next is not None:
                gx = _lowpass_transpose(plan, g_next, j, N)
                filled = True
            else:
                gx = torch.empty((R, N + 2 * mj), device=dev, dtype=dt)
                filled = False
            if j in by_oct:
                k = by_oct[j]
                st = plan.stages[k]
                taps = ctx.tables[k]  # the forward's compact tap tables
                idx = plan._index(k, dev)
                ghs = []
                for grp in _stage_groups(plan, k):
                    S_g = grp.n
                    chunk = max(1, _MorletMixFunction.MIX_CHUNK_BYTES // (S_g * N * C * gy.element_size()))
                    gh_acc = None
                    tg = taps[grp.g0:grp.g1]
                    for r0, r1 in _stage_chunks(R, chunk, D):
                        rc = r1 - r0
                        gw = torch.empty((rc, S_g, N, C), device=dev, dtype=dt)
                        ws_n = L.fdwt_mix_workspace(rc, N, S_g)
                        ws = torch.empty(max(1, ws_n), device=dev, dtype=dt)
                        xj = xs[j][r0:r1]
                        _lib.launch("fdwt_mix_backward", dev, _lib.ptr(xj), _lib.ptr(tg),
                                    _lib.ptr(a), _lib.ptr(b), _lib.ptr(gy[r0:r1]), _lib.ptr(gw),
                                    _lib.ptr(ws), ws_n, rc, xj.shape[1], N, mj, S_g, st.half,
                                    grp.sup, grp.chan, st.dil, C, a.shape[1], D, r0,
                                    _lib.dtype_code(dt), _lib.stream(dev))
                        # (rows, tiles, S_g, 2) -> per weight row d (rows are whole multiples of
                        # D): one reduction, one indexed add (the group's scales are distinct)
                        part = ws[:ws_n].view(-1, D, ws_n // (rc * S_g * 2), S_g, 2).sum((0, 2))
                        gab.index_add_(1, idx[grp.g0:grp.g1], part)
                        gh = _stage_backward(plan, k, grp, xj, gw, S_g, grp.local, taps,
                                             gx[r0:r1], filled, need_h, prec)
                        if gh is not None:
                            gh_acc = gh if gh_acc is None else gh_acc + gh
                        del gw
                    filled = True
                    if gh_acc is not None:
                        ghs.append(gh_acc)
                if ghs:
                    _scatter_gh(plan, gH, k, ghs[0] if len(ghs) == 1 else torch.cat(ghs))
            if not filled:
                gx.zero_()
            g_next = gx
        gx = g_next.to(ctx.x_dtype) if ctx.needs_input_grad[0] else None
        return gx, None, gH, gab[..., 0], gab[..., 1]


def morlet_mix(x: torch.Tensor, plan: MorletPlan, H: torch.Tensor, a: torch.Tensor,
               b: torch.Tensor) -> torch.Tensor:
    """``x (B, D, N)`` -> ``sum_s a[d, s] |W_s| + b[d, s] Re W_s``, shape ``(B, D, N)``
    (reference cwt.py:379-394).  Memory O(B*D*N): the scalogram is never stored."""
    B, D, N = x.shape
    _lib.require_gpu(x)
    x2 = x.reshape(B * D, N).contiguous()
    if x2.dtype not in (torch.float32, torch.float64):
        x2 = x2.float()
    return _MorletMixFunction.apply(x2, plan, H, a, b).view(B, D, N)


class _SpectralSoftmaxFunction(torch.autograd.Function):
    """out[r, n] = sum_f softmax_f(|W_f x_r|(n) / tau) * V_f[r, n] without materialising W
    (reference cwt.py:397-509).  ``V`` is ``(NCH, S)`` (row r uses ``V[r % NCH]``) or
    ``(G, S, N)`` (row r uses ``V[r // NCH]``).  The forward folds every octave into a
    flash-attention style online softmax (m, l, num) and writes out = num / l in its last
    launch; the backward recomputes the chain and one octave of dL/dW at a time."""

    # Row chunks of dL/dW: 2 GiB (the reference uses 256 MiB), as MIX_CHUNK_BYTES above.
    CHUNK_BYTES = 2 * 2**30

    @staticmethod
    def forward(ctx, x, plan: MorletPlan, H, V, nch: int, tau: float, precision: str):
        if not plan.complex:
            raise ValueError("the spectral softmax needs the complex Morlet transform")
        _lib.require_gpu(x, H, V)
        R, N = x.shape
        dt = _out_dtype(x.dtype)
        V_ = V.to(dt).contiguous()
        v_pos = V_.dim() == 3
        H = H.to(dt)
        m = torch.empty((R, N), device=x.device, dtype=dt)
        l = torch.empty_like(m)
        out = torch.empty_like(m)
        by_oct = {st.octave: k for k, st in enumerate(plan.stages)}
        last_j = max(by_oct)
        tables = {}
        xj = x
        first = True
        for j in range(plan.n_octaves):
            if j in by_oct:
                k = by_oct[j]
                st = plan.stages[k]
                taps = tables[k] = plan.stage_taps(H, k)
                groups = _stage_groups(plan, k)
                for gi, grp in enumerate(groups):
                    last = j == last_j and gi + 1 == len(groups)
                    _lib.launch("fdwt_softmax_forward", x.device, _lib.ptr(xj),
                                _lib.ptr(taps[grp.g0:grp.g1]), _lib.ptr(V_), int(v_pos),
                                V_.shape[1], nch, _lib.ptr(m), _lib.ptr(l), _lib.ptr(out), R,
                                xj.shape[1], N, plan.margins[j], grp.n, st.half, grp.sup,
                                grp.chan, st.dil, 1.0 / tau, int(first), int(last),
                                _lib.dtype_code(dt), _lib.stream(x.device))
                    first = False
            if j + 1 < plan.n_octaves and j < last_j:
                xj = _lowpass_step(plan, xj, j, N)
        ctx.plan, ctx.nch, ctx.tau, ctx.precision = plan, nch, tau, precision
        ctx.x_dtype, ctx.v_dtype = x.dtype, V.dtype
        ctx.tables = tables
        ctx.save_for_backward(x, H, V_, m, l, out)
        return out

    @staticmethod
    def backward(ctx, gy):
        plan: MorletPlan = ctx.plan
        x, H, V, m, l, out = ctx.saved_tensors
        gy = gy.contiguous().to(V.dtype)
        prec = ctx.precision
        R, N = gy.shape
        dev, dt = gy.device, gy.dtype
        v_pos = V.dim() == 3
        nch = ctx.nch
        need_h = ctx.needs_input_grad[2]
        gH = torch.zeros_like(H) if need_h else None
        gV = torch.zeros_like(V, memory_format=torch.contiguous_format)
        by_oct = {st.octave: k for k, st in enumerate(plan.stages)}
        xs = _lowpass_chain(plan, x.to(dt))
        L = _lib.lib()
        g_next = None
        for j in range(plan.n_octaves - 1, -1, -1):
            mj = plan.margins[j]
            if g_next is not None:
                gx = _lowpass_transpose(plan, g_next, j, N)
                filled = True
            else:
                gx = torch.empty((R, N + 2 * mj), device=dev, dtype=dt)
                filled = False
            if j in by_oct:
                k = by_oct[j]
                st = plan.stages[k]
                taps = ctx.tables[k]  # the forward's compact tap tables
                idx = plan._index(k, dev)
                ghs = []
                for grp in _stage_groups(plan, k):
                    S_g = grp.n
                    gidx = idx[grp.g0:grp.g1]
                    tg = taps[grp.g0:grp.g1]
                    chunk = max(1, _SpectralSoftmaxFunction.CHUNK_BYTES // (S_g * N * 2 * gy.element_size()))
                    gh_acc = None
                    for r0, r1 in _stage_chunks(R, chunk, nch):
                        rc = r1 - r0
                        gw = torch.empty((rc, S_g, N, 2), device=dev, dtype=dt)
                        ws_n = L.fdwt_softmax_workspace(rc, N, S_g, int(v_pos))
                        ws = torch.empty(max(1, ws_n), device=dev, dtype=dt)
                        xj = xs[j][r0:r1]
                        _lib.launch("fdwt_softmax_backward", dev, _lib.ptr(xj), _lib.ptr(tg),
                                    _lib.ptr(V), int(v_pos), V.shape[1], nch, r0,
                                    _lib.ptr(m[r0:r1]), _lib.ptr(l[r0:r1]), _lib.ptr(out[r0:r1]),
                                    _lib.ptr(gy[r0:r1]), _lib.ptr(gw), _lib.ptr(ws), ws_n, rc,
                                    xj.shape[1], N, mj, S_g, st.half, grp.sup, grp.chan, st.dil,
                                    1.0 / ctx.tau, _lib.dtype_code(dt), _lib.stream(dev))
                        if v_pos:
                            # (rows, S_g, N): the nch rows of each group summed (in row order)
                            # into gV at the group's scale indices, one kernel
                            _lib.launch("fdwt_softmax_dv_reduce", dev, _lib.ptr(ws), _lib.ptr(gV),
                                        rc // nch, nch, S_g, grp.chan, gV.shape[0], gV.shape[1],
                                        N, r0 // nch, _lib.dtype_code(dt), _lib.stream(dev))
                        else:
                            part = ws[:ws_n].view(rc, -1, S_g).sum(1).view(-1, nch, S_g).sum(0)
                            gV[:, gidx] += part
                        gh = _stage_backward(plan, k, grp, xj, gw, S_g, grp.local, taps,
                                             gx[r0:r1], filled, need_h, prec)
                        if gh is not None:
                            gh_acc = gh if gh_acc is None else gh_acc + gh
                        del gw
                    filled = True
                    if gh_acc is not None:
                        ghs.append(gh_acc)
                if ghs:
                    _scatter_gh(plan, gH, k, ghs[0] if len(ghs) == 1 else torch.cat(ghs))
            if not filled:
                gx.zero_()
            g_next = gx
            xs[j] = None  # free each octave signal once its octave is done
        gx = g_next.to(ctx.x_dtype) if ctx.needs_input_grad[0] else None
        return gx, None, gH, gV.to(ctx.v_dtype), None, None, None


def spectral_softmax(x: torch.Tensor, plan: MorletPlan, H: torch.Tensor, V: torch.Tensor,
                     nch: int, tau: float = 1.0) -> torch.Tensor:
    """``x (R, N)`` -> ``sum_f softmax_f(|W_f x|/tau) V_f``, shape ``(R, N)``
    (reference cwt.py:529-549).  ``V`` is ``(nch, S)`` (row r uses ``V[r % nch]``) or
    ``(R // nch, S, N)`` (row r uses ``V[r // nch]``).  Memory O(R*N)."""
    R, N = x.shape
    _lib.require_gpu(x)
    if R % nch:
        raise ValueError(f"the number of rows {R} must be a multiple of nch={nch}")
    prec = resolve_precision(x.dtype)  # the caller's dtype: bf16 / fp16 inputs select bf16
    x2 = x.contiguous()
    if x2.dtype not in (torch.float32, torch.float64):
        x2 = x2.float()
    return _SpectralSoftmaxFunction.apply(x2, plan, H, V, nch, float(tau), prec)


# --------------------------------------------------------------------------- torch paths
def _fft_conv(x, h, n_out, off):
    # y[f, n] = sum_k h[f, k] x[n + off - k] = (h * x)[n + off]   (cwt.py:586-594)
    R, N = x.shape
    K = h.shape[1]
    nfft = 1 << (N + K - 1 - 1).bit_length()
    X = torch.fft.rfft(x.to(h.dtype), nfft)
    Hf = torch.fft.rfft(h, nfft)
    y = torch.fft.irfft(X[:, None, :] * Hf[None], nfft)
    return y[..., off:off + n_out]


def _fft_cwt(x, plan: MorletPlan, H):
    """method="fft": the direct filters through torch.fft on the device (cwt.py:575-576)."""
    R, N = x.shape
    C = plan.channels
    st = plan.stages[0]
    h = H[plan.stage_rows(0)][:, plan.center - st.half:plan.center + st.half + 1].to(x.dtype)
    y = _fft_conv(x, h, N, st.half)  # (R, S*C, N) in stage order
    y = y.reshape(R, len(st.scale_idx), C, N).transpose(-1, -2)
    out = x.new_zeros((R, plan.num_scales, N, C))
    return out.index_copy(1, plan._index(0, x.device), y.to(out.dtype))


# --------------------------------------------------------------------------- public API
def _apply_plan(x: torch.Tensor, plan: MorletPlan, H: torch.Tensor) -> torch.Tensor:
    """cwt.py:600-612.  H must be a Morlet filter bank as :meth:`MorletPlan.filters` builds
    it (real rows even, imaginary rows odd around the centre)."""
    if not x.is_floating_point() or x.is_complex():
        raise TypeError("cwt expects a real floating point tensor")
    _lib.require_gpu(x)
    lead, N = x.shape[:-1], x.shape[-1]
    x2 = x.reshape(-1, N).contiguous()
    if x2.dtype not in (torch.float32, torch.float64):
        x2 = x2.float()
    if plan.method == "fft":
        y = _fft_cwt(x2, plan, H.to(x2.dtype))
    else:
        y = _MorletCWTFunction.apply(x2, plan, H)
    y = y.reshape(*lead, plan.num_scales, N, plan.channels)
    return torch.view_as_complex(y) if plan.complex else y[..., 0]


@lru_cache(maxsize=64)
def _cached_plan(scales: Tuple[float, ...], w0, truncate, norm, complex, method) -> MorletPlan:
    return MorletPlan(scales, w0, truncate, norm, complex, method)


@lru_cache(maxsize=64)
def _cached_filters(plan: MorletPlan, device: torch.device, dtype: torch.dtype):
    s = torch.tensor(plan.scales, dtype=torch.float64, device=device)
    return plan.filters(s, plan.w0, dtype)


def _resolve_scales(scales, freqs, fs, w0) -> List[float]:
    if (scales is None) == (freqs is None):
        raise ValueError("pass exactly one of `scales` or `freqs`")
    s = freqs_to_scales(freqs, fs, w0) if freqs is not None else torch.as_tensor(scales, dtype=torch.float64)
    return [float(v) for v in s.flatten()]


def cwt(x: torch.Tensor, scales: Optional[Sequence[float]] = None, *, freqs=None, fs: float = 1.0,
        w0: float = 6.0, method: str = "fast", norm: str = "l2", complex: bool = True,
        truncate: float = 4.0) -> torch.Tensor:
    """Morlet CWT along the last dimension (cwt.py:633-651): ``(..., N)`` real ->
    ``(..., S, N)`` complex (real if ``complex=False``)."""
    s = _resolve_scales(scales, freqs, fs, w0)
    plan = _cached_plan(tuple(s), float(w0), float(truncate), norm, bool(complex), method)
    dt = torch.float64 if x.dtype == torch.float64 else torch.float32
    return _apply_plan(x, plan, _cached_filters(plan, x.device, dt))


class CWT1D(nn.Module):
    """Morlet continuous wavelet transform as a module (cwt.py:654-716).

    Input ``(..., N)`` real, output ``(..., S, N)`` complex (or real with ``complex=False``).
    With ``learnable=True`` the (log-)scales are parameters; ``learnable_w0`` also learns the
    Morlet wave number.  Parameter / buffer names match the reference for state_dict reuse.
    """

    def __init__(self, freqs=None, scales=None, fs: float = 1.0, w0: float = 6.0,
                 method: str = "fast", norm: str = "l2", complex: bool = True,
                 truncate: float = 4.0, learnable: bool = False, learnable_w0: bool = False,
                 support_margin: Optional[float] = None):
        super().__init__()
        s = _resolve_scales(scales, freqs, fs, w0)
        if support_margin is None:
            support_margin = 1.25 if learnable else 1.0
        self.fs = fs
        self.plan = MorletPlan(s, w0, truncate, norm, complex, method, support_margin)
        log_s = torch.tensor(s, dtype=torch.float64).log().float()
        if learnable:
            self.log_scales = nn.Parameter(log_s)
        else:
            self.register_buffer("log_scales", log_s)
        if learnable_w0:
            self.w0 = nn.Parameter(torch.tensor(float(w0)))
        else:
            self.w0 = float(w0)
        self._learn = learnable or learnable_w0
        self._filter_cache: Dict = {}

    @property
    def scales(self) -> torch.Tensor:
        return self.log_scales.exp()

    @property
    def w0_value(self) -> float:
        return float(self.w0.detach()) if isinstance(self.w0, torch.Tensor) else float(self.w0)

    @property
    def freqs(self) -> torch.Tensor:
        return scales_to_freqs(self.scales.detach(), self.fs, self.w0_value)

    def _filters(self, device, dtype):
        if self._learn:
            return self.plan.filters(self.log_scales.to(torch.float64).exp(), self.w0, dtype)
        key = (device, dtype)
        if key not in self._filter_cache:
            self._filter_cache = {key: self.plan.filters(self.scales.to(torch.float64), self.w0, dtype)}
        return self._filter_cache[key]

    def _apply(self, fn, *args, **kwargs):
        self._filter_cache = {}
        return super()._apply(fn, *args, **kwargs)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dt = torch.float64 if x.dtype == torch.float64 else torch.float32
        return _apply_plan(x, self.plan, self._filters(x.device, dt))

    def extra_repr(self) -> str:
        p = self.plan
        return (f"scales={p.num_scales}, w0={self.w0_value:g}, method={p.method}, norm={p.norm}, "
                f"complex={p.complex}, octaves={p.n_octaves}, learnable={self._learn}")
