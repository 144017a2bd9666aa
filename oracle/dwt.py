"""CPU oracle of the 1-D Mallat DWT (test infrastructure; see ``oracle/__init__.py``).

Restates pytorch_morlet_fdwt src/fdwt/reference.py:15-49 (gather analysis, index_add
synthesis), src/fdwt/kernels/dwt.py:30-49 (modes, periods, the reflect/N=1 rule),
src/fdwt/dwt.py:85-171 (offsets, lengths, idwt as a transpose, the waverec trim rule) and
src/fdwt/wavelets.py:39-64, 86-89 (even padding, reversed synthesis filters).
"""

from __future__ import annotations

import json
import os
from functools import lru_cache

import torch

MODES = {"zero": 0, "periodic": 1, "symmetric": 2, "reflect": 3, "periodization": 4}
ZERO, PERIODIC, SYMMETRIC, REFLECT, PERIODIZATION = range(5)

_TABLE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "pytorch_morlet_fdwt_amd", "data", "filter_banks.json")


@lru_cache(maxsize=None)
def _table():
    with open(_TABLE) as f:
        return json.load(f)["banks"]


def bank(name_or_filters):
    """(dec_lo, dec_hi, rec_lo, rec_hi) padded to a common even length with trailing zeros
    (wavelets.py:39-41, 62-64).  Accepts a PyWavelets name or a 4-sequence."""
    if isinstance(name_or_filters, str):
        filters = _table()[name_or_filters]
    else:
        filters = name_or_filters
    length = max(len(f) for f in filters)
    length += length % 2
    return tuple(tuple(float(v) for v in f) + (0.0,) * (length - len(f)) for f in filters)


def mode_period(mode: int, n: int) -> int:
    """kernels/dwt.py:33-43."""
    return {PERIODIC: n, SYMMETRIC: 2 * n, REFLECT: 2 * n - 2, PERIODIZATION: n + n % 2}.get(mode, 1)


def normalize_mode(mode: int, n: int) -> int:
    """kernels/dwt.py:46-49: reflect on one sample is a constant (period 1) extension."""
    return PERIODIC if (mode == REFLECT and n == 1) else mode


def ext_index(p: torch.Tensor, n: int, mode: int):
    """reference.py:15-30: map extended positions onto [0, n) plus a validity mask."""
    mode = normalize_mode(mode, n)
    if mode == ZERO:
        valid = (p >= 0) & (p < n)
        return p.clamp(0, max(n - 1, 0)), valid
    P = mode_period(mode, n)
    q = torch.remainder(p, P)
    if mode == PERIODIC:
        idx = q
    elif mode == SYMMETRIC:
        idx = torch.where(q < n, q, P - 1 - q)
    elif mode == REFLECT:
        idx = torch.where(q < n, q, P - q)
    else:
        idx = q.clamp(max=n - 1)
    return idx, torch.ones_like(p, dtype=torch.bool)


def _taps(n, n_out, L, mode, off):
    """reference.py:33-36: positions 2*o + off - j of the extended signal."""
    o = torch.arange(n_out)[:, None]
    j = torch.arange(L)[None, :]
    return ext_index(2 * o + off - j, n, mode)


def analysis(x, h0, h1, mode: int, off: int, n_out: int):
    """reference.py:39-42: y_b[o] = sum_j h_b[j] x_ext[2 o + off - j]."""
    idx, valid = _taps(x.shape[-1], n_out, h0.numel(), mode, off)
    xs = x[..., idx] * valid
    return (xs * h0.to(x.dtype)).sum(-1), (xs * h1.to(x.dtype)).sum(-1)


def synthesis(a, d, h0, h1, mode: int, off: int, n: int):
    """reference.py:45-49: the exact transpose of :func:`analysis`."""
    idx, valid = _taps(n, a.shape[-1], h0.numel(), mode, off)
    contrib = (a[..., :, None] * h0.to(a.dtype) + d[..., :, None] * h1.to(a.dtype)) * valid
    y = a.new_zeros(*a.shape[:-1], n)
    return y.index_add(-1, idx.flatten(), contrib.flatten(-2))


def coeff_len(n: int, L: int, mode: str) -> int:
    """dwt.py:97-100."""
    return (n + 1) // 2 if mode == "periodization" else (n + L - 1) // 2


def _filters(w, dtype):
    f = bank(w)
    mk = lambda v: torch.tensor(v, dtype=dtype)  # noqa: E731
    return mk(f[0]), mk(f[1]), mk(f[2][::-1]), mk(f[3][::-1])


def _cdtype(x):
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def dwt(x, w="db4", mode="symmetric"):
    """dwt.py:103-111 (computes in x's dtype; the tests pass float64)."""
    m = MODES[mode]
    h0, h1, _, _ = _filters(w, x.dtype)
    L = h0.numel()
    off = L // 2 if m == PERIODIZATION else 1
    n_out = coeff_len(x.shape[-1], L, mode)
    lead = x.shape[:-1]
    a, d = analysis(x.reshape(-1, x.shape[-1]), h0, h1, m, off, n_out)
    return a.reshape(*lead, n_out), d.reshape(*lead, n_out)


def idwt(cA, cD, w="db4", mode="symmetric"):
    """dwt.py:114-135: transpose of a periodized (or zero-padded, cropped) analysis built on
    the time-reversed synthesis filters."""
    if cA is None and cD is None:
        raise ValueError("at least one of cA, cD must be given")
    cA = torch.zeros_like(cD) if cA is None else cA
    cD = torch.zeros_like(cA) if cD is None else cD
    m = MODES[mode]
    _, _, r0, r1 = _filters(w, cA.dtype)
    L, nc = r0.numel(), cA.shape[-1]
    if m == PERIODIZATION:
        n, off = 2 * nc, L // 2
    else:
        n, off, m = 2 * nc - L + 2, 1, ZERO
        if n <= 0:
            raise ValueError(f"coefficients of length {nc} are too short for a filter of length {L}")
    lead = cA.shape[:-1]
    y = synthesis(cA.reshape(-1, nc), cD.reshape(-1, nc), r0, r1, m, off, n)
    return y.reshape(*lead, n)


def dwt_max_level(n: int, L: int) -> int:
    """dwt.py:138-143."""
    if L < 2 or n < L - 1:
        return 0
    return (n // (L - 1)).bit_length() - 1


def wavedec(x, w="db4", mode="symmetric", level=None):
    """dwt.py:146-158."""
    if level is None:
        level = dwt_max_level(x.shape[-1], len(bank(w)[0]))
    details, a = [], x
    for _ in range(level):
        a, d = dwt(a, w, mode)
        details.append(d)
    return [a] + details[::-1]


def waverec(coeffs, w="db4", mode="symmetric"):
    """dwt.py:161-171 (same trim rule as pywt.waverec)."""
    a = coeffs[0]
    for d in coeffs[1:]:
        if a.shape[-1] == d.shape[-1] + 1:
            a = a[..., :-1]
        a = idwt(a, d, w, mode)
    return a



def wavelet_token_mixer(x, w, mode, level, bands):
    """layers.py:75-109 (WaveletTokenMixer.forward): x (B, L, D) -> wavedec along L of every
    channel, band j of [cA_J, cD_J .. cD_1] mapped across channels by bands[j] -- (W, b) for
    one Linear, (W1, b1, W2, b2) for Linear -> GELU -> Linear -- then waverec, cropped to L."""
    L = x.shape[1]
    coeffs = wavedec(x.transpose(1, 2), w, mode, level)  # (B, D, n_j)
    mixed = []
    for c, p in zip(coeffs, bands):
        t = c.transpose(1, 2)
        if len(p) == 2:
            t = torch.nn.functional.linear(t, p[0], p[1])
        else:
            t = torch.nn.functional.linear(
                torch.nn.functional.gelu(torch.nn.functional.linear(t, p[0], p[1])), p[2], p[3])
        mixed.append(t.transpose(1, 2))
    return waverec(mixed, w, mode)[..., :L].transpose(1, 2)
