"""CPU oracle of the Morlet CWT pyramid, the scalogram mix and the spectral softmax
(test infrastructure; see ``oracle/__init__.py``).

Restates pytorch_morlet_fdwt src/fdwt/cwt.py:54-203 (scale <-> frequency, the Kaiser
half-band, the octave plan and its margins, the sampled Morlet filters), 555-612 (the
PyTorch pyramid and FFT paths), 391-394 (mix definition), 545-549 (spectral softmax
definition), src/fdwt/reference.py:52-66 (filter-bank convolution) and
src/fdwt/layers.py:26-72, 112-262 (module wiring).
"""

from __future__ import annotations

import math
from typing import List

import numpy as np
import torch
import torch.nn.functional as F

PI_M14 = math.pi ** -0.25


def freqs_to_scales(freqs, fs=1.0, w0=6.0):
    """cwt.py:54-57."""
    return w0 * fs / (2 * math.pi * torch.as_tensor(freqs, dtype=torch.float64))


def scales_to_freqs(scales, fs=1.0, w0=6.0):
    """cwt.py:60-62."""
    return w0 * fs / (2 * math.pi * torch.as_tensor(scales, dtype=torch.float64))


def halfband(c: int, beta: float) -> torch.Tensor:
    """cwt.py:65-68: 0.5 sinc(n/2) times a Kaiser window, normalised to unit DC gain."""
    n = torch.arange(-c, c + 1, dtype=torch.float64)
    h = 0.5 * torch.sinc(n / 2) * torch.from_numpy(np.kaiser(2 * c + 1, beta))
    return h / h.sum()


class Plan:
    """cwt.py:88-139: octave grouping, per-scale supports, centre, half-band, margins."""

    def __init__(self, scales, w0=6.0, truncate=4.0, norm="l2", complex=True, method="fast",
                 support_margin=1.0):
        scales = [float(s) for s in scales]
        self.scales, self.w0, self.truncate, self.norm = scales, float(w0), float(truncate), norm
        self.complex, self.method = bool(complex), method
        self.channels = 2 if complex else 1
        reach = truncate * support_margin
        self.s_th = (w0 + truncate) / (0.8 * math.pi)
        groups = {}
        for i, s in enumerate(scales):
            j = 0 if method != "fast" else max(0, math.floor(math.log2(s / self.s_th)))
            groups.setdefault(j, []).append(i)
        # stages: (octave, dil, scale indices sorted by support, half, supports)
        self.stages = []
        for j in sorted(groups):
            dil = 2 ** j
            sup = {i: max(1, math.ceil(reach * scales[i] / dil)) for i in groups[j]}
            idx = sorted(groups[j], key=lambda i: sup[i])
            self.stages.append((j, dil, idx, max(sup.values()), [sup[i] for i in idx]))
        self.n_octaves = self.stages[-1][0] + 1
        self.center = max(st[3] for st in self.stages)
        self.dil = [0.0] * len(scales)
        self.sup = [0.0] * len(scales)
        for j, dil, idx, half, sups in self.stages:
            for i, c in zip(idx, sups):
                self.dil[i], self.sup[i] = float(dil), float(c)
        c_lp, beta = (16, 8.0) if truncate <= 4.5 else (24, 10.0)
        self.lowpass = halfband(c_lp, beta) if self.n_octaves > 1 else torch.zeros(1, dtype=torch.float64)
        self.c_lp = c_lp if self.n_octaves > 1 else 0
        J = self.n_octaves - 1
        by_oct = {st[0]: st for st in self.stages}
        self.margins = [0] * (J + 1)
        for j in range(J, 0, -1):
            own = by_oct[j][3] * 2 ** j if j in by_oct else 0
            nxt = self.margins[j + 1] + self.c_lp * 2 ** j if j < J else 0
            self.margins[j] = max(own, nxt)

    @property
    def num_scales(self):
        return len(self.scales)

    def filters(self, scales: torch.Tensor, w0, dtype=torch.float64) -> torch.Tensor:
        """cwt.py:181-203: (S*C, 2*center+1), row i*C + c, differentiable in scales / w0."""
        f64 = torch.float64
        s = scales.to(f64)[:, None]
        dil = torch.tensor(self.dil, dtype=f64)[:, None]
        sup = torch.tensor(self.sup, dtype=f64)[:, None]
        k = torch.arange(-self.center, self.center + 1, dtype=f64)[None, :]
        t = k * dil / s
        env = torch.exp(-0.5 * t * t) * (k.abs() <= sup)
        amp = PI_M14 * dil / (s.sqrt() if self.norm == "l2" else s)
        w0_ = torch.as_tensor(w0, dtype=f64)
        w0t = w0_ * t
        re = (torch.cos(w0t) - torch.exp(-0.5 * w0_ * w0_)) * env * amp
        if not self.complex:
            return re.to(dtype)
        im = torch.sin(w0t) * env * amp
        return torch.stack([re, im], 1).reshape(-1, k.shape[1]).to(dtype)


def filterbank_conv(x, h, n_out: int, off: int, dil: int = 1):
    """reference.py:52-66: y[..., f, n] = sum_k h[f, k] x[..., n + off - dil k] (zero outside)."""
    lead, N = x.shape[:-1], x.shape[-1]
    Fn, K = h.shape
    left = dil * (K - 1) - off
    right = n_out + off - N
    xp = F.pad(x.reshape(-1, 1, N), (max(left, 0), max(right, 0)))
    if left < 0:
        xp = xp[..., -left:]
    y = F.conv1d(xp, h.flip(-1).to(x.dtype)[:, None, :], dilation=dil)[..., :n_out]
    return y.reshape(*lead, Fn, n_out)


def _stage_rows(plan: Plan, st):
    j, dil, idx, half, sups = st
    C = plan.channels
    rows = [i * C + c for i in idx for c in range(C)]
    cols = slice(plan.center - half, plan.center + half + 1)
    return rows, cols


def lowpass_step(plan: Plan, xj, j: int, N: int):
    """cwt.py:512-519 / 582: x_{j+1} on [-m_{j+1}, N + m_{j+1}) from x_j on [-m_j, N + m_j)."""
    mj, m1 = plan.margins[j], plan.margins[j + 1]
    lp = plan.lowpass.to(xj.dtype)
    return filterbank_conv(xj, lp[None], N + 2 * m1, mj - m1 + plan.c_lp * 2 ** j, 2 ** j)[:, 0]


def torch_cwt(x, plan: Plan, H) -> torch.Tensor:
    """cwt.py:562-583: the pyramid. x (R, N) -> (R, S, N, C)."""
    R, N = x.shape
    C = plan.channels
    out = x.new_zeros((R, plan.num_scales, N, C))
    by_oct = {st[0]: st for st in plan.stages}
    xj = x
    for j in range(plan.n_octaves):
        dil, mj = 2 ** j, plan.margins[j]
        if j in by_oct:
            st = by_oct[j]
            rows, cols = _stage_rows(plan, st)
            h = H[rows][:, cols]
            if plan.method == "fft":
                y = fft_conv(xj, h, N, mj + st[3] * dil)
            else:
                y = filterbank_conv(xj, h, N, mj + st[3] * dil, dil)
            y = y.reshape(R, len(st[2]), C, N).transpose(-1, -2)
            out = out.index_copy(1, torch.tensor(st[2]), y.to(out.dtype))
        if j + 1 < plan.n_octaves:
            xj = lowpass_step(plan, xj, j, N)
    return out


def fft_conv(x, h, n_out, off):
    """cwt.py:586-594."""
    R, N = x.shape
    K = h.shape[1]
    nfft = 1 << (N + K - 1 - 1).bit_length()
    X = torch.fft.rfft(x.to(h.dtype), nfft)
    Hf = torch.fft.rfft(h, nfft)
    y = torch.fft.irfft(X[:, None, :] * Hf[None], nfft)
    return y[..., off:off + n_out]


def apply_plan(x, plan: Plan, H):
    """cwt.py:600-612 (CPU branch): (..., N) -> (..., S, N) complex (or real)."""
    lead, N = x.shape[:-1], x.shape[-1]
    dt = torch.float64 if x.dtype == torch.float64 else torch.float32
    y = torch_cwt(x.reshape(-1, N).to(dt), plan, H.to(dt))
    y = y.reshape(*lead, plan.num_scales, N, plan.channels)
    return torch.view_as_complex(y) if plan.complex else y[..., 0]


def cwt(x, scales=None, *, freqs=None, fs=1.0, w0=6.0, method="fast", norm="l2", complex=True,
        truncate=4.0):
    """cwt.py:633-651."""
    s = freqs_to_scales(freqs, fs, w0) if freqs is not None else torch.as_tensor(scales, dtype=torch.float64)
    plan = Plan([float(v) for v in s.flatten()], w0, truncate, norm, complex, method)
    H = plan.filters(torch.tensor(plan.scales, dtype=torch.float64), plan.w0)
    return apply_plan(x, plan, H)


def morlet_mix(x, plan: Plan, H, a, b):
    """cwt.py:391-394: sum_s a[d, s] |W_s| + b[d, s] Re W_s, x (B, D, N)."""
    w = apply_plan(x, plan, H)
    mag = w.abs()
    re = w.real if plan.complex else w
    return (torch.einsum("bdsn,ds->bdn", mag, a.to(mag.dtype))
            + torch.einsum("bdsn,ds->bdn", re, b.to(mag.dtype)))


def spectral_softmax(x, plan: Plan, H, V, nch: int, tau: float = 1.0):
    """cwt.py:545-549: sum_f softmax_f(|W_f x| / tau) V_f, x (R, N)."""
    R, N = x.shape
    p = torch.softmax(apply_plan(x, plan, H).abs() / tau, dim=-2)
    p = p.view(-1, nch, p.shape[1], N)
    V = V.to(p.dtype)
    Vb = V[None, :, :, None] if V.dim() == 2 else V[:, None]
    return (p * Vb).sum(2).reshape(R, N)


def attention(x, plan: Plan, H, freq_weight, tau):
    """layers.py:155-162, 216-218: MorletAttention on x (B, H, C, T, D)."""
    B, Hh, C, T, D = x.shape
    out = spectral_softmax(x.reshape(B * Hh * C, T * D), plan, H, freq_weight, C, tau)
    return out.reshape(B, Hh, C, T, D).to(x.dtype)


def channel_mix_attention(x, plan: Plan, H, freq_to_channel, tau):
    """layers.py:257-262: U = M x, then the per-position spectral softmax."""
    B, Hh, C, T, D = x.shape
    dt = torch.float64 if x.dtype == torch.float64 else torch.float32
    v = x.reshape(B, Hh, C, T * D).to(dt)
    U = torch.einsum("fk,bhkn->bhfn", freq_to_channel.to(dt), v)
    out = spectral_softmax(x.reshape(B * Hh * C, T * D), plan, H,
                           U.reshape(B * Hh, plan.num_scales, T * D), C, tau)
    return out.reshape(B, Hh, C, T, D).to(x.dtype)


def token_mixer(x, plan: Plan, H, mag_weight, phase_weight, bias, proj_w=None, proj_b=None):
    """layers.py:66-72: (B, L, dim) -> (B, L, dim)."""
    y = morlet_mix(x.transpose(1, 2), plan, H, mag_weight, phase_weight)
    y = y.transpose(1, 2) + bias
    y = y.to(x.dtype)
    return y if proj_w is None else F.linear(y, proj_w, proj_b)


def stage_list(plan: Plan) -> List[list]:
    """Flattened (octave, dil, scale index, half, support) rows, as the fixtures store them."""
    return [[j, dil, i, half, c] for j, dil, idx, half, sups in plan.stages
            for i, c in zip(idx, sups)]
