"""Pins the oracle's module compositions (oracle/cwt.py: attention, channel_mix_attention,
token_mixer; oracle/dwt.py + torch for the wavelet token mixer) on the CPU.

Anchors: the outputs and gradients that the reference's own modules wrote in float64
(tests/golden/make_cwt_golden.py: ``mod/*`` for MorletAttention / MorletChannelMixAttention
at the reference test shapes, ``tm/*`` for MorletTokenMixer), with the modules' stored
parameters.  The oracle rebuilds each module from its definition (layers.py:112-262 and
26-72 of the reference): the default frequency grid, the learnable plan's support margin,
the filters at the stored log-scales and w0, then the CPU pyramid.  Gradients are autograd
through that composition.  The wavelet token mixer has no reference fixture: its oracle is
the composition of ``oracle.dwt.wavedec`` / ``waverec`` (pinned by PyWavelets) and
``torch.nn.functional.linear``, checked here against a dense-matrix form of the same map.
"""

import math

import numpy as np
import pytest
import torch

from golden_io import load
from oracle import cwt as O
from oracle import dwt as OD

G = load("cwt_golden.npz")
f64 = torch.float64

MODS = {
    "att": ("att", dict(num_channels=5, hidden_dim=64, temperature=0.5)),
    "cmix": ("cmix", dict(num_channels=5, hidden_dim=64, temperature=0.5)),
    "att_big": ("att", dict(num_channels=2, hidden_dim=100, temperature=0.01)),
    "att_f4": ("att", dict(num_channels=4, hidden_dim=128, freqs=[2.0, 6.0, 12.0, 25.0])),
    "cmix_f4": ("cmix", dict(num_channels=4, hidden_dim=128, freqs=[2.0, 6.0, 12.0, 25.0])),
}


def _params(prefix):
    n = len(f"{prefix}/param/")
    return {k[n:]: torch.from_numpy(G[k]).clone() for k in G.files
            if k.startswith(f"{prefix}/param/")}


def _patch_plan(kw):
    """layers.py:112-139: fs = hidden_dim / patch_duration, default frequency grid,
    learnable scales and w0 (support margin 1.25)."""
    fs = kw["hidden_dim"] / 1.0
    freqs = kw.get("freqs")
    if freqs is None:
        f_max = min(40.0, fs / 4)
        freqs = torch.logspace(0, math.log10(max(f_max, 1.5)), 16).tolist()
    scales = O.freqs_to_scales(freqs, fs, 6.0).tolist()
    return O.Plan(scales, support_margin=1.25)


@pytest.mark.parametrize("name", sorted(MODS))
def test_attention_oracles_match_reference_modules(name):
    kind, kw = MODS[name]
    prefix = f"mod/{name}"
    p = _params(prefix)
    plan = _patch_plan(kw)
    ls = p["cwt.log_scales"].requires_grad_()
    w0 = p["cwt.w0"].requires_grad_()
    wname = "freq_weight" if kind == "att" else "freq_to_channel"
    W = p[wname].requires_grad_()
    x = torch.from_numpy(G[f"{prefix}/x"]).clone().requires_grad_()
    H = plan.filters(ls.exp(), w0)
    tau = kw.get("temperature", 1.0)
    if kind == "att":
        y = O.attention(x, plan, H, W, tau)
    else:
        y = O.channel_mix_attention(x, plan, H, W, tau)
    y.square().sum().backward()
    tol = 1e-11
    for nm, got in (("y", y.detach()), ("gx", x.grad), (f"grad/{wname}", W.grad),
                    ("grad/cwt.log_scales", ls.grad), ("grad/cwt.w0", w0.grad)):
        ref = G[f"{prefix}/{nm}"]
        np.testing.assert_allclose(got.numpy(), ref, rtol=0,
                                   atol=tol * max(np.abs(ref).max(), 1e-300), err_msg=nm)


TMS = {"tm_f3": dict(scales=None, freqs=[2.0, 8.0, 30.0], fs=250.0),
       "tm_nophase": dict(scales=torch.logspace(0, 6, 16, base=2).tolist(), freqs=None, fs=1.0)}


@pytest.mark.parametrize("name", sorted(TMS))
def test_token_mixer_oracle_matches_reference_module(name):
    kw = TMS[name]
    prefix = f"tm/{name}"
    p = _params(prefix)
    scales = (O.freqs_to_scales(kw["freqs"], kw["fs"], 6.0).tolist() if kw["freqs"] is not None
              else kw["scales"])
    plan = O.Plan(scales, support_margin=1.25)
    for v in p.values():
        v.requires_grad_()
    x = torch.from_numpy(G[f"{prefix}/x"]).clone().requires_grad_()
    H = plan.filters(p["cwt.log_scales"].exp(), plan.w0)
    y = O.token_mixer(x, plan, H, p["mag_weight"], p["phase_weight"], p["bias"],
                      p["out_proj.weight"], p["out_proj.bias"])
    y.square().mean().backward()
    np.testing.assert_allclose(y.detach().numpy(), G[f"{prefix}/y"], rtol=0,
                               atol=1e-11 * np.abs(G[f"{prefix}/y"]).max())
    np.testing.assert_allclose(x.grad.numpy(), G[f"{prefix}/gx"], rtol=0,
                               atol=1e-11 * np.abs(G[f"{prefix}/gx"]).max())
    for pn, v in p.items():
        key = f"{prefix}/grad/{pn}"
        if key in G.files:
            ref = G[key]
            np.testing.assert_allclose(v.grad.numpy(), ref, rtol=0,
                                       atol=1e-11 * max(np.abs(ref).max(), 1e-300), err_msg=pn)


def _dense(fn, n):
    """Matrix of a linear map of (n,) signals, column by column."""
    eye = torch.eye(n, dtype=f64)
    return torch.stack([fn(eye[i]) for i in range(n)], 1)


@pytest.mark.parametrize("wavelet,mode,level", [("db4", "periodization", 3), ("sym4", "symmetric", 2),
                                                ("haar", "zero", 4)])
def test_wavelet_token_mixer_oracle_is_the_band_mixing_map(wavelet, mode, level):
    """oracle.dwt.wavelet_token_mixer (layers.py:75-109) with identity band maps reconstructs
    the input (perfect reconstruction), and with affine channel maps (M_j, b_j) it equals
    sum_j Rec_j (Dec_j x M_j^T + b_j), where Dec_j (signal -> band j of wavedec) and Rec_j
    (band j alone -> waverec) are dense matrices built from the PyWavelets-pinned oracle."""
    g = torch.Generator().manual_seed(3)
    B, L, D = 2, 37, 3
    x = torch.randn(B, L, D, generator=g, dtype=f64)
    eye = [(torch.eye(D, dtype=f64), torch.zeros(D, dtype=f64))] * (level + 1)
    y = OD.wavelet_token_mixer(x, wavelet, mode, level, eye)
    torch.testing.assert_close(y, x, rtol=1e-10, atol=1e-10)

    bands = [(torch.randn(D, D, generator=g, dtype=f64), torch.randn(D, generator=g, dtype=f64))
             for _ in range(level + 1)]
    y = OD.wavelet_token_mixer(x, wavelet, mode, level, bands)
    shapes = [c.shape[-1] for c in OD.wavedec(torch.zeros(1, L, dtype=f64), wavelet, mode, level)]
    ref = torch.zeros_like(x)
    for j, (M, b) in enumerate(bands):
        dec = _dense(lambda s: OD.wavedec(s[None], wavelet, mode, level)[j][0], L)  # (n_j, L)

        def rec_j(c, j=j):
            cs = [torch.zeros(1, n, dtype=f64) for n in shapes]
            cs[j] = c[None]
            return OD.waverec(cs, wavelet, mode)[0, :L]

        rec = _dense(rec_j, shapes[j])  # (L, n_j)
        coef = torch.einsum("nl,bld->bnd", dec, x) @ M.t() + b
        ref = ref + torch.einsum("ln,bnd->bld", rec, coef)
    torch.testing.assert_close(y, ref, rtol=1e-10, atol=1e-10)
