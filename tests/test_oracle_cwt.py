"""Pins the CWT / mix / spectral-softmax oracle (oracle/cwt.py).

Anchors: plan metadata, filters, outputs and gradients written by the reference's own CPU
path (tests/golden/make_cwt_golden.py), the literal O(N^2) Morlet CWT definition
(reference tests/test_cwt.py:16-37), and the fast-vs-direct tolerance (test_cwt.py:40-52).
"""

import math

import numpy as np
import pytest
import torch

from oracle import cwt as O
from golden_io import cwt_compare, load

G = load("cwt_golden.npz")
PLANS = sorted({k.split("/")[1] for k in G.files if k.startswith("plan/")})
FREQS = np.geomspace(0.5, 100, 24)
f64 = torch.float64


def plan_from_fixture(name):
    kw = {k[len(f"plan/{name}/kw_"):]: G[k].item() for k in G.files
          if k.startswith(f"plan/{name}/kw_")}
    return O.Plan(G[f"plan/{name}/scales"].tolist(), **kw)


@pytest.mark.parametrize("name", PLANS)
def test_plan_matches_reference(name):
    p = plan_from_fixture(name)
    assert p.n_octaves == int(G[f"plan/{name}/n_octaves"])
    assert p.center == int(G[f"plan/{name}/center"])
    assert p.margins == G[f"plan/{name}/margins"].tolist()
    assert p.c_lp == int(G[f"plan/{name}/c_lp"])
    assert O.stage_list(p) == G[f"plan/{name}/stages"].tolist()
    np.testing.assert_allclose(p.lowpass.numpy(), G[f"plan/{name}/lowpass"], rtol=0, atol=1e-16)
    assert abs(p.s_th - float(G[f"plan/{name}/s_th"])) < 1e-14
    if f"plan/{name}/H" in G.files:
        H = p.filters(torch.tensor(p.scales, dtype=f64), p.w0)
        np.testing.assert_allclose(H.numpy(), G[f"plan/{name}/H"], rtol=0, atol=1e-15)


CASES = {
    "fast_n7": dict(method="fast"), "fast_n500": dict(method="fast"),
    "fast_n3000": dict(method="fast"), "direct_n500": dict(method="direct"),
    "fast_t5_n4000": dict(method="fast", truncate=5.0),
    "fast_l1_real_n900": dict(method="fast", norm="l1", complex=False),
    "fast_w05_n1100": dict(method="fast", w0=5.0),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_cwt_values_match_reference(case):
    x = torch.from_numpy(G[f"cwt/{case}/x"])
    y = O.cwt(x, freqs=FREQS, fs=250.0, **CASES[case])
    cwt_compare(y, G, f"cwt/{case}/y", 1e-12)


def test_cwt_cfg3_signal_matches_reference():
    x = torch.from_numpy(G["cwt/cfg3/x"])
    y = O.cwt(x, freqs=np.logspace(-0.3, 2, 40), fs=250.0)
    cwt_compare(y, G, "cwt/cfg3/y", 1e-12)


def _naive_cwt(x, scales, w0=6.0, truncate=4.0):
    """Literal definition W[s, n] = sum_m x[m] conj(psi((m - n) / s)) / sqrt(s)."""
    N = x.shape[-1]
    m = torch.arange(N, dtype=f64)
    out = []
    for s in scales:
        t = (m[None, :] - m[:, None]) / s
        env = torch.exp(-0.5 * t ** 2) * ((m[None, :] - m[:, None]).abs() <= math.ceil(truncate * s))
        psi = math.pi ** -0.25 * (torch.exp(1j * w0 * t) - math.exp(-w0 ** 2 / 2)) * env
        out.append((x.to(torch.complex128) @ psi.conj().T) / math.sqrt(s))
    return torch.stack(out, -2)


def test_direct_and_fft_match_definition():
    torch.manual_seed(0)
    x = torch.randn(2, 300, dtype=f64)
    scales = [1.0, 2.5, 7.0, 30.0]
    ref = _naive_cwt(x, scales)
    for method in ("direct", "fft"):
        torch.testing.assert_close(O.cwt(x, scales, method=method), ref, atol=1e-12, rtol=0)


@pytest.mark.parametrize("n", [7, 500, 3000])
def test_fast_close_to_direct(n):
    torch.manual_seed(0)
    x = torch.randn(3, n, dtype=f64)
    ref = O.cwt(x, freqs=FREQS, fs=250, method="direct")
    fast = O.cwt(x, freqs=FREQS, fs=250, method="fast")
    scale = ref.abs().max()
    assert ((fast - ref).abs().max() / scale) < 3e-4
    torch.testing.assert_close(fast[..., -4:, :], ref[..., -4:, :], atol=1e-12 * scale, rtol=0)


@pytest.mark.parametrize("key", ["fast_c", "fast_r", "direct_c", "direct_r"])
def test_cwt_gradients_match_reference(key):
    method, cplx = key.split("_")[0], key.endswith("_c")
    x = torch.from_numpy(G[f"grad/{key}/x"])
    g = torch.Generator().manual_seed(int(G[f"grad/{key}/gy_seed"]))
    torch.randn(3, 2, 600, generator=g, dtype=f64)  # the fixture drew x from this stream first
    gy = torch.randn(3, 2, len(FREQS), 600, 2 if cplx else 1, generator=g, dtype=f64)
    scales = O.freqs_to_scales(FREQS, 250.0)
    plan = O.Plan(scales.tolist(), complex=cplx, method=method, support_margin=1.25)
    ls = torch.tensor(plan.scales, dtype=f64).log().float().to(f64).requires_grad_()
    w0 = torch.tensor(6.0, dtype=f64, requires_grad=True)
    xx = x.clone().requires_grad_()
    y = O.apply_plan(xx, plan, plan.filters(ls.exp(), w0))
    yr = torch.view_as_real(y) if cplx else y[..., None]
    (yr * gy).sum().backward()
    cwt_compare(yr.movedim(-1, -2), G, f"grad/{key}/y", 1e-11)
    cwt_compare(xx.grad, G, f"grad/{key}/gx", 1e-11)
    np.testing.assert_allclose(ls.grad.numpy(), G[f"grad/{key}/g_log_scales"], rtol=1e-9,
                               atol=1e-10 * np.abs(G[f"grad/{key}/g_log_scales"]).max())
    np.testing.assert_allclose(w0.grad.numpy(), G[f"grad/{key}/g_w0"], rtol=1e-9)


@pytest.mark.parametrize("key", ["fast_c", "fast_r", "direct_c", "direct_r"])
def test_mix_matches_reference(key):
    method, cplx = key.split("_")[0], key.endswith("_c")
    plan = O.Plan(O.freqs_to_scales(np.geomspace(1, 60, 12), 250.0).tolist(), complex=cplx,
                  method=method, support_margin=1.25)
    ls = torch.tensor(plan.scales, dtype=f64).log().float().to(f64).requires_grad_()
    x, a, b, gy = (torch.from_numpy(G[f"mix/{key}/{n}"]) for n in ("x", "a", "b", "gy"))
    xx, aa, bb = (t.clone().requires_grad_() for t in (x, a, b))
    y = O.morlet_mix(xx, plan, plan.filters(ls.exp(), plan.w0), aa, bb)
    (y * gy).sum().backward()
    cwt_compare(y, G, f"mix/{key}/y", 1e-11)
    cwt_compare(xx.grad, G, f"mix/{key}/gx", 1e-11)
    for nm, got in (("ga", aa.grad), ("gb", bb.grad), ("g_log_scales", ls.grad)):
        ref = G[f"mix/{key}/{nm}"]
        np.testing.assert_allclose(got.numpy(), ref, rtol=0, atol=1e-11 * np.abs(ref).max())


@pytest.mark.parametrize("key", ["ch", "pos"])
def test_spectral_softmax_matches_reference(key):
    plan = O.Plan([1.5, 3.0, 7.0, 13.0, 26.0], support_margin=1.25)
    x, V, gy = (torch.from_numpy(G[f"ssm/{key}/{n}"]) for n in ("x", "V", "gy"))
    ls = torch.tensor(plan.scales, dtype=f64).log().float().to(f64).requires_grad_()
    w0 = torch.tensor(6.0, dtype=f64, requires_grad=True)
    xx, VV = x.clone().requires_grad_(), V.clone().requires_grad_()
    y = O.spectral_softmax(xx, plan, plan.filters(ls.exp(), w0), VV, 3, 0.7)
    (y * gy).sum().backward()
    for nm, got in (("y", y), ("gx", xx.grad), ("gV", VV.grad), ("g_log_scales", ls.grad),
                    ("g_w0", w0.grad)):
        ref = G[f"ssm/{key}/{nm}"]
        np.testing.assert_allclose(got.detach().numpy(), ref, rtol=0,
                                   atol=1e-11 * max(np.abs(ref).max(), 1e-300))
