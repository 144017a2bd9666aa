"""Pins the DWT oracle (oracle/dwt.py) before anything is checked against it.

Independent anchors: PyWavelets 1.1.1 golden vectors, MATLAB R2012a known answers,
numpy.pad as a second implementation of the four padding modes, the Haar closed form,
adjointness of analysis and synthesis in every mode.
"""

import math

import numpy as np
import pytest
import torch

from oracle import dwt as O
from golden_io import load, pywt_input

MODES = list(O.MODES)
G = load("pywt_dwt.npz")
WAVELETS = [str(w) for w in G["wavelets"]]
SIZES = sorted({int(k.split("/")[3]) for k in G.files if k.startswith("dwt/")})


@pytest.mark.parametrize("wavelet", WAVELETS)
@pytest.mark.parametrize("mode", MODES)
def test_dwt_idwt_match_pywt(wavelet, mode):
    """Grid of the reference's tests/test_dwt.py:21-39."""
    for n in SIZES:
        key = f"dwt/{wavelet}/{mode}/{n}"
        if key + "/seed" not in G.files:
            continue
        x = torch.from_numpy(pywt_input(G[key + "/seed"], (3, n)))
        if key + "/err" in G.files:
            continue
        a, d = O.dwt(x, wavelet, mode)
        np.testing.assert_allclose(a.numpy(), G[key + "/a"], atol=1e-12, rtol=0)
        np.testing.assert_allclose(d.numpy(), G[key + "/d"], atol=1e-12, rtol=0)
        if key + "/idwt" in G.files:
            y = O.idwt(a, d, wavelet, mode)
            np.testing.assert_allclose(y.numpy(), G[key + "/idwt"], atol=1e-12, rtol=0)
        if key + "/idwt_rand" in G.files:
            seed = int(G[key + "/seed"])
            ca = torch.from_numpy(np.random.RandomState(seed + 100000).standard_normal(a.shape))
            cd = torch.from_numpy(np.random.RandomState(seed + 200000).standard_normal(a.shape))
            y = O.idwt(ca, cd, wavelet, mode)
            np.testing.assert_allclose(y.numpy(), G[key + "/idwt_rand"], atol=1e-12, rtol=0)
            if key + "/idwt_a_only" in G.files:
                y = O.idwt(ca, None, wavelet, mode)
                np.testing.assert_allclose(y.numpy(), G[key + "/idwt_a_only"], atol=1e-12, rtol=0)


@pytest.mark.parametrize("wavelet", [str(w) for w in G["dec_wavelets"]])
@pytest.mark.parametrize("mode", MODES)
def test_wavedec_waverec_match_pywt(wavelet, mode):
    """tests/test_dwt.py:42-55 of the reference, all five modes."""
    for n in (64, 1000, 4097):
        key = f"dec/{wavelet}/{mode}/{n}"
        if key + "/seed" not in G.files:
            continue
        x = torch.from_numpy(pywt_input(G[key + "/seed"], (1, n)))
        coeffs = O.wavedec(x, wavelet, mode)
        assert len(coeffs) == int(G[key + "/nlev"])
        for i, c in enumerate(coeffs):
            np.testing.assert_allclose(c.numpy(), G[key + f"/c{i}"], atol=1e-11, rtol=0)
        rec = O.waverec(coeffs, wavelet, mode)
        if key + "/rec" in G.files:
            np.testing.assert_allclose(rec.numpy(), G[key + "/rec"], atol=1e-11, rtol=0)
        np.testing.assert_allclose(rec[..., :n].numpy(), x.numpy(), atol=1e-10, rtol=0)
        if key + "/nlev2" in G.files:
            c2 = O.wavedec(x, wavelet, mode, level=2)
            for i, c in enumerate(c2):
                np.testing.assert_allclose(c.numpy(), G[key + f"/l2c{i}"], atol=1e-11, rtol=0)


def test_dwt_max_level_matches_pywt():
    for n, L, lvl in G["max_level"]:
        assert O.dwt_max_level(int(n), int(L)) == int(lvl)


K = load("matlab_dwt_kat.npz")
KAT_WAVELETS = [str(w) for w in K["wavelets"]]


@pytest.mark.parametrize("mode", MODES)
def test_matlab_known_answers(mode):
    """MATLAB R2012a dwt, run with the same filter coefficients (``_pywtCoeffs``): pins the
    five extension modes independently of PyWavelets' implementation."""
    checked = 0
    for w in KAT_WAVELETS:
        L0 = len(O._table()[w][0])
        for N in (L0, L0 + 1):
            x = torch.from_numpy(K[f"{w}/{N}/x"][None])
            a, d = O.dwt(x, w, mode)
            for part, got in (("ma", a), ("md", d)):
                ref = K[f"{w}/{N}/{mode}/{part}_pywtCoeffs"]
                np.testing.assert_allclose(got[0].numpy(), ref, rtol=1e-10,
                                           atol=1e-10 * np.abs(ref).max())
                checked += 1
    assert checked == 4 * len(KAT_WAVELETS)


def test_filter_table_matches_matlab_builtin_filters():
    """MATLAB's own filters (not PyWavelets') in symmetric mode: pins the coefficient table.
    MATLAB derives db26..db38, coif4 and coif5 numerically and stores them less precisely
    (differences up to 6e-5); every other bank agrees to 1e-9."""
    loose = {f"db{i}" for i in range(26, 39)} | {"coif4", "coif5"}
    for w in KAT_WAVELETS:
        L0 = len(O._table()[w][0])
        x = torch.from_numpy(K[f"{w}/{L0}/x"][None])
        a, d = O.dwt(x, w, "symmetric")
        tol = 1e-4 if w in loose else 1e-9
        np.testing.assert_allclose(a[0].numpy(), K[f"{w}/{L0}/symmetric/ma"], rtol=0, atol=tol)
        np.testing.assert_allclose(d[0].numpy(), K[f"{w}/{L0}/symmetric/md"], rtol=0, atol=tol)


NP_PAD = {"zero": "constant", "periodic": "wrap", "symmetric": "symmetric", "reflect": "reflect"}


def _np_pad_analysis(x, h0, h1, mode, L):
    """Second implementation of one analysis level: explicit numpy.pad extension, then a
    literal loop.  Periodization pads an odd signal with its last sample, then wraps."""
    n = x.shape[-1]
    if mode == "periodization":
        xe = np.concatenate([x, x[-1:]]) if n % 2 else x
        off, n_out, padmode = L // 2, (n + 1) // 2, "wrap"
    else:
        xe, off, n_out, padmode = x, 1, (n + L - 1) // 2, NP_PAD[mode]
    pad = 4 * L + 8
    if padmode == "reflect" and xe.shape[0] == 1:
        padmode = "wrap"  # the reference's rule for reflect on one sample
    xp = np.pad(xe, (pad, pad), mode=padmode)
    y0 = np.zeros(n_out)
    y1 = np.zeros(n_out)
    for o in range(n_out):
        for j in range(L):
            v = xp[pad + 2 * o + off - j]
            y0[o] += h0[j] * v
            y1[o] += h1[j] * v
    return y0, y1


@pytest.mark.parametrize("mode", MODES)
def test_analysis_matches_numpy_pad(mode):
    rng = np.random.RandomState(5)
    for w in ["haar", "db2", "db4", "sym8", "coif3", "bior3.5"]:
        f = O.bank(w)
        L = len(f[0])
        for n in [1, 2, 3, 4, 5, 7, 9, 16, 31]:
            x = rng.standard_normal(n)
            a, d = O.dwt(torch.from_numpy(x[None]), w, mode)
            y0, y1 = _np_pad_analysis(x, f[0], f[1], mode, L)
            np.testing.assert_allclose(a[0].numpy(), y0, atol=1e-12, rtol=0)
            np.testing.assert_allclose(d[0].numpy(), y1, atol=1e-12, rtol=0)


@pytest.mark.parametrize("mode", MODES)
def test_synthesis_is_adjoint(mode):
    m = O.MODES[mode]
    rng = np.random.RandomState(6)
    for w in ["haar", "db3", "sym8", "bior3.5"]:
        f = O.bank(w)
        h0, h1 = torch.tensor(f[0]), torch.tensor(f[1])
        L = h0.numel()
        off = L // 2 if m == O.PERIODIZATION else 1
        for n in [1, 2, 3, 5, 8, 13, 40]:
            n_out = O.coeff_len(n, L, mode)
            x = torch.from_numpy(rng.standard_normal((2, n)))
            ya = torch.from_numpy(rng.standard_normal((2, n_out)))
            yd = torch.from_numpy(rng.standard_normal((2, n_out)))
            a, d = O.analysis(x, h0, h1, m, off, n_out)
            xt = O.synthesis(ya, yd, h0, h1, m, off, n)
            lhs = (a * ya).sum() + (d * yd).sum()
            rhs = (x * xt).sum()
            assert abs(float(lhs - rhs)) < 1e-11 * (1 + abs(float(lhs)))


def test_haar_closed_form():
    x = torch.tensor([[3.0, 1.0, -2.0, 5.0]], dtype=torch.float64)
    a, d = O.dwt(x, "haar", "periodization")
    s = 1 / math.sqrt(2)
    np.testing.assert_allclose(a.numpy(), [[4 * s, 3 * s]], atol=1e-15)
    np.testing.assert_allclose(d.numpy(), [[2 * s, -7 * s]], atol=1e-15)


def test_reflect_single_sample_is_periodic():
    """kernels/dwt.py:47-49 of the reference (PyWavelets 1.1.1 cannot evaluate this case)."""
    x = torch.tensor([[1.7], [-0.3]], dtype=torch.float64)
    for w in ["haar", "db4", "sym5"]:
        for a, b in zip(O.dwt(x, w, "reflect"), O.dwt(x, w, "periodic")):
            torch.testing.assert_close(a, b, rtol=0, atol=0)
