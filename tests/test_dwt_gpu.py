"""DWT parity on the GPU: HIP kernels vs PyWavelets fixtures and the CPU oracle.

Tolerances: float64 to 1e-12 (pywt grid, as the reference's tests/test_dwt.py:21-55) and
float32 to rtol 1e-5 / atol 1e-6 (the north-star parity bar), float16 / bfloat16 as the
reference's test_low_precision_dtypes (1e-2 / 6e-2 of the max).
"""

import numpy as np
import pytest
import torch
from torch.autograd import gradcheck, gradgradcheck

import pytorch_morlet_fdwt_amd as fdwt
from golden_io import load, pywt_input
from oracle import dwt as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
MODES = list(O.MODES)
G = load("pywt_dwt.npz")


@pytest.mark.parametrize("mode", MODES)
def test_dwt_idwt_match_pywt(mode):
    for wavelet in [str(w) for w in G["wavelets"]]:
        for n in (1, 2, 3, 5, 7, 8, 13, 16, 33, 40, 100, 257):
            key = f"dwt/{wavelet}/{mode}/{n}"
            if key + "/seed" not in G.files or key + "/err" in G.files:
                continue
            x = torch.from_numpy(pywt_input(G[key + "/seed"], (3, n))).to(DEV)
            a, d = fdwt.dwt(x, wavelet, mode)
            np.testing.assert_allclose(a.cpu().numpy(), G[key + "/a"], atol=1e-12, rtol=0,
                                       err_msg=key)
            np.testing.assert_allclose(d.cpu().numpy(), G[key + "/d"], atol=1e-12, rtol=0,
                                       err_msg=key)
            if key + "/idwt" in G.files:
                y = fdwt.idwt(a, d, wavelet, mode)
                np.testing.assert_allclose(y.cpu().numpy(), G[key + "/idwt"], atol=1e-12,
                                           rtol=0, err_msg=key)
            if key + "/idwt_rand" in G.files:
                seed = int(G[key + "/seed"])
                ca = torch.from_numpy(np.random.RandomState(seed + 100000).standard_normal(a.shape))
                cd = torch.from_numpy(np.random.RandomState(seed + 200000).standard_normal(a.shape))
                y = fdwt.idwt(ca.to(DEV), cd.to(DEV), wavelet, mode)
                np.testing.assert_allclose(y.cpu().numpy(), G[key + "/idwt_rand"], atol=1e-12,
                                           rtol=0, err_msg=key)
                if key + "/idwt_a_only" in G.files:
                    y = fdwt.idwt(ca.to(DEV), None, wavelet, mode)
                    np.testing.assert_allclose(y.cpu().numpy(), G[key + "/idwt_a_only"],
                                               atol=1e-12, rtol=0, err_msg=key)


@pytest.mark.parametrize("mode", MODES)
def test_wavedec_waverec_match_pywt(mode):
    for wavelet in [str(w) for w in G["dec_wavelets"]]:
        for n in (64, 1000, 4097):
            key = f"dec/{wavelet}/{mode}/{n}"
            if key + "/seed" not in G.files:
                continue
            x = torch.from_numpy(pywt_input(G[key + "/seed"], (1, n))).to(DEV)
            coeffs = fdwt.wavedec(x, wavelet, mode)
            assert len(coeffs) == int(G[key + "/nlev"])
            for i, c in enumerate(coeffs):
                np.testing.assert_allclose(c.cpu().numpy(), G[key + f"/c{i}"], atol=1e-11,
                                           rtol=0, err_msg=key)
            rec = fdwt.waverec(coeffs, wavelet, mode)
            if key + "/rec" in G.files:
                np.testing.assert_allclose(rec.cpu().numpy(), G[key + "/rec"], atol=1e-11,
                                           rtol=0, err_msg=key)
            np.testing.assert_allclose(rec[..., :n].cpu().numpy(), x.cpu().numpy(), atol=1e-10,
                                       rtol=0, err_msg=key)


def _rand(shape, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64).to(dtype)


# filter lengths on the templated path (<= 32 taps) and the runtime-length path (> 32)
LONG = ["coif5", "db17", "dmey", "coif17"]


@pytest.mark.parametrize("mode", MODES)
def test_dwt_matches_oracle_all_lengths(mode):
    seed = 0
    for wavelet in ["haar", "db2", "db4", "sym8", "coif3", "bior3.5", "db10", "sym16"] + LONG:
        for n in (1, 2, 9, 64, 255, 2500, 5001):
            seed += 1
            x = _rand((3, n), seed)
            a, d = fdwt.dwt(x.to(DEV), wavelet, mode)
            ra, rd = O.dwt(x, wavelet, mode)
            torch.testing.assert_close(a.cpu(), ra, atol=1e-12, rtol=1e-12)
            torch.testing.assert_close(d.cpu(), rd, atol=1e-12, rtol=1e-12)
            y = fdwt.idwt(a, d, wavelet, mode)
            torch.testing.assert_close(y.cpu(), O.idwt(ra, rd, wavelet, mode), atol=1e-12,
                                       rtol=1e-12)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_wavedec_waverec_match_oracle(mode, dtype):
    tol = dict(atol=1e-12, rtol=1e-12) if dtype == torch.float64 else dict(atol=1e-6, rtol=1e-5)
    seed = 100
    for wavelet in ["db4", "sym8", "coif3", "haar", "bior2.2", "coif5", "dmey"]:
        for n, level in ((2500, 5), (16384, 6), (16383, 6), (777, None), (40, None)):
            seed += 1
            x = _rand((2, 3, n), seed)
            coeffs = fdwt.wavedec(x.to(DEV, dtype), wavelet, mode, level)
            ref = O.wavedec(x, wavelet, mode, level)
            assert len(coeffs) == len(ref)
            for c, r in zip(coeffs, ref):
                assert c.dtype == dtype
                torch.testing.assert_close(c.cpu().double(), r, **tol)
            rec = fdwt.waverec(coeffs, wavelet, mode)
            rref = O.waverec([r for r in ref], wavelet, mode)
            # the round trip chains 2 x level transforms: the reference's own fp32 CPU path
            # misses the exact result by up to ~1.1e-6 on unit-variance rows (measured), so
            # atol scales with the signal magnitude there
            rtol_ = tol["rtol"]
            atol_ = tol["atol"] * (1.0 if dtype == torch.float64 else max(1.0, rref.abs().max().item()))
            torch.testing.assert_close(rec.cpu().double(), rref, atol=atol_, rtol=rtol_)


@pytest.mark.parametrize("mode", MODES)
def test_fused_backward_matches_oracle(mode):
    """wavedec + waverec forward and backward against torch autograd through the oracle."""
    for wavelet, n, level in (("db4", 2500, 5), ("sym8", 2049, 4), ("coif3", 1001, 3)):
        x = _rand((4, n), 7)
        xg = x.to(DEV).requires_grad_()
        xc = x.clone().requires_grad_()
        cg = fdwt.wavedec(xg, wavelet, mode, level)
        cc = O.wavedec(xc, wavelet, mode, level)
        wts = [_rand(c.shape, 11 + i) for i, c in enumerate(cc)]
        yg = fdwt.waverec([c * w.to(DEV) for c, w in zip(cg, wts)], wavelet, mode)
        yc = O.waverec([c * w for c, w in zip(cc, wts)], wavelet, mode)
        torch.testing.assert_close(yg.detach().cpu(), yc.detach(), atol=1e-12, rtol=1e-12)
        gy = _rand(yc.shape, 23)
        (yg * gy.to(DEV)).sum().backward()
        (yc * gy).sum().backward()
        torch.testing.assert_close(xg.grad.cpu(), xc.grad, atol=1e-11, rtol=1e-11)


def test_analysis_rows_past_one_launch():
    """A launch holds at most 2^32 - 1 threads: the 128-thread analysis chain takes 33,554,431
    rows per launch, so 33,554,433 rows of 2 samples run as two launches over row ranges.
    Rows at the start and end (the second launch) match the oracle; every row matches the
    Haar closed form of its two samples."""
    R = 33_554_433
    x = torch.randn(R, 2, generator=torch.Generator().manual_seed(3))
    xd = x.to(DEV)
    ca, cd = fdwt.wavedec(xd, "haar", "periodization", 1)
    torch.cuda.synchronize()
    for sl in (slice(0, 4), slice(R - 4, R)):
        ra, rd = O.wavedec(x[sl].double(), "haar", "periodization", 1)
        torch.testing.assert_close(ca[sl].cpu().double(), ra, atol=1e-6, rtol=1e-6)
        torch.testing.assert_close(cd[sl].cpu().double(), rd, atol=1e-6, rtol=1e-6)
    s = 2 ** -0.5
    torch.testing.assert_close(ca[:, 0], (xd[:, 0] + xd[:, 1]) * s, atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(cd[:, 0].abs(), (xd[:, 0] - xd[:, 1]).abs() * s, atol=1e-6,
                               rtol=1e-6)


@pytest.mark.parametrize("mode", MODES)
def test_chains_deeper_than_one_launch(mode):
    """More levels than one synthesis launch takes (FDWT_SYN_MAX_LEVELS = 16): lengths
    saturate at a few coefficients, as with pywt when level exceeds dwt_max_level."""
    for wavelet, n, level in (("haar", 100, 20), ("db2", 37, 18)):
        x = _rand((3, n), 5)
        xg = x.to(DEV).requires_grad_()
        xc = x.clone().requires_grad_()
        cg = fdwt.wavedec(xg, wavelet, mode, level)
        cc = O.wavedec(xc, wavelet, mode, level)
        for g, c in zip(cg, cc):
            torch.testing.assert_close(g.detach().cpu(), c.detach(), atol=1e-12, rtol=1e-12)
        wts = [_rand(c.shape, 31 + i) for i, c in enumerate(cc)]
        yg = fdwt.waverec([c * w.to(DEV) for c, w in zip(cg, wts)], wavelet, mode)
        yc = O.waverec([c * w for c, w in zip(cc, wts)], wavelet, mode)
        torch.testing.assert_close(yg.detach().cpu(), yc.detach(), atol=1e-12, rtol=1e-12)
        gy = _rand(yc.shape, 41)
        (yg * gy.to(DEV)).sum().backward()
        (yc * gy).sum().backward()
        torch.testing.assert_close(xg.grad.cpu(), xc.grad, atol=1e-11, rtol=1e-11)


@pytest.mark.parametrize("mode", MODES)
def test_gradcheck_and_gradgradcheck(mode):
    """tests/test_dwt.py:58-72 of the reference, on the HIP kernels in float64."""
    for wavelet in ["haar", "db3", "bior3.5"]:
        for n in [1, 2, 5, 8, 13, 40]:
            x = _rand((2, n), n).to(DEV).requires_grad_()
            assert gradcheck(lambda x: fdwt.dwt(x, wavelet, mode), (x,))
            assert gradgradcheck(lambda x: fdwt.dwt(x, wavelet, mode), (x,))
            a, d = (t.detach().requires_grad_() for t in fdwt.dwt(x, wavelet, mode))
            L = fdwt.get_filter_bank(wavelet).length
            if mode == "periodization" or 2 * a.shape[-1] - L + 2 > 0:
                assert gradcheck(lambda a, d: fdwt.idwt(a, d, wavelet, mode), (a, d))
    x = _rand((2, 70), 3).to(DEV).requires_grad_()
    assert gradcheck(lambda x: fdwt.wavedec(x, "db2", mode, 3), (x,))
    assert gradgradcheck(lambda x: fdwt.wavedec(x, "db2", mode, 3), (x,))
    cs = [c.detach().requires_grad_() for c in fdwt.wavedec(x, "db2", mode, 3)]
    assert gradcheck(lambda *c: fdwt.waverec(list(c), "db2", mode), tuple(cs))
    assert gradgradcheck(lambda *c: fdwt.waverec(list(c), "db2", mode), tuple(cs))


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.float16, 1e-2),
                                       (torch.bfloat16, 6e-2)])
def test_low_precision_dtypes(dtype, tol):
    """tests/test_dwt.py:75-85 of the reference."""
    x = _rand((4, 1000), 0, torch.float32).to(DEV)
    ref = fdwt.wavedec(x.double(), "db4", level=4)
    out = fdwt.wavedec(x.to(dtype), "db4", level=4)
    for o, r in zip(out, ref):
        assert o.dtype == dtype
        torch.testing.assert_close(o.double(), r, atol=tol * r.abs().max().item(), rtol=0)
    rec = fdwt.waverec(out, "db4")
    assert rec.dtype == dtype
    torch.testing.assert_close(rec[..., :1000].double(), x.double(), atol=3 * tol * x.abs().max().item(), rtol=0)


def test_long_rows_and_few_rows():
    """Rows longer than the on-chip chain run their first levels one at a time; few long rows
    spread over several workgroups per row."""
    from pytorch_morlet_fdwt_amd import _lib
    maxlen = _lib.lib().fdwt_chain_max_length(8, 1)
    n = maxlen * 2 + 37
    x = _rand((2, n), 5)
    for mode in ("symmetric", "periodization", "periodic"):
        c = fdwt.wavedec(x.to(DEV), "db4", mode, 4)
        r = O.wavedec(x, "db4", mode, 4)
        for a, b in zip(c, r):
            torch.testing.assert_close(a.cpu(), b, atol=1e-12, rtol=1e-12)
        rec = fdwt.waverec(c, "db4", mode)
        torch.testing.assert_close(rec.cpu(), O.waverec(r, "db4", mode), atol=1e-12, rtol=1e-12)
    x = _rand((3, 200001), 6, torch.float32)
    a, d = fdwt.dwt(x.to(DEV), "sym8", "reflect")
    ra, rd = O.dwt(x.double(), "sym8", "reflect")
    torch.testing.assert_close(a.cpu().double(), ra, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(d.cpu().double(), rd, atol=1e-5, rtol=1e-5)
    y = fdwt.idwt(a, d, "sym8", "reflect")
    torch.testing.assert_close(y.cpu().double(), O.idwt(a.cpu().double(), d.cpu().double(), "sym8",
                                                        "reflect"), atol=1e-5, rtol=1e-5)


def test_chains_at_the_on_chip_limit():
    """Rows exactly as long as the on-chip chain allows (fp32, 16 and 18 taps): the fused
    analysis and synthesis chains of all levels run with LDS close to full."""
    from pytorch_morlet_fdwt_amd import _lib
    for w, taps in (("sym8", 16), ("coif3", 18)):
        n = _lib.lib().fdwt_chain_max_length(taps, 0)
        x = _rand((2, n), 7, torch.float32)
        for mode in ("symmetric", "periodization"):
            c = fdwt.wavedec(x.to(DEV), w, mode, 4)
            r = O.wavedec(x.double(), w, mode, 4)
            for a, b in zip(c, r):
                torch.testing.assert_close(a.cpu().double(), b, atol=1e-5, rtol=1e-5)
            rec = fdwt.waverec(c, w, mode)
            ref = O.waverec([t.cpu().double() for t in c], w, mode)
            torch.testing.assert_close(rec.cpu().double(), ref, atol=2e-5, rtol=1e-5)


@pytest.mark.parametrize("wavelet", ["db1", "db2", "db3", "db4", "sym8", "coif3", "bior3.5"])
def test_periodization_reconstruction_all_offsets(wavelet):
    """Periodization shifts every synthesis position by L/2 - 1, so its outputs sit at each
    offset modulo 4 across these filter lengths (2 .. 18); long fp32 rows exercise the vector
    stores of whole waves."""
    for n in (4099, 4100, 6000):
        x = _rand((3, n), 8, torch.float32)
        c = fdwt.wavedec(x.to(DEV), wavelet, "periodization", 3)
        rec = fdwt.waverec(c, wavelet, "periodization")
        ref = O.waverec([t.cpu().double() for t in c], wavelet, "periodization")
        torch.testing.assert_close(rec.cpu().double(), ref, atol=2e-5, rtol=1e-5)
        a, d = fdwt.dwt(x.to(DEV), wavelet, "periodization")
        y = fdwt.idwt(a, d, wavelet, "periodization")
        yr = O.idwt(a.cpu().double(), d.cpu().double(), wavelet, "periodization")
        torch.testing.assert_close(y.cpu().double(), yr, atol=2e-5, rtol=1e-5)


def test_edge_cases():
    e = torch.empty(0, 5, 100, device=DEV)
    a, d = fdwt.dwt(e, "db4")
    assert a.shape == (0, 5, 53)
    assert fdwt.wavedec(e, "db4", level=2)[0].shape == (0, 5, 30)
    x = torch.tensor([[1.7], [-0.3]], dtype=torch.float64, device=DEV)
    for w in ["haar", "db4"]:
        for p, q in zip(fdwt.dwt(x, w, "reflect"), fdwt.dwt(x, w, "periodic")):
            torch.testing.assert_close(p, q, rtol=0, atol=0)
    with pytest.raises(ValueError):
        fdwt.dwt(torch.empty(3, 0, device=DEV))
    # a zero level decomposition is the signal itself
    assert fdwt.wavedec(x, "db4", level=0)[0] is x


def test_gpu_matches_cpu_large_batch():
    """tests/test_dwt.py:88-99 of the reference (fp32, sym4, reflect)."""
    x = _rand((5, 7, 2049), 0, torch.float32)
    xg = x.to(DEV).requires_grad_()
    xc = x.double().requires_grad_()
    og = fdwt.wavedec(xg, "sym4", "reflect")
    oc = O.wavedec(xc, "sym4", "reflect")
    for a, b in zip(og, oc):
        torch.testing.assert_close(a.detach().cpu().double(), b.detach(), atol=1e-5, rtol=1e-5)
    sum((c * c).sum() for c in og).backward()
    sum((c * c).sum() for c in oc).backward()
    torch.testing.assert_close(xg.grad.cpu().double(), xc.grad, atol=1e-4, rtol=1e-4)


def test_modules():
    x = _rand((2, 128), 1, torch.float32).to(DEV)
    m, im = fdwt.DWT1D("db2", level=3), fdwt.IDWT1D("db2")
    torch.testing.assert_close(im(m(x))[..., :128], x, atol=1e-5, rtol=1e-5)
    custom = fdwt.get_filter_bank(O._table()["db2"])
    torch.testing.assert_close(fdwt.dwt(x, custom)[0], fdwt.dwt(x, "db2")[0])
