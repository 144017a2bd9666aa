"""Morlet CWT, fused mix and spectral softmax on the GPU vs the reference's own outputs
(tests/golden/cwt_golden.npz, written by its CPU path in float64) and the CPU oracle.

Tolerances follow the reference's GPU-vs-CPU tests: float64 to 1e-10 of the max
(tests/test_cwt.py:63-80, test_layers.py:64-79), float32 CWT to 1e-5 relative to the max,
fp16 inputs to 1e-2 (test_cwt.py:103-113); the north-star bar for complex64 is 1e-4.
"""

import math

import numpy as np
import pytest
import torch
from torch.autograd import gradcheck

import pytorch_morlet_fdwt_amd as fdwt
from golden_io import cwt_compare, load
from oracle import cwt as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
G = load("cwt_golden.npz")
FREQS = np.geomspace(0.5, 100, 24)
f64 = torch.float64
CWTM = __import__("importlib").import_module("pytorch_morlet_fdwt_amd.cwt")

CASES = {
    "fast_n7": dict(method="fast"), "fast_n500": dict(method="fast"),
    "fast_n3000": dict(method="fast"), "direct_n500": dict(method="direct"),
    "fast_t5_n4000": dict(method="fast", truncate=5.0),
    "fast_l1_real_n900": dict(method="fast", norm="l1", complex=False),
    "fast_w05_n1100": dict(method="fast", w0=5.0),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_cwt_matches_reference(case):
    x = torch.from_numpy(G[f"cwt/{case}/x"]).to(DEV)
    y = fdwt.cwt(x, freqs=FREQS, fs=250.0, **CASES[case])
    cwt_compare(y, G, f"cwt/{case}/y", 1e-10)


def test_cwt_cfg3_signal_matches_reference():
    x = torch.from_numpy(G["cwt/cfg3/x"]).to(DEV)
    y = fdwt.cwt(x, freqs=np.logspace(-0.3, 2, 40), fs=250.0)
    cwt_compare(y, G, "cwt/cfg3/y", 1e-10)


def test_methods_agree_and_octave0_exact():
    """tests/test_cwt.py:40-52 of the reference."""
    for n in (7, 500, 3000):
        x = torch.randn(3, n, dtype=f64, generator=torch.Generator().manual_seed(n)).to(DEV)
        ref = fdwt.cwt(x, freqs=FREQS, fs=250, method="direct")
        scale = ref.abs().max()
        torch.testing.assert_close(fdwt.cwt(x, freqs=FREQS, fs=250, method="fft"), ref,
                                   atol=1e-12 * scale, rtol=0)
        fast = fdwt.cwt(x, freqs=FREQS, fs=250, method="fast")
        assert ((fast - ref).abs().max() / scale) < 3e-4
        torch.testing.assert_close(fast[..., -4:, :], ref[..., -4:, :], atol=1e-12 * scale, rtol=0)


def test_direct_matches_definition():
    x = torch.randn(2, 300, dtype=f64, generator=torch.Generator().manual_seed(0))
    scales = [1.0, 2.5, 7.0, 30.0]
    ref = O.cwt(x, scales, method="direct")  # pinned to the literal definition on the CPU
    out = fdwt.cwt(x.to(DEV), scales, method="direct").cpu()
    torch.testing.assert_close(out, ref, atol=1e-12, rtol=0)


@pytest.mark.parametrize("key", ["fast_c", "fast_r", "direct_c", "direct_r"])
def test_cwt_gradients_match_reference(key):
    method, cplx = key.split("_")[0], key.endswith("_c")
    x = torch.from_numpy(G[f"grad/{key}/x"])
    g = torch.Generator().manual_seed(int(G[f"grad/{key}/gy_seed"]))
    torch.randn(3, 2, 600, generator=g, dtype=f64)
    gy = torch.randn(3, 2, len(FREQS), 600, 2 if cplx else 1, generator=g, dtype=f64)
    m = fdwt.CWT1D(freqs=FREQS, fs=250, method=method, complex=cplx, learnable=True,
                   learnable_w0=True).to(DEV).double()
    xx = x.to(DEV).requires_grad_()
    y = m(xx)
    yr = torch.view_as_real(y) if cplx else y[..., None]
    (yr * gy.to(DEV)).sum().backward()
    cwt_compare(yr.movedim(-1, -2), G, f"grad/{key}/y", 1e-10)
    cwt_compare(xx.grad, G, f"grad/{key}/gx", 1e-10)
    for nm, got in (("g_log_scales", m.log_scales.grad), ("g_w0", m.w0.grad)):
        ref = G[f"grad/{key}/{nm}"]
        np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=0,
                                   atol=1e-10 * max(np.abs(ref).max(), 1e-300))


@pytest.mark.parametrize("method", ["fast", "direct"])
@pytest.mark.parametrize("cplx", [True, False])
def test_cwt_gradcheck(method, cplx):
    """tests/test_cwt.py:83-100 of the reference."""
    scales = [1.5, 3.0, 6.0, 9.0, 14.0, 23.0]
    m = fdwt.CWT1D(scales=scales, method=method, complex=cplx, learnable=True,
                   learnable_w0=True).to(DEV).double()
    for n in [5, 37, 150]:
        x = torch.randn(2, n, dtype=f64, device=DEV, requires_grad=True)
        ls = m.log_scales.detach().clone().requires_grad_()
        w0 = torch.tensor(6.0, dtype=f64, device=DEV, requires_grad=True)

        def f(ls, w0, x):
            y = CWTM._apply_plan(x, m.plan, m.plan.filters(ls.exp(), w0, f64))
            return torch.view_as_real(y) if cplx else y

        assert gradcheck(f, (ls, w0, x))


def test_fp32_accuracy_and_dtypes():
    """tests/test_cwt.py:103-113 of the reference."""
    x = torch.randn(8, 2500, device=DEV)
    ref = fdwt.cwt(x.double(), freqs=FREQS, fs=250, method="fast")
    out = fdwt.cwt(x, freqs=FREQS, fs=250, method="fast")
    assert out.dtype == torch.complex64
    assert ((out - ref).abs().max() / ref.abs().max()) < 1e-5
    out16 = fdwt.cwt(x.half(), freqs=FREQS, fs=250, method="fast")
    assert out16.dtype == torch.complex64
    assert ((out16 - ref).abs().max() / ref.abs().max()) < 1e-2


def test_frequency_localisation():
    """tests/test_cwt.py:116-129 of the reference."""
    fs, f0 = 250.0, 10.0
    t = torch.arange(5000, dtype=f64, device=DEV) / fs
    x = torch.sin(2 * math.pi * f0 * t)
    freqs = np.geomspace(1, 60, 40)
    for norm in ["l1", "l2"]:
        w = fdwt.cwt(x, freqs=freqs, fs=fs, norm=norm).abs()[:, 2000:3000].mean(-1)
        assert abs(freqs[int(w.argmax())] - f0) / f0 < 0.06
    amps = []
    for f in [3.0, 12.0, 40.0]:
        x = torch.sin(2 * math.pi * f * t)
        amps.append(fdwt.cwt(x, freqs=[f], fs=fs, norm="l1").abs()[0, 2000:3000].mean())
    assert max(amps) / min(amps) < 1.01


@pytest.mark.parametrize("key", ["fast_c", "fast_r", "direct_c", "direct_r"])
def test_mix_matches_reference(key, monkeypatch):
    method, cplx = key.split("_")[0], key.endswith("_c")
    # several row chunks in the backward pass (tests/test_layers.py:32 of the reference)
    monkeypatch.setattr(CWTM._MorletMixFunction, "MIX_CHUNK_BYTES", 4 * 12 * 700 * 16)
    m = fdwt.CWT1D(freqs=np.geomspace(1, 60, 12), fs=250, method=method, complex=cplx,
                   learnable=True).to(DEV).double()
    x, a, b, gy = (torch.from_numpy(G[f"mix/{key}/{n}"]).to(DEV) for n in ("x", "a", "b", "gy"))
    xx, aa, bb = (t.clone().requires_grad_() for t in (x, a, b))
    H = m.plan.filters(m.log_scales.exp(), m.w0, f64)
    y = CWTM.morlet_mix(xx, m.plan, H, aa, bb)
    (y * gy).sum().backward()
    cwt_compare(y, G, f"mix/{key}/y", 1e-10)
    cwt_compare(xx.grad, G, f"mix/{key}/gx", 1e-10)
    for nm, got in (("ga", aa.grad), ("gb", bb.grad), ("g_log_scales", m.log_scales.grad)):
        ref = G[f"mix/{key}/{nm}"]
        np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=0, atol=1e-10 * np.abs(ref).max())


@pytest.mark.parametrize("key", ["ch", "pos"])
def test_spectral_softmax_matches_reference(key, monkeypatch):
    monkeypatch.setattr(CWTM._SpectralSoftmaxFunction, "CHUNK_BYTES", 3 * 5 * 300 * 16)
    m = fdwt.CWT1D(scales=[1.5, 3.0, 7.0, 13.0, 26.0], learnable=True, learnable_w0=True)
    m = m.to(DEV).double()
    x, V, gy = (torch.from_numpy(G[f"ssm/{key}/{n}"]).to(DEV) for n in ("x", "V", "gy"))
    xx, VV = x.clone().requires_grad_(), V.clone().requires_grad_()
    ls = m.log_scales.detach().clone().requires_grad_()
    w0 = torch.tensor(6.0, dtype=f64, device=DEV, requires_grad=True)
    y = CWTM.spectral_softmax(xx, m.plan, m.plan.filters(ls.exp(), w0, f64), VV, 3, 0.7)
    (y * gy).sum().backward()
    for nm, got in (("y", y), ("gx", xx.grad), ("gV", VV.grad), ("g_log_scales", ls.grad),
                    ("g_w0", w0.grad)):
        ref = G[f"ssm/{key}/{nm}"]
        np.testing.assert_allclose(got.detach().cpu().numpy(), ref, rtol=0,
                                   atol=1e-10 * max(np.abs(ref).max(), 1e-300), err_msg=nm)


@pytest.mark.parametrize("per_position", [False, True])
def test_spectral_softmax_gradcheck(per_position):
    """tests/test_layers.py:155-169 of the reference."""
    m = fdwt.CWT1D(scales=[1.5, 3.0, 7.0, 13.0, 26.0], learnable=True, learnable_w0=True)
    m = m.to(DEV).double()
    nch, R, N = 3, 6, 80
    x = torch.randn(R, N, dtype=f64, device=DEV, requires_grad=True)
    shape = (R // nch, 5, N) if per_position else (nch, 5)
    V = torch.randn(shape, dtype=f64, device=DEV, requires_grad=True)
    ls = m.log_scales.detach().clone().requires_grad_()
    w0 = torch.tensor(6.0, dtype=f64, device=DEV, requires_grad=True)
    f = lambda x, V, ls, w0: CWTM.spectral_softmax(  # noqa: E731
        x, m.plan, m.plan.filters(ls.exp(), w0, f64), V, nch, 0.7)
    assert gradcheck(f, (x, V, ls, w0))


MODS = {"att": fdwt.MorletAttention, "cmix": fdwt.MorletChannelMixAttention,
        "att_big": fdwt.MorletAttention, "att_f4": fdwt.MorletAttention,
        "cmix_f4": fdwt.MorletChannelMixAttention}
MOD_KW = {"att": dict(num_channels=5, hidden_dim=64, temperature=0.5),
          "cmix": dict(num_channels=5, hidden_dim=64, temperature=0.5),
          "att_big": dict(num_channels=2, hidden_dim=100, temperature=0.01),
          "att_f4": dict(num_channels=4, hidden_dim=128, freqs=[2.0, 6.0, 12.0, 25.0]),
          "cmix_f4": dict(num_channels=4, hidden_dim=128, freqs=[2.0, 6.0, 12.0, 25.0])}


def _load_module(name, cls, kw, prefix):
    m = cls(**kw).double()
    sd = {k[len(f"{prefix}/param/"):]: torch.from_numpy(G[k]) for k in G.files
          if k.startswith(f"{prefix}/param/")}
    m.load_state_dict(sd)
    return m.to(DEV)


@pytest.mark.parametrize("name", sorted(MODS))
def test_attention_modules_match_reference(name, monkeypatch):
    monkeypatch.setattr(CWTM._SpectralSoftmaxFunction, "CHUNK_BYTES", 7 * 3 * 16 * 384)
    m = _load_module(name, MODS[name], MOD_KW[name], f"mod/{name}")
    x = torch.from_numpy(G[f"mod/{name}/x"]).to(DEV).requires_grad_()
    y = m(x)
    assert y.shape == x.shape and y.dtype == x.dtype
    y.square().sum().backward()
    tol = 1e-10
    np.testing.assert_allclose(y.detach().cpu().numpy(), G[f"mod/{name}/y"], rtol=0,
                               atol=tol * np.abs(G[f"mod/{name}/y"]).max())
    np.testing.assert_allclose(x.grad.cpu().numpy(), G[f"mod/{name}/gx"], rtol=0,
                               atol=tol * np.abs(G[f"mod/{name}/gx"]).max())
    for pn, p in m.named_parameters():
        ref = G[f"mod/{name}/grad/{pn}"]
        np.testing.assert_allclose(p.grad.cpu().numpy(), ref, rtol=0,
                                   atol=tol * max(np.abs(ref).max(), 1e-300), err_msg=pn)


@pytest.mark.parametrize("name", ["tm_f3", "tm_nophase"])
def test_token_mixer_matches_reference(name):
    kw = dict(dim=16, freqs=[2.0, 8.0, 30.0], fs=250) if name == "tm_f3" else dict(dim=16, use_phase=False)
    m = _load_module(name, fdwt.MorletTokenMixer, kw, f"tm/{name}")
    x = torch.from_numpy(G[f"tm/{name}/x"]).to(DEV).requires_grad_()
    y = m(x)
    y.square().mean().backward()
    np.testing.assert_allclose(y.detach().cpu().numpy(), G[f"tm/{name}/y"], rtol=0,
                               atol=1e-10 * np.abs(G[f"tm/{name}/y"]).max())
    np.testing.assert_allclose(x.grad.cpu().numpy(), G[f"tm/{name}/gx"], rtol=0,
                               atol=1e-10 * np.abs(G[f"tm/{name}/gx"]).max())
    for pn, p in m.named_parameters():
        key = f"tm/{name}/grad/{pn}"
        if key in G.files:
            ref = G[key]
            np.testing.assert_allclose(p.grad.cpu().numpy(), ref, rtol=0,
                                       atol=1e-10 * max(np.abs(ref).max(), 1e-300), err_msg=pn)


def test_spectral_softmax_large_amplitudes():
    """tests/test_layers.py:172-182 of the reference: the online softmax stays finite."""
    torch.manual_seed(0)
    m = fdwt.MorletAttention(num_channels=2, hidden_dim=100, temperature=0.01).to(DEV)
    x = (1e3 * torch.randn(1, 1, 2, 10, 100, device=DEV)).requires_grad_()
    y = m(x)
    y.sum().backward()
    assert torch.isfinite(y).all() and torch.isfinite(x.grad).all()
    md = m.cpu().double()
    H = md.cwt._filters("cpu", f64)
    plan = O.Plan(md.cwt.plan.scales, support_margin=1.25)
    ref = O.attention(x.detach().cpu().double(), plan, H, md.freq_weight.detach(), 0.01)
    torch.testing.assert_close(y.detach().cpu().double(), ref, atol=1e-4 * ref.abs().max().item(),
                               rtol=0)


def test_attention_fp32_and_bf16_run():
    m = fdwt.MorletAttention(num_channels=4, hidden_dim=128, freqs=[2.0, 6.0, 12.0, 25.0]).to(DEV)
    x = torch.randn(2, 2, 4, 5, 128, device=DEV)
    for dt in (torch.float32, torch.bfloat16):
        y = m(x.to(dt))
        assert y.dtype == dt and torch.isfinite(y.float()).all()
    np.testing.assert_allclose(m.freqs.cpu().numpy(), [2.0, 6.0, 12.0, 25.0], rtol=1e-5)


def test_bf16_precision_mode_backward(monkeypatch):
    """config.allow_bf16 (the reference's "bf16" precision: bf16 matrix operands, fp32
    accumulation, README.md:206-212) rounds the operands of the bank adjoint -- the upstream
    scalogram gradient and the filters -- and of the matrix-core filter gradient -- the
    upstream gradient and the signal -- to bf16.  CWT: the input gradient matches the float64
    oracle gradient with exactly those operands rounded to bf16 (a CPU emulation of the mode)
    to 2e-3 relative L2 error, while both miss the exact gradient by ~1.6e-2 (the mode's own
    error on this problem: oscillatory filters against a wideband gradient cancel).
    MorletAttention: forward outputs and the mixing weights' gradient unchanged (those kernels
    compute in fp32), the input gradient within 8e-2 relative L2 error of float64 (4.6e-2
    measured), the scale parameters' gradient (through the filter gradient) within 5e-2
    (3.4e-2 measured), and bf16 inputs, which select the mode (cwt.py:540), within 1e-1 (6.1e-2
    and 4.5e-2 measured)."""
    def rel(a, b):
        return ((a - b).norm() / b.norm()).item()

    freqs = torch.logspace(-0.3, 2, 40).tolist()
    sig = torch.randn(4, 2500, generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    scales = O.freqs_to_scales(freqs, 250.0, 6.0).tolist()
    plan = O.Plan(scales)
    H = plan.filters(torch.tensor(scales, dtype=torch.float64), torch.tensor(6.0, dtype=torch.float64))

    def oracle_grad(Hf, round_g):
        xs = sig.clone().requires_grad_()
        yr = torch.view_as_real(O.apply_plan(xs, plan, Hf))
        wt = torch.cos(torch.arange(yr.numel(), dtype=torch.float64)).view_as(yr)
        if round_g:
            wt = wt.to(torch.bfloat16).double()
        (g,) = torch.autograd.grad((yr * wt).sum(), [xs])
        return g

    exact = oracle_grad(H, False)
    emulated = oracle_grad(H.to(torch.bfloat16).double(), True)
    monkeypatch.setattr(fdwt.config, "allow_bf16", True)
    xs = sig.float().to(DEV).requires_grad_()
    yc = torch.view_as_real(fdwt.cwt(xs, freqs=freqs, fs=250, method="fast"))
    wt = torch.cos(torch.arange(yc.numel(), device=DEV, dtype=torch.float64)).view_as(yc)
    (g,) = torch.autograd.grad((yc.double() * wt).sum(), [xs])
    g = g.double().cpu()
    assert rel(g, emulated) < 2e-3, rel(g, emulated)
    assert rel(g, exact) < 2.5e-2, rel(g, exact)
    assert rel(emulated, exact) > 5e-3  # the mode's own error: the comparison above has teeth

    torch.manual_seed(5)
    m = fdwt.MorletAttention(num_channels=6, hidden_dim=200).to(DEV)
    x = torch.randn(2, 2, 6, 10, 200, device=DEV)
    w = torch.cos(torch.arange(x.numel(), device=DEV, dtype=torch.float64).view_as(x))

    def run(dt, bf):
        monkeypatch.setattr(fdwt.config, "allow_bf16", bf)
        mm = m.to(torch.float64 if dt == torch.float64 else torch.float32)
        mm.zero_grad()
        xx = x.detach().to(dt).requires_grad_()
        y = mm(xx)
        (y.double() * w).sum().backward()
        return [t.detach().double() for t in (y, xx.grad, mm.freq_weight.grad,
                                               mm.cwt.log_scales.grad)]

    r64, r32, rb, rbf = (run(torch.float64, False), run(torch.float32, False),
                         run(torch.float32, True), run(torch.bfloat16, False))
    assert torch.equal(rb[0], r32[0]) and torch.equal(rb[2], r32[2])
    assert 1e-6 < rel(rb[1], r64[1]) < 8e-2, rel(rb[1], r64[1])
    assert 1e-4 < rel(rb[3], r64[3]) < 5e-2, rel(rb[3], r64[3])
    assert torch.isfinite(rbf[1]).all() and torch.isfinite(rbf[3]).all()
    assert rel(rbf[1], r64[1]) < 1e-1, rel(rbf[1], r64[1])
    assert rel(rbf[3], r64[3]) < 1e-1, rel(rbf[3], r64[3])


def test_fp32_attention_matches_fp64():
    """north-star fp32 bar on a cfg5-shaped problem: MorletAttention forward + backward."""
    torch.manual_seed(2)
    m = fdwt.MorletAttention(num_channels=19, hidden_dim=200).to(DEV)
    x = torch.randn(2, 2, 19, 30, 200, device=DEV)
    outs = []
    for dt in (torch.float64, torch.float32):
        mm = m.to(dt)
        mm.zero_grad()
        xx = x.to(dt).requires_grad_()
        y = mm(xx)
        (y * torch.cos(torch.arange(y.numel(), device=DEV, dtype=dt).view_as(y))).sum().backward()
        outs.append([t.detach().double() for t in (y, xx.grad, mm.freq_weight.grad,
                                                    mm.cwt.log_scales.grad, mm.cwt.w0.grad)])
    # y and x.grad: 1e-5 of the max.  The parameter gradients are sums over every position of
    # every row; there the reference algorithm's own fp32 CPU path (oracle/, same problem,
    # float32 vs float64) misses by up to 1.6e-5 of the max (freq_weight.grad), so they get
    # 3e-5 of the max.
    for k, (a, b) in enumerate(zip(*outs)):
        frac = 1e-5 if k < 2 else 3e-5
        torch.testing.assert_close(b, a, rtol=1e-4, atol=frac * a.abs().max().item())


def test_token_mixers_run_and_backprop():
    """tests/test_layers.py:45-58 of the reference."""
    torch.manual_seed(0)
    x = torch.randn(2, 300, 16, device=DEV, requires_grad=True)
    for mixer in (fdwt.MorletTokenMixer(16, freqs=[2.0, 8.0, 30.0], fs=250),
                  fdwt.MorletTokenMixer(16, use_phase=False),
                  fdwt.WaveletTokenMixer(16, "db4", hidden=32),
                  fdwt.WaveletTokenMixer(16, "sym4", mode="symmetric", level=3)):
        mixer = mixer.to(DEV)
        y = mixer(x)
        assert y.shape == x.shape
        y.square().mean().backward()
        assert x.grad is not None and torch.isfinite(x.grad).all()
        for p in mixer.parameters():
            if p.requires_grad:
                assert p.grad is not None and torch.isfinite(p.grad).all()
        x.grad = None


def test_channel_mix_attention_map():
    m = fdwt.MorletChannelMixAttention(num_channels=5, hidden_dim=64).to(DEV)
    assert m.attention_map(torch.randn(2, 3, 5, 6, 64, device=DEV)).shape == (2, 3, 6 * 64, 5, 5)


FILTER_PLANS = {
    "complex_l2": dict(scales=[1.5, 3.0, 7.0, 30.0, 90.0], support_margin=1.25),
    "real_l1": dict(scales=[2.0, 5.0, 11.0, 40.0], norm="l1", complex=False),
    "w5_t5": dict(scales=list(np.geomspace(1.2, 200.0, 19)), w0=5.0, truncate=5.0),
}


@pytest.mark.parametrize("name", sorted(FILTER_PLANS))
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_device_filters_match_oracle(name, dtype):
    """The filter-bank kernel against the oracle's direct construction of cwt.py:181-203
    (values), and its gradient kernel against autograd through that construction."""
    kw = dict(FILTER_PLANS[name])
    scales = kw.pop("scales")
    p = fdwt.MorletPlan(scales, **kw)
    op = O.Plan(scales, w0=kw.get("w0", 6.0), truncate=kw.get("truncate", 4.0),
                norm=kw.get("norm", "l2"), complex=kw.get("complex", True),
                support_margin=kw.get("support_margin", 1.0))
    gen = torch.Generator().manual_seed(7)
    ls = (torch.tensor(scales, dtype=f64).log() + 0.05 * torch.randn(len(scales), generator=gen))
    w0v = p.w0 + 0.3
    ls_c = ls.clone().requires_grad_()
    w0_c = torch.tensor(w0v, dtype=f64, requires_grad=True)
    ref = op.filters(ls_c.exp(), w0_c)
    ls_g = ls.to(DEV).requires_grad_()
    w0_g = torch.tensor(w0v, dtype=f64, device=DEV, requires_grad=True)
    H = p.filters(ls_g.exp(), w0_g, dtype)
    assert H.shape == ref.shape and H.dtype == dtype
    tol = 1e-14 if dtype == f64 else 1e-7
    scale = float(ref.abs().max())
    torch.testing.assert_close(H.detach().cpu().double(), ref.detach(), rtol=0, atol=tol * scale)
    # exact symmetry of the device bank
    C = p.channels
    Hc = H.detach().cpu()
    assert torch.equal(Hc[0::C], Hc[0::C].flip(-1))
    if C == 2:
        assert torch.equal(Hc[1::2], -Hc[1::2].flip(-1))
    gH = torch.randn(ref.shape, dtype=f64, generator=gen)
    g_ls, g_w0 = torch.autograd.grad(ref, (ls_c, w0_c), gH)
    d_ls, d_w0 = torch.autograd.grad(H, (ls_g, w0_g), gH.to(DEV, dtype))
    gtol = 1e-12 if dtype == f64 else 1e-5
    gscale = float(max(g_ls.abs().max(), g_w0.abs()))
    torch.testing.assert_close(d_ls.cpu(), g_ls, rtol=0, atol=gtol * gscale)
    torch.testing.assert_close(d_w0.cpu(), g_w0, rtol=0, atol=gtol * gscale)


def test_device_filters_gradcheck():
    """Finite differences pin the analytic derivatives of the gradient kernel."""
    p = fdwt.MorletPlan([1.7, 4.0, 9.0, 25.0], support_margin=1.25)
    ls = torch.tensor(p.scales, dtype=f64, device=DEV).log().requires_grad_()
    w0 = torch.tensor(6.2, dtype=f64, device=DEV, requires_grad=True)
    assert gradcheck(lambda a, b: p.filters(a.exp(), b, f64), (ls, w0), eps=1e-6, atol=1e-8)
    # a float w0 gets no gradient and the scales still do
    H = p.filters(ls.exp(), 6.0, f64)
    (g,) = torch.autograd.grad(H.square().sum(), ls)
    assert torch.isfinite(g).all() and g.abs().max() > 0


MANY = {
    # method "direct" puts every scale in one octave: 150 scales, launched as 64 + 64 + 22
    "direct_150": dict(scales=list(np.geomspace(1.0, 40.0, 150)), method="direct", n=400),
    # a linear grid: octave 5 of the fast plan holds 128 scales (and octave 4 64 + more)
    "fast_255": dict(scales=list(np.arange(1.0, 256.0)), method="fast", n=700),
    # more filters than one filter-kernel launch builds (256): two filter chunks
    "direct_300": dict(scales=list(np.geomspace(1.0, 12.0, 300)), method="direct", n=150),
}


@pytest.mark.parametrize("name", sorted(MANY))
def test_many_scales_per_octave_match_oracle(name):
    """Octaves with more scales than one stage launch takes (FDWT_CWT_MAX_SCALES = 64) and
    banks with more filters than one filter launch builds (256) run as consecutive launch
    groups: values and every gradient against the oracle in float64."""
    kw = MANY[name]
    m = fdwt.CWT1D(scales=kw["scales"], method=kw["method"], learnable=True,
                   learnable_w0=True).to(DEV).double()
    assert max(len(st.scale_idx) for st in m.plan.stages) > 64
    g = torch.Generator().manual_seed(len(kw["scales"]))
    x = torch.randn(3, kw["n"], dtype=f64, generator=g)
    gy = torch.randn(3, len(kw["scales"]), kw["n"], 2, dtype=f64, generator=g)
    xx = x.to(DEV).requires_grad_()
    y = m(xx)
    (torch.view_as_real(y) * gy.to(DEV)).sum().backward()
    plan = O.Plan(m.plan.scales, method=kw["method"], support_margin=1.25)
    ls = m.log_scales.detach().cpu().clone().requires_grad_()
    w0 = torch.tensor(6.0, dtype=f64, requires_grad=True)
    xr = x.clone().requires_grad_()
    ref = O.apply_plan(xr, plan, plan.filters(ls.exp(), w0))
    (torch.view_as_real(ref) * gy).sum().backward()
    for nm, got, want in (("y", y.detach(), ref.detach()), ("gx", xx.grad, xr.grad),
                          ("g_log_scales", m.log_scales.grad, ls.grad), ("g_w0", m.w0.grad, w0.grad)):
        got = got.cpu()
        if got.is_complex():
            got, want = torch.view_as_real(got), torch.view_as_real(want)
        torch.testing.assert_close(got.double(), want.double(), rtol=0,
                                   atol=1e-10 * max(want.abs().max().item(), 1e-300),
                                   msg=lambda s: f"{nm}: {s}")


def test_many_scales_mix_and_softmax_match_oracle():
    """The fused mix and spectral softmax over a 130-scale direct plan (three launch groups
    per octave) against the oracle, with gradients."""
    scales = list(np.geomspace(1.0, 30.0, 130))
    m = fdwt.CWT1D(scales=scales, method="direct", learnable=True, learnable_w0=True)
    m = m.to(DEV).double()
    g = torch.Generator().manual_seed(130)
    B, D, N = 2, 3, 300
    x = torch.randn(B, D, N, dtype=f64, generator=g)
    a = torch.randn(D, 130, dtype=f64, generator=g)
    b = torch.randn(D, 130, dtype=f64, generator=g)
    V = torch.randn(B, 130, N, dtype=f64, generator=g)
    plan = O.Plan(m.plan.scales, method="direct", support_margin=1.25)
    for kind in ("mix", "softmax"):
        m.zero_grad()
        xx, aa, bb, VV = (t.to(DEV).requires_grad_() for t in (x, a, b, V))
        H = m.plan.filters(m.log_scales.exp(), m.w0, f64)
        if kind == "mix":
            y = CWTM.morlet_mix(xx, m.plan, H, aa, bb)
        else:
            y = CWTM.spectral_softmax(xx.reshape(B * D, N), m.plan, H, VV, D, 0.7)
        (y.square()).sum().backward()
        ls = m.log_scales.detach().cpu().clone().requires_grad_()
        w0 = torch.tensor(6.0, dtype=f64, requires_grad=True)
        xr, ar, br, Vr = (t.clone().requires_grad_() for t in (x, a, b, V))
        Hr = plan.filters(ls.exp(), w0)
        if kind == "mix":
            ref = O.morlet_mix(xr, plan, Hr, ar, br)
        else:
            ref = O.spectral_softmax(xr.reshape(B * D, N), plan, Hr, Vr, D, 0.7)
        ref.square().sum().backward()
        pairs = [("y", y.detach(), ref.detach()), ("gx", xx.grad, xr.grad),
                 ("g_log_scales", m.log_scales.grad, ls.grad), ("g_w0", m.w0.grad, w0.grad)]
        if kind == "mix":
            pairs += [("ga", aa.grad, ar.grad), ("gb", bb.grad, br.grad)]
        else:
            pairs += [("gV", VV.grad, Vr.grad)]
        for nm, got, want in pairs:
            torch.testing.assert_close(got.cpu().double(), want.double(), rtol=0,
                                       atol=1e-10 * max(want.abs().max().item(), 1e-300),
                                       msg=lambda s: f"{kind} {nm}: {s}")
