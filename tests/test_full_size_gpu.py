"""Parity at the benchmark's full sizes (BASELINE configs[1]-[4]) in float32.

Every operator here is independent per row, so at full size the oracle (the reference's CPU
algorithm restated, float64) checks a few rows spread over the batch, and size-independent
properties check all of it: perfect reconstruction of orthogonal banks, and the adjoint identity
<A x, c> = <x, A^T c> that ties each forward kernel to its backward kernel.  Tolerances are the
north-star bars (float32 rtol 1e-5 / atol 1e-6 per transform, complex64 CWT 1e-4 relative to
the max); the chained round trip and the module outputs use the calibrated bars of
tests/test_dwt_gpu.py and tests/test_cwt_gpu.py.
"""

import numpy as np
import pytest
import torch

import pytorch_morlet_fdwt_amd as fdwt
from oracle import cwt as OC
from oracle import dwt as OD

pytestmark = pytest.mark.gpu
DEV = "cuda"
f64 = torch.float64
ROWS = [0, 777, 2047]  # rows of the flattened (2048, N) batch checked against the oracle


def _inner(a, b):
    return (a.double() * b.double()).sum().item()


def _norm(t):
    return t.double().pow(2).sum().sqrt().item()


# The adjoint identity in float32: the inner products are sums of random-sign terms, so their
# difference is judged against the Cauchy-Schwarz scale |A x| |c| (rounding of the float32
# kernels: ~1e-11 of it here; an index error on just the boundary samples of every row: > 1e-6).
ADJ_TOL = 1e-7


@pytest.mark.parametrize("mode", ["zero", "periodic", "symmetric", "reflect", "periodization"])
@pytest.mark.parametrize("wavelet", ["sym8", "coif3"])
@pytest.mark.parametrize("n", [16384, 16383])
def test_dwt_sweep_full_size(wavelet, mode, n):
    """wavedec level 6 on x (16, 128, n) fp32."""
    g = torch.Generator().manual_seed(n + len(mode))
    x = torch.randn(16, 128, n, generator=g)
    xd = x.to(DEV).requires_grad_()
    coeffs = fdwt.wavedec(xd, wavelet, mode, 6)
    ref = OD.wavedec(x.reshape(-1, n)[ROWS].double(), wavelet, mode, 6)
    for c, r in zip(coeffs, ref):
        torch.testing.assert_close(c.detach().reshape(-1, c.shape[-1])[ROWS].cpu().double(), r,
                                   atol=1e-6, rtol=1e-5)
    # perfect reconstruction of an orthogonal bank, every row
    rec = fdwt.waverec([c.detach() for c in coeffs], wavelet, mode)[..., :n]
    scale = max(1.0, x.abs().max().item())
    torch.testing.assert_close(rec.cpu(), x, atol=1e-6 * scale, rtol=1e-5)
    # adjoint identity: the fused analysis chain and the synthesis chain that is its backward
    cs = [torch.randn(c.shape, generator=g).to(DEV) for c in coeffs]
    gx, = torch.autograd.grad(coeffs, xd, cs)
    lhs = sum(_inner(c.detach(), u) for c, u in zip(coeffs, cs))
    rhs = _inner(xd.detach(), gx)
    scale = np.sqrt(sum(_norm(c.detach()) ** 2 for c in coeffs) * sum(_norm(u) ** 2 for u in cs))
    assert abs(lhs - rhs) <= ADJ_TOL * scale


def test_cwt_cfg3_full_size():
    """fast CWT, 40 freqs logspace(-0.3, 2) Hz at fs 250 on x (32, 64, 2500)."""
    freqs = np.logspace(-0.3, 2, 40)
    g = torch.Generator().manual_seed(3)
    t = torch.arange(2500, dtype=torch.float32)
    tone = sum(torch.sin(2 * np.pi * f * t / 250.0) for f in (6.0, 10.0, 18.0, 30.0))
    x = torch.randn(32, 64, 2500, generator=g) + tone
    m = fdwt.CWT1D(freqs=freqs, fs=250.0, learnable=True, learnable_w0=True).to(DEV)
    xd = x.to(DEV).requires_grad_()
    y = m(xd)
    assert y.shape == (32, 64, 40, 2500) and y.dtype == torch.complex64
    plan = OC.Plan(m.plan.scales, support_margin=1.25)
    H = plan.filters(m.log_scales.detach().cpu().double().exp(), 6.0)
    ref = OC.apply_plan(x.reshape(-1, 2500)[ROWS].double(), plan, H)
    got = y.detach().reshape(-1, 40, 2500)[ROWS].cpu().to(torch.complex128)
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 1e-4
    # adjoint identity over the whole batch: bank forward vs bank adjoint + half-band transpose
    gy = torch.view_as_complex(torch.randn(*y.shape, 2, generator=g).to(DEV))
    gx, = torch.autograd.grad(y, xd, gy)
    yr, gr = torch.view_as_real(y.detach()), torch.view_as_real(gy)
    lhs = _inner(yr, gr)
    rhs = _inner(xd.detach(), gx)
    assert abs(lhs - rhs) <= ADJ_TOL * _norm(yr) * _norm(gr)


def test_token_mixer_cfg4_full_size():
    """MorletTokenMixer dim 256, 16 freqs logspace(0, 1.8) Hz, fs 250, Xavier
    mixing weights, x (8, 4096, 256); batch element 5 against the oracle."""
    torch.manual_seed(2)
    m = fdwt.MorletTokenMixer(256, freqs=torch.logspace(0, 1.8, 16).tolist(), fs=250.0)
    torch.nn.init.xavier_uniform_(m.mag_weight)
    torch.nn.init.xavier_uniform_(m.phase_weight)
    x = torch.randn(8, 4096, 256, generator=torch.Generator().manual_seed(4))
    y = m.to(DEV)(x.to(DEV))
    plan = OC.Plan(m.cwt.plan.scales, support_margin=1.25)
    H = plan.filters(m.cwt.log_scales.detach().cpu().double().exp(), 6.0)
    p = {k: v.detach().cpu().double() for k, v in m.named_parameters()}
    ref = OC.token_mixer(x[5:6].double(), plan, H, p["mag_weight"], p["phase_weight"], p["bias"],
                         p["out_proj.weight"], p["out_proj.bias"])
    got = y[5:6].detach().cpu().double()
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-5 * ref.abs().max().item())


def test_attention_cfg5_full_size():
    """MorletAttention num_channels 19, hidden_dim 200 on x (8, 4, 19, 30, 200);
    batch element 7 against the oracle."""
    torch.manual_seed(2)
    m = fdwt.MorletAttention(num_channels=19, hidden_dim=200)
    x = torch.randn(8, 4, 19, 30, 200, generator=torch.Generator().manual_seed(5))
    y = m.to(DEV)(x.to(DEV))
    plan = OC.Plan(m.cwt.plan.scales, support_margin=1.25)
    H = plan.filters(m.cwt.log_scales.detach().cpu().double().exp(), 6.0)
    ref = OC.attention(x[7:8].double(), plan, H, m.freq_weight.detach().cpu().double(), 1.0)
    got = y[7:8].detach().cpu().double()
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-5 * ref.abs().max().item())


def test_channel_mix_attention_cfg5_full_size():
    """MorletChannelMixAttention num_channels 19, hidden_dim 200 on x
    (8, 4, 19, 30, 200), forward and backward; batch element 3 against the oracle."""
    torch.manual_seed(2)
    m = fdwt.MorletChannelMixAttention(num_channels=19, hidden_dim=200)
    x = torch.randn(8, 4, 19, 30, 200, generator=torch.Generator().manual_seed(6))
    gy = torch.randn(8, 4, 19, 30, 200, generator=torch.Generator().manual_seed(7))
    m = m.to(DEV)
    xd = x.to(DEV).requires_grad_()
    y = m(xd)
    gx, gM = torch.autograd.grad(y, [xd, m.freq_to_channel], gy.to(DEV))
    plan = OC.Plan(m.cwt.plan.scales, support_margin=1.25)
    H = plan.filters(m.cwt.log_scales.detach().cpu().double().exp(), 6.0)
    xr = x[3:4].double().requires_grad_()
    M = m.freq_to_channel.detach().cpu().double().requires_grad_()
    ref = OC.channel_mix_attention(xr, plan, H, M, 1.0)
    rgx, rgM = torch.autograd.grad(ref, [xr, M], gy[3:4].double())
    torch.testing.assert_close(y[3:4].detach().cpu().double(), ref.detach(), rtol=1e-4,
                               atol=1e-5 * ref.abs().max().item())
    torch.testing.assert_close(gx[3:4].cpu().double(), rgx, rtol=1e-4,
                               atol=1e-5 * rgx.abs().max().item())
    # dL/dM sums over the whole batch: the oracle's one batch element is a partial sum, so the
    # full-batch gradient is checked against a float64 GPU run of the same module instead
    m64 = m.double()
    y64 = m64(xd.detach().double())
    gM64, = torch.autograd.grad(y64, [m64.freq_to_channel], gy.to(DEV).double())
    torch.testing.assert_close(gM.double(), gM64, rtol=1e-4, atol=1e-5 * gM64.abs().max().item())
