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


def test_dwt_cfg0_full_batch():
    """db4, symmetric, level 5 on x (32, 64, 2500) fp32, the benchmark's launch:
    rows spread over the batch against the oracle, perfect reconstruction and the adjoint
    identity over the whole batch."""
    n = 2500
    g = torch.Generator().manual_seed(11)
    x = torch.randn(32, 64, n, generator=g)
    xd = x.to(DEV).requires_grad_()
    coeffs = fdwt.wavedec(xd, "db4", "symmetric", 5)
    assert [c.shape[-1] for c in coeffs] == [84, 84, 162, 318, 630, 1253]
    ref = OD.wavedec(x.reshape(-1, n)[ROWS].double(), "db4", "symmetric", 5)
    for c, r in zip(coeffs, ref):
        torch.testing.assert_close(c.detach().reshape(-1, c.shape[-1])[ROWS].cpu().double(), r,
                                   atol=1e-6, rtol=1e-5)
    rec = fdwt.waverec(coeffs, "db4", "symmetric")
    assert rec.shape == (32, 64, n)
    refr = OD.waverec([r for r in ref], "db4", "symmetric")
    torch.testing.assert_close(rec.detach().reshape(-1, n)[ROWS].cpu().double(), refr,
                               atol=1e-6, rtol=1e-5)
    scale = max(1.0, x.abs().max().item())
    torch.testing.assert_close(rec.detach().cpu(), x, atol=1e-6 * scale, rtol=1e-5)
    # adjoint identity of the benchmark's whole step: forward (analysis then synthesis chain)
    # against its backward (analysis chain of the upstream gradient, then synthesis chain)
    gy = torch.randn(rec.shape, generator=g).to(DEV)
    gx, = torch.autograd.grad(rec, xd, gy)
    lhs = _inner(rec.detach(), gy)
    rhs = _inner(xd.detach(), gx)
    assert abs(lhs - rhs) <= ADJ_TOL * _norm(rec.detach()) * _norm(gy)
    # the round trip is the identity on an orthogonal bank, so is its transpose
    torch.testing.assert_close(gx, gy, atol=1e-6 * max(1.0, gy.abs().max().item()), rtol=1e-5)


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


def _token_mixer_cfg4():
    torch.manual_seed(2)
    m = fdwt.MorletTokenMixer(256, freqs=torch.logspace(0, 1.8, 16).tolist(), fs=250.0)
    torch.nn.init.xavier_uniform_(m.mag_weight)
    torch.nn.init.xavier_uniform_(m.phase_weight)
    return m


def _oracle_token_mixer(m, x):
    plan = OC.Plan(m.cwt.plan.scales, support_margin=1.25)
    p = {k: v.detach().cpu().double().requires_grad_() for k, v in m.named_parameters()}
    H = plan.filters(p["cwt.log_scales"].exp(), 6.0)
    y = OC.token_mixer(x, plan, H, p["mag_weight"], p["phase_weight"], p["bias"],
                       p["out_proj.weight"], p["out_proj.bias"])
    return y, p


def test_token_mixer_cfg4_full_size():
    """MorletTokenMixer dim 256, 16 freqs logspace(0, 1.8) Hz, fs 250, Xavier
    mixing weights, x (8, 4096, 256), forward and backward.  Batch element 5 of the full-batch
    run against the oracle (output and input gradient: rows of different batch elements never
    meet); parameter gradients of the full batch against a float64 GPU run, and of a one-element
    GPU run against the oracle."""
    m = _token_mixer_cfg4().to(DEV)
    x = torch.randn(8, 4096, 256, generator=torch.Generator().manual_seed(4))
    gy = torch.randn(8, 4096, 256, generator=torch.Generator().manual_seed(8))
    xd = x.to(DEV).requires_grad_()
    y = m(xd)
    params = [p for p in m.parameters() if p.requires_grad]
    grads = torch.autograd.grad(y, [xd] + params, gy.to(DEV))
    xr = x[5:6].double().requires_grad_()
    ref, p_ref = _oracle_token_mixer(m, xr)
    names = [n for n, p in m.named_parameters() if p.requires_grad]
    rg = torch.autograd.grad(ref, [xr] + [p_ref[n] for n in names], gy[5:6].double())
    rgx, rp = rg[0], rg[1:]
    torch.testing.assert_close(y[5:6].detach().cpu().double(), ref.detach(), rtol=1e-4,
                               atol=1e-5 * ref.abs().max().item())
    torch.testing.assert_close(grads[0][5:6].cpu().double(), rgx, rtol=1e-4,
                               atol=1e-5 * rgx.abs().max().item())
    # full-batch parameter gradients against float64 on the GPU
    m64 = _token_mixer_cfg4().to(DEV).double()
    m64.load_state_dict(m.state_dict())
    y64 = m64(xd.detach().double())
    p64 = [p for p in m64.parameters() if p.requires_grad]
    g64 = torch.autograd.grad(y64, p64, gy.to(DEV).double())
    for nm, a, b in zip(names, grads[1:], g64):
        torch.testing.assert_close(a.double(), b, rtol=1e-4, atol=3e-5 * b.abs().max().item(),
                                   msg=lambda s: f"{nm}: {s}")
    # one batch element on the GPU: parameter gradients against the oracle
    m.zero_grad()
    y1 = m(x[5:6].to(DEV))
    g1 = torch.autograd.grad(y1, params, gy[5:6].to(DEV))
    for nm, a, b in zip(names, g1, rp):
        torch.testing.assert_close(a.cpu().double(), b, rtol=1e-4, atol=3e-5 * b.abs().max().item(),
                                   msg=lambda s: f"{nm}: {s}")


def test_attention_cfg5_full_size():
    """MorletAttention num_channels 19, hidden_dim 200 on x (8, 4, 19, 30, 200),
    forward and backward: batch element 7 against the oracle (output, input gradient), the
    full batch's parameter gradients against a float64 GPU run, a one-element GPU run's
    parameter gradients against the oracle."""
    torch.manual_seed(2)
    m = fdwt.MorletAttention(num_channels=19, hidden_dim=200).to(DEV)
    x = torch.randn(8, 4, 19, 30, 200, generator=torch.Generator().manual_seed(5))
    gy = torch.randn(8, 4, 19, 30, 200, generator=torch.Generator().manual_seed(9))
    xd = x.to(DEV).requires_grad_()
    y = m(xd)
    names = [n for n, _ in m.named_parameters()]
    params = list(m.parameters())
    grads = torch.autograd.grad(y, [xd] + params, gy.to(DEV))
    plan = OC.Plan(m.cwt.plan.scales, support_margin=1.25)
    p_ref = {n: p.detach().cpu().double().requires_grad_() for n, p in m.named_parameters()}
    H = plan.filters(p_ref["cwt.log_scales"].exp(), p_ref["cwt.w0"])
    xr = x[7:8].double().requires_grad_()
    ref = OC.attention(xr, plan, H, p_ref["freq_weight"], 1.0)
    rg = torch.autograd.grad(ref, [xr] + [p_ref[n] for n in names], gy[7:8].double())
    torch.testing.assert_close(y[7:8].detach().cpu().double(), ref.detach(), rtol=1e-4,
                               atol=1e-5 * ref.abs().max().item())
    torch.testing.assert_close(grads[0][7:8].cpu().double(), rg[0], rtol=1e-4,
                               atol=1e-5 * rg[0].abs().max().item())
    m64 = fdwt.MorletAttention(num_channels=19, hidden_dim=200).to(DEV).double()
    m64.load_state_dict(m.state_dict())
    y64 = m64(xd.detach().double())
    g64 = torch.autograd.grad(y64, list(m64.parameters()), gy.to(DEV).double())
    for nm, a, b in zip(names, grads[1:], g64):
        torch.testing.assert_close(a.double(), b, rtol=1e-4, atol=3e-5 * b.abs().max().item(),
                                   msg=lambda s: f"{nm}: {s}")
    y1 = m(x[7:8].to(DEV))
    g1 = torch.autograd.grad(y1, params, gy[7:8].to(DEV))
    for nm, a, b in zip(names, g1, rg[1:]):
        torch.testing.assert_close(a.cpu().double(), b, rtol=1e-4, atol=3e-5 * b.abs().max().item(),
                                   msg=lambda s: f"{nm}: {s}")


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


SCALED = (64, 8, 64, 60, 256)


@pytest.mark.parametrize("cls", ["MorletAttention", "MorletChannelMixAttention"])
def test_attention_scaled_cfg5_group(cls):
    """The scaled configs[4] shape (64, 8, 64, 60, 256): its own plan (fs 256), the largest
    R x N of the benchmark (32768 x 15360) and dL/dW chunks near the 2 GiB default.  The full
    batch runs forward and backward on the GPU; one whole (b, h) group of 64 channels (the
    channel mix couples a group's channels, never two groups) is checked against the oracle:
    output and input gradient."""
    torch.set_num_threads(max(1, min(16, len(__import__("os").sched_getaffinity(0)))))
    torch.manual_seed(2)
    m = getattr(fdwt, cls)(num_channels=64, hidden_dim=256).to(DEV)
    B, Hh, C, T, D = SCALED
    gen = torch.Generator(device=DEV).manual_seed(12)
    xd = torch.randn(SCALED, device=DEV, generator=gen).requires_grad_()
    gy = torch.randn(SCALED, device=DEV, generator=gen)
    y = m(xd)
    gx, = torch.autograd.grad(y, [xd], gy)
    assert torch.isfinite(gx).all()
    b, h = 41, 5
    plan = OC.Plan(m.cwt.plan.scales, support_margin=1.25)
    H = plan.filters(m.cwt.log_scales.detach().cpu().double().exp(), m.cwt.w0.detach().cpu().double())
    xr = xd.detach()[b:b + 1, h:h + 1].cpu().double().requires_grad_()
    W = (m.freq_weight if cls == "MorletAttention" else m.freq_to_channel).detach().cpu().double()
    if cls == "MorletAttention":
        ref = OC.attention(xr, plan, H, W, 1.0)
    else:
        ref = OC.channel_mix_attention(xr, plan, H, W, 1.0)
    rgx, = torch.autograd.grad(ref, [xr], gy[b:b + 1, h:h + 1].cpu().double())
    torch.testing.assert_close(y[b:b + 1, h:h + 1].detach().cpu().double(), ref.detach(), rtol=1e-4,
                               atol=1e-5 * ref.abs().max().item())
    torch.testing.assert_close(gx[b:b + 1, h:h + 1].cpu().double(), rgx, rtol=1e-4,
                               atol=1e-5 * rgx.abs().max().item())
