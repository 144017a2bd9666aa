"""Layers on the GPU: WaveletTokenMixer against the oracle composition, the inspection paths
(``_probs``, ``attention_map``) against the oracle's softmax, and an end-to-end training smoke
test shaped like the reference's demo (examples/token_mixer_demo.py:1-111).

Tolerances: float64 to 1e-10 of the max (the reference's GPU-vs-CPU bar, test_layers.py:64-79);
float32 to the north-star bars, rtol 1e-5 with atol 1e-6 per transform scaled by the
magnitude of the chained result (a DWT, a per-band Linear and an inverse DWT).
"""

import math

import pytest
import torch
from torch import nn

import pytorch_morlet_fdwt_amd as fdwt
from oracle import cwt as OC
from oracle import dwt as OD

pytestmark = pytest.mark.gpu
DEV = "cuda"
f64 = torch.float64


def _bands(m):
    out = []
    for b in m.bands:
        if isinstance(b, nn.Linear):
            out.append((b.weight, b.bias))
        else:
            out.append((b[0].weight, b[0].bias, b[2].weight, b[2].bias))
    return out


WTM = [("db4", "periodization", 4, 0, 256), ("db4", "periodization", 3, 32, 300),
       ("sym4", "symmetric", 3, 0, 257), ("coif2", "zero", 2, 16, 101),
       ("haar", "reflect", 5, 0, 64), ("sym8", "periodic", 2, 0, 1000)]


@pytest.mark.parametrize("wavelet,mode,level,hidden,L", WTM)
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_wavelet_token_mixer_matches_oracle(wavelet, mode, level, hidden, L, dtype):
    """layers.py:75-109: fused wavedec / waverec with per-band Linear or MLP maps, forward and
    backward (input and every parameter gradient) against the oracle composition on the CPU
    in float64."""
    torch.manual_seed(7)
    D = 16
    m = fdwt.WaveletTokenMixer(D, wavelet, mode=mode, level=level, hidden=hidden)
    x = torch.randn(3, L, D, generator=torch.Generator().manual_seed(L))
    gy = torch.randn(3, L, D, generator=torch.Generator().manual_seed(L + 1))
    mg = m.to(DEV).to(dtype)
    xd = x.to(DEV, dtype).requires_grad_()
    y = mg(xd)
    assert y.shape == x.shape and y.dtype == dtype
    params = list(mg.parameters())
    grads = torch.autograd.grad(y, [xd] + params, gy.to(DEV, dtype))
    mc = fdwt.WaveletTokenMixer(D, wavelet, mode=mode, level=level, hidden=hidden).double()
    mc.load_state_dict({k: v.detach().cpu().double() for k, v in mg.state_dict().items()})
    xr = x.double().requires_grad_()
    ref = OD.wavelet_token_mixer(xr, wavelet, mode, level, _bands(mc))
    rg = torch.autograd.grad(ref, [xr] + list(mc.parameters()), gy.double())
    if dtype == f64:
        def tol(r):
            return dict(rtol=0, atol=1e-10 * max(r.abs().max().item(), 1e-300))
    else:
        def tol(r):
            return dict(rtol=1e-5, atol=1e-6 * max(1.0, r.abs().max().item()) * 4)
    torch.testing.assert_close(y.detach().cpu().double(), ref.detach(), **tol(ref))
    for k, (a, b) in enumerate(zip(grads, rg)):
        torch.testing.assert_close(a.cpu().double(), b, **tol(b), msg=lambda s: f"grad {k}: {s}")


def test_attention_probs_match_oracle_softmax():
    """layers.py:149-153: the materialised softmax over frequencies of |W_f x| / tau."""
    torch.manual_seed(3)
    m = fdwt.MorletAttention(num_channels=5, hidden_dim=64, temperature=0.5).to(DEV).double()
    x = torch.randn(2, 3, 5, 6, 64, dtype=f64, generator=torch.Generator().manual_seed(1))
    p = m._probs(x.to(DEV))
    B, H, C, T, D = x.shape
    assert p.shape == (B, H, C, m.num_freqs, T * D)
    plan = OC.Plan(m.cwt.plan.scales, support_margin=1.25)
    Hf = plan.filters(m.cwt.log_scales.detach().cpu().exp(), m.cwt.w0.detach().cpu())
    w = OC.apply_plan(x.reshape(B, H, C, T * D), plan, Hf)
    ref = torch.softmax(w.abs() / 0.5, dim=-2)
    torch.testing.assert_close(p.cpu(), ref, rtol=0, atol=1e-12)
    torch.testing.assert_close(p.sum(-2).cpu(), torch.ones(B, H, C, T * D, dtype=f64),
                               rtol=0, atol=1e-12)


def test_channel_mix_attention_map_matches_oracle():
    """layers.py:252-255: A[b, h, n, c, k] = sum_f P[b, h, c, f, n] M[f, k]; applying the map
    to x (out[c, n] = sum_k A[n, c, k] x_k[n]) reproduces the fused module's output."""
    torch.manual_seed(4)
    m = fdwt.MorletChannelMixAttention(num_channels=5, hidden_dim=64, temperature=0.5)
    m = m.to(DEV).double()
    x = torch.randn(2, 3, 5, 6, 64, dtype=f64, generator=torch.Generator().manual_seed(2))
    A = m.attention_map(x.to(DEV)).cpu()
    B, H, C, T, D = x.shape
    plan = OC.Plan(m.cwt.plan.scales, support_margin=1.25)
    Hf = plan.filters(m.cwt.log_scales.detach().cpu().exp(), m.cwt.w0.detach().cpu())
    P = torch.softmax(OC.apply_plan(x.reshape(B, H, C, T * D), plan, Hf).abs() / 0.5, dim=-2)
    ref = torch.einsum("bhcfn,fk->bhnck", P, m.freq_to_channel.detach().cpu())
    torch.testing.assert_close(A, ref, rtol=0, atol=1e-12 * ref.abs().max().item())
    out = torch.einsum("bhnck,bhkn->bhcn", A, x.reshape(B, H, C, T * D)).reshape(x.shape)
    y = m(x.to(DEV)).cpu()
    torch.testing.assert_close(y, out, rtol=0, atol=1e-10 * out.abs().max().item())


# ------------------------------------------------------------------ demo-shaped training smoke
FS = 250.0
CLASS_FREQS = [6.0, 10.0, 18.0, 30.0]


def _batch(gen, batch, length):
    """1/f-like noise plus a Gaussian-windowed burst whose frequency is the class."""
    t = torch.arange(length, dtype=torch.float32) / FS
    y = torch.randint(len(CLASS_FREQS), (batch,), generator=gen)
    f = torch.tensor(CLASS_FREQS)[y]
    centre = torch.rand(batch, generator=gen) * (t[-1] - 1.0) + 0.5
    env = torch.exp(-0.5 * ((t[None] - centre[:, None]) / 0.25) ** 2)
    ph = torch.rand(batch, 1, generator=gen)
    burst = env * torch.sin(2 * math.pi * (f[:, None] * t[None] + ph))
    walk = torch.cumsum(torch.randn(batch, length, generator=gen), -1)
    walk = (walk - walk.mean(-1, keepdim=True)) / walk.std(-1, keepdim=True)
    x = 0.6 * burst + 0.5 * walk + 0.3 * torch.randn(batch, length, generator=gen)
    return x.to(DEV), y.to(DEV)


class _Block(nn.Module):
    def __init__(self, dim, mixer):
        super().__init__()
        self.n1, self.n2 = nn.LayerNorm(dim), nn.LayerNorm(dim)
        if mixer == "morlet":
            self.mix = fdwt.MorletTokenMixer(dim, freqs=torch.logspace(0, math.log10(60), 16).tolist(),
                                             fs=FS)
        else:
            self.mix = fdwt.WaveletTokenMixer(dim, "db4", hidden=dim)
        self.ffn = nn.Sequential(nn.Linear(dim, 4 * dim), nn.GELU(), nn.Linear(4 * dim, dim))

    def forward(self, x):
        x = x + self.mix(self.n1(x))
        return x + self.ffn(self.n2(x))


class _Model(nn.Module):
    def __init__(self, dim, depth, mixer):
        super().__init__()
        self.embed = nn.Linear(1, dim)
        self.blocks = nn.Sequential(*(_Block(dim, mixer) for _ in range(depth)))
        self.head = nn.Linear(dim, len(CLASS_FREQS))

    def forward(self, x):
        return self.head(self.blocks(self.embed(x[..., None])).mean(1))


@pytest.mark.parametrize("mixer", ["morlet", "dwt"])
def test_demo_training_smoke(mixer):
    """Two blocks, AdamW, 60 steps on the burst-classification task: every step's gradients
    are finite and the loss falls (mean of the last 10 steps below the first 10)."""
    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(0)
    model = _Model(32, 2, mixer).to(DEV)
    opt = torch.optim.AdamW(model.parameters(), lr=3e-3)
    losses = []
    for _ in range(60):
        x, y = _batch(gen, 32, 1000)
        loss = nn.functional.cross_entropy(model(x), y)
        opt.zero_grad(set_to_none=True)
        loss.backward()
        for p in model.parameters():
            if p.grad is not None:
                assert torch.isfinite(p.grad).all()
        opt.step()
        losses.append(loss.item())
    assert all(math.isfinite(v) for v in losses)
    assert sum(losses[-10:]) / 10 < sum(losses[:10]) / 10 - 0.05, losses
    if mixer == "morlet":
        f = model.blocks[0].mix.cwt.freqs
        assert torch.isfinite(f).all() and (f > 0).all()
