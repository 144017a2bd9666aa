"""Host-side CWT logic on the CPU: the octave plan and the Morlet filters of the product
against the reference's own values (tests/golden/cwt_golden.npz), and the error paths."""

import math

import numpy as np
import pytest
import torch

import pytorch_morlet_fdwt_amd as fdwt
from golden_io import load
from oracle import cwt as O

G = load("cwt_golden.npz")
PLANS = sorted({k.split("/")[1] for k in G.files if k.startswith("plan/")})


def product_plan(name):
    kw = {k[len(f"plan/{name}/kw_"):]: G[k].item() for k in G.files
          if k.startswith(f"plan/{name}/kw_")}
    return fdwt.MorletPlan(G[f"plan/{name}/scales"].tolist(), **kw)


@pytest.mark.parametrize("name", PLANS)
def test_plan_matches_reference(name):
    p = product_plan(name)
    assert p.n_octaves == int(G[f"plan/{name}/n_octaves"])
    assert p.center == int(G[f"plan/{name}/center"])
    assert p.margins == G[f"plan/{name}/margins"].tolist()
    assert p.c_lp == int(G[f"plan/{name}/c_lp"])
    st = [[s.octave, s.dil, i, s.half, c] for s in p.stages for i, c in zip(s.scale_idx, s.support)]
    assert st == G[f"plan/{name}/stages"].tolist()
    np.testing.assert_allclose(p.lowpass.numpy(), G[f"plan/{name}/lowpass"], rtol=0, atol=1e-16)
    if f"plan/{name}/H" in G.files:
        H = p.filters(torch.tensor(p.scales, dtype=torch.float64), p.w0, torch.float64)
        np.testing.assert_allclose(H.numpy(), G[f"plan/{name}/H"], rtol=0, atol=1e-15)


def test_filters_are_exactly_symmetric_and_differentiable():
    p = fdwt.MorletPlan([1.5, 3.0, 7.0, 30.0, 90.0], support_margin=1.25)
    ls = torch.tensor(p.scales, dtype=torch.float64).log().requires_grad_()
    w0 = torch.tensor(6.0, dtype=torch.float64, requires_grad=True)
    H = p.filters(ls.exp(), w0, torch.float64)
    re, im = H[0::2], H[1::2]
    assert torch.equal(re, re.flip(-1))
    assert torch.equal(im, -im.flip(-1))
    # same values as the oracle's direct (non-mirrored) construction
    ref = O.Plan(p.scales, support_margin=1.25).filters(ls.detach().exp(), 6.0)
    torch.testing.assert_close(H.detach(), ref, rtol=0, atol=1e-15)
    H.square().sum().backward()
    assert ls.grad is not None and w0.grad is not None


def test_stage_taps_layout():
    p = fdwt.MorletPlan([2.0, 5.0, 11.0, 40.0], support_margin=1.0)
    H = p.filters(torch.tensor(p.scales, dtype=torch.float64), p.w0, torch.float64)
    for k, st in enumerate(p.stages):
        taps = p.stage_taps(H, k)
        assert taps.shape == (len(st.scale_idx), st.half + 1, 2)
        for s, i in enumerate(st.scale_idx):
            for t in range(st.half + 1):
                assert taps[s, t, 0] == H[2 * i, p.center + t]
                assert taps[s, t, 1] == H[2 * i + 1, p.center + t]


def test_cwt_errors_and_module_api():
    x = torch.randn(4, 5, 200)
    with pytest.raises(ValueError):
        fdwt.cwt(x, scales=[1.0], freqs=[1.0])
    with pytest.raises(ValueError):
        fdwt.cwt(x, [1.0], method="nope")
    with pytest.raises(ValueError):
        fdwt.MorletPlan([1.0], norm="l3")
    with pytest.raises(ValueError):
        fdwt.MorletPlan([-1.0])
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fdwt.cwt(x, freqs=[2.0, 10.0], fs=250)
    with pytest.raises(TypeError):
        fdwt.cwt(torch.arange(10), [1.0])
    m = fdwt.CWT1D(freqs=[2.0, 10.0, 40.0], fs=250)
    np.testing.assert_allclose(m.freqs.numpy(), [2.0, 10.0, 40.0])
    assert not any(True for _ in m.parameters())
    m2 = fdwt.CWT1D(freqs=[2.0, 10.0], fs=250, learnable=True, learnable_w0=True)
    assert sorted(n for n, _ in m2.named_parameters()) == ["log_scales", "w0"]
    assert "log_scales" in m.state_dict()


@pytest.mark.parametrize("cls", [fdwt.MorletAttention, fdwt.MorletChannelMixAttention])
def test_attention_errors(cls):
    """tests/test_layers.py:185-198 of the reference."""
    m = cls(num_channels=3, hidden_dim=32)
    with pytest.raises(ValueError):
        m(torch.randn(2, 3, 4, 32))
    with pytest.raises(ValueError):
        m(torch.randn(1, 1, 4, 2, 32))
    with pytest.raises(ValueError):
        cls(num_channels=3, hidden_dim=32, freqs=[20.0])  # Nyquist = 16 Hz


def test_module_parameters_match_reference_names():
    a = fdwt.MorletAttention(num_channels=5, hidden_dim=64)
    keys = set(a.state_dict())
    assert {"freq_weight", "cwt.log_scales", "cwt.w0"} <= keys
    c = fdwt.MorletChannelMixAttention(num_channels=5, hidden_dim=64)
    assert c.freq_to_channel.shape == (16, 5)
    t = fdwt.MorletTokenMixer(16, freqs=[2.0, 8.0, 30.0], fs=250)
    assert {"mag_weight", "phase_weight", "bias", "out_proj.weight", "cwt.log_scales"} <= set(t.state_dict())
    for name in ("att", "cmix", "att_f4", "cmix_f4"):
        stored = {k[len(f"mod/{name}/param/"):] for k in G.files if k.startswith(f"mod/{name}/param/")}
        assert stored, name
    stored = {k[len("tm/tm_f3/param/"):] for k in G.files if k.startswith("tm/tm_f3/param/")}
    assert stored == set(t.state_dict())


def test_resolve_precision_rule():
    """src/fdwt/kernels/conv.py:332-338: fp64 is always exact, bf16 / fp16 inputs or
    allow_bf16 give bf16 operands, allow_tf32 alone gives tf32."""
    from pytorch_morlet_fdwt_amd import config
    saved = config.allow_tf32, config.allow_bf16
    try:
        config.allow_tf32, config.allow_bf16 = False, False
        assert config.resolve_precision(torch.float32) == "ieee"
        assert config.resolve_precision(torch.float64) == "ieee"
        assert config.resolve_precision(torch.bfloat16) == "bf16"
        assert config.resolve_precision(torch.float16) == "bf16"
        assert config.resolve_precision(torch.float16, torch.float64) == "ieee"
        config.allow_tf32 = True
        assert config.resolve_precision(torch.float32) == "tf32"
        config.allow_bf16 = True
        assert config.resolve_precision(torch.float32) == "bf16"
        assert config.resolve_precision(torch.float64) == "ieee"
    finally:
        config.allow_tf32, config.allow_bf16 = saved
