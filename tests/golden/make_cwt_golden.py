"""Write golden vectors for the Morlet CWT pyramid, the fused mix and the spectral softmax.

The octave plan of the fast CWT (scale grouping, supports, margins, the Kaiser half-band)
and the values it produces are only pinned bit-faithfully by the reference itself, so this
script imports the reference package from a source checkout (CPU, float64 -- its pure
PyTorch fallback path, src/fdwt/cwt.py:555-583, 379-394, 529-549) and stores inputs and
outputs as fixtures::

    python make_cwt_golden.py /path/to/pytorch_morlet_fdwt/src     # writes cwt_golden.npz

Large outputs are stored as their first ``HEAD`` samples plus ``K`` random projections
along time (``sketch``): any error in a coefficient changes a projection.
"""

import importlib
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
HEAD = 64
K = 6
FREQS = np.geomspace(0.5, 100, 24)


def sketch_vectors(n, seed=12345):
    return np.random.RandomState(seed).standard_normal((n, K))


def put_big(out, key, t):
    """Store t (..., N) as its head and K projections along the last axis."""
    a = t.detach().cpu()
    if a.is_complex():
        a = torch.view_as_real(a).movedim(-1, -2)  # (..., 2, N)
    a = a.numpy()
    n = a.shape[-1]
    if n <= 2 * HEAD:
        out[key] = a
        return
    out[key + "@head"] = a[..., :HEAD]
    out[key + "@sketch"] = a @ sketch_vectors(n)


def plan_meta(out, key, plan):
    out[key + "/scales"] = np.array(plan.scales)
    out[key + "/n_octaves"] = np.array(plan.n_octaves)
    out[key + "/center"] = np.array(plan.center)
    out[key + "/margins"] = np.array(plan.margins)
    out[key + "/c_lp"] = np.array(plan.c_lp)
    out[key + "/lowpass"] = plan.lowpass.numpy()
    out[key + "/s_th"] = np.array(plan.s_th)
    st = []
    for s in plan.stages:
        for i, c in zip(s.scale_idx, s.support):
            st.append([s.octave, s.dil, i, s.half, c])
    out[key + "/stages"] = np.array(st)


def main(src):
    sys.path.insert(0, src)
    fdwt = importlib.import_module("fdwt")
    cwtm = importlib.import_module("fdwt.cwt")
    out = {}
    f64 = torch.float64

    # ---- plans: the reference test grid and every BASELINE config
    plans = {
        "grid24": dict(scales=cwtm.freqs_to_scales(FREQS, 250.0).tolist()),
        "grid24_t5": dict(scales=cwtm.freqs_to_scales(FREQS, 250.0).tolist(), truncate=5.0),
        "grid24_direct": dict(scales=cwtm.freqs_to_scales(FREQS, 250.0).tolist(), method="direct"),
        "gc6": dict(scales=[1.5, 3.0, 6.0, 9.0, 14.0, 23.0]),
        "gc6_m125": dict(scales=[1.5, 3.0, 6.0, 9.0, 14.0, 23.0], support_margin=1.25),
        "cfg3": dict(scales=cwtm.freqs_to_scales(np.logspace(-0.3, 2, 40), 250.0).tolist()),
        "cfg4": dict(scales=cwtm.freqs_to_scales(np.logspace(0, 1.8, 16), 250.0).tolist(),
                     support_margin=1.25),
        "cfg5": dict(scales=cwtm.freqs_to_scales(
            torch.logspace(0, math.log10(max(min(40.0, 200.0 / 4), 1.5)), 16).tolist(), 200.0
        ).tolist(), support_margin=1.25),
        "cfg5s": dict(scales=cwtm.freqs_to_scales(
            torch.logspace(0, math.log10(max(min(40.0, 256.0 / 4), 1.5)), 16).tolist(), 256.0
        ).tolist(), support_margin=1.25),
        "w0_5_l1_real": dict(scales=[2.0, 5.0, 11.0, 40.0, 90.0], w0=5.0, norm="l1",
                             complex=False),
    }
    for name, kw in plans.items():
        p = cwtm.MorletPlan(**kw)
        plan_meta(out, "plan/" + name, p)
        for k, v in kw.items():
            if k != "scales":
                out[f"plan/{name}/kw_{k}"] = np.array(v)
        if p.method == "fast":  # direct filters are long; the closed-form tests pin them
            H = p.filters(torch.tensor(p.scales, dtype=f64), p.w0, f64)
            out[f"plan/{name}/H"] = H.numpy()

    # ---- cwt values (fast / direct, complex / real, l1 / l2, truncate 4 / 5)
    cases = [
        ("fast_n7", 7, dict(method="fast")),
        ("fast_n500", 500, dict(method="fast")),
        ("fast_n3000", 3000, dict(method="fast")),
        ("direct_n500", 500, dict(method="direct")),
        ("fast_t5_n4000", 4000, dict(method="fast", truncate=5.0)),
        ("fast_l1_real_n900", 900, dict(method="fast", norm="l1", complex=False)),
        ("fast_w05_n1100", 1100, dict(method="fast", w0=5.0)),
    ]
    for i, (name, n, kw) in enumerate(cases):
        g = torch.Generator().manual_seed(100 + i)
        x = torch.randn(2, n, generator=g, dtype=f64)
        y = fdwt.cwt(x, freqs=FREQS, fs=250.0, **kw)
        out[f"cwt/{name}/x"] = x.numpy()
        put_big(out, f"cwt/{name}/y", y)
    # cfg3-shaped signal: one row of N(0,1) plus the 6/10/18/30 Hz sinusoids
    g = torch.Generator().manual_seed(7)
    t = torch.arange(2500, dtype=f64)
    x = torch.randn(1, 2500, generator=g, dtype=f64)
    x = x + sum(torch.sin(2 * math.pi * f * t / 250.0) for f in (6.0, 10.0, 18.0, 30.0))
    y = fdwt.cwt(x, freqs=np.logspace(-0.3, 2, 40), fs=250.0)
    out["cwt/cfg3/x"] = x.numpy()
    put_big(out, "cwt/cfg3/y", y)

    # ---- CWT1D gradients (learnable scales and w0), fast and direct, complex and real
    for method in ("fast", "direct"):
        for cplx in (True, False):
            key = f"grad/{method}_{'c' if cplx else 'r'}"
            g = torch.Generator().manual_seed(11)
            x = torch.randn(3, 2, 600, generator=g, dtype=f64)
            gy = torch.randn(3, 2, len(FREQS), 600, 2 if cplx else 1, generator=g, dtype=f64)
            m = fdwt.CWT1D(freqs=FREQS, fs=250, method=method, complex=cplx, learnable=True,
                           learnable_w0=True).double()
            xx = x.clone().requires_grad_()
            y = m(xx)
            yr = torch.view_as_real(y) if cplx else y[..., None]
            (yr * gy).sum().backward()
            out[key + "/x"] = x.numpy()
            out[key + "/gy_seed"] = np.array(11)
            put_big(out, key + "/y", yr.movedim(-1, -2))
            put_big(out, key + "/gx", xx.grad)
            out[key + "/g_log_scales"] = m.log_scales.grad.numpy()
            out[key + "/g_w0"] = m.w0.grad.numpy()

    # ---- fused mix (MorletTokenMixer core), the unfused definition on CPU
    for method in ("fast", "direct"):
        for cplx in (True, False):
            key = f"mix/{method}_{'c' if cplx else 'r'}"
            g = torch.Generator().manual_seed(21)
            m = fdwt.CWT1D(freqs=np.geomspace(1, 60, 12), fs=250, method=method, complex=cplx,
                           learnable=True).double()
            B, D, N = 2, 3, 700
            x = torch.randn(B, D, N, generator=g, dtype=f64)
            a = torch.randn(D, 12, generator=g, dtype=f64)
            b = torch.randn(D, 12, generator=g, dtype=f64)
            gy = torch.randn(B, D, N, generator=g, dtype=f64)
            xx, aa, bb = (t_.clone().requires_grad_() for t_ in (x, a, b))
            H = m.plan.filters(m.log_scales.exp(), m.w0, f64)
            y = cwtm.morlet_mix(xx, m.plan, H, aa, bb)
            (y * gy).sum().backward()
            for nm, v in (("x", x), ("a", a), ("b", b), ("gy", gy)):
                out[f"{key}/{nm}"] = v.numpy()
            put_big(out, key + "/y", y)
            put_big(out, key + "/gx", xx.grad)
            out[key + "/ga"] = aa.grad.numpy()
            out[key + "/gb"] = bb.grad.numpy()
            out[key + "/g_log_scales"] = m.log_scales.grad.numpy()

    # ---- spectral softmax, per-channel and per-position V
    for per_pos in (False, True):
        key = f"ssm/{'pos' if per_pos else 'ch'}"
        g = torch.Generator().manual_seed(31)
        m = fdwt.CWT1D(scales=[1.5, 3.0, 7.0, 13.0, 26.0], learnable=True, learnable_w0=True).double()
        nch, R, N = 3, 6, 300
        x = torch.randn(R, N, generator=g, dtype=f64)
        V = torch.randn((R // nch, 5, N) if per_pos else (nch, 5), generator=g, dtype=f64)
        gy = torch.randn(R, N, generator=g, dtype=f64)
        xx, VV = x.clone().requires_grad_(), V.clone().requires_grad_()
        ls = m.log_scales.detach().clone().requires_grad_()
        w0 = torch.tensor(6.0, dtype=f64, requires_grad=True)
        y = cwtm.spectral_softmax(xx, m.plan, m.plan.filters(ls.exp(), w0, f64), VV, nch, 0.7)
        (y * gy).sum().backward()
        for nm, v in (("x", x), ("V", V), ("gy", gy)):
            out[f"{key}/{nm}"] = v.numpy()
        out[key + "/y"] = y.detach().numpy()
        out[key + "/gx"] = xx.grad.numpy()
        out[key + "/gV"] = VV.grad.numpy()
        out[key + "/g_log_scales"] = ls.grad.numpy()
        out[key + "/g_w0"] = w0.grad.numpy()

    # ---- attention modules (the reference test shapes), parameters stored explicitly
    mods = [
        ("att", fdwt.MorletAttention, dict(num_channels=5, hidden_dim=64, temperature=0.5),
         (2, 3, 5, 6, 64), 1.0),
        ("cmix", fdwt.MorletChannelMixAttention,
         dict(num_channels=5, hidden_dim=64, temperature=0.5), (2, 3, 5, 6, 64), 1.0),
        ("att_big", fdwt.MorletAttention, dict(num_channels=2, hidden_dim=100, temperature=0.01),
         (1, 1, 2, 10, 100), 1e3),
        ("att_f4", fdwt.MorletAttention, dict(num_channels=4, hidden_dim=128,
                                               freqs=[2.0, 6.0, 12.0, 25.0]), (2, 2, 4, 5, 128), 1.0),
        ("cmix_f4", fdwt.MorletChannelMixAttention, dict(num_channels=4, hidden_dim=128,
                                                          freqs=[2.0, 6.0, 12.0, 25.0]),
         (2, 2, 4, 5, 128), 1.0),
    ]
    for name, cls, kw, shape, amp in mods:
        torch.manual_seed(41)
        m = cls(**kw).double()
        g = torch.Generator().manual_seed(43)
        x = amp * torch.randn(*shape, generator=g, dtype=f64)
        xx = x.clone().requires_grad_()
        y = m(xx)
        y.square().sum().backward()
        key = "mod/" + name
        out[key + "/x"] = x.numpy()
        for pn, pv in m.state_dict().items():
            out[f"{key}/param/{pn}"] = pv.detach().numpy()
        out[key + "/y"] = y.detach().numpy()
        out[key + "/gx"] = xx.grad.numpy()
        for pn, pv in m.named_parameters():
            out[f"{key}/grad/{pn}"] = pv.grad.numpy()

    # ---- token mixer
    for name, kw in (("tm_f3", dict(dim=16, freqs=[2.0, 8.0, 30.0], fs=250)),
                     ("tm_nophase", dict(dim=16, use_phase=False))):
        torch.manual_seed(51)
        m = fdwt.MorletTokenMixer(**kw).double()
        g = torch.Generator().manual_seed(53)
        x = torch.randn(2, 300, 16, generator=g, dtype=f64)
        xx = x.clone().requires_grad_()
        y = m(xx)
        y.square().mean().backward()
        key = "tm/" + name
        out[key + "/x"] = x.numpy()
        for pn, pv in m.state_dict().items():
            out[f"{key}/param/{pn}"] = pv.detach().numpy()
        out[key + "/y"] = y.detach().numpy()
        out[key + "/gx"] = xx.grad.numpy()
        for pn, pv in m.named_parameters():
            if pv.grad is not None:
                out[f"{key}/grad/{pn}"] = pv.grad.numpy()

    out["meta/head"] = np.array(HEAD)
    out["meta/k"] = np.array(K)
    out["meta/torch"] = np.array(torch.__version__)
    np.savez_compressed(os.path.join(HERE, "cwt_golden.npz"), **out)
    print(f"cwt_golden.npz: {len(out)} arrays")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
