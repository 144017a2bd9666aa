"""The Morlet bank's adjoint (fdwt_morlet_backward_x) and filter gradient
(fdwt_morlet_backward_h) through the C ABI, against autograd of the bank forward.

The forward of one stage is the dilated filter bank of the reference's conv kernels
(src/fdwt/kernels/conv.py:38-134, cwt.py:213-244):
    W[r, s, n, ch] = sum_k H[s, k, ch] x[r, n + x_off - dil (k - half)],  k = 0 .. 2 half,
with x zero outside [0, n_in) and the Morlet symmetry of the taps: the real filter is even
around k = half and the imaginary one odd, both zero beyond the scale's support.  Here that
forward is written as a gather + einsum in float64 on the CPU; torch autograd then gives the
exact adjoint (w.r.t. x) and the exact tap gradient (w.r.t. H), which the two entry points
must reproduce.  The grid covers every code path: dilations 1..128 (power-of-two windowed
adjoint with every residue-group size, and the tiled kernel for a non-power-of-two
dilation), tap counts on both sides of the matrix-core limit (K <= 128), real and complex
banks, accumulate on/off, margins inside and beyond g's reach, float32 and float64.
"""

import ctypes

import pytest
import torch

from pytorch_morlet_fdwt_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _i32(v):
    return (ctypes.c_int32 * len(v))(*v)


def _full_taps(taps, sup):
    """(S, half + 1, C) compact taps -> (S, 2 half + 1, C) full filters (even real, odd
    imaginary, zero beyond each scale's support)."""
    S, h1, C = taps.shape
    half = h1 - 1
    k = torch.arange(-half, half + 1)
    full = taps[:, k.abs(), :].clone()
    if C == 2:
        full[:, :, 1] *= torch.sign(k).to(taps.dtype)[None, :]
    mask = (k.abs()[None, :] <= torch.tensor(sup)[:, None]).to(taps.dtype)
    return full * mask[:, :, None]


def _forward(x, Hf, half, dil, x_off, n_out):
    """W[r, s, n, ch] = sum_k Hf[s, k, ch] x[r, n + x_off - dil (k - half)]."""
    R, n_in = x.shape
    n = torch.arange(n_out)[:, None]
    k = torch.arange(2 * half + 1)[None, :]
    idx = n + x_off - dil * (k - half)
    ok = (idx >= 0) & (idx < n_in)
    xs = x[:, idx.clamp(0, n_in - 1)] * ok.to(x.dtype)  # (R, n_out, K)
    return torch.einsum("rnk,skc->rsnc", xs, Hf)


CASES = [
    # (dil, half, sups, C, margin, accumulate)
    (1, 3, [1, 3], 2, 0, 0),
    (1, 40, [12, 30, 40], 2, 0, 1),
    (2, 17, [17], 1, 60, 0),
    (3, 9, [4, 9], 2, 40, 1),         # non-power-of-two dilation: tiled kernel
    (8, 40, [25, 40], 2, 900, 0),     # margin beyond g's reach: zero fill
    (8, 70, [50, 70], 2, 0, 1),       # K = 141: filter gradient on the vector kernel
    (64, 20, [10, 20], 2, 1400, 1),
    (64, 38, [38], 1, 2500, 0),
    (128, 9, [5, 9], 2, 1300, 0),     # dilation above 64: residue groups of at most 64
    # more scales than one matrix-core group of 16 / C: a trailing single scale (9 = 8 + 1) on
    # the vector kernel, its partial sums after the matrix-core ones in the same workspace;
    # 18 = 16 + 2: a second, partly filled matrix-core group
    (4, 12, [4, 5, 6, 7, 8, 9, 10, 11, 12], 2, 30, 1),
    (2, 10, [1 + s * 9 // 17 for s in range(18)], 1, 0, 0),
]


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32], ids=["f64", "f32"])
@pytest.mark.parametrize("case", CASES, ids=[f"d{c[0]}h{c[1]}C{c[3]}m{c[4]}a{c[5]}" for c in CASES])
def test_bank_adjoint_and_filter_gradient(case, dtype):
    dil, half, sup, C, margin, acc = case
    R, n_out, S, g_scales = 3, 700, len(sup), len(sup) + 2
    chan = [(2 * s + 1) % g_scales for s in range(S)]  # a non-trivial scale -> channel map
    n_in, x_off = n_out + 2 * margin, margin
    gen = torch.Generator().manual_seed(dil * 1000 + half)
    f64 = torch.float64
    x = torch.randn(R, n_in, dtype=f64, generator=gen, requires_grad=True)
    taps = torch.randn(S, half + 1, C, dtype=f64, generator=gen)
    Hf = _full_taps(taps, sup)
    g = torch.randn(R, g_scales, n_out, C, dtype=f64, generator=gen)
    (gx_ref,) = torch.autograd.grad(_forward(x, Hf, half, dil, x_off, n_out), [x], g[:, chan])
    gx0 = torch.randn(R, n_in, dtype=f64, generator=gen)
    if acc:
        gx_ref = gx_ref + gx0

    dt = _lib.dtype_code(dtype)
    gd = g.to(DEV, dtype).contiguous()
    td = taps.to(DEV, dtype).contiguous()
    gx = gx0.to(DEV, dtype).contiguous() if acc else torch.full((R, n_in), float("nan"),
                                                                device=DEV, dtype=dtype)
    _lib.launch("fdwt_morlet_backward_x", torch.device(DEV), _lib.ptr(gd), _lib.ptr(td),
                _lib.ptr(gx), R, n_in, n_out, x_off, S, half, _i32(sup), _i32(chan), dil, C,
                g_scales, acc, dt, _lib.stream(torch.device(DEV)))
    xd = x.detach().to(DEV, dtype).contiguous()
    L = _lib.lib()
    ws_n = L.fdwt_morlet_backward_h_workspace(R, n_out, S, half, C)
    ws = torch.empty(max(1, ws_n), device=DEV, dtype=dtype)
    gh = torch.empty(S, 2 * half + 1, C, device=DEV, dtype=dtype)
    _lib.launch("fdwt_morlet_backward_h", torch.device(DEV), _lib.ptr(xd), _lib.ptr(gd),
                _lib.ptr(ws), ws_n, _lib.ptr(gh), R, n_in, n_out, x_off, S, half, _i32(sup),
                _i32(chan), dil, C, g_scales, 0, dt, _lib.stream(torch.device(DEV)))
    torch.cuda.synchronize()
    tol = 1e-10 if dtype == f64 else 2e-5
    gx_c = gx.cpu().to(f64)
    assert torch.isfinite(gx_c).all(), "positions outside g's reach must be written"
    torch.testing.assert_close(gx_c, gx_ref, rtol=0, atol=tol * gx_ref.abs().max().item())
    # the kernel returns the gradient of every tap, inside a scale's support or not (the
    # reference's backward_h does too): the gradient of the forward w.r.t. unmasked filters
    ref_h = _tap_gradient(x.detach(), g[:, chan], half, dil, x_off, n_out)
    torch.testing.assert_close(gh.cpu().to(f64), ref_h, rtol=0,
                               atol=tol * ref_h.abs().max().item())


def _tap_gradient(x, g, half, dil, x_off, n_out):
    """d/dH of sum(W * g) for unmasked full filters: the correlation of g with x."""
    S, C = g.shape[1], g.shape[3]
    H = torch.zeros(S, 2 * half + 1, C, dtype=x.dtype, requires_grad=True)
    (gH,) = torch.autograd.grad(_forward(x, H, half, dil, x_off, n_out), [H], g)
    return gH


# stages the bf16 matrix-core adjoint takes (power-of-two dilation, at most 56 taps per side);
# the others compute in fp32 (bf16 operands are a permission, not a requirement)
BF16_CASES = [c for c in CASES if c[1] <= 56 and c[0] & (c[0] - 1) == 0]


@pytest.mark.parametrize("case", BF16_CASES, ids=[f"d{c[0]}h{c[1]}C{c[3]}m{c[4]}a{c[5]}" for c in BF16_CASES])
def test_bank_adjoint_bf16_operands(case):
    """FDWT_F32_BF16 (the reference's "bf16" precision, conv.py:192-196): g and the taps are
    rounded to bf16, products and sums are fp32.  Against the adjoint of the bf16-rounded
    operands computed in float64 the kernel must agree to fp32 accumulation (1e-5 of the
    largest value); against the exact adjoint to the reference's ~5e-3 (README.md:206-212)."""
    dil, half, sup, C, margin, acc = case
    R, n_out, S, g_scales = 3, 700, len(sup), len(sup) + 2
    chan = [(2 * s + 1) % g_scales for s in range(S)]
    n_in, x_off = n_out + 2 * margin, margin
    gen = torch.Generator().manual_seed(dil * 1000 + half + 7)
    f64 = torch.float64
    taps = torch.randn(S, half + 1, C, dtype=f64, generator=gen).float()
    g = torch.randn(R, g_scales, n_out, C, dtype=f64, generator=gen).float()
    gx0 = torch.randn(R, n_in, dtype=f64, generator=gen).float()

    def adjoint(t, gg):
        x = torch.zeros(R, n_in, dtype=f64, requires_grad=True)
        (gx,) = torch.autograd.grad(_forward(x, _full_taps(t.double(), sup), half, dil, x_off,
                                             n_out), [x], gg[:, chan].double())
        return gx + gx0.double() if acc else gx

    bf = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
    ref_bf = adjoint(bf(taps), bf(g))
    ref = adjoint(taps, g)
    gd, td = g.to(DEV).contiguous(), taps.to(DEV).contiguous()
    gx = gx0.to(DEV).contiguous() if acc else torch.full((R, n_in), float("nan"), device=DEV)
    _lib.launch("fdwt_morlet_backward_x", torch.device(DEV), _lib.ptr(gd), _lib.ptr(td),
                _lib.ptr(gx), R, n_in, n_out, x_off, S, half, _i32(sup), _i32(chan), dil, C,
                g_scales, acc, _lib.F32_BF16, _lib.stream(torch.device(DEV)))
    torch.cuda.synchronize()
    got = gx.cpu().double()
    assert torch.isfinite(got).all()
    scale = ref_bf.abs().max().item()
    torch.testing.assert_close(got, ref_bf, rtol=0, atol=1e-5 * scale)
    err = (got - ref).abs().max().item() / ref.abs().max().item()
    assert err < 1e-2, err


# stages whose filter gradient runs on the matrix cores (K = 2 half + 1 <= 128)
GH_BF16_CASES = [c for c in CASES if 2 * c[1] + 1 <= 128]


@pytest.mark.parametrize("case", GH_BF16_CASES,
                         ids=[f"d{c[0]}h{c[1]}C{c[3]}m{c[4]}" for c in GH_BF16_CASES])
def test_filter_gradient_bf16_operands(case):
    """FDWT_F32_BF16 for the filter gradient (the reference's "bf16" precision for backward_h,
    conv.py:372-408): on the matrix cores g and x are rounded to bf16 and the products summed
    in fp32.  Those scales must match the tap gradient of the bf16-rounded operands computed in
    float64 to fp32 accumulation (1e-5 of the largest value) and the exact gradient to the
    mode's ~5e-3 (README.md:206-212).  With bf16 operands every scale runs on the matrix cores
    (no trailing group on the vector kernel)."""
    dil, half, sup, C, margin, _ = case
    R, n_out, S, g_scales = 3, 700, len(sup), len(sup) + 2
    chan = [(2 * s + 1) % g_scales for s in range(S)]
    n_in, x_off = n_out + 2 * margin, margin
    gen = torch.Generator().manual_seed(dil * 1000 + half + 11)
    f64 = torch.float64
    x = torch.randn(R, n_in, dtype=f64, generator=gen).float()
    g = torch.randn(R, g_scales, n_out, C, dtype=f64, generator=gen).float()
    bf = lambda t: t.to(torch.bfloat16).double()  # noqa: E731
    ref_bf = _tap_gradient(bf(x), bf(g)[:, chan], half, dil, x_off, n_out)
    ref = _tap_gradient(x.double(), g.double()[:, chan], half, dil, x_off, n_out)
    L = _lib.lib()
    ws_n = L.fdwt_morlet_backward_h_workspace(R, n_out, S, half, C)
    ws = torch.empty(max(1, ws_n), device=DEV)
    gh = torch.full((S, 2 * half + 1, C), float("nan"), device=DEV)
    xd, gd = x.to(DEV).contiguous(), g.to(DEV).contiguous()
    _lib.launch("fdwt_morlet_backward_h", torch.device(DEV), _lib.ptr(xd), _lib.ptr(gd),
                _lib.ptr(ws), ws_n, _lib.ptr(gh), R, n_in, n_out, x_off, S, half, _i32(sup),
                _i32(chan), dil, C, g_scales, 0, _lib.F32_BF16, _lib.stream(torch.device(DEV)))
    torch.cuda.synchronize()
    got = gh.cpu().double()
    assert torch.isfinite(got).all()
    scale = ref_bf.abs().max().item()
    torch.testing.assert_close(got, ref_bf, rtol=0, atol=1e-5 * scale)
    err = (got - ref).abs().max().item() / ref.abs().max().item()
    assert err < 1e-2, err
