"""The allocation-free filter gradient (fdwt_morlet_backward_h_noalloc) through the C ABI,
against the workspace entry point (fdwt_morlet_backward_h) on the same inputs.

Both run the same kernels with the same column count and reduction order, so the results
must agree bit for bit.  Calls in a row share the library's fixed scratch array: the second
call of each pair is smaller than the first, so a column left over from the first would show.
A call too large for the scratch must be refused (FDWT_ERR_SCRATCH) before any launch.
"""

import ctypes

import pytest
import torch

from pytorch_morlet_fdwt_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _i32(v):
    return (ctypes.c_int32 * len(v))(*v)


def _inputs(R, n_out, sup, C, margin, dtype, seed):
    S, g_scales = len(sup), len(sup) + 2
    gen = torch.Generator().manual_seed(seed)
    n_in = n_out + 2 * margin
    x = torch.randn(R, n_in, generator=gen, dtype=torch.float64).to(DEV, dtype)
    g = torch.randn(R, g_scales, n_out, C, generator=gen, dtype=torch.float64).to(DEV, dtype)
    chan = [(2 * s + 1) % g_scales for s in range(S)]
    return x, g, n_in, chan, g_scales


def _args(x, g, R, n_in, n_out, margin, sup, chan, half, dil, C, g_scales, acc, dtype):
    return (R, n_in, n_out, margin, len(sup), half, _i32(sup), _i32(chan), dil, C, g_scales,
            acc, _lib.dtype_code(dtype), _lib.stream(torch.device(DEV)))


def _both(R, n_out, sup, half, dil, C, margin, acc, dtype, seed):
    x, g, n_in, chan, g_scales = _inputs(R, n_out, sup, C, margin, dtype, seed)
    S = len(sup)
    gh0 = torch.randn(S, 2 * half + 1, C, generator=torch.Generator().manual_seed(seed + 1),
                      dtype=torch.float64).to(DEV, dtype)
    rest = _args(x, g, R, n_in, n_out, margin, sup, chan, half, dil, C, g_scales, acc, dtype)
    L = _lib.lib()
    ws_n = L.fdwt_morlet_backward_h_workspace(R, n_out, S, half, C)
    ws = torch.empty(max(1, ws_n), device=DEV, dtype=dtype)
    ref = gh0.clone()
    rc = L.fdwt_morlet_backward_h(_lib.ptr(x), _lib.ptr(g), _lib.ptr(ws), ws_n, _lib.ptr(ref),
                                  *rest)
    assert rc == 0, _lib.lib().fdwt_error_string(rc)
    got = gh0.clone()
    rc = L.fdwt_morlet_backward_h_noalloc(_lib.ptr(x), _lib.ptr(g), _lib.ptr(got), *rest)
    assert rc == 0, _lib.lib().fdwt_error_string(rc)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert torch.equal(got, ref), (got - ref).abs().max().item()


# (R, n_out, sup, half, dil, C, margin, accumulate): the first of each pair takes the
# matrix-core path with hundreds of resident workgroups, the second a smaller stage
# (supports ascending, as every stage orders its scales)
PAIRS = [
    ((512, 3000, [20, 33, 40, 40], 40, 1, 2, 100, 0), (3, 700, [5, 9], 9, 4, 2, 30, 1)),
    ((96, 2100, [55, 70], 70, 8, 2, 600, 1), (5, 300, [12], 12, 2, 1, 0, 0)),  # K = 141: vector
    # 8 + 1 and 16 + 2 scales: matrix cores, then the vector kernel for the trailing group
    ((64, 2000, [4, 5, 6, 7, 8, 9, 10, 11, 12], 12, 4, 2, 30, 1),
     (3, 700, [1 + s * 9 // 17 for s in range(18)], 10, 2, 1, 0, 0)),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("pair", PAIRS, ids=["mfma", "vector", "split"])
def test_noalloc_filter_gradient_matches_workspace_entry(pair, dtype):
    for k, case in enumerate(pair):
        print(f"noalloc case {k}: {case} {dtype}", flush=True)
        _both(*case, dtype=dtype, seed=17 + 100 * k)


def test_noalloc_refuses_calls_beyond_its_scratch():
    """K = 141 runs on the vector kernel, whose partial sums take rows x tiles x n_scales x K x
    channels elements: 2000 rows of one tile, 16 scales, complex -> 9.0 M floats > 32 MiB."""
    L = _lib.lib()
    cap = L.fdwt_morlet_backward_h_noalloc_capacity()
    assert cap == 32 << 20
    R, n_out, half, C = 2000, 700, 70, 2
    sup = [70] * 16
    assert R * 1 * len(sup) * (2 * half + 1) * C * 4 > cap
    x, g, n_in, chan, g_scales = _inputs(R, n_out, sup, C, 0, torch.float32, 5)
    gh = torch.zeros(len(sup), 2 * half + 1, C, device=DEV)
    rc = L.fdwt_morlet_backward_h_noalloc(
        _lib.ptr(x), _lib.ptr(g), _lib.ptr(gh),
        *_args(x, g, R, n_in, n_out, 0, sup, chan, half, 8, C, g_scales, 0, torch.float32))
    assert rc == _lib.ERR_SCRATCH, rc
    assert b"scratch" in L.fdwt_error_string(rc)
    torch.cuda.synchronize()
    assert not gh.any(), "nothing may be launched for a refused call"
