"""fdwt_softmax_dv_reduce through the C ABI: the per-position spectral softmax's dL/dV
partials ((groups * nch) rows, S_g, N) summed over each group's nch rows and added into the
V gradient (G, S_total, N) at the stage's scale indices -- what the reference accumulates with
atomics in its backward stage (src/fdwt/kernels/softmax.py:121-127).  Checked against the same
reduction written with torch on the CPU in float64 (sum over the channel rows, then index_add
at the scale indices), for float32 and float64, with a row-group offset, a scale mapping that
is neither ordered nor contiguous, and lengths that end inside a tile.
"""

import ctypes

import pytest
import torch

from pytorch_morlet_fdwt_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _i32(v):
    return (ctypes.c_int32 * len(v))(*v)


def _reference(part, gv0, groups, nch, chan, g0):
    p = part.double().view(groups, nch, len(chan), -1).sum(1)
    out = gv0.double().clone()
    out[g0:g0 + groups].index_add_(1, torch.tensor(chan, dtype=torch.long), p)
    return out


CASES = [
    # (groups, nch, chan, v_groups, v_s_total, n_out, g0, dtype)
    (4, 19, [5, 2, 9], 6, 12, 6000, 1, torch.float32),
    (3, 1, [0], 3, 1, 1024, 0, torch.float32),
    (2, 7, [3, 0, 7, 1, 6], 5, 8, 1025, 3, torch.float64),
    (5, 3, list(range(16)), 5, 16, 333, 0, torch.float32),
]


@pytest.mark.parametrize("case", CASES, ids=[f"G{c[0]}c{c[1]}S{len(c[2])}n{c[5]}" for c in CASES])
def test_softmax_dv_reduce_matches_torch(case):
    groups, nch, chan, v_groups, v_s_total, n_out, g0, dt = case
    gen = torch.Generator().manual_seed(groups * 100 + nch)
    part = torch.randn(groups * nch, len(chan), n_out, generator=gen, dtype=torch.float64)
    gv0 = torch.randn(v_groups, v_s_total, n_out, generator=gen, dtype=torch.float64)
    ref = _reference(part, gv0, groups, nch, chan, g0)
    p_d = part.to(DEV, dt).contiguous()
    gv = gv0.to(DEV, dt).contiguous()
    L = _lib.lib()
    code = L.fdwt_softmax_dv_reduce(p_d.data_ptr(), gv.data_ptr(), groups, nch, len(chan),
                                    _i32(chan), v_groups, v_s_total, n_out, g0,
                                    _lib.dtype_code(dt), _lib.stream(gv.device))
    assert code == 0, _lib.lib().fdwt_error_string(code)
    torch.cuda.synchronize()
    tol = 1e-12 if dt == torch.float64 else 2e-5 * (nch ** 0.5)
    err = (gv.double().cpu() - ref).abs().max().item()
    assert err < tol, err
    # untouched group rows stay as they were
    keep = [g for g in range(v_groups) if not g0 <= g < g0 + groups]
    if keep:
        assert torch.equal(gv.cpu()[keep], gv0.to(dt)[keep])


def test_softmax_dv_reduce_rejects_bad_arguments():
    """Argument checks run before any launch: a scale index outside V, a group range past V's
    groups, or more scales than a stage holds return FDWT_ERR_ARG."""
    L = _lib.lib()
    p = torch.zeros(2 * 3 * 4, device=DEV)
    gv = torch.zeros(2 * 5 * 4, device=DEV)
    st = _lib.stream(gv.device)
    f32 = _lib.dtype_code(torch.float32)
    ok = L.fdwt_softmax_dv_reduce(p.data_ptr(), gv.data_ptr(), 2, 3, 1, _i32([4]), 2, 5, 4, 0,
                                  f32, st)
    assert ok == 0
    for chan, groups, g0 in (([5], 2, 0), ([0], 2, 1), ([-1], 1, 0)):
        code = L.fdwt_softmax_dv_reduce(p.data_ptr(), gv.data_ptr(), groups, 3, 1, _i32(chan), 2,
                                        5, 4, g0, f32, st)
        assert code != 0
    torch.cuda.synchronize()
