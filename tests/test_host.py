"""CPU-side checks: the C-ABI library loads and exports every declared symbol, the product
refuses CPU tensors, and the host-side validation raises the reference's errors."""

import os
import re

import pytest
import torch

import pytorch_morlet_fdwt_amd as fdwt
from pytorch_morlet_fdwt_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            names |= set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(fdwt_\w+)\s*\(", src, re.M))
    return names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _declared()
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(lib, name), name
    assert set(_lib.SIGNATURES) == declared
    assert lib.fdwt_version().startswith(b"fdwt-hip")
    assert lib.fdwt_error_string(-1).startswith(b"fdwt")


def test_argument_errors_are_rejected_before_launch():
    lib = _lib.lib()
    # odd filter length, bad mode, bad dtype: rejected without touching the GPU
    args = [None] * 5
    assert lib.fdwt_dwt_analysis(*args, 1, 10, 5, 3, 0, 1, 0, None) == -1
    assert lib.fdwt_dwt_analysis(*args, 1, 10, 5, 4, 9, 1, 0, None) == -1
    assert lib.fdwt_dwt_analysis(*args, 1, 10, 5, 4, 0, 1, 7, None) == -1
    assert lib.fdwt_chain_max_length(16, 0) > 16384


def test_bank_entry_points_reject_empty_input_rows():
    """A bank stage stages x into LDS, so rows of zero samples with outputs to produce are an
    argument error (returned before any launch; the pointers are never dereferenced)."""
    import ctypes
    lib = _lib.lib()
    dummy = ctypes.c_void_p(256)
    sup = (ctypes.c_int32 * 1)(2)
    chan = (ctypes.c_int32 * 1)(0)
    # x, taps, y, rows, n_in, n_out, x_off, n_scales, half, support, chan, dil, channels,
    # s_total, dtype, stream
    assert lib.fdwt_morlet_forward(dummy, dummy, dummy, 1, 0, 5, 0, 1, 2, sup, chan, 1, 2, 1,
                                   0, None) == -1
    # no rows, or no outputs: nothing to do
    assert lib.fdwt_morlet_forward(dummy, dummy, dummy, 0, 0, 5, 0, 1, 2, sup, chan, 1, 2, 1,
                                   0, None) == 0
    assert lib.fdwt_morlet_forward(dummy, dummy, dummy, 1, 0, 0, 0, 1, 2, sup, chan, 1, 2, 1,
                                   0, None) == 0
    # x, taps, v, v_per_position, v_s_total, nch, m, l, num, rows, n_in, n_out, x_off,
    # n_scales, half, support, chan, dil, inv_tau, first, last, dtype, stream
    assert lib.fdwt_softmax_forward(dummy, dummy, dummy, 0, 1, 1, dummy, dummy, dummy, 1, 0, 5,
                                    0, 1, 2, sup, chan, 1, 1.0, 1, 1, 0, None) == -1


def test_cpu_tensors_fail_loudly():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fdwt.dwt(torch.randn(2, 64), "db4")
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fdwt.wavedec(torch.randn(2, 64), "db4", level=2)


def test_reference_errors():
    x = torch.randn(2, 128)
    with pytest.raises(ValueError):
        fdwt.dwt(x, "morl")
    with pytest.raises(ValueError):
        fdwt.dwt(x, "db2", mode="smooth")
    with pytest.raises(ValueError):
        fdwt.idwt(None, None)
    with pytest.raises(ValueError):
        fdwt.idwt(torch.randn(3), torch.randn(4))
    with pytest.raises(ValueError):
        fdwt.idwt(torch.randn(2), torch.randn(2), "db4")  # too short for 8 taps
    with pytest.raises(ValueError):
        fdwt.wavedec(x, "db2", level=-1)
    with pytest.raises(ValueError):
        fdwt.waverec([])
    with pytest.raises(TypeError):
        fdwt.dwt(torch.arange(8), "haar")
    with pytest.raises(ValueError):
        fdwt.get_filter_bank([[1.0, 2.0]])
    with pytest.raises(ValueError):
        fdwt.DWT1D("db2", mode="nope")


def test_filter_banks_and_max_level():
    assert fdwt.get_filter_bank("db4").length == 8
    assert fdwt.get_filter_bank("sym8").length == 16
    assert fdwt.get_filter_bank("coif3").length == 18
    assert fdwt.get_filter_bank("bior3.5").length == 12
    b = fdwt.get_filter_bank(([1.0, 1.0, 1.0], [1.0, -1.0, 0.5], [1, 1, 1], [1, -1, 1]))
    assert b.length == 4 and b.dec_lo[-1] == 0.0
    assert fdwt.dwt_max_level(1000, "db4") == 7
    assert fdwt.dwt_max_level(5, "db4") == 0
    t = fdwt.get_filter_bank("db2").tensors("cpu", torch.float64)
    assert torch.equal(t["rec_lo_rev"], torch.tensor(fdwt.get_filter_bank("db2").rec_lo[::-1],
                                                     dtype=torch.float64))
