"""ctypes binding of libfdwt_hip.so (the C ABI declared in include/fdwt_hip.h).

The library is built in-tree by ``__graft_entry__.build()`` (or ``csrc/build.py``) and loaded
after torch, so that it binds to the HIP runtime torch already loaded.  There is no CPU
fallback: every operator of this package raises if its inputs are not on a ROCm device or
if the library is missing.
"""

from __future__ import annotations

import ctypes
import os
import threading
from functools import lru_cache

import torch

_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libfdwt_hip.so")
_LOCK = threading.Lock()
_LIB = None

DTYPE = {torch.float32: 0, torch.float64: 1, torch.float16: 2, torch.bfloat16: 3}
F32_BF16 = 4  # fp32 storage, bf16 matrix-core operands (FDWT_F32_BF16)
ERR_TOO_LONG = -2
ERR_SCRATCH = -3

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_PP = ctypes.POINTER(ctypes.c_void_p)
_PI64 = ctypes.POINTER(ctypes.c_int64)
_PI32 = ctypes.POINTER(ctypes.c_int32)
_DBL = ctypes.c_double

# name -> argument types (restype int unless listed in _RESTYPE)
SIGNATURES = {
    "fdwt_error_string": [ctypes.c_int],
    "fdwt_version": [],
    "fdwt_dwt_analysis": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P],
    "fdwt_dwt_synthesis": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P],
    "fdwt_analysis_chain": [_P, _PP, _P, _P, _P, _I64, _PI64, _PI64, _I32, _I32, _I32, _I32,
                            _I32, _P],
    "fdwt_synthesis_chain": [_P, _PP, _P, _P, _P, _I64, _PI64, _PI64, _I32, _I32, _I32, _I32,
                             _I32, _P],
    "fdwt_chain_max_length": [_I32, _I32],
    "fdwt_halfband": [_P, _P, _P, _I64, _I64, _I64, _I32, _I64, _I32, _I32, _I32, _P],
    "fdwt_morlet_forward": [_P, _P, _P, _I64, _I64, _I64, _I64, _I32, _I32, _PI32, _PI32, _I32,
                            _I32, _I32, _I32, _P],
    "fdwt_morlet_backward_x": [_P, _P, _P, _I64, _I64, _I64, _I64, _I32, _I32, _PI32, _PI32,
                               _I32, _I32, _I32, _I32, _I32, _P],
    "fdwt_morlet_backward_h_workspace": [_I64, _I64, _I32, _I32, _I32],
    "fdwt_morlet_backward_h": [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I32, _I32, _PI32,
                               _PI32, _I32, _I32, _I32, _I32, _I32, _P],
    "fdwt_morlet_backward_h_noalloc_capacity": [],
    "fdwt_morlet_backward_h_noalloc": [_P, _P, _P, _I64, _I64, _I64, _I64, _I32, _I32, _PI32,
                                       _PI32, _I32, _I32, _I32, _I32, _I32, _P],
    "fdwt_mix_workspace": [_I64, _I64, _I32],
    "fdwt_mix_forward": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _I32, _PI32, _PI32,
                         _I32, _I32, _I32, _I32, _I64, _I32, _I32, _P],
    "fdwt_mix_backward": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32,
                          _PI32, _PI32, _I32, _I32, _I32, _I32, _I64, _I32, _P],
    "fdwt_softmax_forward": [_P, _P, _P, _I32, _I64, _I32, _P, _P, _P, _I64, _I64, _I64, _I64,
                             _I32, _I32, _PI32, _PI32, _I32, _DBL, _I32, _I32, _I32, _P],
    "fdwt_softmax_workspace": [_I64, _I64, _I32, _I32],
    "fdwt_softmax_dv_reduce": [_P, _P, _I64, _I32, _I32, _PI32, _I64, _I64, _I64, _I64, _I32,
                               _P],
    "fdwt_morlet_filters": [_P, _P, _PI32, _PI32, _I32, _I32, _I32, _I32, _P, _I32, _P],
    "fdwt_morlet_filters_backward": [_P, _P, _PI32, _PI32, _I32, _I32, _I32, _I32, _P, _I32, _P,
                                     _P, _P],
    "fdwt_softmax_backward": [_P, _P, _P, _I32, _I64, _I32, _I64, _P, _P, _P, _P, _P, _P, _I64,
                              _I64, _I64, _I64, _I64, _I32, _I32, _PI32, _PI32, _I32, _DBL,
                              _I32, _P],
}
_RESTYPE = {"fdwt_error_string": ctypes.c_char_p, "fdwt_version": ctypes.c_char_p,
            "fdwt_chain_max_length": ctypes.c_int64,
            "fdwt_morlet_backward_h_workspace": ctypes.c_int64,
            "fdwt_morlet_backward_h_noalloc_capacity": ctypes.c_int64,
            "fdwt_mix_workspace": ctypes.c_int64, "fdwt_softmax_workspace": ctypes.c_int64}


def library_path() -> str:
    return _PATH


def lib():
    """Load the HIP library (once)."""
    global _LIB
    if _LIB is None:
        with _LOCK:
            if _LIB is None:
                if not os.path.exists(_PATH):
                    raise RuntimeError(
                        f"{_PATH} is missing: build the HIP kernels first "
                        "(python -c 'import __graft_entry__ as g; g.build()')")
                handle = ctypes.CDLL(_PATH)
                for name, args in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.argtypes = args
                    fn.restype = _RESTYPE.get(name, ctypes.c_int)
                _LIB = handle
    return _LIB


_EXT = None
_EXT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_fdwt_autograd.so")


def ext():
    """The C++ autograd nodes of the DWT chains (csrc/autograd.cpp), wired to this library's
    entry points on first use; None when the extension is not built or a launch timer is
    installed (the timer brackets Python-level launches only)."""
    global _EXT
    if _TIMER is not None or not os.path.exists(_EXT_PATH):
        return None
    if _EXT is None:
        with _LOCK:
            if _EXT is None:
                L = lib()
                from . import _fdwt_autograd as m
                addr = lambda f: ctypes.cast(f, ctypes.c_void_p).value  # noqa: E731
                m.set_entry_points(addr(L.fdwt_analysis_chain), addr(L.fdwt_synthesis_chain),
                                   addr(L.fdwt_error_string))
                _EXT = m
    return _EXT


class KernelTimer:
    """Optional per-entry-point timing: when installed (``set_timer``), every launch made
    through :func:`launch` is bracketed by HIP events on the stream it is enqueued on.
    ``summary()`` then gives, per entry point, the number of launches and their mean
    duration (ms), read after a synchronize."""

    def __init__(self):
        self.events = {}

    def record(self, name, device):
        s = torch.cuda.current_stream(device)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        return e0, e1, s

    def summary(self):
        out = {}
        for name, evs in self.events.items():
            ts = [a.elapsed_time(b) for a, b in evs]
            out[name] = (len(ts), sum(ts) / max(1, len(ts)))
        return out


_TIMER = None


def set_timer(timer):
    global _TIMER
    _TIMER = timer


def launch(name: str, device, *args):
    """Call entry point ``name`` with ``args`` on ``device`` and raise on failure."""
    fn = getattr(lib(), name)
    idx = device.index if isinstance(device, torch.device) else device
    if _TIMER is None and (idx is None or idx == torch.cuda.current_device()):
        check(fn(*args), name)  # already the current device: no device switch
        return
    with torch.cuda.device(device):
        if _TIMER is None:
            check(fn(*args), name)
            return
        e0, e1, s = _TIMER.record(name, device)
        code = fn(*args)
        e1.record(s)
        _TIMER.events.setdefault(name, []).append((e0, e1))
        check(code, name)


def check(code: int, what: str = ""):
    if code != 0:
        msg = lib().fdwt_error_string(code).decode()
        raise RuntimeError(f"{what}: {msg} (code {code})" if what else msg)


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "pytorch_morlet_fdwt_amd runs its operators with HIP kernels on ROCm GPU "
                f"tensors only; got a tensor on {t.device}")


def stream(device) -> int:
    """torch's current stream on ``device`` as a raw hipStream_t (an int for the c_void_p
    argument): inside torch.cuda.graph capture this is the capturing stream."""
    idx = device.index if isinstance(device, torch.device) else device
    return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device() if idx is None else idx)


def ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def ptr_array(tensors):
    return (ctypes.c_void_p * max(1, len(tensors)))(
        *[0 if t is None else t.data_ptr() for t in tensors])


def i64_array(values):
    """A C int64 array of ``values``; arrays of tuples are built once and shared (the entry
    points only read them)."""
    if isinstance(values, tuple):
        return _i64_tuple(values)
    return (ctypes.c_int64 * max(1, len(values)))(*[int(v) for v in values])


@lru_cache(maxsize=4096)
def _i64_tuple(values: tuple):
    return (ctypes.c_int64 * max(1, len(values)))(*[int(v) for v in values])


def dtype_code(dtype) -> int:
    try:
        return DTYPE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None
