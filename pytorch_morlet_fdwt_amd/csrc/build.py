"""Build libfdwt_hip.so (all HIP sources of this directory) for gfx950 with hipcc.

    python build.py [-j JOBS]

Objects go to ``_build/`` next to this file; the library is written into the package
directory (``pytorch_morlet_fdwt_amd/libfdwt_hip.so``), where the loader finds it.
"""

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
OUT = os.path.join(PKG, "libfdwt_hip.so")
ARCH = os.environ.get("FDWT_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-I", os.path.join(ROOT, "include"),
    # packed fp32 (v_pk_*_f32) stays off: plain fp32 FMAs only
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def compile_one(src, obj):
    cmd = [hipcc(), *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{out}")
    return out


def build(jobs=None):
    bdir = os.path.join(HERE, "_build")
    os.makedirs(bdir, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(HERE, "*.hip")))
    objs = [os.path.join(bdir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        for msg in ex.map(compile_one, srcs, objs):
            if msg.strip():
                print(msg)
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}")
    os.replace(tmp, OUT)
    return OUT


EXT = os.path.join(PKG, "_fdwt_autograd.so")


def build_ext():
    """The C++ autograd nodes of the DWT chains (autograd.cpp), a torch extension built with
    torch.utils.cpp_extension (g++, torch and ROCm headers) into ``_build/ext`` and copied into
    the package as ``_fdwt_autograd.so``."""
    import torch
    from torch.utils import cpp_extension
    bdir = os.path.join(HERE, "_build", "ext")
    os.makedirs(bdir, exist_ok=True)
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    cpp_extension.load(
        name="_fdwt_autograd", sources=[os.path.join(HERE, "autograd.cpp")],
        extra_include_paths=["/opt/rocm/include"],
        extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1"],
        extra_ldflags=[f"-L{torch_lib}", "-lc10_hip"], build_directory=bdir, with_cuda=False,
        verbose=False, is_python_module=True)
    shutil.copyfile(os.path.join(bdir, "_fdwt_autograd.so"), EXT + ".tmp")
    os.replace(EXT + ".tmp", EXT)
    return EXT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    print(build(ap.parse_args().j))
    print(build_ext())
