"""HIP graph capture of the DWT hot path: wavedec -> waverec forward plus backward (the
configs[0] step, on fewer rows) captured with torch.cuda.graph and replayed.

Capture rules this follows:
* the leaf that receives the gradient is created after every earlier autograd graph that
  used it is gone, and the warm-up runs on the capture's side stream, so no autograd node
  made on the default stream is reached inside the capture (such a node makes the autograd
  engine synchronise the default stream with the capturing one);
* the entry points are launched on torch's current stream, which inside the capture is the
  capturing stream, and make no allocation, copy or synchronisation of their own.
Every replay, with eager work and a synchronisation in between, must equal the eager result
bit for bit (same kernels, same inputs).
"""

import pytest
import torch

import pytorch_morlet_fdwt_amd as fdwt

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("wavelet,mode,level,shape,n",
                         [("db4", "symmetric", 5, (4, 64), 2500),
                          ("sym8", "periodization", 4, (2, 8), 5000)])
def test_dwt_step_graph_replays_match_eager(wavelet, mode, level, shape, n):
    gen = torch.Generator().manual_seed(n)
    x = torch.randn(*shape, n, generator=gen).to(DEV)
    gy_host = torch.randn(*shape, n, generator=gen)

    def step(xl, gy):
        y = fdwt.waverec(fdwt.wavedec(xl, wavelet, mode, level), wavelet, mode)
        (gx,) = torch.autograd.grad(y, xl, gy)
        return y.detach(), gx

    # eager reference on a leaf of its own
    xe = x.clone().requires_grad_()
    y_ref, gx_ref = step(xe, gy_host.to(DEV)[..., : n])
    del xe
    torch.cuda.synchronize()

    xg = x.clone().requires_grad_()
    gy = gy_host.to(DEV).contiguous()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step(xg, gy)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    print(f"capture {wavelet}/{mode}/{level} {shape}x{n}", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_out, gx_out = step(xg, gy)
    torch.cuda.synchronize()
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_out, y_ref), f"replay {r}: y"
        assert torch.equal(gx_out, gx_ref), f"replay {r}: gx"
        # eager work between replays, on the same tensors' memory pool neighbours
        z = fdwt.wavedec(x * (r + 2), wavelet, mode, level)
        torch.cuda.synchronize()
        del z
    # the graph reads xg's storage: a new input copied in is transformed on replay
    xg.data.mul_(-1.0)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y_out, -y_ref) and torch.equal(gx_out, gx_ref)
    del g
