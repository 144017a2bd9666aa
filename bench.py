"""Benchmark of the fdwt hot path on one MI355X (driver contract: one JSON line).

Workload (the DWT mode/filter sweep): for wavelet in
{sym8, coif3} x mode in {zero, periodic, symmetric, reflect, periodization} x length in
{16384, 16383}: ``y = waverec(wavedec(x, level=6))`` on x fp32 (16, 128, N) ~ N(0, 1), then the
backward of y against a random-normal upstream gradient.  One step = all 20 combinations,
forward + backward.  Inputs are synthetic and resident in HBM before the timed region.

value = algorithmic HBM bytes of the step / step time (GB/s): every input of each of the
four fused launches per combination read once, every output written once
(2 N + 2 M + 4 C samples per row, N input, M = waverec length, C = coefficient count).

roofline: the dominant kernel's algorithmic bytes per launch / its mean launch time, timed
live with HIP events on its stream during the timed steps, against 8 TB/s.
cpu_baseline: the CPU oracle (oracle/, the reference's PyTorch fallback restated) on a
bounded row sample of the same step, timed on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12
WAVELETS = ("sym8", "coif3")
MODES = ("zero", "periodic", "symmetric", "reflect", "periodization")
LENGTHS = (16384, 16383)
SHAPE = (16, 128)
LEVEL = 6


def coeff_lengths(n, L, mode, level):
    out = []
    for _ in range(level):
        n = (n + 1) // 2 if mode == "periodization" else (n + L - 1) // 2
        out.append(n)
    return out


def combo_geometry(wavelet, mode, n):
    import pytorch_morlet_fdwt_amd as fdwt
    L = fdwt.get_filter_bank(wavelet).length
    lens = coeff_lengths(n, L, mode, LEVEL)
    C = sum(lens) + lens[-1]  # details of every level + the final approximation
    # waverec length (zero-mode or periodization synthesis with the trim rule)
    m = lens[-1]
    for d in reversed(lens):
        if m == d + 1:
            m = d
        m = 2 * d if mode == "periodization" else 2 * d - L + 2
    return C, m


def make_inputs(dev):
    R = SHAPE[0] * SHAPE[1]
    data = {}
    for n in LENGTHS:
        g = torch.Generator().manual_seed(0)
        x = torch.randn(*SHAPE, n, generator=g)
        data[n] = x.to(dev)
    grads = {}
    for w in WAVELETS:
        for mode in MODES:
            for n in LENGTHS:
                _, m = combo_geometry(w, mode, n)
                if (m,) not in grads:
                    g = torch.Generator().manual_seed(1)
                    grads[(m,)] = torch.randn(*SHAPE, m, generator=g).to(dev)
    return R, data, grads


def step_gpu(fdwt, data, grads):
    for w in WAVELETS:
        for mode in MODES:
            for n in LENGTHS:
                x = data[n].requires_grad_(True)
                coeffs = fdwt.wavedec(x, w, mode, LEVEL)
                y = fdwt.waverec(coeffs, w, mode)
                (gx,) = torch.autograd.grad(y, x, grads[(y.shape[-1],)])
                x.requires_grad_(False)


def step_bytes(R):
    total = 0
    per_kernel = {"fdwt_analysis_chain": [], "fdwt_synthesis_chain": []}
    for w in WAVELETS:
        for mode in MODES:
            for n in LENGTHS:
                C, m = combo_geometry(w, mode, n)
                total += 4 * R * (2 * n + 2 * m + 4 * C)
                per_kernel["fdwt_analysis_chain"] += [4 * R * (n + C), 4 * R * (m + C)]
                per_kernel["fdwt_synthesis_chain"] += [4 * R * (C + m), 4 * R * (C + n)]
    return total, per_kernel


def cpu_baseline(rows=16, reps=3):
    """The oracle (reference CPU fallback restated, fp32) on `rows` rows of every combo."""
    from oracle import dwt as O
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    xs = {}
    for n in LENGTHS:
        g = torch.Generator().manual_seed(0)
        xs[n] = torch.randn(*SHAPE, n, generator=g).reshape(-1, n)[:rows].contiguous()

    def run():
        for w in WAVELETS:
            for mode in MODES:
                for n in LENGTHS:
                    x = xs[n].clone().requires_grad_()
                    y = O.waverec(O.wavedec(x, w, mode, LEVEL), w, mode)
                    g = torch.Generator().manual_seed(1)
                    gy = torch.randn(y.shape, generator=g)
                    torch.autograd.grad(y, x, gy)

    run()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    total, _ = step_bytes(rows)
    return {"value": total / t / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the full 20-combination step on {rows} of {SHAPE[0] * SHAPE[1]} rows, "
                      f"fp32, torch {torch.__version__} CPU, median of {reps} after 1 warm-up "
                      f"({t:.2f} s per step)"}


ATT_SHAPE = (8, 4, 19, 30, 200)  # (B, H, C, T, D)
FP32_PEAK = 157.3e12


def attention_flops(m, R, N):
    """Algorithmic FLOPs of one MorletAttention forward + backward (2 per real filter-tap
    MAC, unfolded taps, half-band chain included): forward = chain + filter bank; backward =
    chain recompute + bank recompute + grad-x + grad-h + transposed chain."""
    plan = m.cwt.plan
    bank = 0
    for st in plan.stages:
        for sup in st.support:
            bank += 2 * 2 * (2 * sup + 1) * plan.channels * R * N
    chain = 0
    for j in range(plan.n_octaves - 1):
        chain += 2 * (2 * plan.c_lp + 1) * R * (N + 2 * plan.margins[j + 1])
    return 4 * bank + 3 * chain


def attention_gpu(steps, warmup, dev):
    import pytorch_morlet_fdwt_amd as fdwt
    B, H, C, T, D = ATT_SHAPE
    torch.manual_seed(2)
    m = fdwt.MorletAttention(num_channels=C, hidden_dim=D).to(dev)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(*ATT_SHAPE, generator=g).to(dev).requires_grad_()
    gy = torch.randn(*ATT_SHAPE, generator=torch.Generator().manual_seed(1)).to(dev)
    params = [x] + list(m.parameters())

    def step():
        y = m(x)
        torch.autograd.grad(y, params, gy)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    R, N = B * H * C, T * D
    fl = attention_flops(m, R, N)
    tokens = B * C * T
    return {"metric": "MorletAttention fwd+bwd tokens/s (B*C*T per step)",
            "value": tokens / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms,
            "config": {"shape_BHCTD": list(ATT_SHAPE), "freqs": "16 logspace(0, log10(40)) Hz",
                       "fs": D, "learnable": True, "temperature": 1.0},
            "roofline": {"bound": "valu", "achieved": fl / (ms * 1e-3) / 1e12,
                         "peak": FP32_PEAK / 1e12, "unit": "TFLOP/s",
                         "frac": fl / (ms * 1e-3) / FP32_PEAK, "alg_flops": fl}}


def attention_cpu(batch=1, reps=3):
    """The oracle (reference CPU fallback restated, fp32) on a batch-`batch` sample."""
    from oracle import cwt as O
    import pytorch_morlet_fdwt_amd as fdwt
    B, H, C, T, D = ATT_SHAPE
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    torch.manual_seed(2)
    m = fdwt.MorletAttention(num_channels=C, hidden_dim=D)
    plan = O.Plan(m.cwt.plan.scales, support_margin=1.25)
    x = torch.randn(batch, H, C, T, D, generator=torch.Generator().manual_seed(0))
    ls = m.cwt.log_scales.detach().clone().requires_grad_()
    w0 = torch.tensor(6.0, requires_grad=True)
    fw = m.freq_weight.detach().clone().requires_grad_()

    def run():
        xx = x.clone().requires_grad_()
        Hf = plan.filters(ls.double().exp(), w0.double(), torch.float32)
        y = O.attention(xx, plan, Hf, fw, 1.0)
        torch.autograd.grad(y, [xx, ls, w0, fw], torch.ones_like(y))

    run()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    return {"value": batch * C * T / t, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"B={batch} of {B} (shape {[batch, H, C, T, D]}), fp32, learnable scales "
                      f"and w0, median of {reps} after 1 warm-up ({t:.2f} s per step)"}


def measured_traffic(kernel):
    """HBM bytes per launch of ``kernel`` on this workload, as measured by the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (calibrated against a plain copy), or None."""
    path = os.path.join(ROOT, "profiles", "dwt_sweep_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)[kernel]["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-attention", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=64)
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 256 MiB device copy (HBM counter calibration)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's hot path is a per-row transform "
              "with no cross-GPU exchange, so run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if a.copy_probe:
        src = torch.randn(64 * 2**20, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_each_way": src.numel() * 4, "launches": 5}))
        return

    import pytorch_morlet_fdwt_amd as fdwt
    from pytorch_morlet_fdwt_amd import _lib

    R, data, grads = make_inputs(dev)
    for _ in range(a.warmup):
        step_gpu(fdwt, data, grads)
    torch.cuda.synchronize()

    timer = _lib.KernelTimer()
    _lib.set_timer(timer)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(a.steps):
        step_gpu(fdwt, data, grads)
    e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _lib.set_timer(None)
    ms = e0.elapsed_time(e1) / a.steps
    wall_ms = (t1 - t0) * 1e3 / a.steps
    total, per_kernel = step_bytes(R)
    value = total / (ms * 1e-3) / 1e9

    kernels = {}
    for name, (count, mean_ms) in timer.summary().items():
        b = per_kernel.get(name)
        if not b:
            continue
        avg_bytes = sum(b) / len(b)
        kernels[name] = {"launches": count, "mean_ms": mean_ms, "alg_bytes": avg_bytes,
                         "gbps": avg_bytes / (mean_ms * 1e-3) / 1e9}
    dom = max(kernels, key=lambda k: kernels[k]["launches"] * kernels[k]["mean_ms"])
    ach = kernels[dom]["gbps"]
    roofline = {"kernel": dom, "bound": "hbm", "achieved": ach, "peak": HBM_PEAK / 1e9,
                "unit": "GB/s", "frac": ach / (HBM_PEAK / 1e9), "traffic": measured_traffic(dom),
                "alg_bytes_per_launch": kernels[dom]["alg_bytes"],
                "mean_launch_ms": kernels[dom]["mean_ms"]}

    line = {
        "metric": "wavedec+waverec fwd+bwd GB/s (algorithmic HBM bytes / step time)",
        "value": value, "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": ms, "wall_ms_per_step": wall_ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "frac_hbm_peak": value / (HBM_PEAK / 1e9),
        "samples_per_s": len(WAVELETS) * len(MODES) * sum(LENGTHS) * R / (ms * 1e-3),
        "config": {"workload": "DWT mode/filter sweep (BASELINE configs[1]): waverec(wavedec(x)) "
                               "fwd+bwd, wavelets sym8/coif3, 5 modes, level 6, x fp32 "
                               "(16,128,16384) and (16,128,16383)",
                   "rows": R, "lengths": list(LENGTHS), "wavelets": list(WAVELETS),
                   "modes": list(MODES), "level": LEVEL, "parallelism": "single GPU"},
        "roofline": roofline,
        "kernels": kernels,
    }
    if not a.no_attention:
        att = attention_gpu(max(3, a.steps // 2), a.warmup, dev)
        if not a.no_cpu_baseline:
            att["cpu_baseline"] = attention_cpu()
        line["morlet_attention"] = att
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(a.cpu_rows)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
