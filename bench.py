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


def cpu_model() -> str:
    """The host CPU's model name (first processor in /proc/cpuinfo), for the baseline record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


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
            "cpu_model": cpu_model(),
            "sample": f"the full 20-combination step on {rows} of {SHAPE[0] * SHAPE[1]} rows, "
                      f"fp32, torch {torch.__version__} CPU, median of {reps} after 1 warm-up "
                      f"({t:.2f} s per step)"}


ATT_SHAPE = (8, 4, 19, 30, 200)  # (B, H, C, T, D)
FP32_PEAK = 157.3e12


def attention_flops(m, R, N):
    """Algorithmic FLOPs of one MorletAttention forward + backward (2 per real filter-tap
    MAC, unfolded taps, half-band chain included): forward = chain + filter bank; backward =
    chain recompute + bank recompute + grad-x + grad-h + transposed chain."""
    bank, chain = bank_chain_flops(m.cwt.plan, R, N)
    return 4 * bank + 3 * chain


ATT_SCALED = (64, 8, 64, 60, 256)  # BASELINE configs[4]'s scaled shape


def _att_module(fdwt, channel_mix, C, D):
    cls = fdwt.MorletChannelMixAttention if channel_mix else fdwt.MorletAttention
    return cls(num_channels=C, hidden_dim=D)


def attention_gpu(steps, warmup, dev, shape=ATT_SHAPE, channel_mix=False):
    """MorletAttention (or, with ``channel_mix``, MorletChannelMixAttention) forward +
    backward on x of ``shape``; learnable scales and w0, module-default weights (seed 2)."""
    import pytorch_morlet_fdwt_amd as fdwt
    B, H, C, T, D = shape
    torch.manual_seed(2)
    m = _att_module(fdwt, channel_mix, C, D).to(dev)
    x = torch.randn(*shape, generator=torch.Generator(device=dev).manual_seed(0),
                    device=dev).requires_grad_()
    gy = torch.randn(*shape, generator=torch.Generator(device=dev).manual_seed(1), device=dev)
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
    if channel_mix:  # U = M x (f x C by C x N per (b, h)): forward, grad-x and grad-M
        fl += 3 * 2 * m.num_freqs * C * N * B * H
    tokens = B * C * T
    name = "MorletChannelMixAttention" if channel_mix else "MorletAttention"
    return {"metric": f"{name} fwd+bwd tokens/s (B*C*T per step)",
            "value": tokens / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms,
            "config": {"shape_BHCTD": list(shape), "freqs": "16 logspace(0, log10(40)) Hz",
                       "fs": D, "learnable": True, "temperature": 1.0},
            "roofline": {"bound": "valu", "achieved": fl / (ms * 1e-3) / 1e12,
                         "peak": FP32_PEAK / 1e12, "unit": "TFLOP/s",
                         "frac": fl / (ms * 1e-3) / FP32_PEAK, "alg_flops": fl}}


def bf16_mode(leg, *args):
    """The same leg with ``config.allow_bf16`` set (the reference's "bf16" precision: bf16
    matrix-core operands with fp32 accumulation in the bank adjoint and filter gradient): its
    step time and throughput, reported beside the fp32 line (a mode the reference offers for
    speed, not the headline's arithmetic)."""
    import pytorch_morlet_fdwt_amd as fdwt
    saved = fdwt.config.allow_bf16
    fdwt.config.allow_bf16 = True
    try:
        r = leg(*args)
    finally:
        fdwt.config.allow_bf16 = saved
    return {"ms_per_step": r["ms_per_step"], "value": r["value"], "unit": r["unit"],
            "precision": "bf16 operands, fp32 accumulation (config.allow_bf16)"}


def attention_cpu(batch=1, reps=3, channel_mix=False):
    """The oracle (reference CPU fallback restated, fp32) on a batch-`batch` sample."""
    from oracle import cwt as O
    import pytorch_morlet_fdwt_amd as fdwt
    B, H, C, T, D = ATT_SHAPE
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    torch.manual_seed(2)
    m = _att_module(fdwt, channel_mix, C, D)
    plan = O.Plan(m.cwt.plan.scales, support_margin=1.25)
    x = torch.randn(batch, H, C, T, D, generator=torch.Generator().manual_seed(0))
    ls = m.cwt.log_scales.detach().clone().requires_grad_()
    w0 = torch.tensor(6.0, requires_grad=True)
    fw = (m.freq_to_channel if channel_mix else m.freq_weight).detach().clone().requires_grad_()
    op = O.channel_mix_attention if channel_mix else O.attention

    def run():
        xx = x.clone().requires_grad_()
        Hf = plan.filters(ls.double().exp(), w0.double(), torch.float32)
        y = op(xx, plan, Hf, fw, 1.0)
        torch.autograd.grad(y, [xx, ls, w0, fw], torch.ones_like(y))

    run()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    return {"value": batch * C * T / t, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"B={batch} of {B} (shape {[batch, H, C, T, D]}), fp32, learnable scales "
                      f"and w0, median of {reps} after 1 warm-up ({t:.2f} s per step)"}


def _timed(step, steps, warmup):
    """Mean ms per call of ``step`` over ``steps`` calls after ``warmup`` untimed ones
    (torch events on the current stream, which is the stream every entry point launches on)."""
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
    return e0.elapsed_time(e1) / steps


def _graph_timed(step, steps):
    """Mean ms per replay of ``step`` captured in one HIP graph.  The warm-up runs on the
    capture's side stream and no autograd graph from before the capture is alive, so every
    node the capture reaches was made on the capturing stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    return _timed(g.replay, steps, 2)


def _cpu_median(run, reps=3):
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    run()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), threads


def bank_chain_flops(plan, R, N):
    """(bank, chain) FLOPs of one pass of a plan over R rows of N samples: 2 per real
    filter-tap MAC, unfolded taps, real and imaginary parts; the half-band chain over the
    margins it runs on."""
    bank = 0
    for st in plan.stages:
        for sup in st.support:
            bank += 2 * plan.channels * (2 * sup + 1) * R * N
    chain = 0
    for j in range(plan.n_octaves - 1):
        chain += 2 * (2 * plan.c_lp + 1) * R * (N + 2 * plan.margins[j + 1])
    return bank, chain


DWT1_SHAPE, DWT1_N, DWT1_LEVEL = (32, 64), 2500, 5


def dwt_cfg1(steps, warmup, dev, cpu):
    """wavedec(x, 'db4', 'symmetric', 5) -> waverec, forward plus
    backward, x fp32 (32, 64, 2500)."""
    import pytorch_morlet_fdwt_amd as fdwt
    x = torch.randn(*DWT1_SHAPE, DWT1_N, generator=torch.Generator().manual_seed(0))
    xd = x.to(dev).requires_grad_()
    with torch.no_grad():  # the output shape only: no autograd graph is kept
        y0 = fdwt.waverec(fdwt.wavedec(xd, "db4", "symmetric", DWT1_LEVEL), "db4", "symmetric")
    gy = torch.randn(y0.shape, generator=torch.Generator().manual_seed(1)).to(dev)

    def step():
        y = fdwt.waverec(fdwt.wavedec(xd, "db4", "symmetric", DWT1_LEVEL), "db4", "symmetric")
        torch.autograd.grad(y, xd, gy)

    ms = _timed(step, steps, warmup)
    gms = _graph_timed(step, steps)
    R = DWT1_SHAPE[0] * DWT1_SHAPE[1]
    lens = coeff_lengths(DWT1_N, 8, "symmetric", DWT1_LEVEL)
    C = sum(lens) + lens[-1]
    m = y0.shape[-1]
    byts = 4 * R * (2 * DWT1_N + 2 * m + 4 * C)
    out = {"metric": "wavedec+waverec fwd+bwd GB/s (algorithmic HBM bytes / step time)",
           "value": byts / (ms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": ms,
           "samples_per_s": R * DWT1_N / (ms * 1e-3),
           "config": {"workload": "BASELINE configs[0]: db4, symmetric, level 5, x fp32 "
                                  "(32,64,2500), waverec(wavedec(x)) fwd+bwd"},
           "graph": {"ms_per_step": gms, "value": byts / (gms * 1e-3) / 1e9,
                     "note": "the same step captured once in a HIP graph (torch.cuda.graph) "
                             "and replayed: kernel time without the host's launch work"},
           "roofline": {"bound": "hbm", "achieved": byts / (ms * 1e-3) / 1e9,
                        "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                        "frac": byts / (ms * 1e-3) / HBM_PEAK, "alg_bytes": byts}}
    if cpu:
        from oracle import dwt as O
        rows = R  # the whole workload
        xs = x.reshape(R, DWT1_N)[:rows].contiguous()
        gys = gy.cpu().reshape(R, -1)[:rows].contiguous()

        def run():
            xx = xs.clone().requires_grad_()
            y = O.waverec(O.wavedec(xx, "db4", "symmetric", DWT1_LEVEL), "db4", "symmetric")
            torch.autograd.grad(y, xx, gys)

        t, threads = _cpu_median(run)
        out["cpu_baseline"] = {
            "value": 4 * rows * (2 * DWT1_N + 2 * m + 4 * C) / t / 1e9, "unit": "GB/s",
            "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{rows} of {R} rows, fp32, median of 3 after 1 warm-up ({t:.3f} s)"}
    return out


CWT3_SHAPE, CWT3_N, CWT3_FS = (32, 64), 2500, 250.0


def cwt3_signal(shape, n, gen):
    t = torch.arange(n, dtype=torch.float32)
    tone = sum(torch.sin(2 * torch.pi * f * t / CWT3_FS) for f in (6.0, 10.0, 18.0, 30.0))
    return torch.randn(*shape, n, generator=gen) + tone


def cwt_cfg3(steps, warmup, dev, cpu):
    """fast Morlet CWT, 40 centre frequencies logspace(-0.3, 2) Hz at
    fs = 250, w0 = 6, truncate = 4, l2 norm, learnable frequencies and w0; forward (complex64
    scalogram (32, 64, 40, 2500)) plus backward on a random-normal upstream gradient."""
    import pytorch_morlet_fdwt_amd as fdwt
    freqs = torch.logspace(-0.3, 2, 40).tolist()
    torch.manual_seed(2)
    m = fdwt.CWT1D(freqs=freqs, fs=CWT3_FS, w0=6.0, truncate=4.0, norm="l2", learnable=True,
                   learnable_w0=True).to(dev)
    x = cwt3_signal(CWT3_SHAPE, CWT3_N, torch.Generator().manual_seed(0))
    xd = x.to(dev).requires_grad_()
    S = m.plan.num_scales
    gen = torch.Generator(device=dev).manual_seed(1)
    gy = torch.view_as_complex(torch.randn(*CWT3_SHAPE, S, CWT3_N, 2, generator=gen, device=dev))
    params = [xd] + list(m.parameters())

    def step():
        y = m(xd)
        torch.autograd.grad(y, params, gy)

    ms = _timed(step, steps, warmup)
    R = CWT3_SHAPE[0] * CWT3_SHAPE[1]
    bank, chain = bank_chain_flops(m.plan, R, CWT3_N)
    fl = 3 * bank + 2 * chain  # forward, grad-x and grad-h of the bank; chain and its transpose
    byts = 4 * R * CWT3_N * 3 + 8 * R * S * CWT3_N * 2  # x twice, gx; W written, gW read
    s = ms * 1e-3
    out = {"metric": "Morlet CWT fwd+bwd samples/s (R*N per step)",
           "value": R * CWT3_N / s, "unit": "samples/s", "ms_per_step": ms,
           "gbps_alg": byts / s / 1e9, "frac_hbm_peak": byts / s / HBM_PEAK,
           "config": {"workload": "BASELINE configs[2]: fast Morlet CWT, 40 freqs "
                                  "logspace(-0.3,2) Hz, fs 250, w0 6, truncate 4, l2, learnable "
                                  "freqs and w0, x fp32 (32,64,2500) N(0,1) + 6/10/18/30 Hz",
                      "octaves": m.plan.n_octaves},
           "roofline": {"bound": "valu", "achieved": fl / s / 1e12, "peak": FP32_PEAK / 1e12,
                        "unit": "TFLOP/s", "frac": fl / s / FP32_PEAK, "alg_flops": fl,
                        "alg_bytes": byts}}
    if cpu:
        from oracle import cwt as O
        rows = 64
        plan = O.Plan(m.plan.scales, w0=6.0, truncate=4.0, norm="l2", support_margin=1.25)
        xs = x.reshape(R, CWT3_N)[:rows].contiguous()
        ls = m.log_scales.detach().cpu().clone().requires_grad_()
        w0 = torch.tensor(6.0, requires_grad=True)
        g = torch.view_as_complex(torch.randn(rows, S, CWT3_N, 2,
                                              generator=torch.Generator().manual_seed(1)))

        def run():
            xx = xs.clone().requires_grad_()
            y = O.apply_plan(xx, plan, plan.filters(ls.double().exp(), w0.double(),
                                                    torch.float32))
            torch.autograd.grad(y, [xx, ls, w0], g)

        t, threads = _cpu_median(run)
        out["cpu_baseline"] = {"value": rows * CWT3_N / t, "unit": "samples/s",
                               "cores": threads, "kind": "port", "cpu_model": cpu_model(),
                               "sample": f"{rows} of {R} rows, fp32, median of 3 after 1 "
                                         f"warm-up ({t:.3f} s)"}
    return out


MIX4_SHAPE, MIX4_DIM = (8, 4096, 256), 256


def token_mixer_cfg4(steps, warmup, dev, cpu):
    """MorletTokenMixer(dim=256, 16 freqs logspace(0, 1.8) Hz, fs=250),
    Xavier-initialised mixing weights, input (8, 4096, 256) fp32; forward plus backward."""
    import pytorch_morlet_fdwt_amd as fdwt
    freqs = torch.logspace(0, 1.8, 16).tolist()
    torch.manual_seed(2)
    m = fdwt.MorletTokenMixer(MIX4_DIM, freqs=freqs, fs=250.0)
    torch.nn.init.xavier_uniform_(m.mag_weight)
    torch.nn.init.xavier_uniform_(m.phase_weight)
    m = m.to(dev)
    x = torch.randn(*MIX4_SHAPE, generator=torch.Generator().manual_seed(0))
    xd = x.to(dev).requires_grad_()
    gy = torch.randn(*MIX4_SHAPE, generator=torch.Generator().manual_seed(1)).to(dev)
    params = [xd] + list(m.parameters())

    def step():
        y = m(xd)
        torch.autograd.grad(y, params, gy)

    ms = _timed(step, steps, warmup)
    B, N, D = MIX4_SHAPE
    R = B * D
    bank, chain = bank_chain_flops(m.cwt.plan, R, N)
    fl = 4 * bank + 3 * chain  # forward; backward recomputes W, then grad-x and grad-h
    s = ms * 1e-3
    out = {"metric": "MorletTokenMixer fwd+bwd tokens/s (B*L per step)",
           "value": B * N / s, "unit": "tokens/s", "ms_per_step": ms,
           "config": {"workload": "BASELINE configs[3]: MorletTokenMixer dim 256, 16 freqs "
                                  "logspace(0,1.8) Hz, fs 250, Xavier mixing weights, x fp32 "
                                  "(8,4096,256), out_proj included"},
           "roofline": {"bound": "valu", "achieved": fl / s / 1e12, "peak": FP32_PEAK / 1e12,
                        "unit": "TFLOP/s", "frac": fl / s / FP32_PEAK, "alg_flops": fl}}
    if cpu:
        from oracle import cwt as O
        p = m.cwt.plan
        plan = O.Plan(p.scales, support_margin=1.25)
        rows = 64
        xs = x[:1, :, :rows].contiguous()  # batch 1, `rows` of the 256 feature rows
        ls = m.cwt.log_scales.detach().cpu().clone().requires_grad_()
        a = m.mag_weight.detach().cpu()[:rows].clone().requires_grad_()
        b = m.phase_weight.detach().cpu()[:rows].clone().requires_grad_()
        bias = m.bias.detach().cpu()[:rows].clone().requires_grad_()
        g = gy.cpu()[:1, :, :rows]

        def run():
            xx = xs.clone().requires_grad_()
            y = O.token_mixer(xx, plan, plan.filters(ls.double().exp(), 6.0, torch.float32),
                              a, b, bias)
            torch.autograd.grad(y, [xx, ls, a, b, bias], g)

        t, threads = _cpu_median(run)
        out["cpu_baseline"] = {"value": N * rows / D / t, "unit": "tokens/s",
                               "cores": threads, "kind": "port", "cpu_model": cpu_model(),
                               "sample": f"batch 1 of {B}, {rows} of {D} feature rows (tokens "
                                         f"counted pro rata), no out_proj, fp32, median of 3 "
                                         f"after 1 warm-up ({t:.3f} s)"}
    return out


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
    ap.add_argument("--no-legs", action="store_true",
                    help="skip the configs[0], configs[2] and configs[3] legs")
    ap.add_argument("--cpu-rows", type=int, default=192)
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

    # the same step captured once in a HIP graph and replayed: its 80 dependent launches
    # without the host's launch work between them (reported beside the eager value)
    gms = _graph_timed(lambda: step_gpu(fdwt, data, grads), a.steps)
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
        "graph": {"ms_per_step": gms, "value": total / (gms * 1e-3) / 1e9,
                  "note": "the same 20-combination step captured once in a HIP graph "
                          "(torch.cuda.graph) and replayed: kernel time without the host's "
                          "launch work"},
    }
    if not a.no_attention:
        att = attention_gpu(max(3, a.steps // 2), a.warmup, dev)
        att["bf16_mode"] = bf16_mode(attention_gpu, max(3, a.steps // 2), a.warmup, dev)
        if not a.no_cpu_baseline:
            att["cpu_baseline"] = attention_cpu()
        line["morlet_attention"] = att
        cmix = attention_gpu(max(3, a.steps // 2), a.warmup, dev, channel_mix=True)
        if not a.no_cpu_baseline:
            cmix["cpu_baseline"] = attention_cpu(channel_mix=True)
        line["channel_mix_attention"] = cmix
    if not a.no_legs:
        cpu = not a.no_cpu_baseline
        k = max(3, a.steps // 2)
        line["cwt_cfg3"] = cwt_cfg3(k, a.warmup, dev, cpu)
        line["token_mixer_cfg4"] = token_mixer_cfg4(k, a.warmup, dev, cpu)
        line["dwt_cfg1"] = dwt_cfg1(k, a.warmup, dev, cpu)
        scaled = attention_gpu(2, 1, dev, ATT_SCALED)
        scaled["bf16_mode"] = bf16_mode(attention_gpu, 2, 1, dev, ATT_SCALED)
        scaled["cpu_baseline"] = None  # the CPU oracle needs minutes per step at this size
        line["morlet_attention_scaled"] = scaled
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(a.cpu_rows)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
