#!/usr/bin/env python3
"""Throughput of the fused CLIP / LiT contrastive loss (forward + backward) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--no-cpu]

A step is one ``loss = module(a, b); loss.backward()`` through the drop-in
``nn.Module`` on synthetic inputs already resident in HBM.  The default
workload is the headline configuration (CLIP, N=32768, D=1152, fp32,
normalized_inputs=False, T=0.07); ``--config`` selects another row of the
benchmark table for exploration.  Rank 0 prints ONE JSON line:

* ``value``: whole-job TFLOP/s, algorithmic flop 8 N^2 D (CLIP) / 6 N^2 D
  (LiT) per step (the backward counts the similarity recompute) over the
  wall-clock of K timed steps;
* ``roofline``: the dominant kernel's algorithmic flop per launch over its
  average launch time, measured with HIP events on the stream the library
  launches on (torch's current stream), against the dense MFMA peak of the
  input dtype;
* ``cpu_baseline``: the dense PyTorch loss (fp32) on the host cores at the
  same workload (same N, D and generator; a smaller N only with
  ``--cpu-n``), timed forward and backward, reported as the flop the dense
  path performs (6 N^2 D for CLIP: logits, then the two gradient products;
  4 N^2 D for LiT) per second, with the core count and CPU model;
* ``configs``: every benchmark configuration (1-5) timed for a few steps
  through the same module (the headline's row repeats its numbers), with
  forward / backward / step ms, TFLOP/s, fraction of the input dtype's MFMA
  peak and peak extra HBM bytes (``--no-table`` skips the other four).

``--precision high`` runs fp32 inputs under
``torch.set_float32_matmul_precision("high")``: the products are formed from
bf16 terms (hi*hi + lo*hi + hi*lo) on the bf16 MFMA.  ``dtype`` is then
"bf16x3", ``value`` stays in algorithmic (fp32-equivalent) flop, and the
roofline counts the three MFMA products per algorithmic one against the bf16
peak.  ``--precision medium`` multiplies bf16-rounded values ("bf16").  The
default, "highest", is IEEE fp32 on the fp32 MFMA.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "CLIP fwd+bwd ms & TFLOP/s (% MFMA peak) at N=32768 D=1152, 1 MI355X"
# MI355X published dense MFMA peaks (256 CUs at 2.4 GHz), TFLOP/s.
PEAK_TFLOPS = {"f32": 157.3, "bf16": 2516.6, "f16": 2516.6}
TORCH_DTYPE = {"f32": "float32", "bf16": "bfloat16", "f16": "float16"}

# config -> (mode, n, d, dtype, normalized_inputs, temperature, generator, CPU baseline n)
# (the CPU baseline runs dense at the configuration's own N up to 32768; the
# 4.3 GB logits of N = 32768 take about 10 s per fwd+bwd on 16 host threads)
CONFIGS = {
    1: ("clip", 1024, 512, "f32", False, 0.07, "randn", 1024),
    2: ("clip", 32768, 1152, "f32", False, 0.07, "randn", 32768),
    3: ("lit", 32768, 1152, "f32", False, 0.07, "randn", 32768),
    4: ("clip", 65536, 768, "bf16", True, 0.07, "correlated", 32768),
    5: ("clip", 262144, 1152, "bf16", True, 0.05, "correlated", 32768),
}
# steps, warm-up steps of each configuration in the table (configuration 1:
# a step is ~0.1 ms of host-bound work, so 300 of them, 30 ms, for a stable
# mean)
TABLE_STEPS = {1: (300, 20), 2: (5, 2), 3: (5, 2), 4: (5, 2), 5: (3, 1)}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(n, d, gen, seed=0):
    """Seeded host generator (bitwise reproducible), fp32 math."""
    import torch
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(seed)
    if gen == "randn":
        a = torch.randn(n, d, generator=g)
        b = torch.randn(n, d, generator=g)
    else:
        a = F.normalize(torch.randn(n, d, generator=g), dim=1)
        b = F.normalize(a + 0.5 * torch.randn(n, d, generator=g), dim=1)
    return a, b


def algo_flop(mode, n, d):
    return (8.0 if mode == "clip" else 6.0) * n * n * d


def time_stage(fn, reps, stream):
    """Average launch time (ms) of fn() over reps, HIP events on `stream`."""
    import torch
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for s, e in ev:
        s.record(stream)
        fn()
        e.record(stream)
    torch.cuda.synchronize()
    return statistics.mean(s.elapsed_time(e) for s, e in ev)


def grad_step_flop(n, d, bs, nb, sides):
    """Algorithmic flop of each backward pipeline step t = 0..nb: step t
    recomputes the similarity blocks of diagonal t (2 d per pair) and
    contracts diagonal t-1 (2 d per pair and side)."""
    rows = [min(bs, n - i * bs) for i in range(nb)]
    pairs = [sum(rows[i] * rows[(i + s) % nb] for i in range(nb)) for s in range(nb)]
    out = []
    for t in range(nb + 1):
        f = 2.0 * d * pairs[t] if t < nb else 0.0
        if t >= 1:
            f += sides * 2.0 * d * pairs[t - 1]
        out.append(f)
    return out


def kernel_leg(x, y, mode, dtc, normalize, temperature, reps):
    """Times each C-ABI stage of the path on its own (same inputs, same stream);
    dtc is the C-ABI dtype code.

    Returns {stage: (avg ms per launch, launches per step, algorithmic flop per launch)}."""
    import torch
    from memoryefficientclip_amd import _lib
    lib = _lib.load()
    n, d = x.shape
    m = _lib.MODE_CLIP if mode == "clip" else _lib.MODE_LIT
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    ws = torch.empty(lib.mec_workspace_floats_for(n, d, dtc), device=x.device)
    loss = torch.empty((), device=x.device)
    nbytes = lib.mec_grad_scratch_bytes(n, d, dtc)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    acc_x = torch.empty(n, d, device=x.device)
    acc_y = torch.empty(n, d, device=x.device) if m == _lib.MODE_CLIP else None
    out_x = torch.empty(n, d, dtype=x.dtype, device=x.device)
    out_y = torch.empty(n, d, dtype=x.dtype, device=x.device) if acc_y is not None else None
    pa = acc_y.data_ptr() if acc_y is not None else None
    X, Y = x.data_ptr(), y.data_ptr()
    norm = int(normalize)
    bs, nb = _lib.grad_blocking(n, d, dtc)
    sides = 2 if m == _lib.MODE_CLIP else 1

    def prepass():
        _lib.call("mec_prepass", X, d, Y, d, n, d, dtc, norm, ws.data_ptr(), sp)

    def sumexp():
        _lib.call("mec_sumexp", X, d, Y, d, n, d, dtc, m, norm, temperature, ws.data_ptr(), sp)

    def finalize():
        _lib.call("mec_finalize", n, m, temperature, ws.data_ptr(), loss.data_ptr(), sp)

    def grad_step(t):
        _lib.call("mec_grad_step", X, d, Y, d, n, d, dtc, m, norm, temperature, ws.data_ptr(), t,
                  scratch.data_ptr(), nbytes, acc_x.data_ptr(), pa, sp)

    def postpass():
        # the fp32 accumulators are converted into separate outputs so repeated calls stay valid
        _lib.call("mec_postpass", X, d, Y, d, n, d, dtc, m, norm, 1.0 / temperature, ws.data_ptr(), None,
                  acc_x.data_ptr(), pa, out_x.data_ptr(), None if out_y is None else out_y.data_ptr(), sp)

    prepass()
    sumexp()
    finalize()
    torch.cuda.synchronize()
    res = {}
    res["prepass"] = (time_stage(prepass, reps, stream), 1, 0.0)
    prepass()
    res["sumexp"] = (time_stage(sumexp, reps, stream), 1, 2.0 * n * n * d)
    prepass()
    sumexp()
    res["finalize"] = (time_stage(finalize, reps, stream), 1, 0.0)
    # every launch of the backward pipeline, in order, reps times
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(nb + 1)]
          for _ in range(reps)]
    for r in range(reps):
        for t in range(nb + 1):
            ev[r][t][0].record(stream)
            grad_step(t)
            ev[r][t][1].record(stream)
    torch.cuda.synchronize()
    per_step = [statistics.mean(ev[r][t][0].elapsed_time(ev[r][t][1]) for r in range(reps)) for t in range(nb + 1)]
    flops = grad_step_flop(n, d, bs, nb, sides)
    res["grad_step"] = (statistics.mean(per_step), nb + 1, sum(flops) / (nb + 1))
    res["postpass"] = (time_stage(postpass, reps, stream), sides, 0.0)
    return res, {"block_rows": bs, "num_blocks": nb, "step_ms": [round(v, 4) for v in per_step]}


def measured_traffic(workload, kernels):
    """HBM bytes of one launch of each of `kernels` at `workload`, summed, from
    the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summaries
    (profiles/traffic_<workload>.md, machine-readable copy in
    profiles/traffic.json), or None if not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)[workload]
        return sum(t[k]["bytes"] for k in kernels)
    except (OSError, KeyError, ValueError):
        return None


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def dense_flop(mode, n, d):
    """Flop the dense PyTorch path performs: the logits (2 N^2 D) and, in the
    backward, dX = G Y (2 N^2 D) and for CLIP dY = G^T X (2 N^2 D)."""
    return (6.0 if mode == "clip" else 4.0) * n * n * d


def cpu_baseline(mode, d, dt, normalized, temperature, gen, n_cpu, runs=3):
    """Dense PyTorch loss on the host cores at (n_cpu, d) of the workload:
    one warm-up, then the median of `runs` timed fwd+bwd steps."""
    import torch
    from oracle.cpu_baseline import dense_step
    a, b = make_inputs(n_cpu, d, gen, seed=0)
    if dt != "f32":
        tdt = getattr(torch, TORCH_DTYPE[dt])
        a, b = a.to(tdt).float(), b.to(tdt).float()
    dense_step(a, b, temperature, mode == "lit", normalized)  # warm-up
    times, fwd, bwd = [], [], []
    for _ in range(runs):
        t = {}
        t0 = time.perf_counter()
        dense_step(a, b, temperature, mode == "lit", normalized, times=t)
        times.append(time.perf_counter() - t0)
        fwd.append(t["fwd"])
        bwd.append(t["bwd"])
        log(f"bench: CPU baseline step {len(times)}: {times[-1] * 1e3:.0f} ms")
    med = statistics.median(times)
    return {
        "value": round(dense_flop(mode, n_cpu, d) / med / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"dense fp32 PyTorch {mode.upper()} fwd+bwd (F.normalize, logits, cross_entropy, autograd) "
                   f"at N={n_cpu}, D={d}, same generator; 1 warm-up, median of {runs} runs; value counts the "
                   f"{'6' if mode == 'clip' else '4'}*N^2*D flop the dense path performs"),
        "n": n_cpu,
        "ms_per_step": round(med * 1e3, 1),
        "fwd_ms": round(statistics.median(fwd) * 1e3, 1),
        "bwd_ms": round(statistics.median(bwd) * 1e3, 1),
        "value_8n2d": round(algo_flop(mode, n_cpu, d) / med / 1e12, 4),
        "threads": torch.get_num_threads(),
        "os_cpu_count": os.cpu_count(),
        "cpu_model": cpu_model(),
    }


def measure(cfg, dt, steps, warmup, with_events=True, calling_thread=False):
    """Times `steps` fwd+bwd steps of configuration `cfg` (input dtype dt)
    through the drop-in module, after `warmup` steps.  Returns (row, a, b)
    with the device inputs a, b.  calling_thread: the timed loop runs under
    torch.autograd.set_multithreading_enabled(False), so that loss.backward()
    runs the backward on the calling thread instead of handing it to the
    autograd engine's device thread (a diagnostic of host overhead)."""
    import torch
    from memoryefficientclip_amd import MemoryEfficientCLIPLoss, MemoryEfficientLiTLoss
    mode, n, d, _, normalized, temperature, gen, _ = CONFIGS[cfg]
    dev = torch.device("cuda:0")
    tdtype = getattr(torch, TORCH_DTYPE[dt])
    a_h, b_h = make_inputs(n, d, gen, seed=0)
    a = a_h.to(dev, tdtype).requires_grad_(True)
    b = b_h.to(dev, tdtype).requires_grad_(mode == "clip")
    del a_h, b_h
    module = (MemoryEfficientCLIPLoss if mode == "clip" else MemoryEfficientLiTLoss)(temperature, normalized)

    def step(evs=None):
        if evs is not None:
            evs[0].record()
        loss = module(a, b)
        if evs is not None:
            evs[1].record()
        loss.backward()
        if evs is not None:
            evs[2].record()
        a.grad = None
        b.grad = None
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    loss = step()
    torch.cuda.synchronize()
    peak_extra = torch.cuda.max_memory_allocated(dev) - base
    loss_val = float(loss.detach())
    # the timed loop records no events (host work that is not the step's own);
    # the forward / backward split comes from a separate loop of evented steps
    with torch.autograd.set_multithreading_enabled(not calling_thread):
        for _ in range(warmup if calling_thread else 0):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms = wall * 1e3 / steps
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(min(steps, 10))]
    if with_events:
        for e in evs:
            step(e)
        torch.cuda.synchronize()
    row = {"config": cfg, "workload": f"{mode}_loss_fwd_bwd", "n": n, "d": d, "dtype": dt,
           "normalized_inputs": normalized, "temperature": temperature, "steps": steps,
           "ms_per_step": round(ms, 4),
           "tflops": round(algo_flop(mode, n, d) / (ms * 1e-3) / 1e12, 3),
           "peak_extra_hbm_bytes": int(peak_extra), "loss": loss_val}
    if with_events:
        row["fwd_ms"] = round(statistics.median(e[0].elapsed_time(e[1]) for e in evs), 4)
        row["bwd_ms"] = round(statistics.median(e[1].elapsed_time(e[2]) for e in evs), 4)
    return row, a, b


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--dtype", choices=sorted(PEAK_TFLOPS), default=None,
                    help="input dtype instead of the config's own (e.g. --config 4 --dtype f16)")
    ap.add_argument("--precision", choices=["highest", "high", "medium"], default="highest",
                    help="float32 matmul precision for fp32 inputs: highest = IEEE fp32 MFMA, "
                         "high = three bf16 MFMA products per fp32 product (bf16x3), medium = bf16 products")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-n", type=int, default=0,
                    help="N of the CPU baseline sample (default: the configuration's own N, at most 32768)")
    ap.add_argument("--no-table", action="store_true", help="skip timing the other benchmark configurations")
    ap.add_argument("--no-alt", action="store_true",
                    help="skip the fp32 'high' precision side leg (e.g. for per-kernel profiles of the IEEE path)")
    ap.add_argument("--kernel-reps", type=int, default=0, help="launches per stage in the kernel leg (default: steps)")
    ap.add_argument("--probe", choices=["copy", "gemm"], default=None,
                    help="copy: only run 5 plain device copies of 1 GiB (calibrates the rocprofv3 byte counters); "
                         "gemm: only time the vendor library's bf16 GEMM (torch.matmul, hipBLASLt) at the "
                         "contraction and similarity shapes (calibrates the MFMA rate)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs the whole N x N loss on one GPU (no collectives); "
              f"--gpus {args.gpus} / WORLD_SIZE={world} is not supported, run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (torch.cuda.is_available() is False)", file=sys.stderr)
        sys.exit(1)
    if args.probe == "copy":
        src = torch.ones(1 << 28, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"probe": "copy", "bytes_read_per_copy": src.numel() * 4,
                          "bytes_written_per_copy": dst.numel() * 4}), flush=True)
        return
    if args.probe == "gemm":
        res = []
        for m, nn, k in [(16384, 768, 16384), (16384, 2304, 16384), (16384, 16384, 4096), (32768, 32768, 768)]:
            a = torch.randn(m, k, device="cuda:0", dtype=torch.bfloat16)
            b = torch.randn(k, nn, device="cuda:0", dtype=torch.bfloat16)
            for _ in range(2):
                c = a @ b
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(6):
                c = a @ b
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / 6
            res.append({"m": m, "n": nn, "k": k, "ms": round(ms, 4), "tflops": round(2 * m * nn * k / ms / 1e9, 1)})
            log(f"bench: probe gemm bf16 {m}x{nn}x{k}: {ms:.3f} ms, {res[-1]['tflops']} TFLOP/s")
            del a, b, c
        print(json.dumps({"probe": "gemm", "dtype": "bf16", "library": "torch.matmul (hipBLASLt)", "shapes": res}),
              flush=True)
        return
    from memoryefficientclip_amd import MemoryEfficientCLIPLoss, MemoryEfficientLiTLoss, _lib
    _lib.load()  # fail loudly if the HIP library is missing

    mode, n, d, dt, normalized, temperature, gen, n_cpu = CONFIGS[args.config]
    dt = args.dtype or dt
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    # arithmetic: the input dtype's MFMA, or for fp32 inputs below "highest"
    # precision bf16x3 (three bf16 products per fp32 product) or bf16
    x3 = args.precision == "high"
    lowp = args.precision != "highest"
    if lowp and dt != "f32":
        print(f"bench.py: --precision {args.precision} applies to fp32 inputs only", file=sys.stderr)
        sys.exit(2)
    torch.set_float32_matmul_precision(args.precision)
    arith = "bf16x3" if x3 else "bf16" if lowp else dt
    mfma_per_flop = 3 if x3 else 1
    peak = PEAK_TFLOPS["bf16" if lowp else dt]
    dtc = {"f32": _lib.DTYPE_F32, "bf16": _lib.DTYPE_BF16, "f16": _lib.DTYPE_F16}[dt]
    if lowp:
        dtc = _lib.DTYPE_F32_BF16X3 if x3 else _lib.DTYPE_F32_BF16
    log(f"bench: config {args.config} {mode} n={n} d={d} {dt} normalized_inputs={normalized} T={temperature}"
        f" arithmetic={arith}")
    head, a, b = measure(args.config, dt, args.steps, args.warmup)
    ms, fwd_ms, bwd_ms = head["ms_per_step"], head["fwd_ms"], head["bwd_ms"]
    peak_extra, loss_val = head["peak_extra_hbm_bytes"], head["loss"]
    flop = algo_flop(mode, n, d)
    tflops = flop / (ms * 1e-3) / 1e12
    log(f"bench: {args.steps} steps, {ms:.3f} ms/step (fwd {fwd_ms:.3f}, bwd {bwd_ms:.3f}), {tflops:.2f} TFLOP/s, "
        f"loss {loss_val:.6f}")

    # fp32 inputs at "highest" precision: the same steps once more under "high"
    # (bf16x3), reported beside the IEEE line (not as its value)
    alt = None
    if dt == "f32" and not lowp and not args.no_alt:
        torch.set_float32_matmul_precision("high")
        hi, _, _ = measure(args.config, dt, args.steps, args.warmup, with_events=False)
        torch.set_float32_matmul_precision("highest")
        ms_hi = hi["ms_per_step"]
        alt = {"float32_matmul_precision": "high", "dtype": "bf16x3", "ms_per_step": round(ms_hi, 4),
               "value": round(flop / (ms_hi * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
               "frac_of_bf16_peak": round(3 * flop / (ms_hi * 1e-3) / 1e12 / PEAK_TFLOPS["bf16"], 4)}
        log(f"bench: float32 matmul precision high (bf16x3): {ms_hi:.3f} ms/step, {alt['value']:.2f} TFLOP/s")

    # kernel leg: per-stage launch times on the library's stream
    x = a.detach()
    y = b.detach()
    reps = args.kernel_reps or args.steps
    stages, blocking = kernel_leg(x, y, mode, dtc, not normalized, temperature, reps)
    for k, (t, nl, fl) in stages.items():
        log(f"bench: stage {k:9s} {t:9.3f} ms x {nl:3d}" + (f"  {fl / (t * 1e-3) / 1e12:8.2f} TFLOP/s" if fl else ""))
    log(f"bench: backward blocking {blocking}")
    # dominant kernel: the backward pipeline step, nb + 1 launches of mec_grad_step per
    # step, about 3/4 of the step's flop: k_grad_step (fp32: gradient-matrix tiles and
    # contractions in one kernel; 16-bit: the gradient-matrix tiles, chained in
    # k_grad_g_chain for normalized inputs, with the contractions in k_grad_contract
    # before them)
    # (bf16x3: MFMA flop = 3 x algorithmic flop, against the bf16 peak)
    t_k, nl_k, f_k = stages["grad_step"]
    achieved = mfma_per_flop * f_k / (t_k * 1e-3) / 1e12
    # (16-bit data with normalized inputs: the gradient-matrix tiles run chained, in k_grad_g_chain)
    gkern = "k_grad_g_chain" if (normalized and not x3) else "k_grad_step"
    kernels = ["k_grad_step"] if arith == "f32" else ["k_grad_contract", gkern]
    traffic = measured_traffic(f"{mode}_n{n}_d{d}_{arith}", kernels)
    if traffic is not None and len(kernels) > 1:
        # each kernel runs in nb of the nb + 1 pipeline launches
        nbk = blocking["num_blocks"]
        traffic = int(traffic * nbk / (nbk + 1))
    roofline = {"bound": "mfma", "kernel": "+".join(kernels), "achieved": round(achieved, 3), "peak": peak,
                "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic,
                "launch_ms": round(t_k, 4), "flop_per_launch": mfma_per_flop * f_k, "launches_per_step": nl_k}
    t_f, _, f_f = stages["sumexp"]
    # (bf16/fp16 products on inputs already normalized: the forward runs the
    # chained block walk, k_sumexp_det, with its O(N) reduction)
    fkern = "k_sumexp_det+k_det_reduce" if (arith != "f32" and normalized) else "k_sumexp"
    roofline_fwd = {"kernel": fkern, "achieved": round(mfma_per_flop * f_f / (t_f * 1e-3) / 1e12, 3),
                    "frac": round(mfma_per_flop * f_f / (t_f * 1e-3) / 1e12 / peak, 4), "launch_ms": round(t_f, 4),
                    "flop_per_launch": mfma_per_flop * f_f}

    del a, b
    torch.cuda.empty_cache()

    # every benchmark configuration (the headline's own row from the run above)
    table = None
    if not args.no_table and args.precision == "highest":
        table = []
        for cfg in sorted(CONFIGS):
            if cfg == args.config and dt == CONFIGS[cfg][3]:
                row = dict(head)
            else:
                st, wu = TABLE_STEPS[cfg]
                row, ta, tb = measure(cfg, CONFIGS[cfg][3], st, wu)
                del ta, tb
                torch.cuda.empty_cache()
            row["frac_of_peak"] = round(row["tflops"] / PEAK_TFLOPS[row["dtype"]], 4)
            if CONFIGS[cfg][1] <= 4096:
                # small N: the host, not the GPU, sets the step; the same loop with
                # the backward on the calling thread shows how much of it is the
                # autograd engine's hand-off to its device thread
                ct, ta, tb = measure(cfg, CONFIGS[cfg][3], *TABLE_STEPS[cfg], calling_thread=True)
                del ta, tb
                row["ms_per_step_backward_on_calling_thread"] = ct["ms_per_step"]
            table.append(row)
            log(f"bench: table config {cfg}: {row['ms_per_step']:.3f} ms/step (fwd {row['fwd_ms']:.3f}, "
                f"bwd {row['bwd_ms']:.3f}), {row['tflops']:.1f} TFLOP/s, {100 * row['frac_of_peak']:.1f}% of "
                f"{row['dtype']} peak, extra HBM {row['peak_extra_hbm_bytes'] / 1e9:.2f} GB")
            if "ms_per_step_backward_on_calling_thread" in row:
                log(f"bench: table config {cfg}, backward on the calling thread: "
                    f"{row['ms_per_step_backward_on_calling_thread']:.3f} ms/step")

    cpu = None
    if not args.no_cpu:
        n_cpu = args.cpu_n or n_cpu
        log(f"bench: CPU baseline at n={n_cpu} ...")
        cpu = cpu_baseline(mode, d, dt, normalized, temperature, gen, n_cpu)
        log(f"bench: CPU baseline {cpu['ms_per_step']} ms/step, {cpu['value']} TFLOP/s on {cpu['cores']} threads "
            f"({cpu['os_cpu_count']} CPUs, {cpu['cpu_model']})")

    out = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": arith,
        "data": "synthetic",
        "config": {"workload": f"{mode}_loss_fwd_bwd", "n": n, "d": d, "temperature": temperature,
                   "normalized_inputs": normalized, "input_dtype": dt, "float32_matmul_precision": args.precision,
                   "parallelism": "none (1 GPU)"},
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "frac_of_peak": round(mfma_per_flop * tflops / peak, 4),
        "peak_extra_hbm_bytes": int(peak_extra),
        "peak_extra_hbm_note": ("PyTorch allocator peak above the inputs during one step; it excludes the "
                                "library's resident 256 MiB no-allocation scratch array (one per GPU it runs on, "
                                "part of the code object)"),
        "loss": loss_val,
        "stages_ms": {k: round(v[0], 4) for k, v in stages.items()},
        "roofline": roofline,
        "roofline_forward": roofline_fwd,
        "backward_blocking": blocking,
        "precision_high": alt,
        "cpu_baseline": cpu,
        "configs": table,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
