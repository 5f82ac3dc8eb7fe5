#!/usr/bin/env python3
"""Benchmark of the Continuum Attention operator on one MI355X.

Workload: the isolated CA operator at
[B,H,T,D] = [2,16,2048,64] fp32, forward + backward, causal full context,
Q,K,V ~ N(0,1) with the op's own 1/sqrt(64) scale, log_gain = 0 (tau = 1),
upstream grad ~ N(0,1), seed 0.  One "step" is one forward + backward of the
operator with inputs already resident in HBM.

Prints ONE JSON line (rank 0).  `value` is the median fwd+bwd milliseconds
(lower is better) of uninstrumented steps.  Before the warm-up steps the same
operator step runs for --clock-warmup-s seconds (default 0.25) so that the
GPU clock has ramped up (line field `clock_warmup`).  `roofline` is for the dominant
kernel, from HIP events recorded around each kernel launch on the launch
stream during a second run of the same steps; `cpu_baseline` times the CPU
port of the reference's PyTorch CPU path (oracle/ca_cpu_port.py) on the same
workload in full (and on config 1).

Two more BASELINE workloads ride along on the same line (skip with
--no-models): `ca_s`, the CA-S decoder training step in tokens/s (config 4,
the metric's "CA-S tokens/s"), and `ca_p`, the small CA-P decoder step
(config 3); each reports its step time and the share spent in CA kernels.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 MFMA
PEAK_BF16_MFMA_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
LIMB_PRODUCTS = 6               # bf16 MFMA products per fp32 product (bf16x6)
SHAPE = (2, 16, 2048, 64)


def pairs(B, H, T):
    return B * H * T * (T + 1) // 2


# algorithmic flops per causal (query, key) pair, per kernel (D = head dim)
def kernel_flops_per_pair(D):
    return {"ca_fwd": 4 * D,        # S = QK^T, O = WV
            "ca_bwd_dkdv": 8 * D,   # S recompute, dP = dY V^T, dV = W^T dY, dK = dS^T Q
            "ca_bwd_dq": 2 * D}     # dQ = dS K


def _cpu_model():
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _time_port(P, shape, seed_order, reps):
    """Median forward and backward seconds of the CPU port on one shape."""
    import torch
    B, H, T, D = shape
    if seed_order:
        torch.manual_seed(0)  # manual_seed(0), then q, k, v, dY
        q, k, v, dy = (torch.randn(shape) for _ in range(4))
    else:
        g = torch.Generator().manual_seed(0)
        q, k, v, dy = (torch.randn(shape, generator=g) for _ in range(4))
    rho = torch.zeros(H)
    P.port_forward(q, k, v, rho, 128)  # warm-up
    P.port_backward(q, k, v, rho, dy, 128)
    fw, bw = [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        P.port_forward(q, k, v, rho, 128)
        t1 = time.perf_counter()
        P.port_backward(q, k, v, rho, dy, 128)
        t2 = time.perf_counter()
        fw.append(t1 - t0)
        bw.append(t2 - t1)
    return statistics.median(fw), statistics.median(bw)


def cpu_baseline(reps=3):
    """The reference's PyTorch CPU path (its restatement in
    oracle/ca_cpu_port.py, query_tile=128) timed on this host's cores at
    BASELINE config 2 in full, and at config 1."""
    import torch
    from oracle import ca_cpu_port as P
    affinity = len(os.sched_getaffinity(0))
    torch.set_num_threads(affinity)
    f2, b2 = _time_port(P, SHAPE, False, reps)
    f1, b1 = _time_port(P, (1, 2, 64, 16), True, 20)
    return {"value": round((f2 + b2) * 1e3, 1), "unit": "ms per fwd+bwd",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"BASELINE config 2 in full ([2,16,2048,64] fp32 fwd+bwd, seed 0, "
                       f"query_tile=128), median of {reps} after 1 warm-up"),
            "fwd_ms": round(f2 * 1e3, 1), "bwd_ms": round(b2 * 1e3, 1),
            "config1": {"shape": [1, 2, 64, 16], "fwd_ms": round(f1 * 1e3, 3),
                        "bwd_ms": round(b1 * 1e3, 3), "sample": "median of 20 after 1 warm-up"},
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(), "affinity": affinity,
            "torch_threads": torch.get_num_threads(),
            "note": "threads = the affinity set; the reference launcher's OMP_NUM_THREADS=2 "
                    "(cuda/run.sh:8) is overridden"}


def _time_steps(step, steps, warmup, first=0):
    """Runs `warmup` untimed and `steps` timed calls of step(i), i counting
    from `first`; returns (ms per step from HIP events on the current stream,
    the last step's output)."""
    import torch
    for i in range(warmup):
        step(first + i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        out = step(first + warmup + i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, out


def _clock_warmup(step, seconds):
    """Runs step(0) (synchronising every 10 calls) for `seconds` of wall time so
    that the GPU clock has ramped up; returns {"s": ..., "steps": ...}."""
    import torch
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            step(0)
        torch.cuda.synchronize()
        n += 10
    return {"s": round(time.perf_counter() - t0, 3), "steps": n}


def _ca_kernel_ms(ca, step, steps, first=0):
    """CA kernel ms per step of an instrumented run of `steps` calls (its
    per-kernel events do not load the timed steps)."""
    import torch
    ca.native.timing_enable(True)
    for i in range(steps):
        step(first + i)
    torch.cuda.synchronize()
    kt = ca.native.timing_read()
    ca.native.timing_enable(False)
    return sum(t for t, c in kt.values()) / steps


def _timed_steps(ca, step, steps, warmup):
    """(ms per step, CA kernel ms per step, last output) of step(i)."""
    ms, out = _time_steps(step, steps, warmup)
    return ms, _ca_kernel_ms(ca, step, steps, warmup + steps), out


def time_operator(ca, dev, q, k, v, rho, dy, steps, warmup, clock_warmup_s=0.0):
    """Forward + backward of the operator on resident inputs: median fwd, bwd
    and total ms of `steps` uninstrumented steps (HIP events on the current
    stream around each half), then the same steps with HIP events around every
    kernel launch on its stream (per-kernel times).

    `clock_warmup_s` > 0 first runs the same step for that many seconds of
    wall time, before the `warmup` steps: the GPU clock ramps up under load
    (medians of 20 steps of the [2,16,2048,64] step from a cold start read
    0.630, 0.557, 0.542, then a steady 0.537 ms), so with a handful of
    warm-up steps the timed steps would otherwise land on the ramp."""
    import torch
    q, k, v = (x.to(dev).requires_grad_(True) for x in (q, k, v))
    rho = rho.to(dev).requires_grad_(True)
    dy = dy.to(dev)
    B, H, T, D = q.shape

    def step():
        y = ca.continuum_attention(q, k, v, rho, 128)
        torch.autograd.grad(y, (q, k, v, rho), dy)
        return y

    clock = _clock_warmup(lambda i: step(), clock_warmup_s)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = []
    t_start = time.perf_counter()
    for _ in range(steps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        ev[0].record()
        y = ca.continuum_attention(q, k, v, rho, 128)
        ev[1].record()
        torch.autograd.grad(y, (q, k, v, rho), dy)
        ev[2].record()
        evs.append(ev)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    fwd = statistics.median(ev[0].elapsed_time(ev[1]) for ev in evs)
    bwd = statistics.median(ev[1].elapsed_time(ev[2]) for ev in evs)
    tot = statistics.median(ev[0].elapsed_time(ev[2]) for ev in evs)
    ca.native.timing_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kt = ca.native.timing_read()
    ca.native.timing_enable(False)
    P = pairs(B, H, T)
    fpp = kernel_flops_per_pair(D)
    per_kernel = {}
    for n, (t, c) in kt.items():
        if c:
            per_kernel[n] = {"avg_ms": round(t / c, 4), "launches": c}
            if n in fpp:
                # the kernel's algorithmic flops per step over its time per step
                per_kernel[n]["tflops"] = round(fpp[n] * P / (t / steps * 1e-3) / 1e12, 2)
    return {"fwd_ms": round(fwd, 4), "bwd_ms": round(bwd, 4), "total_ms": round(tot, 4),
            "fwd_tflops": round(4 * D * P / (fwd * 1e-3) / 1e12, 2),
            "bwd_tflops": round(10 * D * P / (bwd * 1e-3) / 1e12, 2),
            "tflops": round(14 * D * P / (tot * 1e-3) / 1e12, 2),
            "roofline_frac": round(14 * D * P / (tot * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
            "wall_s": round(wall, 3),
            "clock_warmup": clock,
            "kernels": per_kernel, "kt": kt}


def config5_inputs(T=8192):
    """[1,16,T,64]; heads 0-7 near-duplicate adjacent keys
    k_j = k_{j-1} + N(0, 1e-4^2) (delta ~ 1e-4, the Taylor branch), heads 8-15
    keys 4 N(0,1) (large delta); q, v, dY ~ N(0,1); seed 0."""
    import torch
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 16, T, 64, generator=g)
    k0 = torch.randn(8, 1, 64, generator=g)
    walk = torch.cumsum(torch.randn(8, T - 1, 64, generator=g) * 1e-4, 1)
    k = torch.cat([torch.cat([k0, k0 + walk], 1), 4.0 * torch.randn(8, T, 64, generator=g)], 0)[None]
    v = torch.randn(1, 16, T, 64, generator=g)
    dy = torch.randn(1, 16, T, 64, generator=g)
    return q, k.contiguous(), v, torch.zeros(16), dy


def operator_leg(ca, dev, name, shape, steps, warmup, clock_warmup_s=0.0):
    """One more operator shape on the same line: fwd, bwd, total ms and
    TFLOP/s (algorithmic: 4 D, 10 D, 14 D flops per causal pair)."""
    import torch
    B, H, T, D = shape
    if name == "config5":
        q, k, v, rho, dy = config5_inputs(T)
        inputs = ("BASELINE config 5: heads 0-7 k_j = k_{j-1} + N(0,1e-4^2), heads 8-15 "
                  "keys 4 N(0,1); q, v, dY ~ N(0,1), seed 0")
    else:
        g = torch.Generator().manual_seed(0)
        q, k, v, dy = (torch.randn(shape, generator=g) for _ in range(4))
        rho = torch.zeros(H)
        inputs = "q, k, v, dY ~ N(0,1), seed 0 (one CA-S layer's operator shape, fp32)"
    lib = ca.native.load()
    ws_f, ws_b = lib.ca_fwd_workspace_bytes(*shape), lib.ca_bwd_workspace_bytes(*shape)
    prev = ca.ops.workspace_cap()
    ca.ops.set_workspace_cap(0)
    full_b = lib.ca_bwd_workspace_bytes(*shape)
    ca.ops.set_workspace_cap(prev)
    op = time_operator(ca, dev, q, k, v, rho, dy, steps, warmup, clock_warmup_s)
    op.pop("kt")
    op.update({"shape": list(shape), "inputs": inputs, "steps": steps, "warmup": warmup,
               "workspace_cap_bytes": prev, "fwd_workspace_bytes": ws_f,
               "bwd_workspace_bytes": ws_b, "bwd_workspace_unbounded_bytes": full_b,
               "bwd_passes_note": ("the backward runs in passes under the cap"
                                   if full_b > ws_b else "one backward pass")})
    torch.cuda.empty_cache()
    return op


def bench_ca_s(ca, dev, steps=20, warmup=5, clock_warmup_s=0.0):
    """one CA-S decoder training step (101,205,120 params,
    T=2048, batch 1, bf16 autocast with fp32 CA scores, AdamW + clip 1.0 as
    the library's fused HIP optimizer) on uniform-random bytes, random-init
    weights.  The timed step is decoder.GraphedTrainStep: forward and backward
    replayed as one HIP graph, then the eager clip + AdamW (the eager step
    issues ~270 launches from Python, and on a slow host its launch time
    exceeds its GPU time); the eager step's time and its CA kernel time are
    reported beside it."""
    import torch
    Dm = ca.decoder
    torch.manual_seed(0)
    cfg = Dm.ContinuumDecoderConfig()
    model = Dm.ContinuumDecoderLM(cfg).to(dev)
    nparams = Dm.count_parameters(model)["total"]
    opt = Dm.build_fused_adamw(model)
    g = torch.Generator().manual_seed(1)
    batches = [torch.randint(0, 256, (1, cfg.block_size), generator=g).to(dev) for _ in range(4)]
    eager_ms, ca_ms, _ = _timed_steps(ca, lambda i: Dm.train_step(model, opt, batches[i % 4]),
                                      steps, warmup)
    # the graph holds the gradient buffers from here on (no eager step after it)
    graphed = Dm.GraphedTrainStep(model, opt, batches[0])
    # the GPU idles while the graph is captured: ramp its clock up again
    clock = _clock_warmup(lambda i: graphed(batches[i % 4]), clock_warmup_s)
    ms, loss = _time_steps(lambda i: graphed(batches[i % 4]), steps, warmup)
    del graphed
    tokens = cfg.block_size
    res = {"metric": "CA-S tokens/s", "tokens_per_s": round(tokens / (ms * 1e-3), 1),
           "ms_per_step": round(ms, 3), "ca_kernels_ms_per_step": round(ca_ms, 3),
           "eager_ms_per_step": round(eager_ms, 3), "step": "GraphedTrainStep",
           "steps": steps, "warmup": warmup, "clock_warmup": clock, "params": nparams,
           "loss": round(float(loss), 4),
           "dtype": "bf16 autocast, f32 CA scores", "data": "synthetic uniform bytes",
           "config": {"workload": "CA-S decoder train step (BASELINE config 4)", "d_model": cfg.d_model,
                      "n_layers": cfg.n_layers, "n_heads": cfg.n_heads, "T": cfg.block_size,
                      "batch": 1, "optimizer": "AdamW lr 3e-4 wd 0.1 betas (.9,.95), clip 1.0 "
                                               "(HIP clip + AdamW, bf16 shadows of the Linear weights)"}}
    del model, opt
    torch.cuda.empty_cache()
    return res


def bench_ca_p(ca, dev, steps=30, warmup=10, clock_warmup_s=0.0):
    """small CA-P decoder (TinyLM backbone with 4 blocks,
    d 256, 4 heads, fixed tau 0.30, T=512, batch 16), one fp32 step on
    uniform-random bytes, random-init weights.  Timed as
    decoder.GraphedTrainStep (forward and backward replayed as one HIP graph,
    the clip + AdamW eager), with the eager step's time beside it."""
    import torch
    import torch.nn.functional as F
    A = ca.architecture
    torch.manual_seed(0)
    model = A.TinyLM(variant="P", backend="hip", seq_len=512, width=256, hidden=720, heads=4,
                     fixed_tau=0.30, layers=4).to(dev)
    opt = A.build_fused_adamw(model)
    g = torch.Generator().manual_seed(2)
    data = [torch.randint(0, 256, (16, 513), generator=g).to(dev) for _ in range(4)]
    # torch's plain fp32 GEMMs of this small model through rocBLAS ("cublas" on
    # ROCm): lower launch cost and faster kernels than hipBLASLt at these shapes
    # (3.54 against 3.77 ms/step measured)
    prev_blas = torch.backends.cuda.preferred_blas_library()
    torch.backends.cuda.preferred_blas_library("cublas")
    step_kind = "GraphedTrainStep"
    clock = None
    try:
        eager_ms, ca_ms, loss = _timed_steps(
            ca, lambda i: A.train_step(model, opt, data[i % 4][:, :-1], data[i % 4][:, 1:]), steps,
            warmup)
        ms = eager_ms
        # the same step replayed as one HIP graph (forward + backward), the
        # clip + AdamW eager after it; a capture the graph step refuses keeps
        # the eager time
        loss_fn = lambda m, x, t: F.cross_entropy(m(x).reshape(-1, 256), t.reshape(-1))
        try:
            graphed = ca.decoder.GraphedTrainStep(model, opt, (data[0][:, :-1], data[0][:, 1:]),
                                                  amp_dtype=None, loss_fn=loss_fn)
        except ValueError:
            step_kind = "eager"
        else:
            clock = _clock_warmup(lambda i: graphed(data[i % 4][:, :-1], data[i % 4][:, 1:]),
                                  clock_warmup_s)
            ms, loss = _time_steps(lambda i: graphed(data[i % 4][:, :-1], data[i % 4][:, 1:]),
                                   steps, warmup)
            del graphed
    finally:
        torch.backends.cuda.preferred_blas_library(prev_blas)
    tokens = 16 * 512
    res = {"metric": "CA-P tokens/s", "tokens_per_s": round(tokens / (ms * 1e-3), 1),
           "ms_per_step": round(ms, 3), "ca_kernels_ms_per_step": round(ca_ms, 3),
           "eager_ms_per_step": round(eager_ms, 3), "step": step_kind,
           "steps": steps, "warmup": warmup, "clock_warmup": clock, "params": A.parameters(model),
           "loss": round(float(loss), 4), "dtype": "f32", "data": "synthetic uniform bytes",
           "config": {"workload": "CA-P TinyLM train step (BASELINE config 3)", "layers": 4,
                      "width": 256, "heads": 4, "T": 512, "batch": 16, "fixed_tau": 0.30,
                      "optimizer": "AdamW lr 4e-4 wd 0.1 (gains 8x lr, no decay), clip 1.0 (HIP)",
                      "blas": "rocBLAS for torch's fp32 GEMMs"}}
    del model, opt
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20, help="untimed steps before the timed ones")
    ap.add_argument("--clock-warmup-s", type=float, default=0.25,
                    help="seconds of operator steps run before the warm-up steps so that the GPU "
                         "clock has ramped up (it takes ~60 steps of the [2,16,2048,64] operator "
                         "from a cold start: medians of 20 steps 0.630, 0.557, 0.542, then "
                         "0.537 ms); reported as `clock_warmup` on the line, 0 turns it off")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-models", action="store_true",
                    help="skip the CA-S (config 4) and CA-P (config 3) training-step legs")
    ap.add_argument("--no-extra-shapes", action="store_true",
                    help="skip the config-5 [1,16,8192,64] and CA-S layer [1,16,2048,64] "
                         "operator legs")
    ap.add_argument("--shape", default=None,
                    help="B,H,T,D of the operator leg (diagnostics; default is BASELINE config 2)")
    ap.add_argument("--only", choices=["ca_s", "ca_p", "config5", "ca_s_layer_op"], default=None,
                    help="run only one leg (a model step, or one of the extra operator shapes) and "
                         "print its JSON (for profiling)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy (to scale rocprof FETCH/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the CA operator shards over independent (batch, head) slices with no communication",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calibration:
        n = 64 * 1024 * 1024  # 256 MiB of fp32 read + 256 MiB written per copy
        src = torch.randn(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": 4 * n, "copy_calibration_bytes_written": 4 * n,
                          "launches": 5}), flush=True)
        return
    ca = importlib.import_module("continuum-attention_amd")
    ca.native.load()
    dev = torch.device("cuda:0")
    if args.only in ("ca_s", "ca_p"):
        leg = {"ca_s": bench_ca_s, "ca_p": bench_ca_p}[args.only]
        print(json.dumps(leg(ca, dev, steps=args.steps, warmup=args.warmup,
                             clock_warmup_s=args.clock_warmup_s)), flush=True)
        return
    if args.only:
        name, shape = {"config5": ("config5", (1, 16, 8192, 64)),
                       "ca_s_layer_op": ("ca_s_layer", (1, 16, 2048, 64))}[args.only]
        print(json.dumps(operator_leg(ca, dev, name, shape, steps=args.steps, warmup=args.warmup,
                                      clock_warmup_s=args.clock_warmup_s)), flush=True)
        return
    torch.backends.cuda.matmul.allow_tf32 = False

    shape = tuple(int(x) for x in args.shape.split(",")) if args.shape else SHAPE
    B, H, T, D = shape
    g = torch.Generator().manual_seed(0)
    q, k, v, dy = (torch.randn(shape, generator=g) for _ in range(4))
    op = time_operator(ca, dev, q, k, v, torch.zeros(H), dy, args.steps, args.warmup,
                       args.clock_warmup_s)
    ms, kt, per_kernel = op["total_ms"], op["kt"], op["kernels"]
    P = pairs(B, H, T)
    flops_total = 14 * D * P
    fpp = kernel_flops_per_pair(D)
    dom = max((n for n in per_kernel if n in fpp), key=lambda n: per_kernel[n]["avg_ms"])
    dom_ms = kt[dom][0] / kt[dom][1]
    achieved = fpp[dom] * P / (dom_ms * 1e-3) / 1e12
    op_tflops = flops_total / (ms * 1e-3) / 1e12

    out = {
        "metric": "CA fwd+bwd ms @[2,16,2048,64] fp32; % of fp32-MFMA roofline; CA-S tokens/s",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) q,k,v,dY, seed 0",
        "config": {"workload": (f"CA operator fwd+bwd [B,H,T,D]=[{B},{H},{T},{D}] fp32, causal, "
                                "log_gain=0" + (" (BASELINE config 2)" if shape == SHAPE else "")),
                   "B": B, "H": H, "T": T, "D": D, "query_tile": 128},
        "fwd_ms": op["fwd_ms"],
        "bwd_ms": op["bwd_ms"],
        "op_tflops": round(op_tflops, 2),
        "op_roofline_frac": round(op_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
        "fwd_tflops": op["fwd_tflops"],
        "bwd_tflops": op["bwd_tflops"],
        "algorithmic_gflop": round(flops_total / 1e9, 3),
        "wall_s_timed_region": op["wall_s"],
        "clock_warmup": dict(op["clock_warmup"], note=(
            "operator steps run for this long before the warm-up steps, so that the timed steps "
            "see a ramped GPU clock")),
        "kernels": per_kernel,
        # achieved = algorithmic fp32 flops of the dominant kernel / its launch
        # time, against the fp32-MFMA peak the metric names.  The products run
        # as bf16x6 on the bf16 matrix cores (fp32-accurate); the bf16 MFMA
        # work actually issued is LIMB_PRODUCTS x the algorithmic flops.
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                     "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4), "traffic": None,
                     "mfma_path": "bf16x6: six bf16 limb products per fp32 product, fp32 accumulation",
                     "bf16_mfma_frac": round(LIMB_PRODUCTS * achieved / PEAK_BF16_MFMA_TFLOPS, 4)},
        "cpu_baseline": None,
    }
    traffic_file = os.path.join(ROOT, "profiles", "ca_op_2x16x2048x64_hbm_traffic.json")
    if os.path.exists(traffic_file):
        # HBM bytes per launch of the dominant kernel, from the committed
        # rocprofv3 FETCH_SIZE / WRITE_SIZE passes (copy-calibrated)
        tr = json.load(open(traffic_file))
        for name, rec in tr.get("kernels", {}).items():
            if name.startswith(dom + "_kernel") or name.startswith(dom + "<"):
                out["roofline"]["traffic"] = rec["total_bytes"]
                out["roofline"]["traffic_source"] = (
                    f"profiles/ca_op_2x16x2048x64_hbm_traffic.md (commit {tr.get('commit')})")
    if not args.no_extra_shapes and not args.shape:
        # BASELINE config 5 (the long-context stress inputs; the backward in
        # passes under the default 1 GiB workspace cap) and one CA-S layer's
        # operator shape
        out["config5"] = operator_leg(ca, dev, "config5", (1, 16, 8192, 64), steps=20, warmup=10,
                                      clock_warmup_s=args.clock_warmup_s)
        out["ca_s_layer_op"] = operator_leg(ca, dev, "ca_s_layer", (1, 16, 2048, 64),
                                            steps=args.steps, warmup=args.warmup,
                                            clock_warmup_s=args.clock_warmup_s)
    if not args.no_models:
        out["ca_s"] = bench_ca_s(ca, dev, clock_warmup_s=args.clock_warmup_s)
        out["ca_p"] = bench_ca_p(ca, dev, clock_warmup_s=args.clock_warmup_s)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
