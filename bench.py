#!/usr/bin/env python
"""Throughput of the fused optimizer update on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3p]

One "step" is one ``AdamBridge.step()`` over the whole parameter list of the
configuration: one kernel launch that reads every gradient, master and moment
once and writes the master, the moments and the bf16 working weights.  Inputs
are synthetic and already resident in HBM when the timed region starts (bf16
weights ~ N(0, 0.02), bf16 gradients ~ N(0, 1) times a per-tensor scale drawn
log-uniformly from a seeded generator, the same gradients every step; c1 as
BASELINE.json specifies it: an FP32 master ~ N(0, 0.02) and a gradient
~ N(0, 1e-3) regenerated for every step from (seed, step), all made before
the timed region).

Prints ONE JSON line: ``value`` = parameters updated per second (wall clock
over the K timed steps, bracketed by device synchronisations); ``roofline``
for the update kernel = algorithmic bytes per launch (the reference's minimum
bytes, benchmarks/bench_kernels.py:63-65, times the parameters) divided by its
mean launch duration, timed with HIP events on the stream the kernel runs on;
``copy_ceiling`` = a plain copy of the same bytes (half read, half written)
by the library's k_stream_copy, the rate a 1:1 read/write stream reaches here;
``cpu_baseline`` = the reference's own native kernel (oracle/_ref, compiled
from its C source) timed on this host's cores over a bounded sample of the
same parameter list.

Configurations: c1 one flat 16.8M tensor, FP32 moments; c2
Qwen2.5-0.5B list, bf16 moments; c3 Llama-7B list, FP8 moments; c3p (default,
the north star) Llama-7B list, bf16 moments; c4 Qwen2.5-1.5B list, Lion with a
bf16 moment.
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "params updated/sec and achieved HBM GB/s (% roofline), AdamW bf16 moments @7B"
HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the update kernel, measured with rocprofv3 FETCH_SIZE + WRITE_SIZE, each
# scaled by its reading for a copy of known size, in separate profiling runs of this script (the
# counters cannot be read from inside the process they profile); each figure's run is in its file.
MEASURED_TRAFFIC = {"c3p": 134.767e9, "c1": 469.84e6, "c2": 9.8808e9, "c3": 108.67e9, "c4": 24.700e9}
TRAFFIC_PROFILE = {"c3p": "profiles/k_update_packed_c3p_hbm_traffic.md",
                   "c1": "profiles/k_update_f32rec_c1_packed_c2_trace_traffic.md",
                   "c2": "profiles/k_update_f32rec_c1_packed_c2_trace_traffic.md",
                   "c3": "profiles/k_update_fp8_c3_trace_traffic_instructions.md",
                   "c4": "profiles/k_update_lion_rec_c4_trace_traffic.md"}
# the same with an FP24 master (--master fp24), where measured
MEASURED_TRAFFIC_FP24 = {"c3p": 60.646e9 + 60.632e9, "c3": 47.59e9 + 47.58e9, "c4": 10.806e9 + 10.804e9}
TRAFFIC_PROFILE_FP24 = {"c3p": "profiles/k_update_f24rec_fp24_master_trace_valu.md",
                        "c3": "profiles/k_update_fp8_c3_trace_traffic_instructions.md",
                        "c4": "profiles/k_update_f24rec_fp24_master_trace_valu.md"}


# ------------------------------------------------------------ parameter lists

def qwen_like(vocab, hidden, inter, layers, kv) -> list[tuple[str, tuple]]:
    out = [("embed", (vocab, hidden))]
    for i in range(layers):
        out += [(f"l{i}.q", (hidden, hidden)), (f"l{i}.q.b", (hidden,)), (f"l{i}.k", (kv, hidden)),
                (f"l{i}.k.b", (kv,)), (f"l{i}.v", (kv, hidden)), (f"l{i}.v.b", (kv,)), (f"l{i}.o", (hidden, hidden)),
                (f"l{i}.gate", (inter, hidden)), (f"l{i}.up", (inter, hidden)), (f"l{i}.down", (hidden, inter)),
                (f"l{i}.norm1", (hidden,)), (f"l{i}.norm2", (hidden,))]
    out.append(("norm", (hidden,)))
    return out


def llama7b() -> list[tuple[str, tuple]]:
    h, inter = 4096, 11008
    out = [("embed", (32000, h))]
    for i in range(32):
        out += [(f"l{i}.q", (h, h)), (f"l{i}.k", (h, h)), (f"l{i}.v", (h, h)), (f"l{i}.o", (h, h)),
                (f"l{i}.gate", (inter, h)), (f"l{i}.up", (inter, h)), (f"l{i}.down", (h, inter)),
                (f"l{i}.norm1", (h,)), (f"l{i}.norm2", (h,))]
    out += [("norm", (h,)), ("lm_head", (32000, h))]
    return out


CONFIGS = {
    "c1": dict(desc="AdamW, FP32 moments, one flat tensor of 16,777,216 params", shapes=lambda: [("flat", (1 << 24,))],
               algo="adamw", precision="fp32", lr=1e-4, betas=(0.9, 0.999), wd=0.01, gscale=(1e-3, 1e-3),
               warm_steps=5, rotate=4, master_init="fp32", grads_per_step=True),
    "c2": dict(desc="AdamW, bf16 moments, Qwen2.5-0.5B parameter list",
               shapes=lambda: qwen_like(151936, 896, 4864, 24, 128),
               algo="adamw", precision="bf16", lr=2e-5, betas=(0.9, 0.999), wd=0.01, gscale=(1e-5, 1e-2),
               warm_steps=10),
    "c3": dict(desc="AdamW, FP8 moments, Llama-7B parameter list", shapes=llama7b,
               algo="adamw", precision="fp8", lr=1e-5, betas=(0.9, 0.999), wd=0.01, gscale=(1e-5, 1e-2)),
    "c3p": dict(desc="AdamW, bf16 moments, Llama-7B parameter list", shapes=llama7b,
                algo="adamw", precision="bf16", lr=1e-5, betas=(0.9, 0.999), wd=0.01, gscale=(1e-5, 1e-2)),
    "c4": dict(desc="Lion, bf16 moment, Qwen2.5-1.5B parameter list",
               shapes=lambda: qwen_like(151936, 1536, 8960, 28, 256),
               algo="lion", precision="bf16", lr=3e-6, betas=(0.9, 0.99), wd=0.1, gscale=(1e-6, 1e-2),
               grads="elementwise", zeros=0.01),
}


def min_bytes(precision: str, algo: str, grad_bytes: int = 2, out_bytes: int = 2, master: str = "fp32") -> float:
    """Minimum bytes per parameter: master read+write, gradient, moments read+write, output
    (reference benchmarks/bench_kernels.py:63-65; an FP24 master is 3 bytes)."""
    mv = {"fp32": 4, "bf16": 2, "fp8": 1 + 4 / 128}[precision]
    return (3 if master == "fp24" else 4) * 2 + grad_bytes + mv * 2 * (1 if algo == "lion" else 2) + out_bytes


# ----------------------------------------------------------------- GPU side

def build(cfg: dict, device, seed: int = 0, layout: str = "auto", double_buffer: bool = False):
    import torch
    import adambridge_amd as ab

    # Allocated in the order a training job allocates them: every weight when the model is built, the
    # gradients during the first backward pass (last layer first), the optimizer state at the first
    # step.
    gen = torch.Generator(device=device).manual_seed(seed)
    shapes = [shape for _, shape in cfg["shapes"]()]
    masters = None
    if cfg.get("master_init") == "fp32":   # c1: an FP32 master ~ N(0, 0.02), the weights its bf16
        masters = [torch.randn(shape, generator=gen, device=device, dtype=torch.float32).mul_(0.02) for shape in shapes]
        params = [torch.nn.Parameter(m.to(torch.bfloat16)) for m in masters]
    else:
        params = [torch.nn.Parameter(torch.randn(shape, generator=gen, device=device, dtype=torch.bfloat16).mul_(0.02))
                  for shape in shapes]
    grads = step_grads(cfg, params, 1, seed)
    if grads is None:
        grads = [None] * len(shapes)
        for k in reversed(range(len(shapes))):
            grads[k] = synthetic_grad(cfg, k, shapes[k], gen, device, seed)
    kw = dict(lr=cfg["lr"], betas=cfg["betas"], weight_decay=cfg["wd"], precision=cfg["precision"],
              master_precision=cfg.get("master", "fp32"), state_layout=layout, double_buffer=double_buffer)
    opt = ab.LionBridge(params, **kw) if cfg["algo"] == "lion" else ab.AdamBridge(params, **kw)
    if masters is not None:   # the state built now (lazily it would take the bf16 weights), masters loaded
        opt._engine.initialize(list(opt._ordered))
        for slot, m in zip(opt._ordered, masters):
            slot.state.load(master=m.reshape(-1))
        del masters
    for p, g in zip(params, grads):
        p.grad = g
    return opt, params


def step_grads(cfg: dict, params, t: int, seed: int = 0):
    """The gradients of step ``t`` (1, 2, ...) where a configuration regenerates them every step
    (cfg['grads_per_step'], c1: N(0, 1e-3) from a generator seeded by (seed, t)); None where the
    build's gradients serve every step."""
    if not cfg.get("grads_per_step"):
        return None
    import torch

    device = params[0].device
    gen = torch.Generator(device=device).manual_seed((seed << 32) + t)
    return [synthetic_grad(cfg, k, tuple(p.shape), gen, device, seed) for k, p in enumerate(params)]


def use_step_grads(cfg: dict, params, t: int, seed: int = 0) -> None:
    """Point the parameters' gradients at step ``t``'s (step_grads) where the configuration regenerates
    them every step; otherwise leave the build's in place."""
    grads = step_grads(cfg, params, t, seed)
    if grads is not None:
        for p, g in zip(params, grads):
            p.grad = g


def synthetic_grad(cfg: dict, k: int, shape, gen, device, seed: int = 0):
    """Tensor k's bf16 gradient.  Default: N(0, 1) times one scale per tensor, drawn log-uniformly over
    cfg['gscale'] from a generator seeded by (seed, k) (c2, c3).  grads='elementwise' (c4): every
    element's magnitude log-uniform over cfg['gscale'], a random sign, and exact zeros at density
    cfg['zeros'] (sign(0) = 0 in Lion)."""
    import numpy as np
    import torch

    lo, hi = cfg["gscale"]
    if cfg.get("grads") == "elementwise":
        u = torch.rand(shape, generator=gen, device=device)
        g = torch.exp(u.mul_(math.log(hi) - math.log(lo)).add_(math.log(lo)))
        sign = torch.rand(shape, generator=gen, device=device) < 0.5
        g = torch.where(sign, -g, g)
        g[torch.rand(shape, generator=gen, device=device) < cfg.get("zeros", 0.0)] = 0.0
        return g.to(torch.bfloat16)
    u = float(np.random.default_rng((seed, k)).random())
    scale = math.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))
    return torch.randn(shape, generator=gen, device=device, dtype=torch.bfloat16).mul_(scale)


def gpu_bench(cfg: dict, steps: int, warmup: int, layout: str = "auto", double_buffer: bool = False,
              keep: list | None = None) -> dict:
    """Time ``steps`` optimizer steps after ``warmup`` untimed ones.  A configuration with
    ``rotate`` = R builds R independent copies (weights, gradients, state) and steps them in turn,
    so that consecutive launches stream from HBM, not from the 256 MB Infinity Cache (c1 moves
    470 MB per step); each timed step is still one full step of one copy.  ``keep``: a list that
    receives the optimizers and parameters instead of their being released (the caller closes the
    optimizers)."""
    import torch

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    copies = [build(cfg, device, seed=k, layout=layout, double_buffer=double_buffer)
              for k in range(cfg.get("rotate", 1))]
    opts = [opt for opt, _ in copies]
    n = sum(p.numel() for p in copies[0][1])
    # per-step gradients (c1): made before timing, for every copy's warm-up and timed steps; a step
    # only points its parameters' .grad at them
    per_step = {}
    if cfg.get("grads_per_step"):
        for k in range(warmup * len(opts) + steps):
            c, t = k % len(opts), k // len(opts) + 1
            per_step[k] = step_grads(cfg, copies[c][1], t, seed=c) if t > 1 else [p.grad for p in copies[c][1]]

    def step(k: int) -> None:
        grads = per_step.get(k)
        if grads is not None:
            for p, g in zip(copies[k % len(opts)][1], grads):
                p.grad = g
        opts[k % len(opts)].step()

    # No garbage collection inside the timed region (as timeit does): a collection pauses the host
    # for tens of milliseconds, and where a launch is shorter than the host's lead (the 0.5B list:
    # 1.6 ms) the device then idles -- between a launch's start event and the launch, inflating it.
    # The collection runs before the warm-up, not between it and the timed steps: after the idle
    # stretch it leaves (55-87 ms) the first launches ran slower (the 7B list 21.5 against 20.6 ms;
    # the 0.5B list several launches of 1.6-1.8 against 1.55 ms), as traces of this script showed.
    gc.collect()
    gc.disable()
    try:
        for k in range(warmup * len(opts)):
            step(k)
        torch.cuda.synchronize()
        log: list = []
        for opt in opts:
            opt._engine.launch_log = log
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(steps):
            step(warmup * len(opts) + k)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    finally:
        gc.enable()
    for opt in opts:
        opt._engine.launch_log = None
    durs = [a.elapsed_time(b) / 1e3 for a, b, _ in log]
    if os.environ.get("ADAMBRIDGE_BENCH_TRACE"):   # diagnostic: launch durations in order, 10 per line
        for k in range(0, len(durs), 10):
            print(f"[bench] launches {k}..: " + " ".join(f"{d * 1e3:.2f}" for d in durs[k:k + 10]), file=sys.stderr,
                  flush=True)
    launches_per_step = len(log) / steps
    bpp = min_bytes(cfg["precision"], cfg["algo"], master=cfg.get("master", "fp32"))
    kernel_s = sum(durs) / len(durs)
    elems_per_launch = sum(e for _, _, e in log) / len(log)
    achieved = elems_per_launch * bpp / kernel_s / 1e9
    layouts = sorted({s.state.layout for s in opts[0]._ordered})
    state_layout = ", ".join(layouts) + (" (double-buffered)" if double_buffer else "")
    stats = dict(params=n, tensors=len(copies[0][1]), wall=wall, launches_per_step=launches_per_step,
                 layout=state_layout, state_bytes=opts[0].memory_report()["total"], copies=len(opts),
                 kernel_ms=kernel_s * 1e3, kernel_ms_min=min(durs) * 1e3, kernel_ms_max=max(durs) * 1e3,
                 achieved_gbs=achieved, bytes_per_param=bpp)
    if keep is not None:
        keep.extend(copies)
        return stats
    for opt in opts:
        opt.close()
    del opts, copies
    torch.cuda.empty_cache()
    return stats


def torch_release() -> None:
    """Return cached device memory to the driver (after the held builds are dropped)."""
    import torch

    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def calibrate_copy(nbytes: int) -> None:
    """Three copies of ``nbytes`` between two device buffers by the library's k_stream_copy -- the
    update kernels' 16-byte non-temporal loads and stores and tile order: under rocprofv3 --pmc, its
    FETCH_SIZE and WRITE_SIZE readings against ``nbytes`` give the counters' scale factors."""
    import torch
    from adambridge_amd import _hip

    nbytes = nbytes // 16 * 16
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        _hip.load().stream_copy(src, dst)
    torch.cuda.synchronize()
    print(f"[bench] calibration: 3 copies of {nbytes} bytes", file=sys.stderr, flush=True)
    del src, dst
    torch.cuda.empty_cache()


def copy_ceiling(total_bytes: float, reps: int = 10) -> dict:
    """The rate of a plain copy moving the update's bytes -- half read, half written -- by the
    library's k_stream_copy (16-byte non-temporal loads and stores, 4 KiB tiles handed out XCD by
    XCD), timed with HIP events on the stream it runs on: what a 1:1 read/write stream of the same
    size reaches on this device.  Copies under 4 GB rotate over four buffer pairs, so that each
    streams from HBM rather than the 256 MB Infinity Cache.  Median over ``reps`` launches after 3
    untimed ones."""
    import statistics

    import torch
    from adambridge_amd import _hip

    k = _hip.load()
    half = int(total_bytes / 2) // 16 * 16
    pairs = [(torch.ones(half, dtype=torch.uint8, device="cuda"), torch.empty(half, dtype=torch.uint8, device="cuda"))
             for _ in range(4 if 2 * half < 4e9 else 1)]
    times = []
    for i in range(3 + reps):
        src, dst = pairs[i % len(pairs)]
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        k.stream_copy(src, dst)
        b.record()
        b.synchronize()
        if i >= 3:
            times.append(a.elapsed_time(b) / 1e3)
    del pairs
    torch.cuda.empty_cache()
    t = statistics.median(times)
    gbs = 2 * half / t / 1e9
    return dict(kernel="k_stream_copy", bytes=2 * half, ms=t * 1e3, gbs=gbs, frac=gbs / HBM_PEAK_GBS)


# ------------------------------------------------------- hooked pipeline (c5)

PIPELINE = dict(layers=24, hidden=2048, inter=8192, batch=8, seq=512, lr=1e-4, wd=0.01)


def pipeline_model(device, dtype=None):
    """24 x [LayerNorm(2048) -> Linear(2048 -> 8192) -> GELU -> Linear(8192 -> 2048)] with a residual,
    the reference's benchmark block (benchmarks/bench_pipeline.py:20-28), bf16 by default:
    805,650,432 parameters (48 weight matrices with a hook each; 48 biases and 48 LayerNorm weights
    and biases batched at step_sync)."""
    import torch

    class Block(torch.nn.Module):
        def __init__(self, h, i):
            super().__init__()
            self.norm = torch.nn.LayerNorm(h)
            self.up = torch.nn.Linear(h, i)
            self.down = torch.nn.Linear(i, h)

        def forward(self, x):
            return x + self.down(torch.nn.functional.gelu(self.up(self.norm(x))))

    torch.manual_seed(0)
    c = PIPELINE
    return torch.nn.Sequential(*[Block(c["hidden"], c["inter"]) for _ in range(c["layers"])]).to(
        device=device, dtype=dtype or torch.bfloat16)


PIPELINE_RUNS = {
    "floor": "fwd+bwd only",
    "torch": "torch.optim.AdamW(fused=True), bf16 params and state, no master",
    "torch-fp32": "torch.optim.AdamW(fused=True), fp32 params + bf16 autocast",
    "step": "AdamBridge bf16 step()",
    "hooked": "AdamBridge bf16 attach_hooks + step_sync",
    "delayed": "AdamBridge bf16 attach_hooks + delay_updates",
    "step-side": "AdamBridge bf16 step(), update_stream='side'",
    "hooked-side": "AdamBridge bf16 attach_hooks + step_sync, update_stream='side'",
}


def pipeline_bench(steps: int, warmup: int, runs=None) -> dict:
    """Training-step wall time of the c5 stack (reference benchmarks/bench_pipeline.py:58-128) with:
    no optimizer (the floor), torch's fused AdamW on the bf16 model, torch's fused AdamW on an fp32
    model under bf16 autocast (the reference's GPU baseline), AdamBridge.step() after backward,
    attach_hooks + step_sync, and attach_hooks + delay_updates; each with the peak device memory
    allocated during its steps (bench_pipeline.py:37-50), and, for the hooked runs, the GPU time of
    the updates and the exposed tail (last gradient ready -> last update done) from the optimizer's
    timing events, taken over 3 more steps after the timed ones (the timed steps run without those
    events, as the optimizer does by default).  The AdamBridge runs take the default in-order
    updates on the current stream; the "-side" runs put them on a side stream.  ``runs``: the keys
    of PIPELINE_RUNS to time (default: all, in that order)."""
    import statistics

    import torch
    import adambridge_amd as ab

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    c = PIPELINE
    gen = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(c["batch"] * c["seq"], c["hidden"], generator=gen, device=device, dtype=torch.bfloat16)
    target = torch.randn(x.shape, generator=gen, device=device, dtype=torch.bfloat16)

    def loss_of(model):
        return torch.nn.functional.mse_loss(model(x).float(), target.float())

    def timed(step, engine=None):
        times, upd, tail, bwd = [], [], [], []
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(device)
        for i in range(warmup + steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            step()
            torch.cuda.synchronize()
            if i >= warmup:
                times.append(time.perf_counter() - t0)
        out = dict(step_ms=statistics.median(times) * 1e3,
                   peak_gib=torch.cuda.max_memory_allocated(device) / 2**30)
        if engine is not None:   # the update's GPU span and exposed tail, from the timing events
            engine.timing = True
            for _ in range(3):
                st = step()
                torch.cuda.synchronize()
                upd.append(st.gpu_update or 0.0)
                tail.append(st.exposed_tail or 0.0)
                bwd.append(st.gpu_backward or 0.0)
            engine.timing = False
        if upd:
            out.update(gpu_update_ms=statistics.median(upd) * 1e3, exposed_tail_ms=statistics.median(tail) * 1e3,
                       gpu_backward_ms=statistics.median(bwd) * 1e3)
        return out

    def release():
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    results = {}
    runs = list(PIPELINE_RUNS) if runs is None else list(runs)
    n = sum(p.numel() for p in pipeline_model("meta").parameters())
    for key in runs:
        name = PIPELINE_RUNS[key]
        print(f"[bench] c5 run: {name}", file=sys.stderr, flush=True)
        if key == "floor":
            model = pipeline_model(device)

            def step():
                loss_of(model).backward()
                for p in model.parameters():
                    p.grad = None
            results[name] = timed(step)
            del model
        elif key in ("torch", "torch-fp32"):
            fp32 = key == "torch-fp32"
            model = pipeline_model(device, torch.float32 if fp32 else torch.bfloat16)
            opt = torch.optim.AdamW(model.parameters(), lr=c["lr"], weight_decay=c["wd"], fused=True)

            def step():
                with torch.autocast("cuda", dtype=torch.bfloat16, enabled=fp32):
                    loss_of(model).backward()
                opt.step()
                opt.zero_grad(set_to_none=True)
            results[name] = timed(step)
            del opt, model
        else:
            hooks, delay = key in ("hooked", "delayed", "hooked-side"), key == "delayed"
            model = pipeline_model(device)
            opt = ab.AdamBridge(model.parameters(), lr=c["lr"], weight_decay=c["wd"], precision="bf16",
                                delay_updates=delay, update_stream="side" if key.endswith("-side") else "current")
            if hooks:
                opt.attach_hooks(model)

                def step():
                    loss_of(model).backward()
                    return opt.step_sync()
            else:
                def step():
                    loss_of(model).backward()
                    opt.step()
                    opt.zero_grad(set_to_none=True)
            results[name] = timed(step, opt._engine if hooks else None)
            opt.close()
            del opt, model
        release()
    return dict(params=n, results=results)


# ----------------------------------------------------------------- CPU side

def host_cpus() -> dict:
    """The CPUs this process may run on: logical count, physical cores among them, model and the
    widest x86 vector ISA (from /proc/cpuinfo)."""
    try:
        allowed = sorted(os.sched_getaffinity(0))
    except AttributeError:
        allowed = list(range(os.cpu_count() or 1))
    cores, model, flags = set(), "unknown", set()
    try:
        proc = None
        phys = core = None
        for line in Path("/proc/cpuinfo").read_text().splitlines() + [""]:
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "processor":
                proc = int(val)
            elif key == "physical id":
                phys = val
            elif key == "core id":
                core = val
            elif key == "model name":
                model = val
            elif key == "flags":
                flags = set(val.split())
            elif not line and proc is not None:
                if proc in allowed:
                    cores.add((phys, core) if core is not None else proc)
                proc = phys = core = None
    except OSError:
        pass
    isa = "avx512" if "avx512f" in flags else "avx2" if "avx2" in flags else "sse"
    return dict(logical=len(allowed), physical=len(cores) or len(allowed), model=model, isa=isa)


# The GPU box gives a one-GPU job a share of 16 CPUs, whatever the machine has in all.
CPU_SHARE = 16


def cpu_bench(cfg: dict, budget_params: int, steps: int) -> dict:
    """The reference's native kernel (oracle/_ref, compiled from its C source) over the first tensors
    of the same list, up to ``budget_params`` parameters, timed at the reference's default thread
    count -- min(32, 2/3 of the CPUs, engine.py:635), the CPUs being this job's share of the host --
    and on every physical core of that share.  Where the reference library was not built (no
    reference tree at build time), the oracle's C restatement of the same algorithm
    (oracle/liboracle.so, OpenMP) is timed instead, kind "port"."""
    import ctypes

    import numpy as np
    from oracle import oracle as O

    use_ref = O.reference_available()
    lib = O.load_reference() if use_ref else O.load_oracle()
    host = host_cpus()
    share = max(1, min(CPU_SHARE, host["logical"]))
    plans = {"default": max(1, min(32, (2 * share) // 3)), "all_cores": max(1, min(share, host["physical"]))}
    shapes, total = [], 0
    for name, shape in cfg["shapes"]():
        numel = math.prod(shape)
        if shapes and total + numel > budget_params:
            break
        shapes.append((name, numel))
        total += numel
    rng = np.random.default_rng(0)
    # one random pattern tiled over every tensor: each buffer is written once (timing does not depend on values)
    pat_p = ((rng.random(1 << 20, dtype=np.float32) - 0.5) * 0.04).astype(np.float32)
    pat_g = O.bf16_bits((rng.random(1 << 20, dtype=np.float32) - 0.5) * 2e-3)
    mv_dt = {"fp32": O.DT_F32, "bf16": O.DT_BF16, "fp8": O.DT_FP8}[cfg["precision"]]
    lion = cfg["algo"] == "lion"
    group = O.Group(cfg["lr"], cfg["betas"][0], cfg["betas"][1], 0.0 if lion else 1e-8, cfg["wd"], 0, 1, 0)
    keep, segs = [], []
    f24 = cfg.get("master", "fp32") == "fp24"
    for k, (name, numel) in enumerate(shapes):
        p = np.resize(pat_p, numel)
        p_lo = None
        if f24:   # hi plane (the bf16 bits) and lo plane of the same values
            bits = p.view(np.uint32)
            p, p_lo = (bits >> 16).astype(np.uint16), ((bits >> 8) & 0xFF).astype(np.uint8)
        g = np.resize(pat_g, numel)
        out = np.empty(numel, np.uint16)
        if mv_dt == O.DT_FP8:
            nb = -(-numel // 128)
            m, v = np.zeros(nb * 128, np.uint8), np.zeros(nb * 128, np.uint8)
            ms, vs = np.ones(nb, np.float32), np.ones(nb, np.float32)
        else:
            dt = np.float32 if mv_dt == O.DT_F32 else np.uint16
            m, v, ms, vs = np.zeros(numel, dt), np.zeros(numel, dt), None, None
        keep.append(dict(p=p, p_lo=p_lo, g=g, m=m, v=None if lion else v, m_scale=ms, v_scale=None if lion else vs,
                         out=out))
        segs.append(O.Segment(p=p.ctypes.data, p_lo=None if p_lo is None else p_lo.ctypes.data,
                              g=g.ctypes.data, m=m.ctypes.data,
                              v=None if lion else v.ctypes.data, m_scale=None if ms is None else ms.ctypes.data,
                              v_scale=None if (lion or vs is None) else vs.ctypes.data, out=out.ctypes.data,
                              group=ctypes.pointer(group), n=numel, step=1, index=k, offset=0, g_dtype=O.DT_BF16,
                              mv_dtype=mv_dt, out_dtype=O.DT_BF16, algorithm=1 if lion else 0,
                              p_dtype=O.DT_F24 if f24 else O.DT_F32))
    arr = (ctypes.POINTER(O.Segment) * len(segs))(*[ctypes.pointer(s) for s in segs])
    bpp = min_bytes(cfg["precision"], cfg["algo"], master=cfg.get("master", "fp32"))
    level = None
    if use_ref:
        lib.adambridge_set_simd_level(-1)
        level = lib.adambridge_simd_level()
    runs = {}
    step = 1
    for plan, threads in plans.items():
        pool = lib.adambridge_pool_create(threads, None, 0) if use_ref else None
        try:
            def one():
                nonlocal step
                for seg in segs:
                    seg.step = step
                step += 1
                rc = (lib.adambridge_multi_step(pool, arr, len(segs), threads) if use_ref
                      else lib.abo_multi_step(arr, len(segs), 16, threads))
                if rc:
                    raise RuntimeError(f"CPU multi_step returned {rc}")
            one()   # warm-up (bench_kernels.py:30-37)
            times = []
            for _ in range(steps):
                t0 = time.perf_counter()
                one()
                times.append(time.perf_counter() - t0)
        finally:
            if pool:
                lib.adambridge_pool_destroy(pool)
        med = sorted(times)[len(times) // 2]
        runs[plan] = dict(threads=threads, value=total / med, ms_per_step=med * 1e3, gbs=total * bpp / med / 1e9)
    what = (f"reference native kernel (oracle/_ref, compiled from adambridge_kernels.c, SIMD level {level})"
            if use_ref else "oracle C restatement of the reference kernel (oracle/liboracle.so, scalar C, OpenMP)")
    d = runs["default"]
    return dict(value=d["value"], unit="params/s", cores=d["threads"], kind="reference" if use_ref else "port",
                sample=(f"{what} on the first {len(shapes)} tensors of the same list ({total:,} params), median of "
                        f"{steps} steps after 1 warm-up, at the reference's default thread count "
                        f"min(32, 2/3 x {share} CPUs) = {d['threads']} and on all {runs['all_cores']['threads']} "
                        f"physical cores of this job's {share}-CPU share"),
                ms_per_step=d["ms_per_step"], gbs=d["gbs"],
                all_cores=runs["all_cores"],
                host=dict(model=host["model"], logical_cpus=host["logical"], physical_cores=host["physical"],
                          cpu_share=share, isa=host["isa"], reference_simd_level=level))


# --------------------------------------------------------------------- main

def config_of(name: str, master: str = "fp32", precision: str | None = None) -> tuple[dict, bool]:
    """The workload of configuration ``name`` with ``master`` and, when given, ``precision`` for its
    moments; and whether the moments are the configuration's own (its measured traffic applies)."""
    cfg = dict(CONFIGS[name], master=master)
    own = cfg["precision"] == (precision or cfg["precision"])
    if not own:
        names = {"fp32": "FP32", "bf16": "bf16", "fp8": "FP8"}
        cfg["desc"] = cfg["desc"].replace(names[cfg["precision"]], names[precision], 1)
        cfg["precision"] = precision
    return cfg, own


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3p", choices=sorted(CONFIGS) + ["c5"],
                    help="c5: the hooked training pipeline (prints its own JSON line)")
    ap.add_argument("--cpu-params", type=int, default=1 << 30, help="CPU baseline sample size (parameters)")
    ap.add_argument("--cpu-steps", type=int, default=80,
                    help="timed steps of each CPU-baseline run (about 10 s of CPU work at the default sample)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-copy-ceiling", action="store_true",
                    help="skip timing a plain copy of the update's bytes (the copy_ceiling object)")
    ap.add_argument("--layout", default="auto", choices=["auto", "packed", "separate"],
                    help="optimizer state layout in HBM (AdamBridge state_layout)")
    ap.add_argument("--double-buffer", action="store_true", help="AdamBridge double_buffer=True")
    ap.add_argument("--master", default="fp32", choices=["fp32", "fp24"],
                    help="master weight precision (AdamBridge master_precision); the configurations' own is fp32")
    ap.add_argument("--precision", default=None, choices=["fp32", "bf16", "fp8"],
                    help="moment precision (AdamBridge / LionBridge precision); default: the configuration's own")
    ap.add_argument("--traffic", type=float, default=None,
                    help="HBM bytes per launch measured by rocprofv3 (FETCH_SIZE+WRITE_SIZE, scaled); "
                         "default: the figure measured for this configuration, when there is one")
    ap.add_argument("--rebuilds", type=int, default=1, metavar="N",
                    help="diagnostic: build and time the state N times in this process, printing each "
                         "on stderr (the GPU's power state can change between them); the JSON line "
                         "reports the first")
    ap.add_argument("--no-second-build", action="store_true",
                    help="skip timing a second state built while the first is alive (the placement object)")
    ap.add_argument("--pipeline-runs", default="", metavar="RUNS",
                    help="c5: comma-separated runs to time, of " + ",".join(PIPELINE_RUNS) + " (default: all)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="first run 3 device-to-device copies of BYTES bytes (a known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "sharded, each rank would update its 128-aligned element ranges of every state buffer "
              "between a reduce-scatter of the gradients and an all-gather of the weights", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0 or args.rebuilds < 1:
        ap.error("--steps and --rebuilds must be >= 1 and --warmup >= 0")
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
    if args.config == "c5":
        return main_pipeline(args)
    cfg, own = config_of(args.config, args.master, args.precision)
    print(f"[bench] config {args.config}: {cfg['desc']}; warmup {args.warmup}, steps {args.steps}",
          file=sys.stderr, flush=True)
    held: list = []
    g = gpu_bench(cfg, args.steps, args.warmup, args.layout, args.double_buffer, keep=held)
    print(f"[bench] GPU: {g['kernel_ms']:.3f} ms/launch, {g['achieved_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    placement = None
    if not args.no_second_build:
        # The state a fresh process builds first can land where HBM serves this update's traffic
        # more slowly; a second state, built while the first is still allocated, shows the rate the
        # same kernel reaches elsewhere in HBM.  The line's value and roofline are the first build's.
        s2 = gpu_bench(cfg, args.steps, args.warmup, args.layout, args.double_buffer)
        placement = {"first_build_kernel_ms": g["kernel_ms"], "second_build_kernel_ms": s2["kernel_ms"],
                     "second_build_gbs": s2["achieved_gbs"], "second_build_frac": s2["achieved_gbs"] / HBM_PEAK_GBS,
                     "note": "value and roofline are the first build's; the second state is built and timed "
                             "while the first is still allocated"}
        print(f"[bench] second build: {s2['kernel_ms']:.3f} ms/launch, {s2['achieved_gbs']:.0f} GB/s",
              file=sys.stderr, flush=True)
    for opt, _ in held:
        opt.close()
    del held
    torch_release()
    for k in range(1, args.rebuilds):
        r = gpu_bench(cfg, args.steps, args.warmup, args.layout, args.double_buffer)
        print(f"[bench] rebuild {k}: {r['kernel_ms']:.3f} ms/launch, {r['achieved_gbs']:.0f} GB/s", file=sys.stderr,
              flush=True)
    ceiling = None
    if not args.no_copy_ceiling:
        ceiling = copy_ceiling(g["params"] * g["bytes_per_param"])
        ceiling["update_vs_copy"] = g["achieved_gbs"] / ceiling["gbs"]
        print(f"[bench] copy of the same bytes: {ceiling['ms']:.3f} ms, {ceiling['gbs']:.0f} GB/s; "
              f"update / copy {ceiling['update_vs_copy']:.3f}", file=sys.stderr, flush=True)
    cpu = None if args.no_cpu else cpu_bench(cfg, args.cpu_params, args.cpu_steps)
    if cpu is not None:
        print(f"[bench] CPU reference: {cpu['ms_per_step']:.1f} ms/step on {cpu['cores']} threads, "
              f"{cpu['all_cores']['ms_per_step']:.1f} ms/step on {cpu['all_cores']['threads']} ({cpu['host']})",
              file=sys.stderr, flush=True)
    ms_per_step = g["wall"] / args.steps * 1e3
    # the traffic measured for each configuration and master
    measured, profiled = ((MEASURED_TRAFFIC, TRAFFIC_PROFILE) if args.master == "fp32" else
                          (MEASURED_TRAFFIC_FP24, TRAFFIC_PROFILE_FP24))
    if not own:   # the measured traffic figures are the configurations' own moments'
        measured, profiled = {}, {}
    line = {
        "metric": METRIC if args.config == "c3p" and args.master == "fp32" and own else
        f"params updated/sec and achieved HBM GB/s (% roofline), {cfg['desc']} ({args.config}"
        f"{', FP24 master' if args.master == 'fp24' else ''})",
        "value": g["params"] * args.steps / g["wall"],
        "unit": "params/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": ("synthetic (bf16 weights ~N(0,0.02); bf16 grads with per-element log-uniform magnitudes in "
                 f"{cfg['gscale']} and {cfg['zeros']:.0%} exact zeros)" if cfg.get("grads") == "elementwise" else
                 "synthetic (bf16 weights ~N(0,0.02), bf16 grads ~N(0,1) x log-uniform per-tensor scale)"),
        "config": {"workload": cfg["desc"], "config": args.config, "params": g["params"], "tensors": g["tensors"],
                   "moments": cfg["precision"], "master": cfg["master"], "grad": "bf16", "out": "bf16",
                   "bytes_per_param": g["bytes_per_param"], "launches_per_step": g["launches_per_step"],
                   "state_layout": g["layout"], "state_bytes": g["state_bytes"], "copies_rotated": g["copies"],
                   "wall_gbs": g["params"] * g["bytes_per_param"] / (ms_per_step / 1e3) / 1e9},
        "roofline": {"bound": "hbm", "achieved": g["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": g["achieved_gbs"] / HBM_PEAK_GBS,
                     "traffic": args.traffic if args.traffic is not None else measured.get(args.config),
                     "traffic_source": "--traffic" if args.traffic is not None else profiled.get(args.config),
                     "kernel_ms": g["kernel_ms"]},
        "copy_ceiling": ceiling,
        "placement": placement,
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample",
                                                                      "ms_per_step", "gbs", "all_cores", "host")},
    }
    print(json.dumps(line), flush=True)
    return 0


def main_pipeline(args) -> int:
    c = PIPELINE
    runs = args.pipeline_runs.split(",") if args.pipeline_runs else list(PIPELINE_RUNS)
    unknown = [r for r in runs if r not in PIPELINE_RUNS]
    if unknown:
        print(f"bench.py: unknown --pipeline-runs {unknown}; expected some of {list(PIPELINE_RUNS)}", file=sys.stderr)
        return 2
    print(f"[bench] c5: {c['layers']}-layer bf16 MLP LayerNorm + {c['hidden']}->{c['inter']}->{c['hidden']}, "
          f"{c['batch']}x{c['seq']} tokens; warmup {args.warmup}, steps {args.steps}; runs {','.join(runs)}",
          file=sys.stderr, flush=True)
    r = pipeline_bench(args.steps, args.warmup, runs)
    for name, v in r["results"].items():
        print(f"[bench] {name:<64} " + ", ".join(f"{k} {x:.2f}" for k, x in v.items()), file=sys.stderr, flush=True)
    main = r["results"].get(PIPELINE_RUNS["hooked"]) or next(iter(r["results"].values()))
    line = {
        "metric": "training step wall time, 24-layer bf16 MLP, hooked bf16-moment AdamW (c5)",
        "value": main["step_ms"], "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": main["step_ms"], "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 model, f32 update", "data": "synthetic (N(0,1) tokens and targets, seed 0)",
        "config": {"workload": "c5 hooked pipeline", "params": r["params"], "tokens": c["batch"] * c["seq"],
                   "bytes_per_param": 20, "runs": r["results"]},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
