#!/usr/bin/env python
"""Throughput of the fused optimizer update on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3p]

One "step" is one ``AdamBridge.step()`` over the whole parameter list of the
configuration: one kernel launch that reads every gradient, master and moment
once and writes the master, the moments and the bf16 working weights.  Inputs
are synthetic and already resident in HBM when the timed region starts (bf16
weights ~ N(0, 0.02), bf16 gradients ~ N(0, 1) times a per-tensor scale drawn
log-uniformly; the same gradients every step -- the kernel has no
data-dependent branches).

Prints ONE JSON line: ``value`` = parameters updated per second (wall clock
over the K timed steps, bracketed by device synchronisations); ``roofline``
for the update kernel = algorithmic bytes per launch (the reference's minimum
bytes, benchmarks/bench_kernels.py:63-65, times the parameters) divided by its
mean launch duration, timed with HIP events on the stream the kernel runs on;
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
# scaled by its reading for a copy of known size (profiles/*_hbm_traffic.md).
MEASURED_TRAFFIC = {"c3p": 134.764e9, "c1": 469.84e6, "c2": 9.8808e9, "c3": 108.67e9, "c4": 24.6996e9}


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
               algo="adamw", precision="fp32", lr=1e-4, betas=(0.9, 0.999), wd=0.01, gscale=(1e-3, 1e-3)),
    "c2": dict(desc="AdamW, bf16 moments, Qwen2.5-0.5B parameter list",
               shapes=lambda: qwen_like(151936, 896, 4864, 24, 128),
               algo="adamw", precision="bf16", lr=2e-5, betas=(0.9, 0.999), wd=0.01, gscale=(1e-5, 1e-2)),
    "c3": dict(desc="AdamW, FP8 moments, Llama-7B parameter list", shapes=llama7b,
               algo="adamw", precision="fp8", lr=1e-5, betas=(0.9, 0.999), wd=0.01, gscale=(1e-5, 1e-2)),
    "c3p": dict(desc="AdamW, bf16 moments, Llama-7B parameter list", shapes=llama7b,
                algo="adamw", precision="bf16", lr=1e-5, betas=(0.9, 0.999), wd=0.01, gscale=(1e-5, 1e-2)),
    "c4": dict(desc="Lion, bf16 moment, Qwen2.5-1.5B parameter list",
               shapes=lambda: qwen_like(151936, 1536, 8960, 28, 256),
               algo="lion", precision="bf16", lr=3e-6, betas=(0.9, 0.99), wd=0.1, gscale=(1e-6, 1e-2)),
}


def min_bytes(precision: str, algo: str, grad_bytes: int = 2, out_bytes: int = 2) -> float:
    """Minimum bytes per parameter: master read+write, gradient, moments read+write, output
    (reference benchmarks/bench_kernels.py:63-65)."""
    mv = {"fp32": 4, "bf16": 2, "fp8": 1 + 4 / 128}[precision]
    return 4 * 2 + grad_bytes + mv * 2 * (1 if algo == "lion" else 2) + out_bytes


# ----------------------------------------------------------------- GPU side

def build(cfg: dict, device, seed: int = 0, layout: str = "auto", double_buffer: bool = False):
    import torch
    import adambridge_amd as ab

    gen = torch.Generator(device=device).manual_seed(seed)
    lo, hi = cfg["gscale"]
    params, grads = [], []
    for k, (_, shape) in enumerate(cfg["shapes"]()):
        p = torch.nn.Parameter(torch.randn(shape, generator=gen, device=device, dtype=torch.bfloat16).mul_(0.02))
        u = (k * 0.6180339887) % 1.0
        scale = math.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))
        g = torch.randn(shape, generator=gen, device=device, dtype=torch.bfloat16).mul_(scale)
        params.append(p)
        grads.append(g)
    kw = dict(lr=cfg["lr"], betas=cfg["betas"], weight_decay=cfg["wd"], precision=cfg["precision"],
              state_layout=layout, double_buffer=double_buffer)
    opt = ab.LionBridge(params, **kw) if cfg["algo"] == "lion" else ab.AdamBridge(params, **kw)
    for p, g in zip(params, grads):
        p.grad = g
    return opt, params


def gpu_bench(cfg: dict, steps: int, warmup: int, layout: str = "auto", double_buffer: bool = False) -> dict:
    import torch

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    opt, params = build(cfg, device, layout=layout, double_buffer=double_buffer)
    n = sum(p.numel() for p in params)
    for _ in range(warmup):
        opt.step()
    torch.cuda.synchronize()
    log: list = []
    opt._engine.launch_log = log
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        opt.step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    opt._engine.launch_log = None
    durs = [a.elapsed_time(b) / 1e3 for a, b, _ in log]
    launches_per_step = len(log) / steps
    bpp = min_bytes(cfg["precision"], cfg["algo"])
    kernel_s = sum(durs) / len(durs)
    elems_per_launch = sum(e for _, _, e in log) / len(log)
    achieved = elems_per_launch * bpp / kernel_s / 1e9
    layouts = sorted({s.state.layout for s in opt._ordered})
    state_layout = ", ".join(layouts) + (" (double-buffered)" if double_buffer else "")
    stats = dict(params=n, tensors=len(params), wall=wall, launches_per_step=launches_per_step, layout=state_layout,
                 state_bytes=opt.memory_report()["total"],
                 kernel_ms=kernel_s * 1e3, kernel_ms_min=min(durs) * 1e3, kernel_ms_max=max(durs) * 1e3,
                 achieved_gbs=achieved, bytes_per_param=bpp)
    opt.close()
    del opt, params
    torch.cuda.empty_cache()
    return stats


def calibrate_copy(nbytes: int) -> None:
    """Three copies of ``nbytes`` between two device buffers: under rocprofv3 --pmc, the copy kernel's
    FETCH_SIZE and WRITE_SIZE readings against ``nbytes`` give the counters' scale factors."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[bench] calibration: 3 copies of {nbytes} bytes", file=sys.stderr, flush=True)
    del src, dst
    torch.cuda.empty_cache()


# ------------------------------------------------------- hooked pipeline (c5)

PIPELINE = dict(layers=24, hidden=2048, inter=8192, batch=8, seq=512, lr=1e-4, wd=0.01)


def pipeline_model(device):
    """24 x [Linear(2048 -> 8192) + GELU + Linear(8192 -> 2048)] with a residual, bf16: 805,552,128
    parameters (48 weight matrices with a hook each, 48 biases batched at step_sync)."""
    import torch

    class Block(torch.nn.Module):
        def __init__(self, h, i):
            super().__init__()
            self.up = torch.nn.Linear(h, i)
            self.down = torch.nn.Linear(i, h)

        def forward(self, x):
            return x + self.down(torch.nn.functional.gelu(self.up(x)))

    torch.manual_seed(0)
    c = PIPELINE
    return torch.nn.Sequential(*[Block(c["hidden"], c["inter"]) for _ in range(c["layers"])]).to(
        device=device, dtype=torch.bfloat16)


def pipeline_bench(steps: int, warmup: int) -> dict:
    """Training-step wall time of the c5 stack with: no optimizer (the floor), torch's fused AdamW,
    AdamBridge.step() after backward, attach_hooks + step_sync, and attach_hooks + delay_updates;
    plus, for the hooked runs, the GPU time of the updates and the exposed tail (last gradient ready
    -> last update done), from the side stream's events."""
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

    def timed(step, stats_of=None):
        times, upd, tail, bwd = [], [], [], []
        for i in range(warmup + steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            st = step()
            torch.cuda.synchronize()
            if i >= warmup:
                times.append(time.perf_counter() - t0)
                if st is not None:
                    upd.append(st.gpu_update or 0.0)
                    tail.append(st.exposed_tail or 0.0)
                    bwd.append(st.gpu_backward or 0.0)
        out = dict(step_ms=statistics.median(times) * 1e3)
        if upd:
            out.update(gpu_update_ms=statistics.median(upd) * 1e3, exposed_tail_ms=statistics.median(tail) * 1e3,
                       gpu_backward_ms=statistics.median(bwd) * 1e3)
        return out

    results = {}
    model = pipeline_model(device)
    n = sum(p.numel() for p in model.parameters())

    def floor():
        loss_of(model).backward()
        for p in model.parameters():
            p.grad = None
    results["fwd+bwd only"] = timed(floor)

    opt = torch.optim.AdamW(model.parameters(), lr=c["lr"], weight_decay=c["wd"], fused=True)

    def torch_step():
        loss_of(model).backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
    results["torch.optim.AdamW(fused=True), bf16 state, no master"] = timed(torch_step)
    del opt
    torch.cuda.empty_cache()

    for name, hooks, delay in (("AdamBridge bf16 step()", False, False),
                               ("AdamBridge bf16 attach_hooks + step_sync", True, False),
                               ("AdamBridge bf16 attach_hooks + delay_updates", True, True)):
        model = pipeline_model(device)
        opt = ab.AdamBridge(model.parameters(), lr=c["lr"], weight_decay=c["wd"], precision="bf16",
                            delay_updates=delay)
        opt._engine.timing = hooks
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
        results[name] = timed(step)
        opt.close()
        del opt, model
        torch.cuda.empty_cache()
    return dict(params=n, results=results)


# ----------------------------------------------------------------- CPU side

def cpu_bench(cfg: dict, budget_params: int, steps: int) -> dict:
    """The reference's native kernel (oracle/_ref, compiled from its C source) over the first tensors
    of the same list, up to ``budget_params`` parameters, on this host's CPU share.  Where that
    library was not built (no reference tree at build time), the oracle's C restatement of the same
    algorithm (oracle/liboracle.so, OpenMP) is timed instead and reported as kind "port"."""
    import ctypes

    import numpy as np
    from oracle import oracle as O

    use_ref = O.reference_available()
    lib = O.load_reference() if use_ref else O.load_oracle()
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(16, cores))
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
    for k, (name, numel) in enumerate(shapes):
        p = np.resize(pat_p, numel)
        g = np.resize(pat_g, numel)
        out = np.empty(numel, np.uint16)
        if mv_dt == O.DT_FP8:
            nb = -(-numel // 128)
            m, v = np.zeros(nb * 128, np.uint8), np.zeros(nb * 128, np.uint8)
            ms, vs = np.ones(nb, np.float32), np.ones(nb, np.float32)
        else:
            dt = np.float32 if mv_dt == O.DT_F32 else np.uint16
            m, v, ms, vs = np.zeros(numel, dt), np.zeros(numel, dt), None, None
        arrs = dict(p=p, g=g, m=m, v=None if lion else v, m_scale=ms, v_scale=None if lion else vs, out=out)
        keep.append(arrs)
        seg = O.Segment(p=p.ctypes.data, g=g.ctypes.data, m=m.ctypes.data,
                        v=None if lion else v.ctypes.data, m_scale=None if ms is None else ms.ctypes.data,
                        v_scale=None if (lion or vs is None) else vs.ctypes.data, out=out.ctypes.data,
                        group=ctypes.pointer(group), n=numel, step=1, index=k, offset=0, g_dtype=O.DT_BF16,
                        mv_dtype=mv_dt, out_dtype=O.DT_BF16, algorithm=1 if lion else 0, p_dtype=O.DT_F32)
        segs.append(seg)
    arr = (ctypes.POINTER(O.Segment) * len(segs))(*[ctypes.pointer(s) for s in segs])
    if use_ref:
        lib.adambridge_set_simd_level(-1)
        level = lib.adambridge_simd_level()
        pool = lib.adambridge_pool_create(threads, None, 0)
        run = lambda: lib.adambridge_multi_step(pool, arr, len(segs), threads)  # noqa: E731
        what = f"reference native kernel (oracle/_ref, compiled from adambridge_kernels.c, SIMD level {level})"
    else:
        pool = None
        run = lambda: lib.abo_multi_step(arr, len(segs), 16, threads)  # noqa: E731
        what = "oracle C restatement of the reference kernel (oracle/liboracle.so, scalar C, OpenMP)"
    try:
        def one(step):
            for s in segs:
                s.step = step
            rc = run()
            if rc:
                raise RuntimeError(f"CPU multi_step returned {rc}")
        one(1)
        times = []
        for k in range(steps):
            t0 = time.perf_counter()
            one(k + 2)
            times.append(time.perf_counter() - t0)
    finally:
        if pool:
            lib.adambridge_pool_destroy(pool)
    times.sort()
    med = times[len(times) // 2]
    bpp = min_bytes(cfg["precision"], cfg["algo"])
    return dict(value=total / med, unit="params/s", cores=threads, kind="reference" if use_ref else "port",
                sample=(f"{what} on the first {len(shapes)} tensors of the same list ({total:,} params), "
                        f"median of {steps} steps after 1 warm-up, {threads} threads"),
                ms_per_step=med * 1e3, gbs=total * bpp / med / 1e9)


# --------------------------------------------------------------------- main

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3p", choices=sorted(CONFIGS) + ["c5"],
                    help="c5: the hooked training pipeline (prints its own JSON line)")
    ap.add_argument("--cpu-params", type=int, default=1 << 30, help="CPU baseline sample size (parameters)")
    ap.add_argument("--cpu-steps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--layout", default="auto", choices=["auto", "packed", "separate"],
                    help="optimizer state layout in HBM (AdamBridge state_layout)")
    ap.add_argument("--double-buffer", action="store_true", help="AdamBridge double_buffer=True")
    ap.add_argument("--traffic", type=float, default=None,
                    help="HBM bytes per launch measured by rocprofv3 (FETCH_SIZE+WRITE_SIZE, scaled); "
                         "default: the figure measured for this configuration, when there is one")
    ap.add_argument("--rebuilds", type=int, default=1, metavar="N",
                    help="diagnostic: build and time the state N times in this process, printing each "
                         "on stderr (the GPU's power state can change between them); the JSON line "
                         "reports the first")
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
    if args.config == "c5":
        return main_pipeline(args)
    cfg = CONFIGS[args.config]
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
    print(f"[bench] config {args.config}: {cfg['desc']}; warmup {args.warmup}, steps {args.steps}",
          file=sys.stderr, flush=True)
    g = gpu_bench(cfg, args.steps, args.warmup, args.layout, args.double_buffer)
    print(f"[bench] GPU: {g['kernel_ms']:.3f} ms/launch, {g['achieved_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    for k in range(1, args.rebuilds):
        r = gpu_bench(cfg, args.steps, args.warmup, args.layout, args.double_buffer)
        print(f"[bench] rebuild {k}: {r['kernel_ms']:.3f} ms/launch, {r['achieved_gbs']:.0f} GB/s", file=sys.stderr,
              flush=True)
    cpu = None if args.no_cpu else cpu_bench(cfg, args.cpu_params, args.cpu_steps)
    if cpu is not None:
        print(f"[bench] CPU reference: {cpu['ms_per_step']:.1f} ms/step on {cpu['cores']} threads",
              file=sys.stderr, flush=True)
    ms_per_step = g["wall"] / args.steps * 1e3
    line = {
        "metric": METRIC if args.config == "c3p" else
        f"params updated/sec and achieved HBM GB/s (% roofline), {cfg['desc']} ({args.config})",
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
        "data": "synthetic (bf16 weights ~N(0,0.02), bf16 grads ~N(0,1) x log-uniform per-tensor scale)",
        "config": {"workload": cfg["desc"], "config": args.config, "params": g["params"], "tensors": g["tensors"],
                   "moments": cfg["precision"], "master": "fp32", "grad": "bf16", "out": "bf16",
                   "bytes_per_param": g["bytes_per_param"], "launches_per_step": g["launches_per_step"],
                   "state_layout": g["layout"], "state_bytes": g["state_bytes"],
                   "wall_gbs": g["params"] * g["bytes_per_param"] / (ms_per_step / 1e3) / 1e9},
        "roofline": {"bound": "hbm", "achieved": g["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": g["achieved_gbs"] / HBM_PEAK_GBS,
                     "traffic": args.traffic if args.traffic is not None else MEASURED_TRAFFIC.get(args.config),
                     "kernel_ms": g["kernel_ms"]},
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
    }
    print(json.dumps(line), flush=True)
    return 0


def main_pipeline(args) -> int:
    c = PIPELINE
    print(f"[bench] c5: {c['layers']}-layer bf16 MLP {c['hidden']}->{c['inter']}->{c['hidden']}, "
          f"{c['batch']}x{c['seq']} tokens; warmup {args.warmup}, steps {args.steps}", file=sys.stderr, flush=True)
    r = pipeline_bench(args.steps, args.warmup)
    for name, v in r["results"].items():
        print(f"[bench] {name:<48} " + ", ".join(f"{k} {x:.2f}" for k, x in v.items()), file=sys.stderr, flush=True)
    hooked = r["results"]["AdamBridge bf16 attach_hooks + step_sync"]
    line = {
        "metric": "training step wall time, 24-layer bf16 MLP, hooked bf16-moment AdamW (c5)",
        "value": hooked["step_ms"], "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": hooked["step_ms"], "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 model, f32 update", "data": "synthetic (N(0,1) tokens and targets, seed 0)",
        "config": {"workload": "c5 hooked pipeline", "params": r["params"], "tokens": c["batch"] * c["seq"],
                   "bytes_per_param": 20, "runs": r["results"]},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
