"""The hooked pipeline at its real size (BASELINE config c5) on the GPU.

The 24-layer bf16 MLP of the pipeline benchmark -- LayerNorm, 2048 -> 8192 -> 2048
with GELU and biases, 805,650,432 parameters, batch 8 x 512 tokens, MSE to seeded
targets (reference benchmarks/bench_pipeline.py:20-35, 58-128) -- trained with
AdamBridge(precision='bf16').attach_hooks(), with and without delay_updates, with the
updates in order on the compute stream (the default) and on a side stream:

* every element of every parameter's update is bit-exact against the oracle:
  the state before the step and the gradient the hook saw go through the
  oracle's multi_step with the same index and step number;
* exact mode: the weights are the bf16 of the new master at step_sync; delayed
  mode: they are one step stale -- the previous update's output -- until the
  next step's hooks or flush() write the newer one (test_cuda.py:129-177);
* StepStats carries the overlap measurements the reference asserts
  (test_cuda.py:351-365): gpu_backward > 0, gpu_update > 0 and
  0 <= exposed_tail < gpu_update.
"""

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import adambridge_amd as ab
from oracle import oracle as O

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
import bench  # noqa: E402

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _windows(numel: int) -> list[tuple[int, int]]:
    return [(0, numel)]   # every element


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.float32:
        return t.numpy().copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def _state_arrays(slot, lo: int, hi: int) -> dict:
    return {k: _bits(v) for k, v in slot.state.window(lo, hi).items()}


@pytest.mark.parametrize("stream,delay", [("current", False), ("current", True), ("side", False)])
def test_c5_hooked_pipeline_matches_oracle_and_reports_overlap(stream, delay):
    c = bench.PIPELINE
    torch.cuda.set_device(DEV)
    model = bench.pipeline_model(DEV)
    assert sum(p.numel() for p in model.parameters()) == 805_650_432
    gen = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(c["batch"] * c["seq"], c["hidden"], generator=gen, device=DEV, dtype=torch.bfloat16)
    target = torch.randn(x.shape, generator=gen, device=DEV, dtype=torch.bfloat16)
    params = list(model.parameters())

    # the gradients each step's updates read, copied by a hook that runs before the optimizer's
    grads: dict[int, list[torch.Tensor]] = {}

    def capture(p):
        k = index_of[id(p)]
        grads[k] = [p.grad.detach().reshape(-1)[lo:hi].clone() for lo, hi in _windows(p.numel())]

    index_of = {id(p): k for k, p in enumerate(params)}
    for p in params:
        p.register_post_accumulate_grad_hook(capture)
    opt = ab.AdamBridge(params, lr=c["lr"], weight_decay=c["wd"], precision="bf16", delay_updates=delay,
                        autotune=True, update_stream=stream)   # autotune: StepStats timing on
    opt.attach_hooks(model)
    group = opt.param_groups[0]
    ogroup = {"lr": group["lr"], "beta1": group["betas"][0], "beta2": group["betas"][1], "eps": group["eps"],
              "weight_decay": group["weight_decay"], "seed": 0, "stochastic": 1}

    def train_step():
        torch.nn.functional.mse_loss(model(x).float(), target.float()).backward()
        return opt.step_sync()

    try:
        train_step()   # the first step builds the state
        torch.cuda.synchronize()
        previous_out = None
        for step in range(2):
            before = {s.index: [_state_arrays(s, lo, hi) for lo, hi in _windows(s.numel)] for s in opt._ordered}
            grads.clear()
            stats = train_step()
            torch.cuda.synchronize()
            assert len(grads) == len(params) and stats.num_updates == len(params)
            # StepStats (engine.py:340-349; reference test_cuda.py:351-365)
            assert stats.gpu_backward is not None and stats.gpu_backward > 0
            assert stats.gpu_update is not None and stats.gpu_update > 0
            assert stats.exposed_tail is not None and 0 <= stats.exposed_tail < stats.gpu_update
            cases, where = [], []
            for slot in opt._ordered:
                for w, (lo, hi) in enumerate(_windows(slot.numel)):
                    arrays = dict(before[slot.index][w])
                    arrays["g"] = _bits(grads[slot.index][w])
                    arrays["out"] = np.zeros(hi - lo, np.uint16)
                    case = O.Case(n=hi - lo, algorithm=O.ADAMW, mv_dtype=O.DT_BF16, p_dtype=O.DT_F32,
                                  g_dtype=O.DT_BF16, out_dtype=O.DT_BF16, offset=lo, index=slot.index,
                                  step=slot.step, arrays=arrays)
                    case.group = dict(ogroup)
                    cases.append(case)
                    where.append((slot, lo, hi))
            want = O.run_many(cases, "oracle", 16, threads=O.threads_default(), in_place=True)
            outs = []
            for (slot, lo, hi), w in zip(where, want):
                got = _state_arrays(slot, lo, hi)
                for key in ("p", "m", "v"):
                    assert np.array_equal(got[key].view(np.uint8), w.arrays[key].view(np.uint8)), \
                        f"{stream} delay={delay} step {step}: parameter {slot.index} [{lo}, {hi}) {key}"
                weight = _bits(slot.param.reshape(-1)[lo:hi])
                if not delay:
                    assert np.array_equal(weight, w.arrays["out"]), f"parameter {slot.index} weights"
                elif previous_out is not None:   # one step stale: the previous update's weights
                    assert np.array_equal(weight, previous_out[len(outs)]), f"parameter {slot.index} stale weights"
                outs.append(w.arrays["out"])
            previous_out = outs
        if delay:   # flush() writes the newest update into the weights
            opt.flush()
            torch.cuda.synchronize()
            for (slot, lo, hi), out in zip(where, previous_out):
                assert np.array_equal(_bits(slot.param.reshape(-1)[lo:hi]), out)
    finally:
        opt.close()
        del opt, model
        torch.cuda.empty_cache()
