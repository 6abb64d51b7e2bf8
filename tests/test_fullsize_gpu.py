"""Parity at the benchmark configurations' full sizes (GPU).

Each test builds one BASELINE configuration's whole parameter list on the GPU (up to the 7B
Llama list, 291 tensors), runs warm-up steps through ``AdamBridge.step()`` -- one multi-tensor
launch per step -- and then checks one more step two ways:

* sampled windows, bit for bit: before the step, windows of the optimizer state, gradient and
  master are copied out (the first, a middle and the last 128-aligned elements of several
  tensors, and every tensor's first elements); the oracle updates each window as a segment of
  its own with the parameter's index, the step number and the window's element offset -- the
  rounding stream is keyed by (parameter, step, element index), so a window reproduces exactly
  what the whole-tensor launch must write there;
* every element: the bf16 working weight written by the step equals the round-to-nearest-even
  bf16 of the stored master (kernels.c:108-112 applied to the value actually stored).

``test_full_size_every_element`` checks every element of every tensor bit for bit: the state
before the step is cloned on the device, and after the step the oracle updates the clone chunk
by chunk (host memory bounded by one chunk) for comparison with what the launch wrote.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
import bench  # noqa: E402

pytestmark = pytest.mark.gpu

WINDOW = 4096


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def snapshot(opt, slot, lo: int, hi: int) -> dict:
    """The slot's state, gradient and master over elements [lo, hi) as the oracle's arrays, read
    through the state's own view of its layout (ParamState.window)."""
    a: dict[str, np.ndarray] = {}
    for key, t in slot.state.window(lo, hi).items():
        if t.dtype == torch.float32:
            a[key] = t.detach().contiguous().cpu().numpy().copy()
        elif t.element_size() == 2:
            a[key] = _u16(t)
        else:
            a[key] = _u8(t)
    g = slot.param.grad.reshape(-1)[lo:hi]
    a["g"] = _u16(g) if g.dtype == torch.bfloat16 else g.float().cpu().numpy()
    a["out"] = np.zeros(hi - lo, np.uint16)
    return a


def windows(numel: int) -> list[tuple[int, int]]:
    if numel <= 3 * WINDOW:
        return [(0, numel)]
    mid = (numel // 2) // 128 * 128
    last = (numel - WINDOW) // 128 * 128
    return [(0, WINDOW), (mid, mid + WINDOW), (last, numel)]


def run_config(name: str, warm: int | None = None, tensors: int = 6, cfg: dict | None = None,
               windows_of=None, layout: str = "auto") -> None:
    """Build the configuration, run its warm-up steps (the configuration's own count: c1 5, c2 10,
    else 2), then check one more step on sampled windows against the oracle; then check that
    dropping the optimizer and the model freed all of it."""
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    base = torch.cuda.memory_allocated(dev)
    _sampled_parity(name, warm, tensors, cfg, windows_of, layout)
    _check_released(name, base)


def _sampled_parity(name, warm, tensors, cfg, windows_of, layout) -> None:
    cfg = cfg or bench.CONFIGS[name]
    warm = cfg.get("warm_steps", 2) if warm is None else warm
    dev = torch.device("cuda", 0)
    opt, params = bench.build(cfg, dev, layout=layout)
    windows_of = windows_of or windows
    try:
        for t in range(1, warm + 1):   # c1: the gradient of each step regenerated from (seed, step)
            bench.use_step_grads(cfg, params, t)
            opt.step()
        bench.use_step_grads(cfg, params, warm + 1)
        torch.cuda.synchronize()
        if layout == "separate":
            assert all(s.state.layout == "separate" for s in opt._ordered)
        lion = cfg["algo"] == "lion"
        mv = {"fp32": O.DT_F32, "bf16": O.DT_BF16, "fp8": O.DT_FP8}[cfg["precision"]]
        # the largest tensors (first, middle, last windows) and the first window of every tensor
        by_size = sorted(opt._ordered, key=lambda s: -s.numel)[:tensors]
        picks = []
        for slot in opt._ordered:
            for lo, hi in (windows_of(slot.numel) if slot in by_size else [(0, min(slot.numel, 256))]):
                assert 0 <= lo < hi <= slot.numel, (slot.index, lo, hi, slot.numel)
                picks.append((slot, lo, hi))
        group = opt.param_groups[0]
        cases = []
        for slot, lo, hi in picks:
            arrays = snapshot(opt, slot, lo, hi)
            case = O.Case(n=hi - lo, algorithm=O.LION if lion else O.ADAMW, mv_dtype=mv,
                          p_dtype=O.DT_F24 if "p_lo" in arrays else O.DT_F32, g_dtype=O.DT_BF16,
                          out_dtype=O.DT_BF16, offset=lo, index=slot.index, step=slot.step + 1, arrays=arrays)
            case.group = {"lr": group["lr"], "beta1": group["betas"][0], "beta2": group["betas"][1],
                          "eps": group["eps"], "weight_decay": group["weight_decay"], "seed": 0, "stochastic": 1}
            cases.append(case)
        if cfg.get("zeros"):   # c4: exact-zero gradients at 1% density reach the kernel (sign(0) = 0)
            zero_grads = sum(int(np.count_nonzero((c.arrays["g"] & 0x7FFF) == 0)) for c in cases)
            total = sum(c.n for c in cases)
            assert zero_grads > 0.005 * total, f"{zero_grads} zero gradients in {total} sampled elements"
        want = O.run_many(cases, "oracle", 16, threads=O.threads_default())
        opt.step()
        torch.cuda.synchronize()
        for (slot, lo, hi), w, before in zip(picks, want, cases):
            # the step moves the master (every window has nonzero gradients), so equality below
            # compares two updates, not two copies of the old state
            assert not np.array_equal(before.arrays["p"].view(np.uint8), w.arrays["p"].view(np.uint8))
            got = snapshot(opt, slot, lo, hi)
            got["out"] = _u16(slot.param.detach().reshape(-1)[lo:hi])
            for key in ("p", "p_lo", "m", "v", "m_scale", "v_scale", "out"):
                if key in w.arrays:
                    assert np.array_equal(w.arrays[key].view(np.uint8), got[key].view(np.uint8)), \
                        f"{name}: parameter {slot.index} elements [{lo}, {hi}): {key} differs"
        # every element: working weight == bf16 RNE of the stored master
        for slot in opt._ordered:
            master = slot.state.master_fp32()
            assert torch.equal(slot.param.detach().reshape(-1), master.to(torch.bfloat16)), \
                f"{name}: parameter {slot.index}: bf16 weight != RNE(master)"
    finally:
        opt.close()
        del opt, params
        torch.cuda.empty_cache()


def _check_released(name: str, base: int) -> None:
    """The dropped optimizer and model left nothing allocated: reference counting alone frees the
    state arena, the parameters and the gradients (no cycle waits for the garbage collector)."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    left = torch.cuda.memory_allocated() - base
    assert left < 64 << 20, f"{name}: {left / 2**30:.2f} GiB still allocated after the optimizer was dropped"


@pytest.mark.parametrize("name", ["c3p", "c3", "c4", "c2", "c1"])
def test_full_size_config_sampled_parity(name):
    run_config(name)


def _host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    if t.dtype == torch.float32:
        return t.cpu().numpy()
    return _u16(t) if t.element_size() == 2 else _u8(t)


CHUNK = 1 << 28   # elements per oracle call


@pytest.mark.parametrize("name", ["c1", "c2", "c4", "c3p", "c3", "c3p-fp24", "c3-fp24"])
def test_full_size_every_element(name):
    """One step after the configuration's warm-up steps, every element of every tensor against the
    oracle: master (and its low plane), moments, FP8 block scales and the bf16 working weight.
    'c3p-fp24': the 7B list with an FP24 master (FP24-master records); 'c3-fp24': FP8 moments with
    an FP24 master (the reference's separate arrays)."""
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    base = torch.cuda.memory_allocated(dev)
    _every_element(name)
    _check_released(name, base)


def _every_element(name: str) -> None:
    config, _, master = name.partition("-")
    cfg = dict(bench.CONFIGS[config], master=master or "fp32")
    dev = torch.device("cuda", 0)
    opt, params = bench.build(cfg, dev)
    try:
        warm = cfg.get("warm_steps", 2)
        if cfg.get("master_init") == "fp32":   # c1 starts from an FP32 master ~ N(0, 0.02), not bf16 values
            m = opt._ordered[0].state.master_fp32()
            assert torch.any(m != m.to(torch.bfloat16).float()) and abs(float(m.std()) - 0.02) < 1e-3
            del m
        for t in range(1, warm + 1):   # c1: the gradient of each step regenerated from (seed, step)
            bench.use_step_grads(cfg, params, t)
            opt.step()
        bench.use_step_grads(cfg, params, warm + 1)
        torch.cuda.synchronize()
        if master == "fp24":
            want = {"bf16": "f24-records", "fp8": "fp8-f24-records"}.get(cfg["precision"], "separate")
            assert all(s.state.layout == want for s in opt._ordered)
        before = {s.index: {k: v.clone() for k, v in s.state.window(0, s.numel).items()} for s in opt._ordered}
        opt.step()
        torch.cuda.synchronize()
        lion = cfg["algo"] == "lion"
        mv = {"fp32": O.DT_F32, "bf16": O.DT_BF16, "fp8": O.DT_FP8}[cfg["precision"]]
        group = opt.param_groups[0]
        ogroup = {"lr": group["lr"], "beta1": group["betas"][0], "beta2": group["betas"][1], "eps": group["eps"],
                  "weight_decay": group["weight_decay"], "seed": 0, "stochastic": 1}
        slots, checked = list(opt._ordered), 0
        while slots:
            chunk, size = [], 0
            while slots and (not chunk or size + slots[0].numel <= CHUNK):
                chunk.append(slots.pop(0))
                size += chunk[-1].numel
            cases = []
            for slot in chunk:
                arrays = {k: _host(v) for k, v in before.pop(slot.index).items()}
                arrays["g"] = _host(slot.param.grad.reshape(-1))
                arrays["out"] = np.zeros(slot.numel, np.uint16)
                case = O.Case(n=slot.numel, algorithm=O.LION if lion else O.ADAMW, mv_dtype=mv,
                              p_dtype=O.DT_F24 if "p_lo" in arrays else O.DT_F32, g_dtype=O.DT_BF16,
                              out_dtype=O.DT_BF16, offset=0, index=slot.index, step=slot.step, arrays=arrays)
                case.group = dict(ogroup)
                cases.append(case)
            O.run_many(cases, "oracle", 16, threads=O.threads_default(), in_place=True)
            for slot, want in zip(chunk, cases):
                got = {k: _host(v) for k, v in slot.state.window(0, slot.numel).items()}
                got["out"] = _u16(slot.param.detach().reshape(-1))
                for key in ("p", "p_lo", "m", "v", "m_scale", "v_scale", "out"):
                    if key in want.arrays:
                        assert np.array_equal(want.arrays[key].view(np.uint8), got[key].view(np.uint8)), \
                            f"{name}: parameter {slot.index}: {key} differs"
                checked += slot.numel
            del cases
        assert checked == sum(p.numel() for p in params)
    finally:
        opt.close()
        del opt, params
        before = None
        torch.cuda.empty_cache()


@pytest.mark.parametrize("name", ["c3p", "c3", "c4"])
def test_full_size_separate_layout_sampled_parity(name):
    """The reference's separate state arrays at the 7B list and the Lion list (the default keeps
    AdamW's BF16 moments in pairs, its FP8 moments in block records and Lion's moment in records)."""
    run_config(name, layout="separate")


# one tensor past 2^31 elements: 64-bit element indices, and the rounding stream's 32-bit element
# index wrapping (kernels.c:100-106, idx = uint32(i)); every window lies inside it
BIG = (1 << 31) + 3 * WINDOW + 1152


def _big_windows(numel):
    around = (1 << 31) - 2048
    return [(0, WINDOW), (around, around + WINDOW), ((numel - WINDOW) // 128 * 128, numel)]


@pytest.mark.parametrize("precision", ["bf16", "fp8"])
def test_tensor_beyond_2_31_elements(precision):
    cfg = dict(bench.CONFIGS["c3p"], shapes=lambda: [("big", (BIG,)), ("norm", (4096,))], precision=precision)
    run_config(f"2^31+ {precision}", warm=1, tensors=1, cfg=cfg, windows_of=_big_windows)
