"""Run oracle ``Case``s through the HIP library (test helper).

The case's numpy arrays are copied to device tensors, one multi_apply (or
multi_step) call of libadambridge_hip.so updates them on the current stream,
and the results come back as a new Case for comparison with the oracle.
"""

from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np
import torch

from oracle import oracle as O

from adambridge_amd import _hip

GOLDEN = Path(__file__).resolve().parent / "golden"
WIDTH_LEVEL = {16: "avx512", 8: "avx2", 0: "scalar"}


def to_device(a: np.ndarray, device="cuda") -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).to(device)
    return torch.from_numpy(a.copy()).to(device)


def from_device(t: torch.Tensor, like: np.ndarray) -> np.ndarray:
    return t.cpu().numpy().view(like.dtype).reshape(like.shape)


def hip_segment(case: O.Case, tensors: dict, group: _hip.Group | None) -> _hip.Segment:
    ptr = lambda k: tensors[k].data_ptr() if k in tensors else None  # noqa: E731
    return _hip.Segment(p=ptr("p"), p_lo=ptr("p_lo"), g=ptr("g"), m=ptr("m"), v=ptr("v"), m_scale=ptr("m_scale"),
                        v_scale=ptr("v_scale"), out=ptr("out"),
                        group=ctypes.pointer(group) if group is not None else None, n=case.n, step=case.step,
                        index=case.index, offset=case.offset, g_dtype=case.g_dtype, mv_dtype=case.mv_dtype,
                        out_dtype=case.out_dtype, algorithm=case.algorithm, p_dtype=case.p_dtype)


def run_hip(cases: list[O.Case], width: int = 16, pool: int | None = None,
            tensors_hook=None) -> list[O.Case]:
    """Update copies of ``cases`` in one call of the HIP library; returns them.

    ``tensors_hook(i, tensors)`` may replace device tensors before the call (misalignment tests)."""
    kernels = _hip.load()
    work = [c.copy() for c in cases]
    dev = [{k: to_device(a) for k, a in c.arrays.items()} for c in work]
    if tensors_hook is not None:
        for i, t in enumerate(dev):
            tensors_hook(i, t)
    by_group = all(c.group is not None for c in work)
    groups = [_hip.Group(**{k: c.group[k] for k in ("lr", "beta1", "beta2", "eps", "weight_decay")},
                         seed=c.group["seed"] & (2**64 - 1), stochastic=int(c.group["stochastic"]))
              if by_group else None for c in work]
    segs = [hip_segment(c, t, g) for c, t, g in zip(work, dev, groups)]
    arr = kernels.segment_array([ctypes.pointer(s) for s in segs])
    kernels.set_simd_level(WIDTH_LEVEL[width])
    try:
        kernels.set_stream(torch.cuda.current_stream())
        if by_group:
            kernels.multi_step(pool, arr)
        else:
            hps = [_hip.HParams(**{k: c.hparams[k] for k, _ in _hip.HParams._fields_}) for c in work]
            kernels.multi_apply(pool, arr, hps)
        torch.cuda.synchronize()
    finally:
        kernels.set_simd_level(None)
    for c, t in zip(work, dev):
        for k in list(c.arrays):
            if k in t:
                c.arrays[k] = from_device(t[k], c.arrays[k])
    return work


def golden_cases():
    """(meta, input Case, gradients per step, expected Case) for every golden vector."""
    meta = json.loads((GOLDEN / "vectors.json").read_text())
    data = np.load(GOLDEN / "vectors.npz")
    out = []
    for i, m in enumerate(meta):
        arrays = {k.split(".", 2)[2]: data[k] for k in data.files if k.startswith(f"c{i}.in.")}
        expect = {k.split(".", 2)[2]: data[k] for k in data.files if k.startswith(f"c{i}.out.")}
        grads = [data[f"c{i}.g{k}"] for k in range(m["steps"])]
        case = O.Case(n=m["n"], algorithm=m["algorithm"], mv_dtype=m["mv_dtype"], p_dtype=m["p_dtype"],
                      g_dtype=m["g_dtype"], out_dtype=m["out_dtype"], offset=m["offset"], index=m["index"],
                      step=m["step"], arrays=arrays, hparams=m["hparams"], group=m["group"])
        exp = case.copy()
        exp.arrays = expect
        out.append((m, case, grads, exp))
    return out


def run_steps(case: O.Case, grads: list, runner, width: int) -> O.Case:
    """Apply len(grads) consecutive updates with ``runner(cases, width) -> cases``."""
    state = case.copy()
    for g in grads:
        state.arrays["g"] = g.copy()
        state = runner([state], width)[0]
        state.step += 1
    return state
