"""adambridge_multi_step_noalloc, the entry point that allocates nothing, against
adambridge_multi_step on the same inputs (GPU).

Two calls in a row -- the second smaller, on another stream -- each with more
than 7 segments of some kernel variants, so that their segment tables go through
the library's static device array.  Bit-exact against multi_step's result (and
the oracle's): masters, moments, FP8 codes and scales, outputs.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from hip_cases import Prepared

from adambridge_amd import _hip

pytestmark = pytest.mark.gpu

MVS = [O.DT_F32, O.DT_BF16, O.DT_FP8]
PTS = [O.DT_F32, O.DT_F24]


def mixed_cases(rng, count: int, variants: int, seed: int) -> list[O.Case]:
    """``count`` segments with groups (the multi_step path) over ``variants`` kernel variants."""
    out = []
    for k in range(count):
        v = k % variants
        algo = O.LION if v == 5 else O.ADAMW
        out.append(O.make_case(rng, int(rng.integers(1, 20000)), algorithm=algo, mv_dtype=MVS[v % 3],
                               p_dtype=PTS[(v // 3) % 2], explicit=False, index=k,
                               step=int(rng.integers(1, 50)), offset=128 * int(rng.integers(0, 100)), seed=seed))
    return out


@pytest.mark.parametrize("order", ["noalloc-first", "multi_step-first"])
def test_noalloc_matches_multi_step_on_two_calls(order):
    rng = np.random.default_rng(71)
    kernels = _hip.load()
    side = torch.cuda.Stream()
    # call 1: 200 segments over 6 variants (33-34 each); call 2: 30 over 2 variants (15 each)
    for count, variants, stream in ((200, 6, side), (30, 2, torch.cuda.current_stream())):
        cases = mixed_cases(rng, count, variants, seed=count)
        ref, mine = Prepared(cases), Prepared(cases)
        torch.cuda.synchronize()
        calls = [lambda: ref.call(), lambda: kernels.multi_step_noalloc(stream, mine.arr)]
        if order == "noalloc-first":
            calls.reverse()
        for call in calls:
            call()
        torch.cuda.synchronize()
        want, got = ref.collect(), mine.collect()
        oracle = O.run_many(cases, "oracle", 16)
        for w, g, o in zip(want, got, oracle):
            assert not O.outputs_equal(w, g), f"noalloc differs from multi_step ({count} segments)"
            assert not O.outputs_equal(o, g), f"noalloc differs from the oracle ({count} segments)"


def test_noalloc_call_with_device_tables_replays_from_a_graph():
    """Under stream capture, where a pooled call that needs a segment table is refused (its table
    would come from a reused host slot at replay), the allocation-free call is captured whole: its
    tables are written by kernels whose arguments carry the descriptors.  Each of three replays --
    with eager work and synchronisations between them -- applies the same step again and is checked
    against the oracle on the previous state."""
    from hip_cases import Prepared

    rng = np.random.default_rng(83)
    kernels = _hip.load()
    warm = Prepared(mixed_cases(rng, 12, 1, seed=5))
    kernels.multi_step_noalloc(torch.cuda.current_stream(), warm.arr)   # device array located before capture
    torch.cuda.synchronize()
    cases = mixed_cases(rng, 40, 2, seed=9)   # 20 segments of each of two variants: device tables
    mine = Prepared(cases)
    graph = torch.cuda.CUDAGraph()
    side = torch.zeros(1024, device="cuda")
    with torch.cuda.graph(graph):
        kernels.multi_step_noalloc(torch.cuda.current_stream(), mine.arr)
        side.add_(1.0)
    torch.cuda.synchronize()
    state = mine.collect()   # capturing ran nothing
    for w, g in zip(cases, state):
        assert not O.outputs_equal(w, g), "the capture changed the state"
    for replay in range(3):
        graph.replay()
        torch.cuda.synchronize()
        want = O.run_many(state, "oracle", 16)
        state = mine.collect()
        for w, g in zip(want, state):
            assert not O.outputs_equal(w, g), f"replay {replay} differs from the oracle"
        side.mul_(0.5)   # eager work between replays
        torch.cuda.synchronize()
