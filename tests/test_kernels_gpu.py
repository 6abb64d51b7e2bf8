"""Parity of the HIP fused update with the oracle and the golden vectors (GPU).

Every test calls libadambridge_hip.so through its C ABI (adambridge_multi_apply /
adambridge_multi_step) on device copies of seeded inputs and compares the
updated state with the CPU oracle (oracle/abh_oracle.c) on the same inputs:

* finite inputs: bit-exact -- master (FP32 or FP24 planes), moments (FP32 bits,
  BF16 bits, FP8 codes and scales) and the working-weight output;
* non-finite inputs: bit-exact except that any two NaNs count as equal (the
  payload and sign of a NaN produced where NaNs meet or are generated is not
  fixed by IEEE 754 and differs between x86 and AMD GPUs).
"""

import itertools

import numpy as np
import pytest
import torch

from oracle import oracle as O
from hip_cases import golden_cases, run_hip, run_steps

pytestmark = pytest.mark.gpu

ALGOS = [O.ADAMW, O.LION]
MVS = [O.DT_F32, O.DT_BF16, O.DT_FP8]
PTS = [O.DT_F32, O.DT_F24]


def check(a, b, special=False):
    bad = O.outputs_equal(a, b, nan_equiv=special)
    assert not bad, f"arrays differing: {bad}"


def oracle_runner(cases, width):
    return O.run_many(cases, "oracle", width)


def hip_runner(cases, width):
    return run_hip(cases, width)


@pytest.mark.parametrize("algo", ALGOS)
@pytest.mark.parametrize("mv", MVS)
@pytest.mark.parametrize("pt", PTS)
def test_every_storage_combination_matches_oracle(algo, mv, pt):
    """grad F32/BF16 x out NONE/F32/BF16 x SR on/off x sizes around the vector width and FP8 block."""
    rng = np.random.default_rng(algo * 100 + mv * 10 + pt)
    cases = []
    for gt, ot, sr, n in itertools.product([O.DT_BF16, O.DT_F32], [O.DT_NONE, O.DT_F32, O.DT_BF16], [True, False],
                                           [1, 15, 16, 17, 127, 129, 1000, 8192 + 77, 20000]):
        off = int(rng.integers(0, 50)) * 128 if mv == O.DT_FP8 else int(rng.integers(0, 2**32))
        cases.append(O.make_case(rng, n, algorithm=algo, mv_dtype=mv, p_dtype=pt, g_dtype=gt, out_dtype=ot,
                                 stochastic=sr, offset=off, index=int(rng.integers(0, 1000)),
                                 step=int(rng.integers(1, 50))))
    for width in (16, 8, 0):
        want = O.run_many(cases, "oracle", width)
        got = run_hip(cases, width)   # all segments of all variants in one call
        for w, g in zip(want, got):
            check(w, g)


@pytest.mark.parametrize("algo", ALGOS)
@pytest.mark.parametrize("mv", MVS)
def test_non_finite_inputs_match_oracle_up_to_nan_payload(algo, mv):
    rng = np.random.default_rng(7 + algo + 3 * mv)
    cases = [O.make_case(rng, n, algorithm=algo, mv_dtype=mv, p_dtype=pt, special=True, stochastic=sr)
             for n in (700, 5000) for pt in PTS for sr in (True, False)]
    want = O.run_many(cases, "oracle", 16)
    got = run_hip(cases, 16)
    for w, g in zip(want, got):
        check(w, g, special=True)


def test_golden_vectors():
    """Vectors written by the reference kernel itself (tests/golden/make_golden.py)."""
    for meta, case, grads, expect in golden_cases():
        got = run_steps(case, grads, hip_runner, meta["width"])
        bad = O.outputs_equal(got, expect, nan_equiv=meta["special"])
        assert not bad, f"golden case {meta['desc']!r}: {bad}"


def test_multi_step_coefficients_match_multi_apply():
    """Coefficients computed by the library from group + step (kernels.c:793-809) give the
    same bytes as the oracle's, for several parameters and steps in one call."""
    rng = np.random.default_rng(11)
    cases = [O.make_case(rng, 3000 + 128 * k, mv_dtype=MVS[k % 3], explicit=False, index=k, step=k + 1, lr=1e-3 * (k + 1),
                         seed=99, algorithm=ALGOS[k % 2]) for k in range(10)]
    want = O.run_many(cases, "oracle", 16)
    got = run_hip(cases, 16)
    for w, g in zip(want, got):
        check(w, g)


def test_many_segments_use_the_device_table():
    """More segments than fit in the kernel arguments, mixed sizes and variants."""
    rng = np.random.default_rng(12)
    cases = [O.make_case(rng, int(rng.integers(1, 40000)), mv_dtype=MVS[k % 3], p_dtype=PTS[(k // 3) % 2],
                         index=k, offset=128 * int(rng.integers(0, 1000))) for k in range(60)]
    want = O.run_many(cases, "oracle", 16)
    got = run_hip(cases, 16)
    for w, g in zip(want, got):
        check(w, g)


@pytest.mark.parametrize("mv", MVS)
def test_misaligned_buffers_take_the_scalar_path(mv):
    """Device views that start one element into their allocation: no 16-byte access is legal."""
    rng = np.random.default_rng(13)
    cases = [O.make_case(rng, 3000, mv_dtype=mv, p_dtype=pt) for pt in PTS]

    def shift(i, tensors):
        for k, t in list(tensors.items()):
            if k in ("m_scale", "v_scale"):
                continue
            if mv == O.DT_FP8 and k in ("m", "v"):
                buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
            else:
                buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
            buf[1:].copy_(t)
            view = buf[1:]
            tensors[k] = view
            tensors["_keep" + k] = buf

    def run_shifted(cs, width):
        # results come back through from_device(view), which reads the shifted views
        return run_hip(cs, width, tensors_hook=shift)

    want = O.run_many(cases, "oracle", 16)
    got = run_shifted(cases, 16)
    for w, g in zip(want, got):
        check(w, g)


def test_config1_flat_tensor_bit_exact():
    """one flat 16,777,216-element AdamW step with FP32 moments, seed 0,
    master ~ N(0, 0.02), bf16 grad ~ N(0, 1e-3), m, v from 5 seeded warm-up steps, step 6."""
    n = 1 << 24
    rng = np.random.default_rng(0)
    case = O.make_case(rng, n, mv_dtype=O.DT_F32, explicit=False, lr=1e-4, weight_decay=0.01, seed=0)
    case.arrays["m"][:] = 0.0
    case.arrays["v"][:] = 0.0
    grads = [O.bf16_bits((rng.normal(0.0, 1e-3, n)).astype(np.float32)) for _ in range(6)]
    threads = O.threads_default()
    want = run_steps(case, grads, lambda cs, w: O.run_many(cs, "oracle", w, threads=threads), 16)
    got = run_steps(case, grads, hip_runner, 16)
    assert want.step == got.step == 7
    check(want, got)


def test_rejects_bad_segments_before_touching_any():
    """Negative codes in the reference's order (kernels.c:1537-1553); nothing is updated."""
    rng = np.random.default_rng(14)
    good = O.make_case(rng, 1000)
    bad_offset = O.make_case(rng, 1000, mv_dtype=O.DT_FP8, offset=64)
    with pytest.raises(RuntimeError, match=r"code -11"):
        run_hip([good, bad_offset], 16)
    bad_dtype = O.make_case(rng, 1000)
    bad_dtype.g_dtype = 7
    with pytest.raises(RuntimeError, match=r"code -3"):
        run_hip([good, bad_dtype], 16)
