"""gfx950's conversion instructions against the reference's rounding rules, and the FP8 kernel on
moments whose codes mostly go through them (GPU).

The FP8 kernel encodes full blocks with v_cvt_sr_fp8/bf8_f32 (stochastic) or
v_cvt_pk_fp8/bf8_f32 (nearest-even) wherever those give the codes of kernels.c:857-876, and
writes BF16 with v_cvt_pk_bf16_f32 (kernels.c:108-112).  adambridge_check_conversions compares
the instructions with integer forms of the rules over all 2^32 FP32 inputs; the kernel test
drives realistic moments (mostly the instruction path) and ragged ones (mostly the integer path)
through several steps against the oracle.
"""

import numpy as np
import pytest

from adambridge_amd import _hip
from oracle import oracle as O
from hip_cases import run_hip, run_steps

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", [0, 0x2545F491])
def test_conversion_instructions_equal_the_reference_rules(seed):
    counts = _hip.HipKernels().check_conversions(seed)
    assert set(counts) == set(_hip.HipKernels.CONVERSION_CHECKS)
    assert all(v == 0 for v in counts.values()), counts


def _fresh_fp8_case(rng, n, algo, sr):
    """A segment whose FP8 moments start at zero codes (scale 1): after the first step they hold
    the codes of gradient-shaped values, as in training."""
    case = O.make_case(rng, n, algorithm=algo, mv_dtype=O.DT_FP8, stochastic=sr, offset=128 * 3,
                       index=5, step=1)
    for key in ("m", "v"):
        if key in case.arrays:
            case.arrays[key][:] = 0
            case.arrays[key + "_scale"][:] = 1.0
    return case


@pytest.mark.parametrize("algo", [O.ADAMW, O.LION])
@pytest.mark.parametrize("sr", [True, False])
def test_fp8_steps_from_zero_state_match_oracle(algo, sr):
    rng = np.random.default_rng(11 + algo + 2 * sr)
    n = 128 * 96 + 40                      # full blocks and a partial last block
    case = _fresh_fp8_case(rng, n, algo, sr)
    grads = []
    for k in range(4):
        g = (rng.normal(0.0, 1.0, n) * 10.0 ** rng.uniform(-5, -2)).astype(np.float32)
        g[rng.random(n) < 0.002] = 0.0     # a few exact zeros: lanes that take the integer encoder
        grads.append(O.bf16_bits(g))
    want = run_steps(case, grads, lambda cs, w: O.run_many(cs, "oracle", w), 16)
    got = run_steps(case, grads, run_hip, 16)
    bad = O.outputs_equal(want, got, nan_equiv=False)
    assert not bad, f"arrays differing: {bad}"
