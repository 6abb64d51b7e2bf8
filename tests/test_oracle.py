"""Pinning the oracle (CPU): golden vectors, the compiled reference, closed forms.

The oracle (oracle/abh_oracle.c) is what every GPU parity test compares with,
so it is checked here against everything that fixes the reference's results
independently of it:

* the golden vectors written by the reference kernel itself (tests/golden/);
* the reference kernel compiled from its source (oracle/_ref), on fresh random
  cases over every branch, when that library is present;
* closed forms: FP8 encoding = brute-force nearest code (ties to even) with
  every finite code round-tripping; BF16 RNE = torch's cast; lowbias32 and
  splitmix64 from their published constants; the AdamW step against
  torch.optim.AdamW and the Lion step against its definition; unbiased
  stochastic rounding; seeds independent of how a tensor is chunked.
"""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from hip_cases import golden_cases, run_steps


def oracle_runner(cases, width):
    return O.run_many(cases, "oracle", width)


# ------------------------------------------------------------- golden vectors

def test_golden_vectors_bit_exact():
    cases = golden_cases()
    assert len(cases) >= 70
    for meta, case, grads, expect in cases:
        got = run_steps(case, grads, oracle_runner, meta["width"])
        bad = O.outputs_equal(got, expect, nan_equiv=meta["special"])
        assert not bad, f"golden case {meta['desc']!r}: {bad}"


def test_golden_vectors_are_strict_where_finite():
    """Finite golden cases must match without NaN tolerance (the tolerance is only for specials)."""
    for meta, case, grads, expect in golden_cases():
        if meta["special"]:
            continue
        got = run_steps(case, grads, oracle_runner, meta["width"])
        assert not O.outputs_equal(got, expect), meta["desc"]


# ------------------------------------------------------- compiled reference

needs_ref = pytest.mark.skipif(not O.reference_available(), reason="oracle/_ref not built (no reference tree)")


@needs_ref
@pytest.mark.parametrize("algo", [O.ADAMW, O.LION])
@pytest.mark.parametrize("mv", [O.DT_F32, O.DT_BF16, O.DT_FP8])
def test_oracle_matches_reference_library(algo, mv):
    rng = np.random.default_rng(1000 + 10 * algo + mv)
    for pt, gt, ot, sr, special, n, width in itertools.product(
            [O.DT_F32, O.DT_F24], [O.DT_BF16, O.DT_F32], [O.DT_NONE, O.DT_F32, O.DT_BF16], [True, False],
            [False, True], [1, 37, 1000, 4099], [16, 8, 0]):
        off = int(rng.integers(0, 4)) * 128 * 7 if mv == O.DT_FP8 else int(rng.integers(0, 2**32))
        case = O.make_case(rng, n, algorithm=algo, mv_dtype=mv, p_dtype=pt, g_dtype=gt, out_dtype=ot,
                           stochastic=sr, special=special, offset=off, index=int(rng.integers(0, 300)),
                           step=int(rng.integers(1, 20)), explicit=bool(rng.integers(0, 2)))
        a = O.run(case, "oracle", width)
        b = O.run(case, "ref", width)
        assert not O.outputs_equal(a, b, nan_equiv=special), (pt, gt, ot, sr, special, n, width)


@needs_ref
def test_oracle_matches_reference_multithreaded_multi_segment():
    """One multi_step over many segments, the reference on its thread pool."""
    rng = np.random.default_rng(5)
    cases = [O.make_case(rng, int(rng.integers(1, 300000)), mv_dtype=[O.DT_F32, O.DT_BF16, O.DT_FP8][k % 3],
                         explicit=False, index=k, step=3, seed=7) for k in range(12)]
    a = O.run_many(cases, "oracle", 16, threads=4)
    b = O.run_many(cases, "ref", 16, threads=4)
    for x, y in zip(a, b):
        assert not O.outputs_equal(x, y)


# --------------------------------------------------------------- closed forms

def _brute_nearest(table: np.ndarray, x: float) -> int:
    """Nearest finite code of x's sign (magnitude clamped to the max), ties to the even code."""
    sign = 0x80 if (x < 0 or (x == 0 and math.copysign(1.0, x) < 0)) else 0
    a = min(abs(x), float(np.nanmax(np.where(np.isfinite(table[:128]), table[:128], np.nan))))
    best, best_d = 0, math.inf
    for c in range(128):
        v = float(table[c])
        if not math.isfinite(v):
            continue
        d = abs(v - a)
        if d < best_d or (d == best_d and c % 2 == 0):
            best, best_d = c, d
    return sign | best


@pytest.mark.parametrize("role", [0, 1])
def test_fp8_codec_closed_form(role):
    """kernels.c:857-876 against brute force, every finite code round-trips, NaN -> NaN code."""
    lib = O.load_oracle()
    table = O.fp8_decode_table(role)
    for c in range(256):
        if np.isfinite(table[c]):
            assert lib.abo_fp8_encode(float(table[c]), 0, 0, role) == c
    rng = np.random.default_rng(role)
    fmax = 448.0 if role == 0 else 57344.0
    xs = np.concatenate([rng.uniform(-1.1 * fmax, 1.1 * fmax, 3000),
                         rng.normal(0, 1, 3000) * 2.0 ** rng.integers(-20, 6, 3000),
                         (table[np.isfinite(table)][:, None] + table[np.isfinite(table)][None, :]).ravel()[:4000] / 2])
    for x in xs.astype(np.float32):
        assert lib.abo_fp8_encode(float(x), 0, 0, role) == _brute_nearest(table, float(x)), float(x)
    assert lib.abo_fp8_encode(float("nan"), 0, 0, role) == (0x7F if role == 0 else 0x7E)
    assert lib.abo_fp8_encode(-float("nan"), 0, 0, role) == (0xFF if role == 0 else 0xFE)
    assert table[0x80] == 0 and math.copysign(1, table[0x80]) < 0


def test_fp8_decode_matches_torch_float8():
    """Finite codes decode like torch.float8_e4m3fn / float8_e5m2 (precision.py:77-82)."""
    codes = torch.arange(256, dtype=torch.uint8)
    for role, dtype in ((0, torch.float8_e4m3fn), (1, torch.float8_e5m2)):
        mine = torch.from_numpy(O.fp8_decode_table(role))
        theirs = codes.view(dtype).float()
        fin = torch.isfinite(theirs)
        assert torch.equal(mine[fin], theirs[fin])
        assert torch.equal(torch.isnan(mine), torch.isnan(theirs))


def test_bf16_rne_matches_torch_cast():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(0, 1, 100000), rng.normal(0, 1e-30, 1000), [0.0, -0.0, np.inf, -np.inf]])
    x = x.astype(np.float32)
    mine = O.bf16_bits(x)
    lib = O.load_oracle()
    assert all(lib.abo_bf16_rne(int(b)) >> 16 == int(m) for b, m in zip(x.view(np.uint32)[:2000], mine[:2000]))
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine, theirs)


def test_round_values_follows_the_pinned_element_rules():
    """abo_round_values (the whole-array checker of the plane conversion) against the element rules it
    loops over: FP24 nearest = the top 24 bits to nearest even by integer arithmetic on the bits
    (ties to an even byte 1, carries into the exponent, NaN quietened), BF16 nearest = torch's cast
    (finite and infinite values), stochastic = the element's stream bits added before the cut, with
    the stream index wrapping at 2^32."""
    rng = np.random.default_rng(11)
    bits = np.concatenate([rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32),
                           np.array([0, 0x80000000, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x7FC00001, 0x7F800001,
                                     0x3F8000FF, 0x3F800180, 0x3F800080, 0x3F80017F, 0x007FFFFF], np.uint32)])
    exp = (bits >> 23) & 0xFF
    nan = (exp == 0xFF) & ((bits & 0x7FFFFF) != 0)
    keep = bits >> 8
    rnd = (bits & 0xFF) > 0x80
    tie = (bits & 0xFF) == 0x80
    up = (rnd | (tie & ((keep & 1) == 1))).astype(np.uint64)
    near = (((keep.astype(np.uint64) + up) << 8) & 0xFFFFFFFF).astype(np.uint32)
    near = np.where(nan, bits | 0x00400000, near)
    assert np.array_equal(O.round_values(bits, "fp24"), near)
    fin = ~nan
    theirs = torch.from_numpy(bits[fin].view(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.round_values(bits[fin], "bf16"), theirs)
    lib = O.load_oracle()
    seed, offset = 0x1234567, (1 << 32) - 5
    sr24, sr16 = O.round_values(bits[:64], "fp24", seed, offset), O.round_values(bits[:64], "bf16", seed, offset)
    for i, b in enumerate(bits[:64].tolist()):
        r = lib.abo_hash32(((offset + i) & 0xFFFFFFFF) ^ seed)
        if not nan[i]:
            assert int(sr24[i]) == ((b + (r & 0xFF)) & 0xFFFFFFFF) & 0xFFFFFF00
        assert int(sr16[i]) == ((b + (r & 0xFFFF)) & 0xFFFFFFFF) >> 16


def test_hash_and_seed_constants():
    """lowbias32 (kernels.c:100-106) and the splitmix64 seed chain (kernels.c:774-790), restated in Python."""
    lib = O.load_oracle()

    def hash32(x):
        x ^= x >> 16
        x = (x * 0x7FEB352D) & 0xFFFFFFFF
        x ^= x >> 15
        x = (x * 0x846CA68B) & 0xFFFFFFFF
        return x ^ (x >> 16)

    def mix(*vals):
        h = 0x9E3779B97F4A7C15
        for v in vals:
            h = ((h ^ v) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
            h ^= h >> 31
            h = (h * 0x94D049BB133111EB) & (2**64 - 1)
            h ^= h >> 29
        return h

    rng = np.random.default_rng(4)
    for x in [0, 1, 0xFFFFFFFF, *rng.integers(0, 2**32, 200).tolist()]:
        assert lib.abo_hash32(x) == hash32(x)
    assert hash32(0) == 0  # fixed point of the finaliser
    for base, index, step in [(0, 0, 1), (1234, 7, 3), (2**63, 290, 10**6)]:
        assert lib.abo_step_seed(base, index, step) == mix(base, index, step) & 0xFFFFFFFF


def test_adamw_step_matches_torch_adamw():
    """One FP32-moment step against torch.optim.AdamW(foreach=False) (reference test_kernels.py:35-45)."""
    rng = np.random.default_rng(6)
    n = 10007
    case = O.make_case(rng, n, mv_dtype=O.DT_F32, g_dtype=O.DT_F32, out_dtype=O.DT_NONE, explicit=False,
                       lr=1e-3, weight_decay=0.1, step=5, stochastic=False)
    p = torch.nn.Parameter(torch.from_numpy(case.arrays["p"].copy()))
    ref = torch.optim.AdamW([p], lr=1e-3, weight_decay=0.1, foreach=False)
    ref.state[p] = {"step": torch.tensor(4.0), "exp_avg": torch.from_numpy(case.arrays["m"].copy()),
                    "exp_avg_sq": torch.from_numpy(case.arrays["v"].copy())}
    p.grad = torch.from_numpy(case.arrays["g"].copy())
    ref.step()
    got = O.run(case, "oracle", 16)
    torch.testing.assert_close(torch.from_numpy(got.arrays["p"]), p.detach(), rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(torch.from_numpy(got.arrays["m"]), ref.state[p]["exp_avg"], rtol=1e-6, atol=1e-9)
    torch.testing.assert_close(torch.from_numpy(got.arrays["v"]), ref.state[p]["exp_avg_sq"], rtol=1e-6, atol=1e-12)


def test_adamw_fused_and_tail_forms_differ_only_by_rounding():
    """The scalar-tail form (kernels.c:171-176) and the fused form agree to a few ulp, and a
    case exists where they differ: the tail rule is not vacuous."""
    rng = np.random.default_rng(8)
    case = O.make_case(rng, 4096, mv_dtype=O.DT_F32, out_dtype=O.DT_NONE, stochastic=False)
    a = O.run(case, "oracle", 16).arrays["p"]
    b = O.run(case, "oracle", 0).arrays["p"]
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-9)
    assert np.any(a != b)


def test_lion_step_closed_form():
    """c = b1 m + (1-b1) g; p = p (1 - lr wd) - lr sign(c); m = b2 m + (1-b2) g (kernels.c:1093-1124)."""
    rng = np.random.default_rng(9)
    case = O.make_case(rng, 5000, algorithm=O.LION, mv_dtype=O.DT_F32, g_dtype=O.DT_F32, out_dtype=O.DT_NONE,
                       explicit=False, lr=1e-3, betas=(0.9, 0.99), weight_decay=0.1, stochastic=False)
    case.arrays["g"][::97] = 0.0
    case.arrays["m"][::97] = 0.0
    p, g, m = (case.arrays[k].astype(np.float64) for k in ("p", "g", "m"))
    c = 0.9 * m + 0.1 * g
    want_p = p * (1 - 1e-3 * 0.1) - 1e-3 * np.sign(c)
    want_m = 0.99 * m + 0.01 * g
    got = O.run(case, "oracle", 16)
    np.testing.assert_allclose(got.arrays["p"], want_p, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(got.arrays["m"], want_m, rtol=1e-6, atol=1e-12)
    zero = np.nonzero(c == 0)[0]
    assert zero.size and np.allclose(got.arrays["p"][zero], p[zero] * (1 - 1e-4), rtol=1e-6)


@pytest.mark.parametrize("mv", [O.DT_BF16, O.DT_FP8])
def test_stochastic_rounding_is_unbiased(mv):
    """Many draws of the same value (different element indices) average to the value
    (reference selftest.c:149-156; test_precision.py:42-46)."""
    n = 1 << 16
    rng = np.random.default_rng(10)
    case = O.make_case(rng, n, mv_dtype=mv, out_dtype=O.DT_NONE, g_dtype=O.DT_F32, stochastic=True)
    # p unchanged except by decay; m receives (1-b1)*g exactly once from zero
    case.hparams.update(beta1=0.0, one_minus_beta1=1.0, decay=1.0, step_size=0.0)
    x = np.float32(0.1234567)
    case.arrays["g"][:] = x
    case.arrays["m"][:] = 0
    keep = np.ones(n, bool)
    if mv == O.DT_FP8:  # a constant block scales to exactly 448: give each block a larger first element
        case.arrays["g"][::128] = 1.0
        keep[::128] = False
    got = O.run(case, "oracle", 16)
    if mv == O.DT_FP8:
        vals = O.fp8_decode_table(0)[got.arrays["m"][:n]] * np.repeat(got.arrays["m_scale"], 128)[:n]
    else:
        vals = O.bf16_value(got.arrays["m"])
    vals = vals[keep].astype(np.float64)
    assert len(np.unique(vals)) == 2  # the two neighbours
    assert abs(vals.mean() - x) < 4 * vals.std() / math.sqrt(vals.size) + 1e-7


def test_chunked_segments_equal_the_whole_tensor():
    """Pieces with element offsets draw the same rounding bits as the whole tensor
    (kernels.c:757-760; reference selftest.c:304-336)."""
    rng = np.random.default_rng(12)
    for mv in (O.DT_BF16, O.DT_FP8):
        whole = O.make_case(rng, 5 * 1024 + 3, mv_dtype=mv, p_dtype=O.DT_F24, offset=0, index=4)
        a = O.run(whole, "oracle", 16)
        arrays = {k: v.copy() for k, v in whole.arrays.items()}
        pieces = []
        for lo, hi in ((0, 1024), (1024, 3072), (3072, whole.n)):
            c = whole.copy()
            c.n, c.offset = hi - lo, lo
            for k in c.arrays:
                if k.endswith("_scale"):
                    c.arrays[k] = arrays[k][lo // 128:]
                else:  # FP8 codes are padded to whole blocks
                    extra = -(hi - lo) % 128 if (mv == O.DT_FP8 and k in ("m", "v")) else 0
                    c.arrays[k] = arrays[k][lo:hi + extra]
            pieces.append(c)
        O.run_many(pieces, "oracle", 16, in_place=True)
        for k in ("p", "p_lo", "m", "v", "out", "m_scale", "v_scale"):
            if k in arrays:
                assert np.array_equal(arrays[k], a.arrays[k]), (mv, k)


def test_segment_validation_codes():
    """check_segment's codes and order (kernels.c:1537-1553)."""
    lib = O.load_oracle()
    rng = np.random.default_rng(13)
    case = O.make_case(rng, 100, mv_dtype=O.DT_FP8)
    seg = O.segment_for(case)
    assert lib.abo_check_segment(seg, 0) == 0
    assert lib.abo_check_segment(seg, 1) == -8
    seg.offset = 64
    assert lib.abo_check_segment(seg, 0) == -11
    seg.offset = 0
    seg.m_scale = None
    assert lib.abo_check_segment(seg, 0) == -7
    seg.algorithm = 5
    assert lib.abo_check_segment(seg, 0) == -12


@pytest.mark.parametrize("key,short", [("out", 1), ("g", 1), ("p", 7), ("m", 128)])
@pytest.mark.parametrize("impl", ["oracle", "ref"])
def test_undersized_case_buffers_are_refused_before_any_call(key, short, impl, monkeypatch):
    """A case whose host buffer is shorter than its segment needs -- as when a sampled window of a
    full-size test reaches past the end of its tensor and the slices taken from the tensor come out
    short -- is refused by oracle.check_sizes with a ValueError before the C oracle or the compiled
    reference is handed it: either would write its outputs past the numpy buffer's end, corrupting
    the host heap (glibc then aborts the process)."""
    if impl == "ref" and not O.reference_available():
        pytest.skip("the compiled reference (oracle/_ref) is not built")
    rng = np.random.default_rng(5)
    case = O.make_case(rng, 1000, mv_dtype=O.DT_FP8 if key == "m" else O.DT_BF16)
    case.arrays[key] = case.arrays[key][: case.arrays[key].size - short]
    calls = []
    lib = O.load_oracle() if impl == "oracle" else O.load_reference()
    for name in ("abo_multi_apply", "abo_multi_step") if impl == "oracle" else \
            ("adambridge_multi_apply", "adambridge_multi_step"):
        monkeypatch.setattr(lib, name, lambda *a, _n=name: calls.append(_n) or 0, raising=False)
    with pytest.raises(ValueError, match=f"case buffer '{key}' holds"):
        O.run_many([case], impl, 16)
    assert not calls
