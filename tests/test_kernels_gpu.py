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


def test_graph_capture_inline_launches_and_staged_table_refusal():
    """Under stream capture: a call of at most 7 segments (descriptors in the kernel arguments) is
    captured, and every replay applies the update again -- each checked against the oracle on the
    previous state, with eager work and synchronisations between replays; a call of 8 segments of
    one variant, whose launch would stage its table through a reused host slot, returns -22
    before enqueueing anything."""
    from hip_cases import Prepared
    rng = np.random.default_rng(15)
    seven = [O.make_case(rng, 3000 + 100 * k, mv_dtype=MVS[k % 3], index=k) for k in range(7)]
    eight = [O.make_case(rng, 1000, mv_dtype=O.DT_BF16, index=k) for k in range(8)]
    run_hip(seven, 16)   # eager first: the default launch queue exists before the capture
    small, large = Prepared(seven), Prepared(eight)
    before = large.collect()
    graph = torch.cuda.CUDAGraph()
    side = torch.zeros(1024, device="cuda")
    with torch.cuda.graph(graph):
        small.call()
        with pytest.raises(RuntimeError, match="code -22"):
            large.call()
        side.add_(1.0)
    torch.cuda.synchronize()
    for w, g in zip(before, large.collect()):
        check(w, g)   # the refused call changed nothing
    state = small.collect()   # capturing ran nothing
    for w, g in zip(seven, state):
        check(w, g)
    for replay in range(3):
        graph.replay()
        torch.cuda.synchronize()
        want = O.run_many(state, "oracle", 16)
        state = small.collect()
        for w, g in zip(want, state):
            check(w, g)
        side.mul_(0.5)   # eager work on the same tensors' stream between replays
        torch.cuda.synchronize()


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


# ------------------------------------------------------ interleaved state layout

from hip_cases import run_hip_packed  # noqa: E402


@pytest.mark.parametrize("double_buffer", [False, True])
def test_packed_layout_matches_oracle(double_buffer):
    """ADAMBRIDGE_DT_PACKED (master + BF16 moments interleaved) gives the separate layout's bytes:
    odd sizes, tails of every reproduced ISA, offsets, SR on/off, every grad/out dtype."""
    rng = np.random.default_rng(21)
    cases = []
    for gt, ot, sr, n in itertools.product([O.DT_BF16, O.DT_F32], [O.DT_NONE, O.DT_F32, O.DT_BF16], [True, False],
                                           [1, 2, 15, 16, 17, 33, 1000, 2048 + 77, 5001]):
        cases.append(O.make_case(rng, n, mv_dtype=O.DT_BF16, p_dtype=O.DT_F32, g_dtype=gt, out_dtype=ot,
                                 stochastic=sr, offset=int(rng.integers(0, 2**32)), index=int(rng.integers(0, 999)),
                                 step=int(rng.integers(1, 30))))
    for width in (16, 8, 0):
        want = O.run_many(cases, "oracle", width)
        got = run_hip_packed(cases, width, double_buffer=double_buffer)
        for w, g in zip(want, got):
            check(w, g)


def test_packed_layout_misaligned_gradient_and_specials():
    rng = np.random.default_rng(22)
    cases = [O.make_case(rng, n, mv_dtype=O.DT_BF16, special=sp) for n in (999, 4096) for sp in (False, True)]
    want = O.run_many(cases, "oracle", 16)
    got = run_hip_packed(cases, 16, misalign_g=True)
    for w, g, c in zip(want, got, cases):
        bad = O.outputs_equal(w, g, nan_equiv=True)
        assert not bad, bad


def test_packed_layout_multi_step_groups():
    rng = np.random.default_rng(23)
    cases = [O.make_case(rng, 3000 + 7 * k, mv_dtype=O.DT_BF16, explicit=False, index=k, step=k + 2, seed=3)
             for k in range(12)]
    want = O.run_many(cases, "oracle", 16)
    got = run_hip_packed(cases, 16)
    for w, g in zip(want, got):
        check(w, g)


def test_packed_layout_rejects_bad_segments():
    rng = np.random.default_rng(24)
    lion = O.make_case(rng, 100, mv_dtype=O.DT_BF16)
    lion.algorithm = O.LION
    with pytest.raises(RuntimeError, match=r"code -12"):
        run_hip_packed_unchecked(lion)


def run_hip_packed_unchecked(case):
    """One packed segment with whatever algorithm the case names (validation test)."""
    import ctypes
    from adambridge_amd import _hip
    from hip_cases import pack_state, to_device
    k = _hip.load()
    state = torch.from_numpy(pack_state(case).view(np.int32)).cuda()
    g = to_device(case.arrays["g"])
    seg = _hip.Segment(p=state.data_ptr(), g=g.data_ptr(), n=case.n, step=1, mv_dtype=O.DT_BF16,
                       g_dtype=case.g_dtype, out_dtype=0, algorithm=case.algorithm, p_dtype=_hip.DT_PACKED)
    hp = _hip.HParams(**{kk: case.hparams[kk] for kk, _ in _hip.HParams._fields_})
    k.multi_apply(None, k.segment_array([ctypes.pointer(seg)]), [hp])


# ------------------------------------------------------ FP8 block-record layout

from hip_cases import run_hip_records  # noqa: E402


# (algorithm, master): ADAMBRIDGE_DT_PACKED_FP8, ADAMBRIDGE_DT_PACKED_FP8_F24, ADAMBRIDGE_DT_PACKED_LION_FP8
RECORD_KINDS = [(O.ADAMW, O.DT_F32), (O.ADAMW, O.DT_F24), (O.LION, O.DT_F32), (O.LION, O.DT_F24)]
RECORD_IDS = ["adamw-f32", "adamw-f24", "lion-f32", "lion-f24"]   # the last: ADAMBRIDGE_DT_PACKED_LION_FP8_F24


@pytest.mark.parametrize("algo,pt", RECORD_KINDS, ids=RECORD_IDS)
def test_fp8_records_match_oracle(algo, pt):
    """ADAMBRIDGE_DT_PACKED_FP8 (FP32 master and both FP8 moments in 768-byte block records),
    ADAMBRIDGE_DT_PACKED_FP8_F24 (FP24 master planes and codes in 640-byte records) and
    ADAMBRIDGE_DT_PACKED_LION_FP8 (Lion: FP32 master and m codes in 640-byte records) give the
    separate layout's bytes: ragged and block-aligned sizes, tails of every reproduced ISA,
    128-aligned offsets, SR on/off, every grad/out dtype; an FP24 or Lion record's padding masters
    stay as they were."""
    rng = np.random.default_rng(31 + pt + 7 * algo)
    cases = []
    for gt, ot, sr, n in itertools.product([O.DT_BF16, O.DT_F32], [O.DT_NONE, O.DT_F32, O.DT_BF16], [True, False],
                                           [1, 15, 127, 128, 129, 1000, 2048 + 77, 16384 + 300]):
        cases.append(O.make_case(rng, n, algorithm=algo, mv_dtype=O.DT_FP8, p_dtype=pt, g_dtype=gt, out_dtype=ot,
                                 stochastic=sr, offset=128 * int(rng.integers(0, 2**24)),
                                 index=int(rng.integers(0, 999)), step=int(rng.integers(1, 30))))
    for width in (16, 8, 0):
        want = O.run_many(cases, "oracle", width)
        padding = []
        got = run_hip_records(cases, width, padding=padding)
        for w, g in zip(want, got):
            check(w, g)
        for pad in padding:
            if algo == O.LION and pt == O.DT_F32:
                assert np.all(pad == 0x7F8A5A5A), "a Lion record's padding master was written"
            else:
                hi, lo = pad
                assert np.all(hi == 0xA5A5) and np.all(lo == 0x5A), "an FP24 record's padding master was written"


@pytest.mark.parametrize("algo,pt", RECORD_KINDS, ids=RECORD_IDS)
def test_fp8_records_misaligned_gradient_and_specials(algo, pt):
    rng = np.random.default_rng(32 + pt + 7 * algo)
    cases = [O.make_case(rng, n, algorithm=algo, mv_dtype=O.DT_FP8, p_dtype=pt, special=sp)
             for n in (999, 4096) for sp in (False, True)]
    want = O.run_many(cases, "oracle", 16)
    got = run_hip_records(cases, 16, misalign_g=True)
    for w, g in zip(want, got):
        bad = O.outputs_equal(w, g, nan_equiv=True)
        assert not bad, bad


@pytest.mark.parametrize("algo,pt", RECORD_KINDS, ids=RECORD_IDS)
def test_fp8_records_multi_step_groups_and_steps(algo, pt):
    """Several segments per call through the group path, then three consecutive steps of one."""
    rng = np.random.default_rng(33 + pt + 7 * algo)
    cases = [O.make_case(rng, 3000 + 128 * k + 7, algorithm=algo, mv_dtype=O.DT_FP8, p_dtype=pt, explicit=False,
                         index=k, step=k + 2, seed=3) for k in range(12)]
    want = O.run_many(cases, "oracle", 16)
    got = run_hip_records(cases, 16)
    for w, g in zip(want, got):
        check(w, g)
    case = O.make_case(rng, 5000, algorithm=algo, mv_dtype=O.DT_FP8, p_dtype=pt)
    grads = [O.make_case(rng, 5000, mv_dtype=O.DT_FP8).arrays["g"] for _ in range(3)]
    check(run_steps(case, grads, oracle_runner, 16), run_steps(case, grads, run_hip_records, 16))


@pytest.mark.parametrize("layout", ["fp8-records", "fp8-f24-records", "lion-fp8-records", "lion-fp8-f24-records"])
def test_fp8_records_reject_bad_segments(layout):
    """The other algorithm (-12), a second state buffer (-13), BF16 moments (-4) and a misaligned
    record (-14)."""
    import ctypes
    from adambridge_amd import _hip
    rng = np.random.default_rng(34)
    k = _hip.load()
    case = O.make_case(rng, 300, mv_dtype=O.DT_FP8)
    rec = torch.zeros(3 * 768 + 16, dtype=torch.uint8, device="cuda")
    g = torch.zeros(300, dtype=torch.bfloat16, device="cuda")
    sc = torch.ones(3, dtype=torch.float32, device="cuda")
    hp = _hip.HParams(**{kk: case.hparams[kk] for kk, _ in _hip.HParams._fields_})
    pt = {"fp8-records": _hip.DT_PACKED8, "fp8-f24-records": _hip.DT_PACKED8_F24,
          "lion-fp8-records": _hip.DT_PACKED8_LION, "lion-fp8-f24-records": _hip.DT_PACKED8_LION_F24}[layout]
    algo = 1 if layout.startswith("lion") else 0
    base = dict(p=rec.data_ptr(), g=g.data_ptr(), m_scale=sc.data_ptr(), v_scale=sc.data_ptr(), n=300, step=1,
                mv_dtype=O.DT_FP8, g_dtype=O.DT_BF16, out_dtype=0, algorithm=algo, p_dtype=pt)
    for change, code in ((dict(algorithm=1 - algo), -12), (dict(p_lo=rec.data_ptr()), -13),
                         (dict(mv_dtype=O.DT_BF16), -4), (dict(p=rec.data_ptr() + 8), -14)):
        seg = _hip.Segment(**{**base, **change})
        with pytest.raises(RuntimeError, match=rf"code {code}"):
            k.multi_apply(None, k.segment_array([ctypes.pointer(seg)]), [hp])
    assert torch.count_nonzero(rec).item() == 0   # nothing ran


# ------------------------------------------------------------ Lion record layout

from hip_cases import run_hip_lion_records  # noqa: E402


@pytest.mark.parametrize("double_buffer", [False, True])
def test_lion_records_match_oracle(double_buffer):
    """ADAMBRIDGE_DT_PACKED_LION (master + BF16 m in 1536-byte records) gives the separate layout's
    bytes: sizes around the record and the lane's 4 elements, offsets, SR on/off, every grad/out dtype;
    in place, the padding slots of the last record keep their bits."""
    rng = np.random.default_rng(41)
    cases = []
    for gt, ot, sr, n in itertools.product([O.DT_BF16, O.DT_F32], [O.DT_NONE, O.DT_F32, O.DT_BF16], [True, False],
                                           [1, 2, 3, 5, 255, 256, 257, 1000, 2048 + 77, 5001]):
        cases.append(O.make_case(rng, n, algorithm=O.LION, mv_dtype=O.DT_BF16, g_dtype=gt, out_dtype=ot,
                                 stochastic=sr, offset=int(rng.integers(0, 2**32)), index=int(rng.integers(0, 999)),
                                 step=int(rng.integers(1, 30)), lr=1e-4, betas=(0.9, 0.99), weight_decay=0.1))
    want = O.run_many(cases, "oracle", 16)
    pads: list = []
    got = run_hip_lion_records(cases, 16, double_buffer=double_buffer, padding=pads)
    for w, g in zip(want, got):
        check(w, g)
    if not double_buffer:
        for (pp, pm), c in zip(pads, cases):
            assert (pp == 0x7FA5A5A5).all() and (pm == 0xA5A5).all(), f"padding changed at n={c.n}"


def test_lion_records_zero_gradients_misaligned_and_specials():
    """Exact-zero gradients at 1% (sign(0) = 0, kernels.c:1107-1124), gradients shifted by one
    element (off the vector path's alignment: the element-wise path) and by two, and non-finite
    inputs."""
    rng = np.random.default_rng(42)
    cases = []
    for n, sp in ((999, False), (4096, False), (4096, True), (5001, True)):
        c = O.make_case(rng, n, algorithm=O.LION, mv_dtype=O.DT_BF16, special=sp, lr=3e-6, betas=(0.9, 0.99),
                        weight_decay=0.1)
        if not sp:
            zero = rng.random(n) < 0.01
            c.arrays["g"][zero] = 0
            c.arrays["m"][zero] = 0   # c = 0 exactly where m and g are both zero: u = 0
            assert zero.any()
        cases.append(c)
    want = O.run_many(cases, "oracle", 16)
    for shift in (1, 2):
        got = run_hip_lion_records(cases, 16, misalign_g=shift)
        for w, g in zip(want, got):
            bad = O.outputs_equal(w, g, nan_equiv=True)
            assert not bad, (shift, bad)


def test_lion_records_multi_step_groups_and_steps():
    """Several segments per call through the group path, then three consecutive steps of one."""
    rng = np.random.default_rng(43)
    cases = [O.make_case(rng, 3000 + 64 * k + 3, algorithm=O.LION, mv_dtype=O.DT_BF16, explicit=False, index=k,
                         step=k + 2, seed=5) for k in range(12)]
    want = O.run_many(cases, "oracle", 16)
    got = run_hip_lion_records(cases, 16)
    for w, g in zip(want, got):
        check(w, g)
    case = O.make_case(rng, 5000, algorithm=O.LION, mv_dtype=O.DT_BF16)
    grads = [O.make_case(rng, 5000, algorithm=O.LION, mv_dtype=O.DT_BF16).arrays["g"] for _ in range(3)]
    check(run_steps(case, grads, oracle_runner, 16), run_steps(case, grads, run_hip_lion_records, 16))


def test_lion_records_reject_bad_segments():
    """AdamW (-12), FP8 moments (-4) and misaligned records (-14), before anything runs."""
    import ctypes
    from adambridge_amd import _hip
    rng = np.random.default_rng(44)
    k = _hip.load()
    case = O.make_case(rng, 300, algorithm=O.LION, mv_dtype=O.DT_BF16)
    rec = torch.zeros(2 * 1536 + 16, dtype=torch.uint8, device="cuda")
    g = torch.zeros(300, dtype=torch.bfloat16, device="cuda")
    hp = _hip.HParams(**{kk: case.hparams[kk] for kk, _ in _hip.HParams._fields_})
    base = dict(p=rec.data_ptr(), g=g.data_ptr(), n=300, step=1, mv_dtype=O.DT_BF16, g_dtype=O.DT_BF16,
                out_dtype=0, algorithm=1, p_dtype=_hip.DT_PACKED_LION)
    for change, code in ((dict(algorithm=0), -12), (dict(mv_dtype=O.DT_FP8), -4), (dict(p=rec.data_ptr() + 8), -14),
                         (dict(p_lo=rec.data_ptr() + 4), -14)):
        seg = _hip.Segment(**{**base, **change})
        with pytest.raises(RuntimeError, match=rf"code {code}"):
            k.multi_apply(None, k.segment_array([ctypes.pointer(seg)]), [hp])
    assert torch.count_nonzero(rec).item() == 0   # nothing ran


# ------------------------------------------------ FP32-moment AdamW records

from hip_cases import run_hip_f24_records, run_hip_f32_records  # noqa: E402


@pytest.mark.parametrize("double_buffer", [False, True])
def test_f32_records_match_oracle(double_buffer):
    """ADAMBRIDGE_DT_PACKED_F32 (master, m and v FP32 in 3072-byte records) gives the separate
    layout's bytes: sizes around the record, the lane's 4 elements and the reproduced SIMD widths'
    tails (fused body, unfused scalar tail at widths 16, 8 and 0), offsets, every grad/out dtype; in
    place, the padding slots of the last record keep their bits."""
    rng = np.random.default_rng(51)
    cases = []
    for gt, ot, n in itertools.product([O.DT_BF16, O.DT_F32], [O.DT_NONE, O.DT_F32, O.DT_BF16],
                                       [1, 2, 3, 4, 5, 15, 16, 17, 255, 256, 257, 1000, 2048 + 77, 5001]):
        cases.append(O.make_case(rng, n, mv_dtype=O.DT_F32, g_dtype=gt, out_dtype=ot,
                                 stochastic=bool(rng.integers(0, 2)), offset=int(rng.integers(0, 2**32)),
                                 index=int(rng.integers(0, 999)), step=int(rng.integers(1, 30))))
    for width in (16, 8, 0):
        want = O.run_many(cases, "oracle", width)
        pads: list = []
        got = run_hip_f32_records(cases, width, double_buffer=double_buffer, padding=pads)
        for w, g in zip(want, got):
            check(w, g)
        if not double_buffer:
            for pad, c in zip(pads, cases):
                for k, col in enumerate(pad):
                    assert (col == 0x7FA5A5A5 + k).all(), f"padding changed at n={c.n}"


def test_f32_records_misaligned_gradient_and_specials():
    """Gradients shifted by one element (the element-wise path) and by two, and non-finite inputs
    (zeros, subnormals, infinities, NaNs in every input)."""
    rng = np.random.default_rng(52)
    cases = [O.make_case(rng, n, mv_dtype=O.DT_F32, special=sp) for n, sp in
             ((999, False), (4096, False), (4096, True), (5001, True))]
    want = O.run_many(cases, "oracle", 16)
    for shift in (1, 2):
        got = run_hip_f32_records(cases, 16, misalign_g=shift)
        for w, g in zip(want, got):
            bad = O.outputs_equal(w, g, nan_equiv=True)
            assert not bad, (shift, bad)


def test_f32_records_multi_step_groups_and_steps():
    """Several segments per call through the group path, then three consecutive steps of one."""
    rng = np.random.default_rng(53)
    cases = [O.make_case(rng, 3000 + 64 * k + 3, mv_dtype=O.DT_F32, explicit=False, index=k, step=k + 2, seed=5)
             for k in range(12)]
    want = O.run_many(cases, "oracle", 16)
    got = run_hip_f32_records(cases, 16)
    for w, g in zip(want, got):
        check(w, g)
    case = O.make_case(rng, 5000, mv_dtype=O.DT_F32)
    grads = [O.make_case(rng, 5000, mv_dtype=O.DT_F32).arrays["g"] for _ in range(3)]
    check(run_steps(case, grads, oracle_runner, 16), run_steps(case, grads, run_hip_f32_records, 16))


# (algorithm, moments) of the FP24-master records: ADAMBRIDGE_DT_PACKED_F24, _LION_F24, _F24_F32
F24_KINDS = [(O.ADAMW, O.DT_BF16), (O.LION, O.DT_BF16), (O.ADAMW, O.DT_F32), (O.LION, O.DT_F32)]
F24_IDS = ["adamw-bf16", "lion-bf16", "adamw-f32", "lion-f32"]


@pytest.mark.parametrize("algo,mv", F24_KINDS, ids=F24_IDS)
@pytest.mark.parametrize("double_buffer", [False, True])
def test_f24_records_match_oracle(double_buffer, algo, mv):
    """ADAMBRIDGE_DT_PACKED_F24 (FP24 master planes and BF16 m, v in 1792-byte records), its Lion form
    and ADAMBRIDGE_DT_PACKED_F24_F32 (FP32 m, v in 2816-byte records) give the separate FP24 layout's
    bytes: sizes around the record and the lane's 4 elements, the reproduced SIMD widths' tails,
    offsets, stochastic and nearest rounding, every grad/out dtype, delayed (previous-weight)
    output; in place, the padding slots of the last record keep their bits."""
    from hip_cases import _f24_columns
    rng = np.random.default_rng(61 + algo + 5 * (mv == O.DT_F32))   # ADAMBRIDGE_DT_PACKED_LION_F24_F32 too
    cases = []
    for gt, ot, n in itertools.product([O.DT_BF16, O.DT_F32], [O.DT_NONE, O.DT_F32, O.DT_BF16],
                                       [1, 2, 3, 4, 5, 15, 16, 17, 255, 256, 257, 1000, 2048 + 77, 5001]):
        cases.append(O.make_case(rng, n, algorithm=algo, mv_dtype=mv, p_dtype=O.DT_F24, g_dtype=gt,
                                 out_dtype=ot,
                                 stochastic=bool(rng.integers(0, 2)), offset=int(rng.integers(0, 2**32)),
                                 index=int(rng.integers(0, 999)), step=int(rng.integers(1, 30))))
    for width in (16, 8, 0):
        want = O.run_many(cases, "oracle", width)
        pads: list = []
        got = run_hip_f24_records(cases, width, double_buffer=double_buffer, padding=pads)
        for w, g in zip(want, got):
            check(w, g)
        if not double_buffer:
            for pad, c in zip(pads, cases):
                for col, (_, _, _, fill) in zip(pad, _f24_columns(c)[0]):
                    assert (col == fill).all(), f"padding changed at n={c.n}"


@pytest.mark.parametrize("algo,mv", F24_KINDS, ids=F24_IDS)
def test_f24_records_misaligned_gradient_specials_and_steps(algo, mv):
    """Gradients shifted by one element and by two, non-finite inputs, several segments through the
    group path, and three consecutive steps of one segment."""
    rng = np.random.default_rng(62 + algo + 5 * (mv == O.DT_F32))
    cases = [O.make_case(rng, n, algorithm=algo, mv_dtype=mv, p_dtype=O.DT_F24, special=sp, stochastic=sr)
             for n, sp, sr in ((999, False, True), (4096, False, False), (4096, True, True), (5001, True, False))]
    want = O.run_many(cases, "oracle", 16)
    for shift in (1, 2):
        got = run_hip_f24_records(cases, 16, misalign_g=shift)
        for w, g in zip(want, got):
            bad = O.outputs_equal(w, g, nan_equiv=True)
            assert not bad, (shift, bad)
    cases = [O.make_case(rng, 3000 + 64 * k + 3, algorithm=algo, mv_dtype=mv, p_dtype=O.DT_F24,
                         explicit=False, index=k, step=k + 2, seed=5) for k in range(12)]
    for w, g in zip(O.run_many(cases, "oracle", 16), run_hip_f24_records(cases, 16)):
        check(w, g)
    case = O.make_case(rng, 5000, algorithm=algo, mv_dtype=mv, p_dtype=O.DT_F24)
    grads = [O.make_case(rng, 5000, mv_dtype=mv).arrays["g"] for _ in range(3)]
    check(run_steps(case, grads, oracle_runner, 16), run_steps(case, grads, run_hip_f24_records, 16))


@pytest.mark.parametrize("layout", ["f32-records", "f24-f32-records"])
def test_f32_records_reject_bad_segments(layout):
    """Lion (-12), BF16 moments (-4), a missing gradient (-2) and misaligned records (-14), before
    anything runs."""
    import ctypes
    from adambridge_amd import _hip
    rng = np.random.default_rng(54)
    k = _hip.load()
    case = O.make_case(rng, 300, mv_dtype=O.DT_F32)
    rec = torch.zeros(2 * 3072 + 16, dtype=torch.uint8, device="cuda")
    g = torch.zeros(300, dtype=torch.bfloat16, device="cuda")
    hp = _hip.HParams(**{kk: case.hparams[kk] for kk, _ in _hip.HParams._fields_})
    pt = _hip.DT_PACKED_F32 if layout == "f32-records" else _hip.DT_PACKED_F24_F32
    base = dict(p=rec.data_ptr(), g=g.data_ptr(), n=300, step=1, mv_dtype=O.DT_F32, g_dtype=O.DT_BF16,
                out_dtype=0, algorithm=0, p_dtype=pt)
    for change, code in ((dict(algorithm=1), -12), (dict(mv_dtype=O.DT_BF16), -4), (dict(g=None), -2),
                         (dict(p=rec.data_ptr() + 8), -14), (dict(p_lo=rec.data_ptr() + 4), -14)):
        seg = _hip.Segment(**{**base, **change})
        with pytest.raises(RuntimeError, match=rf"code {code}"):
            k.multi_apply(None, k.segment_array([ctypes.pointer(seg)]), [hp])
    assert torch.count_nonzero(rec).item() == 0   # nothing ran


# ------------------------------------------------ Lion FP32-moment records

from hip_cases import run_hip_lion_f32_records  # noqa: E402


@pytest.mark.parametrize("double_buffer", [False, True])
def test_lion_f32_records_match_oracle(double_buffer):
    """ADAMBRIDGE_DT_PACKED_LION_F32 (master and m FP32 in 2048-byte records) gives the separate
    layout's bytes: sizes around the record and the lane's 4 elements, offsets, every grad/out dtype
    (Lion fuses every element, so no tail forms); in place, the padding slots of the last record keep
    their bits."""
    rng = np.random.default_rng(61)
    cases = []
    for gt, ot, n in itertools.product([O.DT_BF16, O.DT_F32], [O.DT_NONE, O.DT_F32, O.DT_BF16],
                                       [1, 2, 3, 4, 5, 15, 16, 17, 255, 256, 257, 1000, 2048 + 77, 5001]):
        cases.append(O.make_case(rng, n, algorithm=O.LION, mv_dtype=O.DT_F32, g_dtype=gt, out_dtype=ot,
                                 stochastic=bool(rng.integers(0, 2)), offset=int(rng.integers(0, 2**32)),
                                 index=int(rng.integers(0, 999)), step=int(rng.integers(1, 30))))
    want = O.run_many(cases, "oracle", 16)
    pads: list = []
    got = run_hip_lion_f32_records(cases, 16, double_buffer=double_buffer, padding=pads)
    for w, g in zip(want, got):
        check(w, g)
    if not double_buffer:
        for pad, c in zip(pads, cases):
            for k, col in enumerate(pad):
                assert (col == 0x7FA5A5A5 + k).all(), f"padding changed at n={c.n}"


def test_lion_f32_records_zero_gradients_misaligned_and_specials():
    """Exact zero gradients (sign(0) = 0), gradients shifted by one element (the element-wise path)
    and by two, and non-finite inputs (zeros, subnormals, infinities, NaNs in every input)."""
    rng = np.random.default_rng(62)
    cases = [O.make_case(rng, n, algorithm=O.LION, mv_dtype=O.DT_F32, special=sp) for n, sp in
             ((999, False), (4096, False), (4096, True), (5001, True))]
    cases[1].arrays["g"][::3] = 0
    want = O.run_many(cases, "oracle", 16)
    for shift in (0, 1, 2):
        got = run_hip_lion_f32_records(cases, 16, misalign_g=shift)
        for w, g in zip(want, got):
            bad = O.outputs_equal(w, g, nan_equiv=True)
            assert not bad, (shift, bad)


def test_lion_f32_records_multi_step_groups_and_steps():
    """Several segments per call through the group path, then three consecutive steps of one."""
    rng = np.random.default_rng(63)
    cases = [O.make_case(rng, n, algorithm=O.LION, mv_dtype=O.DT_F32, explicit=False, index=i, step=2 + i)
             for i, n in enumerate([700, 4096, 5001])]
    for w, g in zip(O.run_many(cases, "oracle", 16), run_hip_lion_f32_records(cases, 16)):
        check(w, g)
    case = O.make_case(rng, 3000, algorithm=O.LION, mv_dtype=O.DT_F32, explicit=False)
    grads = [O.make_case(rng, 3000, mv_dtype=O.DT_F32).arrays["g"] for _ in range(3)]
    check(run_steps(case, grads, oracle_runner, 16), run_steps(case, grads, run_hip_lion_f32_records, 16))


def test_lion_f32_records_reject_bad_segments():
    """AdamW (-12), a BF16 moment (-4), a missing gradient (-2) and misaligned records (-14), before
    anything runs."""
    import ctypes
    from adambridge_amd import _hip
    rng = np.random.default_rng(64)
    k = _hip.load()
    case = O.make_case(rng, 300, algorithm=O.LION, mv_dtype=O.DT_F32)
    rec = torch.zeros(2 * 2048 + 16, dtype=torch.uint8, device="cuda")
    g = torch.zeros(300, dtype=torch.bfloat16, device="cuda")
    hp = _hip.HParams(**{kk: case.hparams[kk] for kk, _ in _hip.HParams._fields_})
    base = dict(p=rec.data_ptr(), g=g.data_ptr(), n=300, step=1, mv_dtype=O.DT_F32, g_dtype=O.DT_BF16,
                out_dtype=0, algorithm=1, p_dtype=_hip.DT_PACKED_LION_F32)
    for change, code in ((dict(algorithm=0), -12), (dict(mv_dtype=O.DT_BF16), -4), (dict(g=None), -2),
                         (dict(p=rec.data_ptr() + 8), -14), (dict(p_lo=rec.data_ptr() + 4), -14)):
        seg = _hip.Segment(**{**base, **change})
        with pytest.raises(RuntimeError, match=rf"code {code}"):
            k.multi_apply(None, k.segment_array([ctypes.pointer(seg)]), [hp])
    assert torch.count_nonzero(rec).item() == 0   # nothing ran


# ------------------------------------------------ fused_adamw, pools, streams

@pytest.mark.parametrize("mv", [O.DT_F32, O.DT_BF16])
@pytest.mark.parametrize("gt", [O.DT_BF16, O.DT_F32])
@pytest.mark.parametrize("ot", [O.DT_NONE, O.DT_F32, O.DT_BF16])
def test_fused_adamw_updates_a_subrange_like_the_oracle(mv, gt, ot):
    """adambridge_fused_adamw (kernels.c:1518-1535) through HipKernels.fused_adamw: elements
    [lo, hi) of flat tensors, rounding streams at offset lo, the rest untouched."""
    from adambridge_amd import _hip
    from hip_cases import to_device, from_device
    k = _hip.load()
    rng = np.random.default_rng(40 + mv * 10 + gt * 3 + ot)
    n, lo, hi = 10007, 384, 10007 - 5
    whole = O.make_case(rng, n, mv_dtype=mv, g_dtype=gt, out_dtype=ot, stochastic=True)
    dev = {key: to_device(a) for key, a in whole.arrays.items()}
    as_t = lambda key, dt: dev[key].view(dt)  # noqa: E731
    f32, bf16 = torch.float32, torch.bfloat16
    mdt = f32 if mv == O.DT_F32 else bf16
    out = None if ot == O.DT_NONE else as_t("out", f32 if ot == O.DT_F32 else bf16)
    hp = _hip.HParams(**{f: whole.hparams[f] for f, _ in _hip.HParams._fields_})
    k.fused_adamw(as_t("p", f32), as_t("g", f32 if gt == O.DT_F32 else bf16), as_t("m", mdt), as_t("v", mdt),
                  out, hp, lo, hi)
    part = whole.copy()
    part.n, part.offset = hi - lo, lo
    part.arrays = {key: a[lo:hi].copy() for key, a in whole.arrays.items()}
    want = O.run(part, "oracle", 16)
    for key, a in whole.arrays.items():
        got = from_device(dev[key], a)
        assert np.array_equal(got[:lo].view(np.uint8), a[:lo].view(np.uint8)), key
        assert np.array_equal(got[hi:].view(np.uint8), a[hi:].view(np.uint8)), key
        assert np.array_equal(got[lo:hi].view(np.uint8), want.arrays[key].view(np.uint8)), key


def test_fused_adamw_python_checks():
    from adambridge_amd import _hip
    k = _hip.load()
    hp = _hip.HParams(0.9, 0.999, 0.1, 0.001, 1.0, 1e-3, 1.0, 1e-8, 7, 1)
    t = lambda n, dt=torch.float32: torch.zeros(n, dtype=dt, device="cuda")  # noqa: E731
    with pytest.raises(ValueError):
        k.fused_adamw(t(8), t(7), t(8), t(8), None, hp, 0, 8)
    with pytest.raises(TypeError):
        k.fused_adamw(t(8, torch.bfloat16), t(8), t(8), t(8), None, hp, 0, 8)
    with pytest.raises(TypeError):
        k.fused_adamw(t(8), t(8), t(8), t(8, torch.bfloat16), None, hp, 0, 8)
    with pytest.raises(IndexError):
        k.fused_adamw(t(8), t(8), t(8), t(8), None, hp, 4, 9)
    with pytest.raises(ValueError):
        k.fused_adamw(t(8), torch.zeros(8), t(8), t(8), None, hp, 0, 8)


def test_pools_on_two_streams_from_two_threads():
    """Two launch queues bound to two streams, driven from two host threads at once (the GIL is
    released in the C calls): each gets the oracle's bytes; pool_threads reports the CUs."""
    import ctypes
    import threading
    from adambridge_amd import _hip
    from hip_cases import hip_segment, to_device, from_device
    k = _hip.load()
    rng = np.random.default_rng(50)
    sets = [[O.make_case(rng, int(rng.integers(1000, 300000)), mv_dtype=MVS[(i + j) % 3], index=10 * i + j,
                         offset=128 * j) for j in range(9)] for i in range(2)]
    want = [O.run_many(cs, "oracle", 16) for cs in sets]
    pools = [k.create_pool() for _ in range(2)]
    streams = [torch.cuda.Stream() for _ in range(2)]
    try:
        assert k.pool_threads(pools[0]) == torch.cuda.get_device_properties(0).multi_processor_count
        dev = [[{key: to_device(a) for key, a in c.arrays.items()} for c in cs] for cs in sets]
        torch.cuda.synchronize()
        errors = []

        def work(i):
            try:
                k.set_pool_stream(pools[i], streams[i])
                segs = [hip_segment(c, t, None) for c, t in zip(sets[i], dev[i])]
                hps = [_hip.HParams(**{f: c.hparams[f] for f, _ in _hip.HParams._fields_}) for c in sets[i]]
                k.multi_apply(pools[i], k.segment_array([ctypes.pointer(s) for s in segs]), hps)
                k.pool_sync(pools[i])
            except Exception as exc:  # noqa: BLE001 -- reported by the main thread
                errors.append(exc)

        threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
        for th in threads:
            th.start()
        for th in threads:
            th.join()
        assert not errors, errors
        for i in range(2):
            for c, t, w in zip(sets[i], dev[i], want[i]):
                got = c.copy()
                got.arrays = {key: from_device(t[key], a) for key, a in c.arrays.items()}
                check(w, got)
    finally:
        for p in pools:
            k.destroy_pool(p)


_LARGER_FP8_TILE = r"""
import itertools, sys
import numpy as np
sys.path[:0] = sys.argv[1:3]
from oracle import oracle as O
from hip_cases import run_hip, run_hip_records
rng = np.random.default_rng(41)
cases = [O.make_case(rng, n, algorithm=algo, mv_dtype=O.DT_FP8, p_dtype=pt, stochastic=sr,
                     offset=128 * int(rng.integers(0, 2**20)), index=int(rng.integers(0, 999)), step=3)
         for algo, pt, sr, n in itertools.product([O.ADAMW, O.LION], [O.DT_F32, O.DT_F24], [True, False],
                                                  [129, 4096 + 77, 3 * 4096, 20000 + 5])]
records = cases   # every combination has its block records
bad = 0
for runner, subset in ((run_hip, cases), (run_hip_records, records)):
    for w, g in zip(O.run_many(subset, "oracle", 16), runner(subset, 16)):
        diff = O.outputs_equal(w, g)
        if diff:
            print("differ:", w.n, w.algorithm, w.p_dtype, diff, flush=True)
            bad += 1
print("cases", len(cases) + len(records), "bad", bad, flush=True)
sys.exit(1 if bad else 0)
"""


@pytest.mark.parametrize("tile", [4096, 8192])
def test_fp8_larger_tile_matches_oracle(tile):
    """The FP8 kernel's loop over several blocks per 16-lane group, taken only when
    ADAMBRIDGE_TILE_FP8 asks for a tile above 2048 elements (read once per process, hence a child
    process): separate and block-record layouts, AdamW and Lion, FP32 and FP24 masters; 2 and 4
    passes per tile, with partial passes and blocks at the segments' ends."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    env = dict(os.environ, ADAMBRIDGE_TILE_FP8=str(tile))
    print(f"child process: ADAMBRIDGE_TILE_FP8={tile}", flush=True)
    run = subprocess.run([sys.executable, "-c", _LARGER_FP8_TILE, str(root), str(root / "tests")], env=env,
                         capture_output=True, text=True, timeout=110)
    print(run.stdout, flush=True)
    assert run.returncode == 0, run.stdout + run.stderr[-3000:]


def _previous_weight(case):
    """The working weight of the case's master as it is before the update: what
    ADAMBRIDGE_SEG_OUT_PREVIOUS writes to out (kernels.c:108-112 for a bf16 out)."""
    p = case.arrays["p"]
    old = O.f24_value(p, case.arrays["p_lo"]) if case.p_dtype == O.DT_F24 else p.view(np.float32)
    return O.bf16_bits(old) if case.out_dtype == O.DT_BF16 else old.astype(np.float32)


@pytest.mark.parametrize("layout", ["separate", "pairs", "fp8-records", "lion-records", "f32-records", "f24-records",
                                    "lion-f24-records", "fp8-f24-records", "lion-f32-records", "lion-fp8-records",
                                    "f24-f32-records", "lion-f24-f32-records", "lion-fp8-f24-records"])
def test_out_previous_writes_the_weight_from_before_the_update(layout):
    """ADAMBRIDGE_SEG_OUT_PREVIOUS (delayed updates): out receives the weight of the master as stored
    before the update -- FP32, or bf16 by the kernels' rounding of FP32 and decoded FP24 masters,
    NaN masters included -- and the state is updated exactly as without the flag."""
    from hip_cases import (run_hip_f24_records, run_hip_f32_records, run_hip_lion_f32_records, run_hip_lion_records,
                           run_hip_packed, run_hip_records)
    from adambridge_amd import _hip

    rng = np.random.default_rng(31 + len(layout) + (layout == "f24-records"))
    combos = {"separate": [(a, mv, pt) for a in ALGOS for mv in MVS for pt in PTS],
              "pairs": [(O.ADAMW, O.DT_BF16, O.DT_F32)], "fp8-records": [(O.ADAMW, O.DT_FP8, O.DT_F32)],
              "lion-records": [(O.LION, O.DT_BF16, O.DT_F32)], "f32-records": [(O.ADAMW, O.DT_F32, O.DT_F32)],
              "f24-records": [(O.ADAMW, O.DT_BF16, O.DT_F24)], "lion-f24-records": [(O.LION, O.DT_BF16, O.DT_F24)],
              "fp8-f24-records": [(O.ADAMW, O.DT_FP8, O.DT_F24)],
              "lion-f32-records": [(O.LION, O.DT_F32, O.DT_F32)], "lion-fp8-records": [(O.LION, O.DT_FP8, O.DT_F32)],
              "f24-f32-records": [(O.ADAMW, O.DT_F32, O.DT_F24)],
              "lion-f24-f32-records": [(O.LION, O.DT_F32, O.DT_F24)],
              "lion-fp8-f24-records": [(O.LION, O.DT_FP8, O.DT_F24)]}[layout]
    runner = {"separate": run_hip, "pairs": run_hip_packed, "fp8-records": run_hip_records,
              "lion-records": run_hip_lion_records, "f32-records": run_hip_f32_records,
              "f24-records": run_hip_f24_records, "lion-f24-records": run_hip_f24_records,
              "fp8-f24-records": run_hip_records, "lion-f32-records": run_hip_lion_f32_records,
              "lion-fp8-records": run_hip_records, "f24-f32-records": run_hip_f24_records,
              "lion-f24-f32-records": run_hip_f24_records, "lion-fp8-f24-records": run_hip_records}[layout]
    cases = []
    for (algo, mv, pt), gt, ot, sr, n in itertools.product(combos, [O.DT_BF16, O.DT_F32], [O.DT_F32, O.DT_BF16],
                                                             [True, False], [1, 15, 17, 129, 1000, 8192 + 77]):
        off = int(rng.integers(0, 50)) * 128 if mv == O.DT_FP8 else int(rng.integers(0, 2**32))
        cases.append(O.make_case(rng, n, algorithm=algo, mv_dtype=mv, p_dtype=pt, g_dtype=gt, out_dtype=ot,
                                 stochastic=sr, offset=off, index=int(rng.integers(0, 1000)),
                                 step=int(rng.integers(1, 50))))
    regular = len(cases)
    cases += [O.make_case(rng, 3000, algorithm=algo, mv_dtype=mv, p_dtype=pt, special=True)
              for algo, mv, pt in combos]   # zeros, subnormals, infinities and NaNs in every input
    want = O.run_many(cases, "oracle", 16)
    got = runner(cases, 16, seg_flags=_hip.SEG_OUT_PREVIOUS)
    for i, (c, w, g) in enumerate(zip(cases, want, got)):
        prev = _previous_weight(c)
        assert np.array_equal(g.arrays["out"].view(np.uint8), prev.view(np.uint8)), \
            f"{layout}: case {i} (n={c.n}, out_dtype={c.out_dtype}): out is not the weight from before the update"
        w.arrays["out"] = prev
        check(w, g, special=i >= regular)


def test_stream_copy_copies_exactly():
    """adambridge_stream_copy, the counter-calibration copy: every byte, sizes around its 4 KiB tile."""
    from adambridge_amd import _hip
    k = _hip.load()
    g = torch.Generator(device="cuda").manual_seed(3)
    for nbytes in (16, 4096 - 16, 4096, 3 * 4096 + 48, 1 << 24):
        src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=g)
        dst = torch.zeros_like(src)
        k.stream_copy(src, dst)
        torch.cuda.synchronize()
        assert torch.equal(src, dst), nbytes


def test_stream_copy_beyond_one_launch():
    """A copy of more than 64 GiB goes out as two launches; each byte lands once, the ragged end too."""
    from adambridge_amd import _hip
    k = _hip.load()
    torch.cuda.empty_cache()
    nbytes = (64 << 30) + 4096 + 48
    src = torch.empty(nbytes // 8, dtype=torch.int64, device="cuda")
    torch.arange(src.numel(), out=src)
    src.mul_(0x5851F42D4C957F2D)   # wraps: every 8-byte word differs
    dst = torch.zeros_like(src)
    try:
        k.stream_copy(src, dst)
        torch.cuda.synchronize()
        assert torch.equal(src, dst)
    finally:
        del src, dst
        torch.cuda.empty_cache()


def test_recycle_device_memory_holds_nothing_and_clears_its_error():
    """adambridge_recycle_device_memory allocates and frees at once; an allocation the device cannot
    make is reported, holds nothing and leaves no HIP error behind for the next launch check."""
    from adambridge_amd import _hip

    k = _hip.load()
    dev = torch.device("cuda", 0)
    free0 = torch.cuda.mem_get_info(dev)[0]
    assert k.recycle_device_memory(1 << 30, dev)
    assert not k.recycle_device_memory(1 << 50, dev)   # 1 PiB: more than the device has
    assert "recycle" in k.last_error()
    x = torch.arange(1 << 20, device=dev, dtype=torch.float32).mul_(2.0)   # launches and checks succeed
    torch.cuda.synchronize()
    assert float(x[-1]) == 2.0 * ((1 << 20) - 1)
    assert abs(torch.cuda.mem_get_info(dev)[0] - free0) < (256 << 20)
