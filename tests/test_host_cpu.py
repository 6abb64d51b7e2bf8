"""Host logic on the CPU: storage formats, torch-side encoders, argument and checkpoint validation.

The torch-side encoders (``adambridge_amd.precision``) re-encode moments off the step path:
initial state, ``set_precision()`` and loading a checkpoint of another precision.  Here they are
pinned bit for bit against the oracle's encoders (oracle/abh_oracle.c, which the golden vectors
pin to the reference kernel) on finite inputs, and against the formats' behaviour the reference's
own suite checks (reference tests/test_precision.py:8-160).  Optimizer construction and
checkpoint validation need no device and run here too.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O

import adambridge_amd as ab
from adambridge_amd import formats as F
from adambridge_amd import precision as P


# ------------------------------------------------------------ names and sizes

def test_precision_aliases_and_bytes_per_param():
    assert P.canonical_precision("BF16_Moments") == "bf16"
    assert P.canonical_precision("fp8_moments") == "fp8"
    assert P.canonical_precision("float32") == "fp32"
    for bad in ("int4", "fp16", None):
        with pytest.raises(ValueError):
            P.canonical_precision(bad)
    assert P.canonical_master_precision("FP24") == "fp24"
    with pytest.raises(ValueError):
        P.canonical_master_precision("bf16")
    # master + two moments (precision.py:103-108): 4+8, 4+4, 4+2*(1+4/128); FP24 one byte less
    assert P.bytes_per_param("fp32") == 12
    assert P.bytes_per_param("bf16") == 8
    assert P.bytes_per_param("fp8") == pytest.approx(6.0625)
    assert P.bytes_per_param("fp8", master="fp24") == pytest.approx(5.0625)
    assert P.bytes_per_param("bf16", moments=1, master="fp24") == 5


# ------------------------------------------------- rounding streams and codecs

def test_bf16_weight_is_the_kernels_weight_rounding():
    """formats.bf16_weight (the weight written into a parameter for an owed delayed update) rounds as
    the kernels' working-weight output does (kernels.c:108-112): nearest-even, NaN sign and payload
    kept with the quiet bit set -- against the oracle's rule, on special values and random bits."""
    rng = np.random.default_rng(3)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7F800001, 0xFFC00001, 0x7FBFFFFF, 0x7F7FFFFF,
                        0xFF7FFFFF, 0x00000001, 0x8000FFFF, 0x3F808000, 0x3F818000, 0x3F807FFF, 0x7FFF0000,
                        0xFFFF8000], dtype=np.uint32)
    bits = np.concatenate([special, rng.integers(0, 2**32, 1 << 18, dtype=np.uint64).astype(np.uint32)])
    got = F.bf16_weight(torch.from_numpy(bits.view(np.float32).copy()))
    assert got.dtype == torch.bfloat16
    assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), O.bf16_bits(bits.view(np.float32)))


def test_random_bits_is_the_kernels_counter_hash():
    lib = O.load_oracle()
    for offset in (0, 12345, (1 << 31) - 100, (1 << 32) + 7):
        bits = P.random_bits(offset, 200, seed=0xDEADBEEF).numpy().view(np.uint32)
        want = [lib.abo_hash32(((offset + i) & 0xFFFFFFFF) ^ 0xDEADBEEF) for i in range(200)]
        assert bits.tolist() == want, offset
    seed = 0x1234567
    assert P.moment_seed(seed, "m") == seed
    assert P.moment_seed(seed, "v") == lib.abo_hash32(seed ^ 0xA511E9B3)
    assert P.moment_seed(seed, "p") == lib.abo_hash32(seed ^ 0x6C8E9CF5)


def _finite_samples(n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, generator=g) * torch.exp2(torch.randint(-30, 30, (n,), generator=g).float())
    x[::97] = 0.0
    x[1::97] = -0.0
    x[2::97] = 1e-41   # subnormal
    return x


def test_bf16_stochastic_rounding_matches_the_kernels():
    """(bits + (hash & 0xffff)) >> 16, kernels.c:120-126."""
    lib = O.load_oracle()
    x = _finite_samples(20000, 1)
    seed, offset = 0x9E37, 5000
    got = P.round_to_bf16_stochastic(x.clone(), seed, offset).view(torch.int16).numpy().view(np.uint16)
    b = x.numpy().view(np.uint32).astype(np.uint64)
    r = np.array([lib.abo_hash32((offset + i) ^ seed) for i in range(x.numel())], np.uint64)
    want = (((b + (r & 0xFFFF)) & 0xFFFFFFFF) >> 16).astype(np.uint16)
    assert np.array_equal(got, want)


def test_fp24_nearest_matches_the_kernels_and_brute_force():
    lib = O.load_oracle()
    x = _finite_samples(20000, 2)
    got = P.round_to_fp24_nearest_(x.clone()).numpy().view(np.uint32)
    want = np.array([lib.abo_f24_round(int(b), 0, 0) for b in x.numpy().view(np.uint32)], np.uint32)
    assert np.array_equal(got, want)
    # nearest of the two 24-bit neighbours, ties to even
    b = x.numpy().view(np.uint32).astype(np.int64)
    down = b & ~0xFF
    up = down + 0x100
    xv = x.double().numpy()
    dd = np.abs(xv - down.astype(np.uint32).view(np.float32).astype(np.float64))
    du = np.abs(up.astype(np.uint32).view(np.float32).astype(np.float64) - xv)
    pick = np.where(dd < du, down, np.where(du < dd, up, np.where(down & 0x100, up, down))).astype(np.uint32)
    assert np.array_equal(got, pick)
    nan = P.round_to_fp24_nearest_(torch.tensor([float("nan"), -float("inf")]))
    assert nan[0].isnan() and nan[1] == -float("inf")


def test_fp24_stochastic_rounding_is_unbiased():
    x = torch.full((100_000,), 1.0 + 2 ** -17)   # a quarter of the way between two FP24 values
    y = P.round_to_fp24_stochastic(x.clone(), seed=3)
    assert set(y.unique().tolist()) == {1.0, 1.0 + 2 ** -15}
    assert y.mean().item() == pytest.approx(1.0 + 2 ** -17, abs=0.01 * 2 ** -15)


@pytest.mark.parametrize("role", ["m", "v"])
@pytest.mark.parametrize("stochastic", [False, True])
def test_fp8_store_encodes_like_the_kernels_block_path(role, stochastic):
    """Per 128-block: scale = absmax / format max (1 for an all-zero block), codes = the encoder of
    value / scale, v in the sqrt domain (kernels.c:1049-1057, 857-876)."""
    lib = O.load_oracle()
    n = 128 * 20 + 37
    g = torch.Generator().manual_seed(4 + stochastic)
    x = torch.randn(n, generator=g) * torch.exp2(torch.randint(-12, 4, (n,), generator=g).float())
    x[128:256] = 0.0   # an all-zero block
    if role == "v":
        x = x.square()
    seed, offset = 0xABC, 128 * 3
    store = P.FP8Store(n, role)
    store.write(0, n, x.clone(), seed=seed if stochastic else None)
    # the store's block offset is its own element index (0); re-derive with that offset
    del offset
    codes = store.q.view(torch.uint8).numpy()
    scales = store.scale.numpy()
    vals = np.sqrt(np.maximum(x.numpy(), 0)) if role == "v" else x.numpy()
    fmax = 448.0 if role == "m" else 57344.0
    r = 0 if role == "m" else 1
    for blk in range(-(-n // 128)):
        lo, hi = blk * 128, min(blk * 128 + 128, n)
        am = np.float32(np.max(np.abs(vals[lo:hi])))
        sc = np.float32(am / np.float32(fmax)) if am > 0 else np.float32(1.0)
        assert scales[blk].view(np.uint32) == sc.view(np.uint32), blk
        for i in range(lo, hi):
            q = np.float32(vals[i]) / sc
            rb = lib.abo_hash32(i ^ seed) if stochastic else 0
            assert codes[i] == lib.abo_fp8_encode(float(q), int(stochastic), rb, r), (blk, i)
        assert not codes[hi: blk * 128 + 128].any()


def test_fp8_decode_matches_the_kernels_table():
    for role, dtype in ((0, torch.float8_e4m3fn), (1, torch.float8_e5m2)):
        table = O.fp8_decode_table(role)
        got = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(dtype).float().numpy()
        same = (table.view(np.uint32) == got.view(np.uint32)) | (np.isnan(table) & np.isnan(got))
        assert same.all()


def test_fp8_store_chunked_writes_equal_whole():
    n = 1000
    x = torch.randn(n, generator=torch.Generator().manual_seed(5))
    whole = P.make_store("fp8", n, "m")
    whole.write(0, n, x.clone(), seed=77)
    parts = P.make_store("fp8", n, "m")
    for lo in range(0, n, 256):
        hi = min(lo + 256, n)
        parts.write(lo, hi, x[lo:hi].clone(), seed=77)
    assert torch.equal(whole.q.view(torch.uint8), parts.q.view(torch.uint8))
    assert torch.equal(whole.scale, parts.scale)


@pytest.mark.parametrize("prec", ["bf16", "fp8"])
def test_ema_stalls_under_nearest_but_not_under_stochastic_rounding(prec):
    """v <- 0.999 v + 0.001 g^2 cannot leave its starting value under round-to-nearest when each
    increment is below half an ulp; stochastic rounding tracks the exact EMA on average."""
    lib = O.load_oracle()
    n = 4096
    init = torch.ones(n)
    init[::128] = 4.0   # one larger element per block, so FP8 scaling cannot make 1.0 exact
    target = torch.full((n,), 1.5)
    target[::128] = 4.0
    tracked = torch.ones(n, dtype=torch.bool)
    tracked[::128] = False
    out = {}
    for sr in (False, True):
        store = P.make_store(prec, n, "v", init=init)
        for step in range(1, 401):
            v = store.to_fp32()
            v.mul_(0.999).add_(target, alpha=0.001)
            seed = P.moment_seed(lib.abo_step_seed(0, 0, step), "v") if sr else None
            store.write(0, n, v, seed=seed)
        out[sr] = store.to_fp32()[tracked].mean().item()
    exact = 1.5 - 0.5 * 0.999 ** 400
    assert out[False] == pytest.approx(1.0, abs=1e-6)
    assert out[True] == pytest.approx(exact, rel=0.01 if prec == "bf16" else 0.03)


@pytest.mark.parametrize("prec", ["fp32", "bf16", "fp8"])
@pytest.mark.parametrize("role", ["m", "v"])
def test_store_round_trip_and_state_dict(prec, role):
    n = 1000
    x = torch.randn(n, generator=torch.Generator().manual_seed(6)) * 1e-3
    if role == "v":
        x = x.abs()
    store = P.make_store(prec, n, role, init=x)
    tol = {"fp32": 0.0, "bf16": 2 ** -8, "fp8": 0.25}[prec]
    assert (store.to_fp32() - x).abs().max().item() <= tol * x.abs().max().item()
    clone = P.store_from_state_dict(store.state_dict(), n, role)
    assert torch.equal(clone.to_fp32(), store.to_fp32())


def test_store_from_state_dict_rejects_bad_stores():
    n = 300
    good = P.make_store("fp8", n, "m", init=torch.randn(n)).state_dict()
    with pytest.raises(ValueError):
        P.store_from_state_dict({"precision": "int4", "data": torch.zeros(n)}, n, "m")
    with pytest.raises(ValueError):
        P.store_from_state_dict({"precision": "bf16", "data": torch.zeros(n + 1, dtype=torch.bfloat16)}, n, "m")
    with pytest.raises(ValueError):
        P.store_from_state_dict({**good, "role": "w"}, n, "m")
    with pytest.raises(ValueError):
        P.store_from_state_dict({**good, "block": 0}, n, "m")
    with pytest.raises(ValueError):
        P.store_from_state_dict({**good, "scale": good["scale"][:-1]}, n, "m")
    with pytest.raises(ValueError):
        P.check_master_state({"precision": "fp24", "hi": torch.zeros(n, dtype=torch.bfloat16),
                              "lo": torch.zeros(n, dtype=torch.int8)}, n, "master")


@pytest.mark.parametrize("n", [1, 127, 128, 300, 4096 + 77])
def test_fp8_records_layout_offsets_and_views(n):
    """AdamRecordState puts element 128b + 8l + j's master at byte 16l + 4j (j < 4) or 256 + 16l + 4(j - 4)
    of record b, its m code at 512 + 16l + j and its v code at 520 + 16l + j (the kernel's
    ADAMBRIDGE_DT_PACKED_FP8 layout); loading takes codes as they are, and the moments read back as
    separate FP8Stores with the same codes and scales."""
    from adambridge_amd.state import AdamRecordState
    rng = np.random.default_rng(n)
    master = rng.normal(0, 0.02, n).astype(np.float32)
    nb = -(-n // 128)
    codes = {"m": rng.integers(0, 256, nb * 128, dtype=np.uint8),
             "v": rng.integers(0, 0x7c, nb * 128, dtype=np.uint8)}   # finite E5M2 codes
    scale = torch.from_numpy(rng.uniform(1e-6, 1e-3, nb).astype(np.float32))
    separate = {}
    for role, q in codes.items():
        st = P.FP8Store(n, role)
        st.q.copy_(torch.from_numpy(q).view(st.q.dtype))
        st.scale.copy_(scale)
        separate[role] = st
    rs = AdamRecordState(n, "cpu")
    rs.load(master=torch.from_numpy(master), moments=separate)
    rec = rs.current.numpy()
    for e in list(range(min(n, 40))) + list(rng.integers(0, n, 40)):
        b, l, j = e // 128, (e % 128) // 8, e % 8
        off = 16 * l + 4 * j if j < 4 else 256 + 16 * l + 4 * (j - 4)
        assert rec[b, off:off + 4].view(np.float32)[0] == master[e]
        assert rec[b, 512 + 16 * l + j] == codes["m"][e] and rec[b, 520 + 16 * l + j] == codes["v"][e]
    assert np.array_equal(rs.master_fp32().numpy(), master)
    for role, sep in separate.items():
        mom = rs.moment(role)
        assert np.array_equal(mom.q.view(torch.uint8).numpy(), codes[role])
        assert torch.equal(mom.to_fp32().view(torch.int32), sep.to_fp32().view(torch.int32))   # NaN codes too
        sd = mom.state_dict()
        assert sd["precision"] == "fp8" and sd["role"] == role and torch.equal(sd["scale"], scale)
    window = rs.window(128 * (nb - 1), n)
    assert np.array_equal(window["m"].numpy(), codes["m"][128 * (nb - 1):])
    assert rs.footprint() == (4 * n, nb * (768 + 8) - 4 * n)


@pytest.mark.parametrize("n", [1, 2, 255, 256, 601])
def test_lion_and_pair_layout_offsets(n):
    """LionRecordState: element 256r + i (i < 256) keeps its master at byte 4i of record r and its m
    bits at 1024 + 2i (ADAMBRIDGE_DT_PACKED_LION).  PairState: elements 2k, 2k + 1 at words 0, 1 of
    row k, their m and v bits in the halves of words 2 and 3 (ADAMBRIDGE_DT_PACKED)."""
    from adambridge_amd.state import LionRecordState, PairState
    rng = np.random.default_rng(n + 7)
    master = rng.normal(0, 0.02, n).astype(np.float32)
    m = rng.integers(0, 0x7f00, n).astype(np.int16)
    v = rng.integers(0, 0x7f00, n).astype(np.int16)
    stores = {}
    for role, bits in (("m", m), ("v", v)):
        st = P.BF16Store(n)
        st.data.copy_(torch.from_numpy(bits).view(torch.bfloat16))
        stores[role] = st
    lion = LionRecordState(n, "cpu")
    lion.load(master=torch.from_numpy(master), moments={"m": stores["m"]})
    rec = lion.current.numpy()
    for e in range(n):
        r, i = divmod(e, 256)
        assert rec[r, 4 * i:4 * i + 4].view(np.float32)[0] == master[e]
        assert rec[r, 1024 + 2 * i:1026 + 2 * i].view(np.int16)[0] == m[e]
    assert np.array_equal(lion.moment("m").data.view(torch.int16).numpy(), m)
    pairs = PairState(n, "cpu", double_buffer=True)
    pairs.load(master=torch.from_numpy(master), moments=stores)
    rows = pairs.current.numpy().view(np.uint32)
    for e in range(n):
        k, h = divmod(e, 2)
        assert rows[k, h] == master[e:e + 1].view(np.uint32)[0]
        assert (rows[k, 2] >> (16 * h)) & 0xFFFF == np.uint16(m[e]) and (rows[k, 3] >> (16 * h)) & 0xFFFF == np.uint16(v[e])
    assert np.array_equal(pairs.master_fp32().numpy(), master)
    pairs.advance()   # double-buffered: the other buffer is current now
    assert pairs.current.data_ptr() != pairs.buffers[0].data_ptr() and pairs.target is pairs.buffers[0]


@pytest.mark.parametrize("n", [1, 255, 256, 257, 1000])
def test_f32_record_layout_offsets(n):
    """F32RecordState: element 256r + i (i < 256) keeps its master at byte 4i of record r, its m at
    1024 + 4i and its v at 2048 + 4i (ADAMBRIDGE_DT_PACKED_F32); moments and windows read back the
    values loaded, double buffering alternates the buffers."""
    from adambridge_amd.state import F32RecordState
    rng = np.random.default_rng(n + 11)
    vals = {r: rng.normal(0, 1, n).astype(np.float32) for r in ("p", "m", "v")}
    st = F32RecordState(n, "cpu", double_buffer=True)
    assert F32RecordState.buffer_bytes(n) == -(-n // 256) * 3072 == st.current.nbytes
    st.load(master=torch.from_numpy(vals["p"]),
            moments={r: P.FP32Store(n, init=torch.from_numpy(vals[r])) for r in ("m", "v")})
    rec = st.current.numpy()
    for e in range(n):
        r, i = divmod(e, 256)
        for k, role in enumerate(("p", "m", "v")):
            assert rec[r, 1024 * k + 4 * i:1024 * k + 4 * i + 4].view(np.float32)[0] == vals[role][e]
    assert np.array_equal(st.master_fp32().numpy(), vals["p"])
    for role in ("m", "v"):
        assert np.array_equal(st.moment(role).to_fp32().numpy(), vals[role])
    w = st.window(n // 3, n)
    assert np.array_equal(w["v"].numpy(), vals["v"][n // 3:])
    st.advance()
    assert st.target is st.buffers[0] and st.current.data_ptr() == st.buffers[1].data_ptr()


@pytest.mark.parametrize("n", [1, 255, 256, 257, 1000])
def test_f24_record_layout_offsets(n):
    """F24RecordState: element 256r + i (i < 256) keeps its master's hi half at byte 2i of record r,
    its lo byte at 512 + i, its m at 768 + 2i and its v at 1280 + 2i (ADAMBRIDGE_DT_PACKED_F24); the
    master loads rounded to FP24 as the separate store rounds it, reads back through master_fp32,
    the checkpoint planes and windows, and double buffering alternates the buffers."""
    from adambridge_amd.state import F24RecordState
    rng = np.random.default_rng(n + 21)
    master = torch.from_numpy(rng.normal(0, 1, n).astype(np.float32))
    moments = {r: P.BF16Store(n, init=torch.from_numpy(rng.normal(0, 1, n).astype(np.float32))) for r in ("m", "v")}
    st = F24RecordState(n, "cpu", double_buffer=True)
    assert F24RecordState.buffer_bytes(n) == -(-n // 256) * 1792 == st.current.nbytes
    st.load(master=master, moments=moments)
    ref = P.make_master("fp24", n, init=master)
    hi, lo = ref.hi.view(torch.int16).numpy().view(np.uint16), ref.lo.numpy()
    rec = st.current.numpy()
    for e in range(n):
        r, i = divmod(e, 256)
        assert rec[r, 2 * i:2 * i + 2].view(np.uint16)[0] == hi[e] and rec[r, 512 + i] == lo[e]
        for base, role in ((768, "m"), (1280, "v")):
            assert rec[r, base + 2 * i:base + 2 * i + 2].view(np.uint16)[0] == \
                moments[role].data.view(torch.int16).numpy().view(np.uint16)[e]
    assert torch.equal(st.master_fp32(), ref.to_fp32())
    saved = st.export_master()
    assert saved["precision"] == "fp24" and torch.equal(saved["hi"], ref.hi) and torch.equal(saved["lo"], ref.lo)
    for role in ("m", "v"):
        assert torch.equal(st.moment(role).data, moments[role].data)
    w = st.window(n // 3, n)
    assert torch.equal(w["p_lo"], ref.lo[n // 3:]) and torch.equal(w["v"], moments["v"].data[n // 3:])
    other = F24RecordState(n, "cpu")
    other.load(master=saved)   # FP24 planes are taken as they are
    assert torch.equal(other.master_fp32(), ref.to_fp32())
    assert st.footprint() == (3 * n * 2, 2 * st.current.nbytes - 3 * n * 2)
    st.advance()
    assert st.target is st.buffers[0] and st.current.data_ptr() == st.buffers[1].data_ptr()


def test_fp24_master_store_round_trip():
    n = 1000
    x = torch.randn(n) * 3
    store = P.make_master("fp24", n, init=x)
    y = store.to_fp32()
    assert store.nbytes == 3 * n
    assert ((y - x).abs() <= x.abs() * 2 ** -16).all()
    assert (y.view(torch.int32) & 0xFF == 0).all()
    clone = P.FP24Store(n)
    P.load_master_(clone, store.state_dict())
    assert torch.equal(clone.to_fp32(), y)


# ------------------------------------------------------- optimizer, host side

def _params():
    return [torch.nn.Parameter(torch.zeros(10)), torch.nn.Parameter(torch.zeros(3, 3))]


@pytest.mark.parametrize("kwargs", [dict(lr=-1.0), dict(eps=-1.0), dict(betas=(1.0, 0.9)), dict(betas=(0.9, -0.1)),
                                    dict(weight_decay=-0.1), dict(chunk_size=100), dict(precision="int4"),
                                    dict(master_precision="fp16"), dict(accumulation_steps=0),
                                    dict(delay_warmup_steps=-1), dict(gpu_state_budget=-5), dict(backend="torch"),
                                    dict(backend="cuda"), dict(state_layout="rows")])
def test_constructor_validates_like_the_reference(kwargs):
    with pytest.raises(ValueError):
        ab.AdamBridge(_params(), **kwargs)


def test_lion_has_no_eps_and_its_own_defaults():
    with pytest.raises(TypeError):
        ab.LionBridge(_params(), eps=1e-8)
    opt = ab.LionBridge(_params())
    g = opt.param_groups[0]
    assert g["lr"] == 1e-4 and g["betas"] == (0.9, 0.99) and g["weight_decay"] == 0.0
    assert opt.expected_bytes_per_param() == 8
    assert ab.AdamBridge(_params(), precision="fp8").expected_bytes_per_param() == pytest.approx(6.0625)
    assert ab.OptiComputeAdamW is ab.AdamBridge


def test_host_only_knobs_are_accepted():
    opt = ab.AdamBridge(_params(), numa_aware=False, num_threads=3, chunk_size=256, transfer_buffer_mb=64,
                        gpu_state_budget="auto", autotune=ab.AutoTuneConfig(), precision="BF16")
    assert opt.precision == "bf16"
    assert opt.autotune_log and opt.tune_threads() == {}
    assert opt.memory_report()["total"] == 0   # lazy state: nothing allocated before the first update


def test_cpu_parameters_are_refused_at_the_first_update():
    p = torch.nn.Parameter(torch.ones(4))
    opt = ab.AdamBridge([p])
    p.grad = torch.ones(4)
    with pytest.raises(RuntimeError, match="GPU"):
        opt.step()


def test_fresh_state_dict_and_checkpoint_validation():
    params = _params()
    opt = ab.AdamBridge(params, precision="fp8")
    sd = opt.state_dict()
    assert sd["state"] == {}
    assert sd["adambridge"] == {"precision": "fp8", "master_precision": "fp32", "format": 1, "algorithm": "adamw"}
    bad = {"state": {0: {"step": 1, "master": torch.zeros(11), "exp_avg": torch.zeros(10),
                         "exp_avg_sq": torch.zeros(10)}}, "param_groups": sd["param_groups"]}
    with pytest.raises(ValueError, match="11 elements"):
        opt.load_state_dict(bad)
    lion_ckpt = {"state": {0: {"step": 1, "master": torch.zeros(10), "exp_avg": torch.zeros(10)}},
                 "param_groups": sd["param_groups"]}
    with pytest.raises(ValueError, match="exp_avg_sq"):
        opt.load_state_dict(lion_ckpt)
    out_of_range = {"state": {5: {"step": 1, "exp_avg": torch.zeros(10), "exp_avg_sq": torch.zeros(10)}},
                    "param_groups": sd["param_groups"]}
    with pytest.raises(ValueError, match="parameters"):
        opt.load_state_dict(out_of_range)
    assert opt.state_dict()["state"] == {}   # nothing was loaded


def test_segment_struct_mirrors_match_the_library():
    from adambridge_amd import _hip
    lib = _hip.open_library()
    assert ctypes.sizeof(_hip.Segment) == lib.adambridge_segment_size() == ctypes.sizeof(O.Segment)
    assert ctypes.sizeof(_hip.HParams) == lib.adambridge_hparams_size() == ctypes.sizeof(O.HParams)
    assert ctypes.sizeof(_hip.Group) == lib.adambridge_group_size() == ctypes.sizeof(O.Group)


# -------------------------------------- store behaviour (reference tests/test_precision.py,
#                                         tests/test_hardening.py:80-89)

def test_fp8_store_saved_under_the_other_role_is_converted():
    """A checkpointed m store loaded as v is decoded in its own format and re-encoded as v
    (E5M2, sqrt domain), not reinterpreted."""
    n = 256
    x = torch.rand(n, generator=torch.Generator().manual_seed(4)) * 1e-3
    saved = P.make_store("fp8", n, "m", init=x)
    loaded = P.store_from_state_dict(saved.state_dict(), n, "v")
    assert loaded.role == "v" and loaded.dtype == torch.float8_e5m2
    assert torch.equal(loaded.to_fp32(), P.make_store("fp8", n, "v", init=saved.to_fp32()).to_fp32())


def test_fp8_stochastic_rounding_is_unbiased():
    x = torch.full((200_000,), 1.03)
    y = P.round_to_fp8_stochastic(x.clone(), torch.float8_e4m3fn, seed=0).float()
    assert abs(y.mean().item() / 1.03 - 1.0) < 1e-3
    # the two neighbouring codes of 1.03 (1.0 and 1.125) both occur
    assert set(torch.unique(y).tolist()) == {1.0, 1.125}


def test_fp8_store_keeps_small_second_moments():
    """v is stored as sqrt(v): values 2^40 below the block's largest stay non-zero."""
    v = torch.full((128,), 1e-12)
    v[0] = 1.0
    out = P.make_store("fp8", 128, "v", init=v).to_fp32()
    assert abs(out[0].item() - 1.0) < 0.3
    assert (out[1:] > 0).all()


def test_fp24_store_initialises_exactly_from_bf16_and_in_chunks(monkeypatch):
    n = 1000
    x = torch.randn(n, generator=torch.Generator().manual_seed(5)) * 3
    from_bf16 = P.make_master("fp24", n, init=x.to(torch.bfloat16).view(10, 100))
    assert torch.equal(from_bf16.to_fp32(), x.to(torch.bfloat16).float()) and not from_bf16.lo.any()
    whole = P.make_master("fp24", n, init=x)
    monkeypatch.setattr(P.FP24Store, "INIT_CHUNK", 96)
    chunked = P.make_master("fp24", n, init=x.view(20, 50))
    assert torch.equal(chunked.to_fp32(), whole.to_fp32())


# ------------------------------------------ the native module (reference adambridge/native.py)

def test_native_module_mirrors_the_reference_names():
    from adambridge_amd import _hip, native
    assert native.NativeKernels is _hip.HipKernels and native.Group is _hip.Group and native.Segment is _hip.Segment
    assert native.library_path().exists() and native.library_path().parent == native.cache_dir()
    k = native.load(build_if_missing=False)
    assert k is not None and native.available() and native.load_error() is None
    assert k.backend == "hip/gfx950"
    assert issubclass(native.BuildError, RuntimeError)


@pytest.mark.parametrize("step", [1, 2, 7, 100, 5000])
def test_step_coefficients_equal_the_librarys_own(step):
    """StepCoefficients -> multi_apply hparams (reference native.py:243-270, 381-387) carry the
    bits multi_step derives from the group (kernels.c:793-809, restated by the oracle)."""
    from adambridge_amd import _hip, native
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.999, 1e-8, 0.01
    case = O.make_case(np.random.default_rng(0), 16, explicit=False, lr=lr, betas=(b1, b2), eps=eps,
                       weight_decay=wd, step=step)
    want = O.hparams_for(case)
    got = _hip.HipKernels.make_hparams(native.StepCoefficients.for_step(lr, b1, b2, eps, wd, step),
                                      seed=want["seed"], stochastic=True)
    for field, _ in _hip.HParams._fields_:
        a, b = getattr(got, field), want[field]
        if isinstance(a, float):
            assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), (field, a, b)
        else:
            assert a == b, (field, a, b)
    lion = native.StepCoefficients.for_lion(1e-4, 0.9, 0.99, 0.1)
    assert (lion.step_size, lion.inv_sqrt_bc2, lion.eps) == (1e-4, 1.0, 0.0)


def test_optimizer_is_freed_without_the_garbage_collector(monkeypatch):
    """Nothing the optimizer builds at construction refers back to it (the gradient hooks reach it
    through a weak reference): dropping the last reference frees it, and with it its device state,
    at once -- a 7B state is 54 GB of HBM."""
    import gc
    import weakref

    import adambridge_amd as ab
    from adambridge_amd import _hip

    monkeypatch.setattr(_hip, "load", lambda: None)   # no library calls: the engine is never used here
    params = [torch.nn.Parameter(torch.zeros(4, 4)), torch.nn.Parameter(torch.zeros(4))]
    gc.disable()
    try:
        opt = ab.AdamBridge(params, lr=1e-3)
        gone = weakref.ref(opt)
        opt.attach_hooks()
        del opt
        assert gone() is None
    finally:
        gc.enable()


@pytest.mark.parametrize("precision", ["bf16", "fp8"])
def test_dropped_optimizer_leaves_no_cycle_holding_its_state(monkeypatch, precision):
    """With states built (small parameters batched, interleaved states in one shared arena), dropping
    the optimizer frees every slot, batch and state by reference counting alone: nothing is left for
    the garbage collector, so the arena -- 54 GB of HBM at the 7B list -- and the parameters the
    groups hold go at once.  (States are built on the host here, the GPU check bypassed.)"""
    import contextlib
    import gc
    import weakref

    import adambridge_amd as ab
    from adambridge_amd import _hip
    from adambridge_amd.engine import ParamSlot, SmallGroup, UpdateEngine
    from adambridge_amd.state import ParamState

    monkeypatch.setattr(_hip, "load", lambda: None)
    monkeypatch.setattr(UpdateEngine, "check_param", staticmethod(lambda p: None))
    monkeypatch.setattr(torch.cuda, "device", lambda device: contextlib.nullcontext())
    params = [torch.nn.Parameter(torch.randn(512, 256).bfloat16()), torch.nn.Parameter(torch.randn(256).bfloat16()),
              torch.nn.Parameter(torch.randn(300).bfloat16())]
    gc.collect()
    gc.disable()
    gc.set_debug(gc.DEBUG_SAVEALL)
    try:
        opt = ab.AdamBridge(params, lr=1e-3, precision=precision, small_param_threshold=1024)
        slots = list(opt._ordered)
        opt._registry.small.append(SmallGroup(slots[1:]))   # as batch_small does for device parameters
        assert [s.small is not None for s in slots] == [False, True, True]
        opt._engine.initialize(slots)
        states = {type(s.state).__name__ for s in slots}
        assert states & {"PairState", "AdamRecordState"}, states
        buffer = slots[0].state.current
        held = weakref.ref(buffer._base if buffer._base is not None else buffer)
        del slots, opt, buffer
        assert held() is None, "the state arena outlived the optimizer"
        gc.collect()
        left = [o for o in gc.garbage if isinstance(o, (ParamSlot, SmallGroup, ParamState, UpdateEngine))]
        assert not left, f"only the garbage collector frees: {sorted({type(o).__name__ for o in left})}"
    finally:
        gc.set_debug(0)
        gc.garbage.clear()
        gc.enable()


def test_large_state_arenas_follow_an_allocate_free_of_their_size(monkeypatch):
    """new_states allocates an arena of RECYCLE_MIN_BYTES or more right after the library has
    allocated and freed a block of the arena's size (the placement that streams at a copy's rate),
    and so do the separate layout's stores, counted together; smaller state, or the states a
    gradient hook creates, go without it.  (Host tensors stand in for HBM.)"""
    from adambridge_amd import _hip
    from adambridge_amd import state as S

    calls = []

    class Lib:
        def recycle_device_memory(self, nbytes, device):
            calls.append((nbytes, device))
            return True

    monkeypatch.setattr(_hip, "load", lambda: Lib())
    masters = [torch.zeros(3000), torch.zeros(1001)]
    _, total = S.arena_plan("pairs", [m.numel() for m in masters])
    monkeypatch.setattr(S, "RECYCLE_MIN_BYTES", total)
    states = S.new_states("pairs", "adamw", "bf16", "fp32", "cpu", masters)
    assert calls == [(total, torch.device("cpu"))]
    assert states[0].master_fp32().numel() == 3000
    S.new_states("pairs", "adamw", "bf16", "fp32", "cpu", masters, place=False)   # a hook's state
    monkeypatch.setattr(S, "RECYCLE_MIN_BYTES", total + 1)
    S.new_states("pairs", "adamw", "bf16", "fp32", "cpu", masters)
    sep = 4001 * (4 + 2 * 2)   # FP32 master and two BF16 moments of the two parameters
    monkeypatch.setattr(S, "RECYCLE_MIN_BYTES", sep)
    S.new_states("separate", "adamw", "bf16", "fp32", "cpu", masters)
    assert calls[1:] == [(sep, torch.device("cpu"))]
    S.new_states("separate", "adamw", "bf16", "fp32", "cpu", masters, master_params=[masters[0], None])
    assert len(calls) == 2   # the first parameter is its own master: 3000 x 4 bytes fewer, under the minimum


def test_layout_choice_for_every_algorithm_precision_and_master():
    """Each (algorithm, moment precision) with an FP32 master of the optimizer's own gets its
    interleaved layout (Lion with a BF16, FP32 or FP8 moment), and AdamW with BF16, FP8 or FP32 moments
    and Lion with a BF16, FP32 or FP8 moment their FP24 records under an FP24 master; an FP32 parameter
    updated in place and state_layout='separate' keep the reference's arrays."""
    from adambridge_amd.state import choose_layout
    want = {("adamw", "bf16"): "pairs", ("adamw", "fp8"): "fp8-records", ("adamw", "fp32"): "f32-records",
            ("lion", "bf16"): "lion-records", ("lion", "fp8"): "lion-fp8-records", ("lion", "fp32"): "lion-f32-records"}
    for (algo, prec), layout in want.items():
        assert choose_layout(algo, prec, "fp32") == layout, (algo, prec)
        assert choose_layout(algo, prec, "fp24") == {("adamw", "bf16"): "f24-records",
                                                     ("lion", "bf16"): "lion-f24-records",
                                                     ("adamw", "fp8"): "fp8-f24-records",
                                                     ("adamw", "fp32"): "f24-f32-records",
                                                     ("lion", "fp32"): "lion-f24-f32-records",
                                                     ("lion", "fp8"): "lion-fp8-f24-records"}.get((algo, prec), "separate")
        assert choose_layout(algo, prec, "fp24", requested="separate") == "separate"
        assert choose_layout(algo, prec, "fp32", master_is_param=True) == "separate"
        assert choose_layout(algo, prec, "fp32", requested="separate") == "separate"


@pytest.mark.parametrize("layout", ["pairs", "fp8-records", "lion-records", "f32-records", "f24-records",
                                    "lion-f24-records", "fp8-f24-records", "lion-f32-records", "lion-fp8-records",
                                    "f24-f32-records", "lion-f24-f32-records", "lion-fp8-f24-records"])
def test_arena_plan_aligns_large_buffers_and_packs_small_ones(layout):
    """Buffers of 2 MiB or more start on 2 MiB boundaries, smaller ones on 256-byte boundaries (16-byte
    state access needs 16); no two buffers overlap, and many small tensors take little more than
    their own bytes."""
    from adambridge_amd import state as S
    cls = S._INTERLEAVED[layout]
    sizes = [4096, 1 << 20, 3, 896, 300_000, 1 << 18, 4096] * 3
    for double in (False, True):
        offsets, total = S.arena_plan(layout, sizes, double)
        spans = []
        for n, offs in zip(sizes, offsets):
            nbytes = cls.buffer_bytes(n)
            assert len(offs) == (2 if double and layout not in S.IN_PLACE else 1)
            for o in offs:
                assert o % (S.ARENA_ALIGN if nbytes >= S.ARENA_ALIGN else S.SMALL_ALIGN) == 0
                spans.append((o, o + nbytes))
        spans.sort()
        assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:])) and spans[-1][1] <= total
    small = [896] * 1000
    _, total = S.arena_plan(layout, small)
    assert total < 1000 * (cls.buffer_bytes(896) + S.SMALL_ALIGN)


def test_launch_points_fire_at_the_start_of_each_hooked_modules_backward():
    """A hooked update is launched at the next launch point of its backward pass: the hook on the
    gradient of a hooked module's output fires before that module's parameters get their gradients,
    so the update of a parameter is launched beside the next module's GEMMs (and not beside the
    elementwise backward in between).  A forward pass without gradients registers nothing."""
    from adambridge_amd.optimizer import _LaunchPoints

    events = []

    class Owner:
        def launch(self):
            events.append("point")

    owner = Owner()
    points = _LaunchPoints(owner.launch)
    model = torch.nn.Sequential(torch.nn.Linear(4, 8), torch.nn.GELU(), torch.nn.Linear(8, 4))
    points.add([model[0], model[2]])
    for i, p in enumerate([model[0].weight, model[2].weight]):
        p.register_post_accumulate_grad_hook(lambda p, i=i: events.append(f"grad{i}"))
    with torch.no_grad():
        model(torch.randn(3, 4))
    assert not points.armed
    model(torch.randn(3, 4)).sum().backward()
    assert points.armed
    assert events == ["point", "grad1", "point", "grad0"]
    points.clear()
    points.armed = False
    events.clear()
    model(torch.randn(3, 4)).sum().backward()
    assert not points.armed and events == ["grad1", "grad0"]
    del owner   # the hooks hold the owner weakly: a dropped owner is not called
    points.add([model[2]])
    model(torch.randn(3, 4)).sum().backward()
    assert events == ["grad1", "grad0"] * 2


def test_device_fp24_and_weight_conversions_take_the_plane_kernel(monkeypatch):
    """For tensors in device memory, the FP24 master's conversions (rounding into the planes, their
    expansion, a store's writes and reads) and the bf16 working weight of a master are one call of
    the plane-conversion kernel each -- never the torch integer chain, whose int64 temporaries cost
    ~33 bytes per element and ~10 dispatches per tensor.  (The device is stood in for: the calls are
    recorded, the chain's building blocks fail the test if reached.)"""
    from adambridge_amd import _hip

    calls = []
    monkeypatch.setattr(F, "_on_device", lambda x: True)
    monkeypatch.setattr(F, "convert_plane", lambda src, dst, n, device, offset=0, seed=None:
                        calls.append((src.dtype, dst.dtype, n, offset, seed)))

    def forbidden(*args, **kwargs):
        raise AssertionError("the torch FP24 / weight chain was called for a device tensor")

    for name in ("_as_u32", "_from_u32", "round_bits_stochastic", "counter_hash"):
        monkeypatch.setattr(F, name, forbidden)
    x = torch.randn(1000)
    hi, lo = F.fp24_encode(x, 7, 128)
    F.fp24_join(hi, lo)
    F.fp24_split(x)
    F.bf16_weight(x)
    store = P.FP24Store(1000, init=x)
    store.read(0, 1000)
    store.write(256, 512, x[:256], seed=5)
    f32, bf16, f24 = _hip.DT_F32, _hip.DT_BF16, _hip.DT_F24
    assert calls == [(f32, f24, 1000, 128, 7), (f24, f32, 1000, 0, None), (f32, f24, 1000, 0, None),
                     (f32, bf16, 1000, 0, None), (f32, f24, 1000, 0, None), (f24, f32, 1000, 0, None),
                     (f32, f24, 256, 256, 5)]


def test_memory_report_keys():
    """memory_report() has the reference's keys (optimizer.py:496-513) plus ``reserved``; every byte is
    device memory, so ``gpu_state`` equals ``total`` (the reference reports its host bytes as
    ``total`` and its GPU-resident state apart)."""
    import types

    opt = ab.AdamBridge.__new__(ab.AdamBridge)
    opt._registry = types.SimpleNamespace(ordered=[])
    opt._engine = types.SimpleNamespace(_reserved={"slot": [torch.zeros(1000, dtype=torch.uint8),
                                                            torch.zeros(24, dtype=torch.uint8)]})
    rep = ab.AdamBridge.memory_report(opt)
    assert set(rep) == {"master", "moments", "staging", "reserved", "total", "gpu_state"}
    assert rep["reserved"] == 1024 and rep["total"] == 1024 and rep["gpu_state"] == rep["total"]


def test_bench_precision_override_and_one_gpu_only():
    """bench.py's --precision: the configuration's workload with other moments, its description
    renamed and its measured traffic set aside; and --gpus above 1 exits with a message before
    touching a device."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    sys.path.insert(0, str(root))
    import bench
    cfg, own = bench.config_of("c4", "fp32", "fp8")
    assert not own and cfg["precision"] == "fp8" and cfg["desc"].startswith("Lion, FP8 moment")
    assert bench.CONFIGS["c4"]["precision"] == "bf16"   # the table itself is unchanged
    cfg, own = bench.config_of("c3p", "fp24", None)
    assert own and cfg["master"] == "fp24" and cfg["precision"] == "bf16"
    cfg, own = bench.config_of("c1", "fp32", "fp32")
    assert own and cfg["desc"] == bench.CONFIGS["c1"]["desc"]
    run = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120, cwd=root)
    assert run.returncode != 0 and "one GPU" in (run.stdout + run.stderr)
