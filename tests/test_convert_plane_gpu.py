"""adambridge_convert_plane, the kernel behind the FP24 master's conversions and the working weights a
master gives (GPU), bit for bit against the oracle's rounding rules (oracle/abh_oracle.c
abo_f24_round, abo_bf16_rne; kernels.c:108-112, 120-126, 145-160) -- over special values and every
low-byte value of the bits FP24 rounding drops -- and through every state layout's master plane:
records' strided columns, FP8 block records, separate FP24 planes."""

import numpy as np
import pytest
import torch

import adambridge_amd as ab
from adambridge_amd import _hip
from adambridge_amd import formats as F
from adambridge_amd import state as S
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def special_highs() -> np.ndarray:
    """High halves: zeros, the smallest and largest subnormals and normals, one, the largest finite
    (whose rounding may carry into infinity), infinities, quiet and signalling NaNs, each with
    either sign, plus a seeded sample of the rest."""
    base = [0x0000, 0x0001, 0x007F, 0x0080, 0x0081, 0x3F80, 0x3F7F, 0x7F7F, 0x7F7E, 0x7F80, 0x7FC0, 0x7F81,
            0x7FBF, 0x7FFF, 0x4B00, 0x3400]
    rng = np.random.default_rng(7)
    rest = rng.integers(0, 0x8000, 200)
    h = np.unique(np.concatenate([base, rest])).astype(np.uint32)
    return np.concatenate([h, h | 0x8000])


def every_low_byte() -> np.ndarray:
    """FP32 bit patterns: each high half above with middle bytes 0x00, 0x01, 0x7F, 0x80, 0xFE, 0xFF
    (the byte FP24 keeps: its lowest bit decides ties) and all 256 low bytes (the byte it drops)."""
    hi = special_highs()[:, None, None] << 16
    mid = np.array([0x00, 0x01, 0x7F, 0x80, 0xFE, 0xFF], np.uint32)[None, :, None] << 8
    low = np.arange(256, dtype=np.uint32)[None, None, :]
    return (hi | mid | low).reshape(-1).astype(np.uint32)


def device_f32(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.float32).copy()).to(DEV)


def u32(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int32).numpy().view(np.uint32)


def u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("seed", [None, 0x9E3779B9])
def test_fp24_rounding_matches_the_oracle_over_specials_and_every_low_byte(seed):
    bits = every_low_byte()
    offset = (1 << 32) - 1000   # the stream's 32-bit element index wraps inside the array
    hi, lo = F.fp24_encode(device_f32(bits), seed, offset)
    torch.cuda.synchronize()
    want = O.round_values(bits, "fp24", seed, offset) & np.uint32(0xFFFFFF00)   # the planes hold the top 24 bits
    got = (u16(hi).astype(np.uint32) << 16) | (lo.cpu().numpy().astype(np.uint32) << 8)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {bits.size} differ"
    # the planes expand back exactly, and FP24 into FP24 is a bit-for-bit copy (NaN payloads kept)
    assert np.array_equal(u32(F.fp24_join(hi, lo)), want)
    hi2, lo2 = torch.empty_like(hi), torch.empty_like(lo)
    F.convert_plane(_hip.fp24_plane(hi, lo), _hip.fp24_plane(hi2, lo2), hi.numel(), DEV)
    assert torch.equal(hi2.view(torch.int16), hi.view(torch.int16)) and torch.equal(lo2, lo)


@pytest.mark.parametrize("seed", [None, 12345])
def test_bf16_conversion_matches_the_oracle(seed):
    """Nearest: the working weight the kernels write (NaN quietened with sign and payload kept);
    stochastic: the BF16 moment store's rule, low 16 bits of the stream added, no NaN case."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    low = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1234], np.uint32)
    bits = (hi[:, None] | low[None, :]).reshape(-1)
    x = device_f32(bits)
    out = torch.empty(bits.size, dtype=torch.bfloat16, device=DEV)
    F.convert_plane(_hip.plane_of(x), _hip.plane_of(out), bits.size, DEV, 77, seed)
    torch.cuda.synchronize()
    assert np.array_equal(u16(out), O.round_values(bits, "bf16", seed, 77))
    if seed is None:
        assert np.array_equal(u16(F.bf16_weight(x)), O.round_values(bits, "bf16"))


def test_exact_conversions_copy_bits():
    """BF16 into FP32 and FP24, FP24 into FP32: every value copied bit for bit, signalling NaNs
    included (a value the destination holds is not rounded)."""
    codes = torch.arange(1 << 16, dtype=torch.int32, device=DEV).to(torch.int16).view(torch.bfloat16)
    f32 = torch.empty(codes.numel(), dtype=torch.float32, device=DEV)
    F.convert_plane(_hip.plane_of(codes), _hip.plane_of(f32), codes.numel(), DEV)
    hi = torch.empty_like(codes)
    lo = torch.full((codes.numel(),), 0xAB, dtype=torch.uint8, device=DEV)
    F.convert_plane(_hip.plane_of(codes), _hip.fp24_plane(hi, lo), codes.numel(), DEV, 0, 99)   # SR: still exact
    torch.cuda.synchronize()
    want = np.arange(1 << 16, dtype=np.uint32) << 16
    assert np.array_equal(u32(f32), want)
    assert np.array_equal(u16(hi), np.arange(1 << 16, dtype=np.uint16)) and int(lo.max()) == 0


def _values(n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, generator=g) * torch.exp(torch.empty(n).uniform_(-30.0, 30.0, generator=g))
    x[torch.rand(n, generator=g) < 0.01] = float("nan")
    x[torch.rand(n, generator=g) < 0.01] = -float("inf")
    x[torch.rand(n, generator=g) < 0.02] = 0.0
    return x.float()


LAYOUTS = [("pairs", "adamw", "bf16", "fp32"), ("lion-records", "lion", "bf16", "fp32"),
           ("f32-records", "adamw", "fp32", "fp32"), ("f24-records", "adamw", "bf16", "fp24"),
           ("lion-f24-records", "lion", "bf16", "fp24"), ("fp8-records", "adamw", "fp8", "fp32"),
           ("fp8-f24-records", "adamw", "fp8", "fp24"), ("lion-f32-records", "lion", "fp32", "fp32"),
           ("lion-fp8-records", "lion", "fp8", "fp32"), ("f24-f32-records", "adamw", "fp32", "fp24"),
           ("lion-f24-f32-records", "lion", "fp32", "fp24"), ("lion-fp8-f24-records", "lion", "fp8", "fp24"),
           ("separate", "adamw", "bf16", "fp24"), ("separate", "adamw", "fp8", "fp32")]


@pytest.mark.parametrize("layout,algorithm,precision,master", LAYOUTS)
@pytest.mark.parametrize("n", [1, 255, 256, 1000, 4096 + 7])
def test_master_planes_of_every_layout(layout, algorithm, precision, master, n):
    """Through each layout's master plane: a state built from FP32 values holds them rounded as the
    master stores them (FP24: nearest), master_fp32() returns exactly those, the working weights
    equal the oracle's BF16 rounding of them, an FP24 checkpoint's planes load bit for bit, and the
    padding slots of the records are left as they were."""
    x = _values(n, n)
    bits = x.view(torch.int32).numpy().view(np.uint32)
    stored = O.round_values(bits, "fp24") & np.uint32(0xFFFFFF00) if master == "fp24" else bits
    st = S.new_states(layout, algorithm, precision, master, DEV, [x.to(DEV)], place=False)[0]
    assert st.layout == layout
    pad_before = None
    if layout != "separate":   # every byte of the buffer random, then the masters loaded again
        g = torch.Generator(device=DEV).manual_seed(n)
        st.current.view(torch.uint8).copy_(torch.randint(0, 256, st.current.view(torch.uint8).shape, generator=g,
                                                         device=DEV, dtype=torch.uint8))
        pad_before = st.current.clone()
        st.load(master=x.to(DEV))
    got = u32(st.master_fp32())
    assert np.array_equal(got, stored)
    w = torch.empty(n, dtype=torch.bfloat16, device=DEV)
    st.write_weights(w)
    f = torch.empty(n, dtype=torch.float32, device=DEV)
    st.write_weights(f)
    torch.cuda.synchronize()
    assert np.array_equal(u16(w), O.round_values(stored, "bf16"))
    assert np.array_equal(u32(f), stored)
    if pad_before is not None:
        # the load wrote the master slots of elements 0 .. n - 1 and no other byte of the buffer
        written = np.zeros(st.current.nbytes, bool)
        plane = st.master_plane()
        i = np.arange(n, dtype=np.int64)
        if layout in ("fp8-records", "lion-fp8-records"):   # the plane's stride is the record size
            rec = 768 if layout == "fp8-records" else 640
            assert plane.stride in (0, rec) and (plane.stride == rec or layout == "fp8-records")
            offs = [(i >> 7) * rec + np.where(i & 4, 256, 0) + ((i >> 3) & 15) * 16 + (i & 3) * 4 + k for k in range(4)]
        elif master == "fp24":   # hi plane at the record's start, lo plane right after it
            g = plane.group_log2
            at = (i >> g) * plane.stride + (i & ((1 << g) - 1)) * 2
            offs = [at, at + 1, (i >> g) * plane.stride + (2 << g) + (i & ((1 << g) - 1))]
        else:
            at = (i >> plane.group_log2) * plane.stride + (i & ((1 << plane.group_log2) - 1)) * 4
            offs = [at + k for k in range(4)]
        for o in offs:
            written[o] = True
        now = st.current.view(torch.uint8).reshape(-1).cpu().numpy()
        before = pad_before.view(torch.uint8).reshape(-1).cpu().numpy()
        assert np.array_equal(now[~written], before[~written]), "the conversion wrote outside the master slots"
    if master == "fp24":   # checkpoint planes in, bit for bit; export gives them back
        y = _values(n, n + 1).view(torch.int32).numpy().view(np.uint32)
        hi = torch.from_numpy((y >> 16).astype(np.int32).astype(np.int16)).view(torch.bfloat16)
        lo = torch.from_numpy(((y >> 8) & 0xFF).astype(np.uint8))
        st.load(master={"precision": "fp24", "hi": hi, "lo": lo})
        exp = st.export_master()
        assert np.array_equal(u16(exp["hi"]), u16(hi)) and np.array_equal(exp["lo"].cpu().numpy(), lo.numpy())
        assert np.array_equal(u32(st.master_fp32()), y & 0xFFFFFF00)


def test_plane_conversion_argument_codes_on_the_device():
    k = _hip.load()
    x = torch.zeros(16, dtype=torch.float32, device=DEV)
    ok = _hip.plane_of(x)
    lib = k._lib
    import ctypes

    def rc(src, dst, n=16, flags=0):
        return lib.adambridge_convert_plane(ctypes.byref(src), ctypes.byref(dst), n, 0, 0, flags)

    assert rc(ok, ok, 0) == 0
    assert rc(ok, ok, -1) == -1
    assert rc(ok, ok, 16, 2) == -1
    assert rc(_hip.Plane(x.data_ptr(), None, 0, 3, 0), ok) == -13          # FP8 is no plane type
    assert rc(_hip.Plane(x.data_ptr(), None, 0, _hip.DT_F24, 0), ok) == -2   # FP24 without its low bytes
    assert rc(_hip.Plane(x.data_ptr() + 2, None, 0, _hip.DT_F32, 0), ok) == -14
    assert rc(_hip.Plane(x.data_ptr(), None, 6, _hip.DT_F32, 1), ok) == -14  # stride not a multiple of 4
    assert rc(_hip.Plane(x.data_ptr(), None, 16, _hip.DT_F32, 31), ok) == -1
    assert "convert_plane" in k.capabilities


def test_delayed_flush_of_a_large_parameter_allocates_nothing():
    """The weights a delayed optimizer owes are written straight from the masters into the parameters
    (one conversion pass each): flush() of a 2^28-element parameter allocates no device memory."""
    torch.cuda.set_device(DEV)
    n = 1 << 28
    p = torch.nn.Parameter(torch.randn(n, device=DEV, dtype=torch.bfloat16).mul_(0.02))
    opt = ab.AdamBridge([p], lr=1e-3, precision="bf16", delay_updates=True)
    try:
        for _ in range(2):
            p.grad = torch.randn(n, device=DEV, dtype=torch.bfloat16).mul_(1e-3)
            opt.step()
        p.grad = None
        torch.cuda.synchronize()
        master = opt._ordered[0].state.master_fp32()
        want = O.round_values(u32(master), "bf16")
        del master
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(DEV)
        base = torch.cuda.memory_allocated(DEV)
        opt.flush()
        torch.cuda.synchronize()
        assert torch.cuda.max_memory_allocated(DEV) - base < 1 << 20
        assert np.array_equal(u16(p.detach()), want)
    finally:
        opt.close()
