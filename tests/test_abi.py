"""The C-ABI library loads and exports what include/adambridge_hip.h declares (CPU).

No entry point that touches a device is called here: only the ABI version,
struct sizes, the SIMD-level switch and the backend name.
"""

import re
from pathlib import Path

import pytest

from adambridge_amd import _hip

HEADER = Path(__file__).resolve().parents[1] / "include" / "adambridge_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"ADAMBRIDGE_API\s+[\w\s\*]+?\b(adambridge_\w+)\s*\(", text)


def test_header_declares_the_reference_entry_points():
    names = set(declared_symbols())
    # the reference's 14 exports (kernels.c:1427-1641) all have a counterpart
    reference = {"adambridge_abi_version", "adambridge_detected_simd_level", "adambridge_simd_level",
                 "adambridge_set_simd_level", "adambridge_hparams_size", "adambridge_group_size",
                 "adambridge_segment_size", "adambridge_fused_adamw", "adambridge_pool_create",
                 "adambridge_pool_destroy", "adambridge_pool_threads", "adambridge_pool_set_spin",
                 "adambridge_multi_step", "adambridge_multi_apply"}
    assert reference <= names
    assert names == set(_hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _hip.open_library()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_layouts_and_version():
    lib = _hip.open_library()
    assert lib.adambridge_abi_version() == 5
    assert lib.adambridge_segment_size() == 128
    assert lib.adambridge_group_size() == 56
    assert lib.adambridge_hparams_size() == 40
    assert lib.adambridge_backend() == b"hip/gfx950"


def test_header_codes_match_the_python_mirror():
    """The storage codes and the segment flag the header defines are the ones _hip passes."""
    text = HEADER.read_text()
    codes = {name: int(v) for name, v in re.findall(r"ADAMBRIDGE_(DT_\w+)\s*=\s*(\d+)", text)}
    mirror = {"DT_NONE": _hip.DT_NONE, "DT_F32": _hip.DT_F32, "DT_BF16": _hip.DT_BF16, "DT_FP8": _hip.DT_FP8,
              "DT_F24": _hip.DT_F24, "DT_PACKED": _hip.DT_PACKED, "DT_PACKED_FP8": _hip.DT_PACKED8,
              "DT_PACKED_LION": _hip.DT_PACKED_LION, "DT_PACKED_F32": _hip.DT_PACKED_F32,
              "DT_PACKED_F24": _hip.DT_PACKED_F24, "DT_PACKED_LION_F24": _hip.DT_PACKED_LION_F24,
              "DT_PACKED_FP8_F24": _hip.DT_PACKED8_F24, "DT_PACKED_LION_F32": _hip.DT_PACKED_LION_F32,
              "DT_PACKED_LION_FP8": _hip.DT_PACKED8_LION, "DT_PACKED_F24_F32": _hip.DT_PACKED_F24_F32,
              "DT_PACKED_LION_F24_F32": _hip.DT_PACKED_LION_F24_F32,
              "DT_PACKED_LION_FP8_F24": _hip.DT_PACKED8_LION_F24}
    assert codes == mirror
    flag = re.search(r"#define ADAMBRIDGE_SEG_OUT_PREVIOUS (\d+)", text)
    assert flag and int(flag.group(1)) == _hip.SEG_OUT_PREVIOUS


def test_simd_level_switch():
    k = _hip.HipKernels()
    assert k.detected_simd_level == "avx512"
    try:
        assert k.set_simd_level("scalar") == "scalar"
        assert k.simd_level == "scalar"
        assert k.set_simd_level("avx2") == "avx2"
    finally:
        assert k.set_simd_level(None) == "avx512"


def test_library_is_built_for_gfx950():
    data = _hip.LIB_PATH.read_bytes()
    assert b"gfx950" in data


@pytest.mark.parametrize("sym", ["hipMalloc", "hipHostMalloc"])
def test_links_the_hip_runtime(sym):
    assert sym.encode() in _hip.LIB_PATH.read_bytes()


# ------------------------------------------- argument validation, on the host

import ctypes  # noqa: E402

import numpy as np  # noqa: E402

from oracle import oracle as O  # noqa: E402


def _segment_variants():
    """(description, segment mutation, expected code) -- kernels.c:1537-1553 in order; every
    segment is invalid, so no call below reaches the device."""
    def m(**kw):
        return kw
    return [
        ("negative n", m(n=-1), -1),
        ("unknown algorithm", m(algorithm=5), -12),
        ("unknown master format", m(p_dtype=17), -13),
        ("no master", m(p=None), -2),
        ("no gradient", m(g=None), -2),
        ("no first moment", m(m=None), -2),
        ("AdamW without v", m(v=None), -2),
        ("FP24 master without its low plane", m(p_dtype=O.DT_F24, p_lo=None), -2),
        ("gradient dtype", m(g_dtype=O.DT_FP8), -3),
        ("moment dtype", m(mv_dtype=O.DT_F24), -4),
        ("output dtype", m(out_dtype=O.DT_FP8), -5),
        ("output missing", m(out=None), -6),
        ("FP8 without scales", m(mv_dtype=O.DT_FP8, m_scale=None), -7),
        ("negative offset", m(offset=-128), -11),
        ("FP8 offset not a block multiple", m(mv_dtype=O.DT_FP8, offset=64), -11),
    ]


@pytest.mark.parametrize("desc,mut,code", _segment_variants(), ids=[v[0] for v in _segment_variants()])
def test_validation_codes_match_the_reference(desc, mut, code):
    lib = _hip.HipKernels()._lib
    oracle = O.load_oracle()
    rng = np.random.default_rng(3)
    case = O.make_case(rng, 1000, mv_dtype=O.DT_FP8, explicit=False)
    group = O.group_struct(case.group)
    hp = O.HParams(0.9, 0.999, 0.1, 0.001, 1.0, 1e-3, 1.0, 1e-8, 7, 1)
    for need_group in (False, True):
        seg = O.segment_for(case, group)
        for k, val in mut.items():
            setattr(seg, k, val)
        good = O.segment_for(case, group)   # a valid segment first: validation covers every segment
        arr = (ctypes.POINTER(O.Segment) * 2)(ctypes.pointer(good), ctypes.pointer(seg))
        codes = {"oracle": oracle.abo_check_segment(ctypes.byref(seg), int(need_group))}
        hps = (_hip.HParams * 2)(*[_hip.HParams(*[getattr(hp, f) for f, _ in O.HParams._fields_])] * 2)
        harr = ctypes.cast(arr, ctypes.POINTER(ctypes.POINTER(_hip.Segment)))
        codes["hip"] = (lib.adambridge_multi_step(None, harr, 2, 0) if need_group
                        else lib.adambridge_multi_apply(None, harr, hps, 2, 0))
        if O.reference_available():
            ref = O.load_reference()
            rhps = (O.HParams * 2)(hp, hp)
            codes["reference"] = (ref.adambridge_multi_step(None, arr, 2, 1) if need_group
                                  else ref.adambridge_multi_apply(None, arr, rhps, 2, 1))
        assert set(codes.values()) == {code}, (desc, need_group, codes)
    # a valid segment without a group: multi_step refuses it (-8)
    seg = O.segment_for(case, None)
    arr = (ctypes.POINTER(_hip.Segment) * 1)(ctypes.cast(ctypes.pointer(seg), ctypes.POINTER(_hip.Segment)))
    assert lib.adambridge_multi_step(None, arr, 1, 0) == -8


def test_fused_adamw_argument_codes():
    """kernels.c:1518-1535: the same checks and codes; none reaches the device."""
    lib = _hip.HipKernels()._lib
    hp = _hip.HParams(0.9, 0.999, 0.1, 0.001, 1.0, 1e-3, 1.0, 1e-8, 7, 1)
    buf = (ctypes.c_float * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    F32, BF16, FP8 = _hip.DT_F32, _hip.DT_BF16, _hip.DT_FP8
    call = lib.adambridge_fused_adamw
    assert call(p, p, BF16, p, p, BF16, p, BF16, -1, 0, ctypes.byref(hp)) == -1
    assert call(p, p, BF16, p, p, BF16, p, BF16, 8, 0, None) == -1
    assert call(p, p, BF16, p, p, BF16, p, BF16, 0, 0, ctypes.byref(hp)) == 0   # nothing to do
    assert call(None, p, BF16, p, p, BF16, p, BF16, 8, 0, ctypes.byref(hp)) == -2
    assert call(p, p, BF16, p, None, BF16, p, BF16, 8, 0, ctypes.byref(hp)) == -2
    assert call(p, p, FP8, p, p, BF16, p, BF16, 8, 0, ctypes.byref(hp)) == -3
    assert call(p, p, F32, p, p, FP8, p, BF16, 8, 0, ctypes.byref(hp)) == -4
    assert call(p, p, F32, p, p, F32, p, FP8, 8, 0, ctypes.byref(hp)) == -5
    assert call(p, p, F32, p, p, F32, None, BF16, 8, 0, ctypes.byref(hp)) == -6


def test_check_conversions_argument_codes():
    """adambridge_check_conversions rejects a missing or empty result array before any device call."""
    lib = _hip.open_library()
    assert lib.adambridge_check_conversions(0, None, 5) == -2
    buf = (ctypes.c_uint64 * 5)()
    assert lib.adambridge_check_conversions(0, buf, 0) == -2


def test_convert_argument_codes():
    """adambridge_convert's checks; none reaches the device."""
    lib = _hip.open_library()
    buf = (ctypes.c_float * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    F32, BF16, FP8 = _hip.DT_F32, _hip.DT_BF16, _hip.DT_FP8
    assert lib.adambridge_convert(p, None, F32, p, None, BF16, -1, 0) == -1
    assert lib.adambridge_convert(p, None, F32, p, None, 7, 8, 0) == -4
    assert lib.adambridge_convert(p, None, _hip.DT_F24, p, None, F32, 8, 0) == -4
    assert lib.adambridge_convert(p, None, F32, p, None, BF16, 8, 2) == -4
    assert lib.adambridge_convert(p, None, F32, p, None, BF16, 0, 0) == 0
    assert lib.adambridge_convert(None, None, F32, p, None, BF16, 8, 0) == -2
    assert lib.adambridge_convert(p, None, F32, None, None, BF16, 8, 0) == -2
    assert lib.adambridge_convert(p, None, FP8, p, None, F32, 8, 0) == -7
    assert lib.adambridge_convert(p, None, F32, p, None, FP8, 8, 1) == -7


def test_convert_plane_argument_codes_and_capabilities():
    """adambridge_convert_plane's checks of both planes, all made before anything is launched (an
    empty copy of valid planes returns 0); adambridge_capabilities names what the library adds to
    the reference's ABI version 5."""
    lib = _hip.open_library()
    buf = (ctypes.c_uint8 * 64)()
    base = ctypes.addressof(buf) + (-ctypes.addressof(buf) % 16)
    P = _hip.Plane
    F32, BF16, F24, P8 = _hip.DT_F32, _hip.DT_BF16, _hip.DT_F24, _hip.DT_PACKED8

    def rc(src, dst, n=0, flags=0):
        return lib.adambridge_convert_plane(ctypes.byref(src), ctypes.byref(dst), n, 0, 0, flags)

    ok = P(base, None, 0, F32, 0)
    assert rc(ok, ok) == 0
    assert rc(ok, ok, -1) == -1
    assert rc(ok, ok, 0, 2) == -1                                   # unknown flag
    assert lib.adambridge_convert_plane(None, ctypes.byref(ok), 0, 0, 0, 0) == -2
    assert rc(P(None, None, 0, F32, 0), ok) == -2
    assert rc(P(base, None, 0, F24, 0), ok) == -2                   # FP24 needs its low bytes
    assert rc(ok, P(base, None, 0, _hip.DT_FP8, 0)) == -13
    assert rc(ok, P(base, None, 0, _hip.DT_PACKED, 0)) == -13
    assert rc(P(base + 2, None, 0, F32, 0), ok) == -14
    assert rc(P(base + 1, None, 0, BF16, 0), ok) == -14
    assert rc(P(base + 8, None, 0, P8, 0), ok) == -14               # FP8 records are 16-byte aligned
    assert rc(P(base, None, 640, P8, 0), ok) == 0                    # Lion FP8 records: 640-byte stride
    assert rc(P(base, None, 640, P8, 31), ok) == 0                   # group_log2 unused there
    assert rc(P(base, None, 496, P8, 0), ok) == -1                   # shorter than a record's masters
    assert rc(P(base, None, 648, P8, 0), ok) == -14                  # records stay 16-byte aligned
    assert rc(P(base, None, 1536, F32, 31), ok) == -1
    assert rc(P(base, None, -16, F32, 1), ok) == -1
    assert rc(P(base, None, 18, F32, 1), ok) == -14
    assert rc(P(base, base + 1, 1792, F24, 8), P(base, None, 16, F32, 1)) == 0
    assert rc(P(base, base + 256, 640, F24, 7), P(base, None, 16, F32, 1)) == 0   # an FP8 record's FP24 planes
    caps = lib.adambridge_capabilities()
    assert caps == sum(_hip.CAPABILITIES.values())
    assert lib.adambridge_abi_version() == 5


def test_pool_threads_without_a_pool():
    """kernels.c:1484: adambridge_pool_threads(NULL) is 1."""
    lib = _hip.open_library()
    assert lib.adambridge_pool_threads(None) == 1


# ----------------------------------------------------------- the launch plan

MAX_TILES = (0xFFFFFFFF // 256) // 8 * 8   # workgroups of one dispatch: 2^32 - 1 lanes, whole rounds of 8 XCDs


def _fake_segments(specs):
    """Segments over fake 16-byte-aligned device addresses: planning reads no buffer and launches nothing."""
    segs = []
    for k, (n, algo, p_dtype) in enumerate(specs):
        segs.append(_hip.Segment(p=0x10000000, g=0x20000000, out=0x30000000, n=n, step=1, index=k,
                                 g_dtype=_hip.DT_BF16, mv_dtype=_hip.DT_BF16, out_dtype=_hip.DT_BF16,
                                 algorithm=algo, p_dtype=p_dtype))
    k = _hip.HipKernels()
    return k, segs, k.segment_array([ctypes.pointer(s) for s in segs])


def test_launch_plan_splits_a_segment_at_the_dispatch_limit():
    """A segment whose tiles overflow one dispatch continues in the next launch from the tile where
    the first launch stopped (its entry's first tile moved back by the tiles already taken)."""
    big = MAX_TILES * 1024 + 5000   # 1024-element tiles: MAX_TILES + 5 tiles
    k, segs, arr = _fake_segments([(3000, 0, _hip.DT_PACKED), (big, 0, _hip.DT_PACKED), (100, 0, _hip.DT_PACKED)])
    rows = k.plan_launches(arr)
    variant = rows[0][1]
    assert rows == [(0, variant, 0, MAX_TILES), (0, variant, 3, MAX_TILES),
                    (1, variant, -(MAX_TILES - 3), 9), (1, variant, 8, 9)]
    # every tile of every segment in exactly one launch
    launch_tiles = {launch: tiles for launch, _, _, tiles in rows}
    assert sum(launch_tiles.values()) == 3 + (MAX_TILES + 5) + 1


def test_launch_plan_batches_by_variant_and_staging_slot():
    """One launch per kernel variant, split where a variant has more segments than a staging slot
    holds (128 KiB of 152-byte entries: 862); variants in index order, segments in call order."""
    specs = [(1000 + k, 1 if k % 3 == 0 else 0, _hip.DT_PACKED_LION if k % 3 == 0 else _hip.DT_PACKED)
             for k in range(2400)]
    k, segs, arr = _fake_segments(specs)
    rows = k.plan_launches(arr)
    assert len(rows) == 2400
    by_launch: dict = {}
    for launch, variant, first, tiles in rows:
        by_launch.setdefault(launch, []).append((variant, first, tiles))
    sizes = [len(v) for _, v in sorted(by_launch.items())]
    assert sizes == [862, 738, 800]   # AdamW pairs (1600: 862 + 738), then Lion records (800)
    # expected: per variant, segments in call order, each starting where the previous one's tiles end
    order = [n for n, algo, _ in specs if algo == 0] + [n for n, algo, _ in specs if algo == 1]
    chunks = [order[:862], order[862:1600], order[1600:]]
    for (_, entries), ns in zip(sorted(by_launch.items()), chunks):
        assert len({v for v, _, _ in entries}) == 1
        tiles = [-(-n // 512) for n in ns]   # each variant moves fewer than 2^25 elements: 512-element tiles
        assert [f for _, f, _ in entries] == [sum(tiles[:j]) for j in range(len(tiles))]
        assert entries[0][2] == sum(tiles)


def test_launch_tile_follows_the_launch_size():
    """512-element tiles for a launch of at most 2^25 elements of a two- or four-element-per-lane
    kernel, 1024 above; FP8 launches keep 2048 (one 128-element block per 16-lane group)."""
    small = 1 << 24
    for sizes, tile in (([small], 512), ([small, small], 512), ([small, small, 1], 1024), ([3 << 24], 1024)):
        k, segs, arr = _fake_segments([(n, 0, _hip.DT_PACKED) for n in sizes])
        rows = k.plan_launches(arr)
        assert rows[-1][3] == sum(-(-n // tile) for n in sizes), (sizes, tile)
    k, segs, arr = _fake_segments([(small, 0, _hip.DT_PACKED8)])
    for s in segs:
        s.mv_dtype, s.m_scale, s.v_scale = _hip.DT_FP8, 0x40000000, 0x50000000
    assert k.plan_launches(arr)[0][3] == small // 2048


def test_launch_plan_validates_first():
    k, segs, arr = _fake_segments([(100, 0, _hip.DT_PACKED), (100, 0, _hip.DT_PACKED)])
    segs[1].g = None
    with pytest.raises(RuntimeError, match="code -2"):
        k.plan_launches(arr)


def test_noalloc_refuses_more_segments_than_its_array_holds():
    """adambridge_multi_step_noalloc: 1025 valid segments are refused (-9) with the reason, before
    any device call; invalid segments get the validation code first."""
    k, segs, arr = _fake_segments([(100, 0, _hip.DT_PACKED)] * 1025)
    group = _hip.Group(1e-3, 0.9, 0.999, 1e-8, 0.01, 0, 1, 0)
    for s in segs:
        s.group = ctypes.pointer(group)
    with pytest.raises(RuntimeError, match=r"code -9\): .*at most 1024"):
        k.multi_step_noalloc(None, arr)
    segs[3].group = None
    with pytest.raises(RuntimeError, match=r"code -8"):
        k.multi_step_noalloc(None, arr)
    assert k._lib.adambridge_multi_step_noalloc(None, None, 5) == -1
    assert k._lib.adambridge_multi_step_noalloc(None, None, 0) == 0


def test_stream_copy_argument_codes():
    """adambridge_stream_copy's checks; none reaches the device."""
    lib = _hip.open_library()
    buf = (ctypes.c_float * 16)()
    p = ctypes.addressof(buf) // 16 * 16 + 16
    assert lib.adambridge_stream_copy(p, p, -16) == -1
    assert lib.adambridge_stream_copy(p, p, 24) == -1
    assert lib.adambridge_stream_copy(p, p, 0) == 0
    assert lib.adambridge_stream_copy(None, p, 16) == -2
    assert lib.adambridge_stream_copy(p + 4, p, 16) == -14
