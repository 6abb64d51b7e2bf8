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
