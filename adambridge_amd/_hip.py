"""ctypes binding of libadambridge_hip.so (the HIP fused-update library).

Plays the part of the reference's ``adambridge/native.py`` (NativeKernels,
native.py:273-435): the same struct mirrors (``HParams``, ``Group``,
``Segment``), ABI and struct-size checks at load, and a RuntimeError for every
non-zero return code.  Pointers in segments are device pointers; a "pool" is a
launch queue on a HIP stream.

There is no fallback: if the library is missing or fails its checks, ``load()``
raises.  ``torch`` must be imported first so that the library binds to the HIP
runtime torch already loaded (same SONAME), and shares its streams.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

__all__ = ["HipKernels", "HParams", "Group", "Segment", "Plane", "plane_of", "fp24_plane", "load", "LIB_PATH", "DT_NONE", "DT_F32", "DT_BF16",
           "DT_FP8", "DT_F24", "DT_PACKED", "DT_PACKED8", "DT_PACKED_LION", "DT_PACKED_F32", "DT_PACKED_F24", "DT_PACKED_LION_F24",
           "DT_PACKED8_F24", "DT_PACKED_LION_F32", "DT_PACKED8_LION", "DT_PACKED_F24_F32", "DT_PACKED_LION_F24_F32", "DT_PACKED8_LION_F24",
           "SEG_OUT_PREVIOUS", "MOMENT_CODES", "MASTER_CODES",
           "ALGORITHMS", "SIMD_NAMES"]

LIB_PATH = Path(__file__).resolve().with_name("libadambridge_hip.so")
ABI_VERSION = 5

(DT_NONE, DT_F32, DT_BF16, DT_FP8, DT_F24, DT_PACKED, DT_PACKED8, DT_PACKED_LION, DT_PACKED_F32, DT_PACKED_F24,
 DT_PACKED_LION_F24, DT_PACKED8_F24, DT_PACKED_LION_F32, DT_PACKED8_LION, DT_PACKED_F24_F32,
 DT_PACKED_LION_F24_F32, DT_PACKED8_LION_F24) = range(17)
SEG_OUT_PREVIOUS = 1   # Segment.reserved: out receives the weight of the master before the update
_DTYPE_CODES = {torch.float32: DT_F32, torch.bfloat16: DT_BF16}
MOMENT_CODES = {"fp32": DT_F32, "bf16": DT_BF16, "fp8": DT_FP8}
MASTER_CODES = {"fp32": DT_F32, "fp24": DT_F24}
ALGORITHMS = {"adamw": 0, "lion": 1}
SIMD_NAMES = {0: "scalar", 1: "avx2", 2: "avx512"}


class HParams(ctypes.Structure):
    """adambridge_hparams (include/adambridge_hip.h; reference kernels.c:77-88, native.py:58-70)."""
    _fields_ = [("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
                ("one_minus_beta1", ctypes.c_float), ("one_minus_beta2", ctypes.c_float),
                ("decay", ctypes.c_float), ("step_size", ctypes.c_float),
                ("inv_sqrt_bc2", ctypes.c_float), ("eps", ctypes.c_float),
                ("seed", ctypes.c_uint32), ("stochastic", ctypes.c_int32)]


class Group(ctypes.Structure):
    """adambridge_group (reference kernels.c:736-745, native.py:73-85)."""
    _fields_ = [("lr", ctypes.c_double), ("beta1", ctypes.c_double), ("beta2", ctypes.c_double),
                ("eps", ctypes.c_double), ("weight_decay", ctypes.c_double),
                ("seed", ctypes.c_uint64), ("stochastic", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class Segment(ctypes.Structure):
    """adambridge_segment with device pointers (reference kernels.c:747-769, native.py:88-111)."""
    _fields_ = [("p", ctypes.c_void_p), ("p_lo", ctypes.c_void_p), ("g", ctypes.c_void_p),
                ("m", ctypes.c_void_p), ("v", ctypes.c_void_p), ("m_scale", ctypes.c_void_p),
                ("v_scale", ctypes.c_void_p), ("out", ctypes.c_void_p), ("group", ctypes.POINTER(Group)),
                ("n", ctypes.c_int64), ("step", ctypes.c_int64), ("index", ctypes.c_uint64),
                ("offset", ctypes.c_int64), ("g_dtype", ctypes.c_int32), ("mv_dtype", ctypes.c_int32),
                ("out_dtype", ctypes.c_int32), ("algorithm", ctypes.c_int32), ("p_dtype", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


class Plane(ctypes.Structure):
    """adambridge_plane: element i at data + (i >> group_log2) * stride + (i mod 2^group_log2) * size
    (stride 0: contiguous); an FP24 plane's low bytes likewise from ``lo`` (no reference counterpart)."""
    _fields_ = [("data", ctypes.c_void_p), ("lo", ctypes.c_void_p), ("stride", ctypes.c_int64),
                ("dtype", ctypes.c_int32), ("group_log2", ctypes.c_int32)]


CONVERT_STOCHASTIC = 1
CAPABILITIES = {"packed_layouts": 0x01, "out_previous": 0x02, "noalloc": 0x04, "convert": 0x08,
                "convert_plane": 0x10, "stream_copy": 0x20, "fp8_f24_records": 0x40, "lion_f32_records": 0x80,
                "lion_fp8_records": 0x100, "f24_f32_records": 0x200,
                "lion_f24_f32_records": 0x400, "lion_fp8_f24_records": 0x800}


def plane_of(t: torch.Tensor) -> Plane:
    """The plane of a contiguous float32 or bfloat16 device tensor."""
    if not t.is_contiguous() or t.dtype not in _DTYPE_CODES:
        raise ValueError(f"a plane is a contiguous float32 or bfloat16 tensor, got {t.dtype}"
                         f"{'' if t.is_contiguous() else ' (strided)'}")
    return Plane(t.data_ptr(), None, 0, _DTYPE_CODES[t.dtype], 0)


def fp24_plane(hi: torch.Tensor, lo: torch.Tensor) -> Plane:
    """The plane of an FP24 master's contiguous hi (BF16 bits) and lo (uint8) tensors."""
    if not (hi.is_contiguous() and lo.is_contiguous()) or hi.element_size() != 2 or lo.element_size() != 1:
        raise ValueError("an FP24 plane is a contiguous 2-byte hi tensor and a contiguous 1-byte lo tensor")
    return Plane(hi.data_ptr(), lo.data_ptr(), 0, DT_F24, 0)


_SegArray = ctypes.POINTER(ctypes.POINTER(Segment))

# Every symbol include/adambridge_hip.h declares.
EXPORTS = (
    "adambridge_abi_version", "adambridge_detected_simd_level", "adambridge_simd_level",
    "adambridge_set_simd_level", "adambridge_hparams_size", "adambridge_group_size", "adambridge_segment_size",
    "adambridge_fused_adamw", "adambridge_pool_create", "adambridge_pool_destroy", "adambridge_pool_threads",
    "adambridge_pool_set_spin", "adambridge_multi_step", "adambridge_multi_apply", "adambridge_pool_set_stream",
    "adambridge_pool_sync", "adambridge_set_stream", "adambridge_last_error", "adambridge_backend",
    "adambridge_check_conversions", "adambridge_convert", "adambridge_plan_launches",
    "adambridge_multi_step_noalloc", "adambridge_stream_copy", "adambridge_recycle_device_memory",
    "adambridge_convert_plane", "adambridge_capabilities",
)


def open_library(path: Path = LIB_PATH) -> ctypes.CDLL:
    """dlopen the library and declare every entry point; checks the ABI and struct layouts.
    Needs no GPU (no entry point that touches the device is called)."""
    if not path.exists():
        raise RuntimeError(f"{path} is not built: run `python -m adambridge_amd.build` (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(path))
    i32, i64, u64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_void_p
    sig = {
        "adambridge_abi_version": (ctypes.c_int, []),
        "adambridge_detected_simd_level": (ctypes.c_int, []),
        "adambridge_simd_level": (ctypes.c_int, []),
        "adambridge_set_simd_level": (ctypes.c_int, [ctypes.c_int]),
        "adambridge_hparams_size": (ctypes.c_int, []),
        "adambridge_group_size": (ctypes.c_int, []),
        "adambridge_segment_size": (ctypes.c_int, []),
        "adambridge_fused_adamw": (ctypes.c_int, [vp, vp, ctypes.c_int, vp, vp, ctypes.c_int, vp, ctypes.c_int,
                                                  i64, u64, ctypes.POINTER(HParams)]),
        "adambridge_pool_create": (vp, [i32, vp, i32]),
        "adambridge_pool_destroy": (None, [vp]),
        "adambridge_pool_threads": (i32, [vp]),
        "adambridge_pool_set_spin": (None, [vp, i32]),
        "adambridge_multi_step": (ctypes.c_int, [vp, _SegArray, i32, i32]),
        "adambridge_multi_apply": (ctypes.c_int, [vp, _SegArray, ctypes.POINTER(HParams), i32, i32]),
        "adambridge_pool_set_stream": (ctypes.c_int, [vp, vp]),
        "adambridge_pool_sync": (ctypes.c_int, [vp]),
        "adambridge_set_stream": (ctypes.c_int, [vp]),
        "adambridge_last_error": (ctypes.c_char_p, []),
        "adambridge_backend": (ctypes.c_char_p, []),
        "adambridge_check_conversions": (ctypes.c_int, [ctypes.c_uint32, ctypes.POINTER(u64), i32]),
        "adambridge_convert": (ctypes.c_int, [vp, vp, i32, vp, vp, i32, i64, i32]),
        "adambridge_plan_launches": (ctypes.c_int, [_SegArray, i32, ctypes.POINTER(i64), i32]),
        "adambridge_multi_step_noalloc": (ctypes.c_int, [vp, _SegArray, i32]),
        "adambridge_stream_copy": (ctypes.c_int, [vp, vp, i64]),
        "adambridge_recycle_device_memory": (ctypes.c_int, [i64]),
        "adambridge_convert_plane": (ctypes.c_int, [ctypes.POINTER(Plane), ctypes.POINTER(Plane), i64, u64,
                                                    ctypes.c_uint32, i32]),
        "adambridge_capabilities": (ctypes.c_uint32, []),
    }
    for name in EXPORTS:
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = sig[name]
    if lib.adambridge_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI {lib.adambridge_abi_version()}, expected {ABI_VERSION}")
    for fn, struct in (("adambridge_hparams_size", HParams), ("adambridge_group_size", Group),
                       ("adambridge_segment_size", Segment)):
        if getattr(lib, fn)() != ctypes.sizeof(struct):
            raise RuntimeError(f"{fn}: struct layout mismatch between the library and Python")
    return lib


class HipKernels:
    """The loaded library (reference counterpart: NativeKernels, native.py:273-435)."""

    def __init__(self, path: Path = LIB_PATH):
        self.path = path
        self._lib = open_library(path)

    # -- identity and the SIMD level reproduced ------------------------------

    @property
    def backend(self) -> str:
        return self._lib.adambridge_backend().decode()

    CONVERSION_CHECKS = ("stochastic E4M3", "stochastic E5M2", "nearest-even E4M3", "nearest-even E5M2",
                         "nearest-even BF16", "square roots", "FP8 decode",
                         "divisions (sampled)", "reciprocals")

    def check_conversions(self, seed: int = 0) -> dict[str, int]:
        """Differing results between the current device's conversion instructions and the
        reference's rounding rules over every FP32 input in the ranges the kernels use them
        (adambridge_check_conversions); all zero on a conforming device."""
        out = (ctypes.c_uint64 * len(self.CONVERSION_CHECKS))()
        rc = self._lib.adambridge_check_conversions(seed & 0xFFFFFFFF, out, len(out))
        if rc < 0:
            raise RuntimeError(f"adambridge_check_conversions: {rc} {self._lib.adambridge_last_error().decode()}")
        return dict(zip(self.CONVERSION_CHECKS, (int(x) for x in out)))

    @property
    def simd_level(self) -> str:
        return SIMD_NAMES[self._lib.adambridge_simd_level()]

    @property
    def detected_simd_level(self) -> str:
        return SIMD_NAMES[self._lib.adambridge_detected_simd_level()]

    def set_simd_level(self, name: str | None) -> str:
        """Reproduce another reference ISA's rounding (``None`` restores AVX-512)."""
        code = -1 if name is None else {v: k for k, v in SIMD_NAMES.items()}[name]
        return SIMD_NAMES[self._lib.adambridge_set_simd_level(code)]

    @staticmethod
    def supports(grad_dtype: torch.dtype, moment_precision: str, out_dtype: torch.dtype | None) -> bool:
        return (grad_dtype in _DTYPE_CODES and moment_precision in MOMENT_CODES
                and (out_dtype is None or out_dtype in _DTYPE_CODES))

    @staticmethod
    def dtype_code(dtype: torch.dtype | None) -> int:
        return DT_NONE if dtype is None else _DTYPE_CODES[dtype]

    # -- queues --------------------------------------------------------------

    def create_pool(self) -> int:
        """A launch queue on the current device (reference: adambridge_pool_create)."""
        handle = self._lib.adambridge_pool_create(0, None, 0)
        if not handle:
            raise RuntimeError(f"adambridge_pool_create failed: {self.last_error()}")
        return handle

    def destroy_pool(self, handle: int) -> None:
        self._lib.adambridge_pool_destroy(handle)

    def pool_threads(self, handle: int) -> int:
        return self._lib.adambridge_pool_threads(handle)

    def set_pool_stream(self, handle: int, stream: torch.cuda.Stream | int | None) -> None:
        self._lib.adambridge_pool_set_stream(handle, _stream_handle(stream))

    def pool_sync(self, handle: int | None) -> None:
        self._check(self._lib.adambridge_pool_sync(handle), "adambridge_pool_sync")

    def set_stream(self, stream: torch.cuda.Stream | int | None) -> None:
        """The calling thread's stream for pool-less calls."""
        self._lib.adambridge_set_stream(_stream_handle(stream))

    def last_error(self) -> str:
        return self._lib.adambridge_last_error().decode(errors="replace")

    # -- updates ---------------------------------------------------------------

    @staticmethod
    def segment_array(segments: list) -> ctypes.Array:
        """Array of Segment pointers for multi_step / multi_apply."""
        return (ctypes.POINTER(Segment) * len(segments))(*segments)

    def multi_step(self, pool: int | None, segments: ctypes.Array, threads: int = 0) -> None:
        """Enqueue an update of every segment; coefficients from each segment's group and step."""
        self._check(self._lib.adambridge_multi_step(pool, segments, len(segments), threads), "adambridge_multi_step")

    def multi_step_noalloc(self, stream: torch.cuda.Stream | int | None, segments: ctypes.Array) -> None:
        """multi_step on ``stream`` without any allocation (adambridge_multi_step_noalloc): segment
        tables in the library's static device array, at most 1024 segments per call; calls that
        overlap on one GPU race."""
        rc = self._lib.adambridge_multi_step_noalloc(_stream_handle(stream), segments, len(segments))
        if rc != 0:
            raise RuntimeError(f"adambridge_multi_step_noalloc rejected the update (code {rc}): {self.last_error()}")

    def multi_apply(self, pool: int | None, segments: ctypes.Array, hparams: list, threads: int = 0) -> None:
        """Like multi_step with explicit coefficients, one ``HParams`` per segment."""
        hps = (HParams * len(hparams))(*hparams)
        self._check(self._lib.adambridge_multi_apply(pool, segments, hps, len(segments), threads),
                    "adambridge_multi_apply")

    def plan_launches(self, segments: ctypes.Array) -> list[tuple[int, int, int, int]]:
        """(launch, kernel variant, first tile, launch tiles) of every entry of the launches a
        multi_apply / multi_step call over ``segments`` would make (adambridge_plan_launches); no
        device work."""
        count = self._lib.adambridge_plan_launches(segments, len(segments), None, 0)
        if count < 0:
            self._check(count, "adambridge_plan_launches")
        rows = (ctypes.c_int64 * (4 * max(count, 1)))()
        got = self._lib.adambridge_plan_launches(segments, len(segments), rows, count)
        if got != count:
            raise RuntimeError(f"adambridge_plan_launches returned {got}, then {count}")
        return [tuple(rows[4 * k: 4 * k + 4]) for k in range(count)]

    def stream_copy(self, src: torch.Tensor, dst: torch.Tensor) -> None:
        """Copy ``src`` into ``dst`` (same byte size, a multiple of 16) on the current stream with the
        update kernels' access type (adambridge_stream_copy): the known-size kernel that byte
        counters are calibrated with."""
        if src.nbytes != dst.nbytes or not (src.is_cuda and dst.is_cuda and src.is_contiguous() and dst.is_contiguous()):
            raise ValueError("stream_copy: two contiguous device tensors of the same byte size")
        with torch.cuda.device(dst.device):
            self.set_stream(torch.cuda.current_stream(dst.device))
            self._check(self._lib.adambridge_stream_copy(src.data_ptr(), dst.data_ptr(), dst.nbytes),
                        "adambridge_stream_copy")

    def recycle_device_memory(self, nbytes: int, device: torch.device) -> bool:
        """Allocate ``nbytes`` on ``device`` and free them at once (adambridge_recycle_device_memory),
        ahead of allocating a buffer of that size; False if the allocation failed (nothing held)."""
        with torch.cuda.device(device):
            return self._lib.adambridge_recycle_device_memory(int(nbytes)) == 0

    _CONVERT_DTYPES = {torch.float32: DT_F32, torch.bfloat16: DT_BF16, torch.float8_e4m3fn: DT_FP8,
                       torch.float8_e5m2: DT_FP8, torch.uint8: DT_FP8}

    def convert(self, src: torch.Tensor, src_scale: torch.Tensor | None, dst: torch.Tensor,
                dst_scale: torch.Tensor | None, n: int, role: str) -> None:
        """Re-encode ``n`` values of moment ``role`` ('m' or 'v') from ``src`` into ``dst`` on the current
        stream (adambridge_convert).  Formats follow the dtypes: float32, bfloat16, or FP8 codes (an
        FP8 / uint8 tensor padded to whole 128-element blocks, with one float32 scale per block)."""
        if role not in ("m", "v"):
            raise ValueError(f"role must be 'm' or 'v', got {role!r}")
        codes = []
        for what, t, scale in (("source", src, src_scale), ("destination", dst, dst_scale)):
            if t.device.type != "cuda" or not t.is_contiguous():
                raise ValueError(f"convert: the {what} must be a contiguous device tensor")
            code = self._CONVERT_DTYPES.get(t.dtype)
            if code is None:
                raise TypeError(f"convert: unsupported {what} dtype {t.dtype}")
            nb = -(-n // 128)
            need = nb * 128 if code == DT_FP8 else n
            if t.numel() < need:
                raise ValueError(f"convert: the {what} holds {t.numel()} values, {need} needed")
            if code == DT_FP8:
                if scale is None or scale.dtype != torch.float32 or not scale.is_contiguous() or scale.numel() < nb:
                    raise ValueError(f"convert: the FP8 {what} needs {nb} contiguous float32 scales")
                if scale.device != t.device:
                    raise ValueError("convert: scales on another device")
            codes.append(code)
        if src.device != dst.device:
            raise ValueError("convert: source and destination on different devices")
        with torch.cuda.device(dst.device):
            self._lib.adambridge_set_stream(torch.cuda.current_stream(dst.device).cuda_stream)
            rc = self._lib.adambridge_convert(src.data_ptr(), src_scale.data_ptr() if codes[0] == DT_FP8 else None,
                                              codes[0], dst.data_ptr(),
                                              dst_scale.data_ptr() if codes[1] == DT_FP8 else None, codes[1], n,
                                              0 if role == "m" else 1)
        self._check(rc, "adambridge_convert")

    @property
    def capabilities(self) -> set[str]:
        """What the library adds to the reference's ABI (adambridge_capabilities), by name."""
        bits = self._lib.adambridge_capabilities()
        return {name for name, bit in CAPABILITIES.items() if bits & bit}

    def convert_plane(self, src: Plane, dst: Plane, n: int, device: torch.device, offset: int = 0,
                      seed: int | None = None) -> None:
        """Copy ``n`` values from plane ``src`` to plane ``dst`` on ``device``'s current stream,
        converting between their types (adambridge_convert_plane): exact where the destination
        represents the value, else rounded as the kernels round -- to nearest, or stochastically with
        the 32-bit stream ``seed`` and element index ``offset + i``.  The planes' memory must stay
        alive until the stream has run the copy."""
        if n < 0:
            raise ValueError(f"convert_plane: n = {n}")
        with torch.cuda.device(device):
            self._lib.adambridge_set_stream(torch.cuda.current_stream(device).cuda_stream)
            rc = self._lib.adambridge_convert_plane(ctypes.byref(src), ctypes.byref(dst), int(n), int(offset),
                                                    0 if seed is None else seed & 0xFFFFFFFF,
                                                    0 if seed is None else CONVERT_STOCHASTIC)
        self._check(rc, "adambridge_convert_plane")

    def fused_adamw(self, master: torch.Tensor, grad: torch.Tensor, m: torch.Tensor, v: torch.Tensor,
                    out: torch.Tensor | None, hp: HParams, lo: int, hi: int) -> None:
        """Update elements ``[lo, hi)`` of flat contiguous device tensors in place, synchronously
        (reference: NativeKernels.fused_adamw, native.py:389-435, with the same checks)."""
        n = master.numel()
        tensors = {"master": master, "grad": grad, "m": m, "v": v, **({} if out is None else {"out": out})}
        for name, t in tensors.items():
            if not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous device tensor")
            if t.numel() != n:
                raise ValueError(f"{name} has {t.numel()} elements, master has {n}")
            if t.device != master.device:
                raise ValueError(f"{name} is on {t.device}, master on {master.device}")
        if master.dtype != torch.float32:
            raise TypeError("master must be float32")
        for name, t in tensors.items():
            if name != "master" and t.dtype not in _DTYPE_CODES:
                raise TypeError(f"{name} must be float32 or bfloat16, got {t.dtype}")
        if m.dtype != v.dtype:
            raise TypeError("m and v must have the same dtype")
        if not 0 <= lo <= hi <= n:
            raise IndexError(f"range [{lo}, {hi}) outside 0..{n}")
        with torch.cuda.device(master.device):
            self.set_stream(torch.cuda.current_stream())
            rc = self._lib.adambridge_fused_adamw(
                master.data_ptr() + lo * 4, grad.data_ptr() + lo * grad.element_size(), _DTYPE_CODES[grad.dtype],
                m.data_ptr() + lo * m.element_size(), v.data_ptr() + lo * v.element_size(), _DTYPE_CODES[m.dtype],
                None if out is None else out.data_ptr() + lo * out.element_size(),
                DT_NONE if out is None else _DTYPE_CODES[out.dtype], hi - lo, lo, ctypes.byref(hp))
        self._check(rc, "adambridge_fused_adamw")

    @staticmethod
    def make_hparams(c, seed: int, stochastic: bool) -> HParams:
        """From ``StepCoefficients`` (reference native.py:381-387)."""
        return HParams(c.beta1, c.beta2, 1.0 - c.beta1, 1.0 - c.beta2, c.decay, c.step_size, c.inv_sqrt_bc2,
                       c.eps, seed & 0xFFFFFFFF, int(stochastic))

    def _check(self, rc: int, what: str) -> None:
        if rc != 0:
            detail = self.last_error() if rc in (-20, -22) else ""   # codes that set the error text
            raise RuntimeError(f"{what} rejected the update (code {rc}){': ' + detail if detail else ''}")


def _stream_handle(stream) -> int | None:
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


_lock = threading.Lock()
_loaded: HipKernels | None = None


def load() -> HipKernels:
    """The library, loaded once.  Raises RuntimeError if it is missing or inconsistent: there is no
    other implementation to fall back to."""
    global _loaded
    with _lock:
        if _loaded is None:
            _loaded = HipKernels()
        return _loaded
