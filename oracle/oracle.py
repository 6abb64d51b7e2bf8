"""ctypes access to the parity checkers (test infrastructure only).

Two CPU implementations of the reference's fused update can be driven through
the same case description:

* ``liboracle.so``   -- this directory's C restatement (abh_oracle.c);
* ``_ref/libadambridge_ref.so`` -- the reference kernel compiled from its own
  source by oracle/Makefile (present where /root/reference was at build time).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg import
this module.  The product package (adambridge_amd) never does.

A :class:`Case` holds numpy arrays in the reference's storage layout (BF16 as
uint16 bits, FP8 as uint8 codes with one float32 scale per 128 elements, the
FP24 master as a uint16 hi plane and a uint8 lo plane) plus the segment's
scalars; :func:`run` copies the arrays, updates the copies with one
implementation and returns them.
"""

from __future__ import annotations

import ctypes
import dataclasses
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libadambridge_ref.so"

DT_NONE, DT_F32, DT_BF16, DT_FP8, DT_F24 = 0, 1, 2, 3, 4
ADAMW, LION = 0, 1
FP8_BLOCK = 128
# SIMD level (kernels.c:73-74) -> width of the reference's vector body; 0 = scalar level
LEVEL_WIDTH = {0: 0, 1: 8, 2: 16}


class HParams(ctypes.Structure):
    """adambridge_hparams, kernels.c:77-88."""
    _fields_ = [("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
                ("one_minus_beta1", ctypes.c_float), ("one_minus_beta2", ctypes.c_float),
                ("decay", ctypes.c_float), ("step_size", ctypes.c_float),
                ("inv_sqrt_bc2", ctypes.c_float), ("eps", ctypes.c_float),
                ("seed", ctypes.c_uint32), ("stochastic", ctypes.c_int32)]


class Group(ctypes.Structure):
    """adambridge_group, kernels.c:736-745."""
    _fields_ = [("lr", ctypes.c_double), ("beta1", ctypes.c_double), ("beta2", ctypes.c_double),
                ("eps", ctypes.c_double), ("weight_decay", ctypes.c_double),
                ("seed", ctypes.c_uint64), ("stochastic", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class Segment(ctypes.Structure):
    """adambridge_segment, kernels.c:747-769 (raw addresses)."""
    _fields_ = [("p", ctypes.c_void_p), ("p_lo", ctypes.c_void_p), ("g", ctypes.c_void_p),
                ("m", ctypes.c_void_p), ("v", ctypes.c_void_p), ("m_scale", ctypes.c_void_p),
                ("v_scale", ctypes.c_void_p), ("out", ctypes.c_void_p), ("group", ctypes.POINTER(Group)),
                ("n", ctypes.c_int64), ("step", ctypes.c_int64), ("index", ctypes.c_uint64),
                ("offset", ctypes.c_int64), ("g_dtype", ctypes.c_int32), ("mv_dtype", ctypes.c_int32),
                ("out_dtype", ctypes.c_int32), ("algorithm", ctypes.c_int32), ("p_dtype", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


SegArray = ctypes.POINTER(ctypes.POINTER(Segment))

_oracle = None
_ref = None


def load_oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.exists():
            raise FileNotFoundError(f"{ORACLE_LIB} is not built (make -C oracle)")
        lib = ctypes.CDLL(str(ORACLE_LIB))
        lib.abo_hash32.restype = ctypes.c_uint32
        lib.abo_hash32.argtypes = [ctypes.c_uint32]
        lib.abo_step_seed.restype = ctypes.c_uint32
        lib.abo_step_seed.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int64]
        lib.abo_bf16_rne.restype = ctypes.c_uint32
        lib.abo_bf16_rne.argtypes = [ctypes.c_uint32]
        lib.abo_f24_round.restype = ctypes.c_uint32
        lib.abo_f24_round.argtypes = [ctypes.c_uint32, ctypes.c_int, ctypes.c_uint32]
        lib.abo_round_values.restype = None
        lib.abo_round_values.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_uint32, ctypes.c_uint64]
        lib.abo_fp8_decode.restype = ctypes.c_float
        lib.abo_fp8_decode.argtypes = [ctypes.c_uint32, ctypes.c_int]
        lib.abo_fp8_encode.restype = ctypes.c_uint32
        lib.abo_fp8_encode.argtypes = [ctypes.c_float, ctypes.c_int, ctypes.c_uint32, ctypes.c_int]
        lib.abo_hparams_for.restype = None
        lib.abo_hparams_for.argtypes = [ctypes.POINTER(Segment), ctypes.POINTER(HParams)]
        lib.abo_check_segment.restype = ctypes.c_int
        lib.abo_check_segment.argtypes = [ctypes.POINTER(Segment), ctypes.c_int]
        lib.abo_multi_apply.restype = ctypes.c_int
        lib.abo_multi_apply.argtypes = [SegArray, ctypes.POINTER(HParams), ctypes.c_int32, ctypes.c_int64,
                                        ctypes.c_int32]
        lib.abo_multi_step.restype = ctypes.c_int
        lib.abo_multi_step.argtypes = [SegArray, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32]
        for fn, st in (("abo_hparams_size", HParams), ("abo_group_size", Group), ("abo_segment_size", Segment)):
            if getattr(lib, fn)() != ctypes.sizeof(st):
                raise RuntimeError(f"{fn}: layout mismatch")
        _oracle = lib
    return _oracle


def reference_available() -> bool:
    return REF_LIB.exists()


def load_reference() -> ctypes.CDLL:
    """The reference kernel built from its own source (oracle/Makefile); raises if absent."""
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            raise FileNotFoundError(f"{REF_LIB} is not built (make -C oracle ref, with the reference tree)")
        lib = ctypes.CDLL(str(REF_LIB))
        for fn in ("adambridge_abi_version", "adambridge_simd_level", "adambridge_detected_simd_level",
                   "adambridge_set_simd_level", "adambridge_hparams_size", "adambridge_group_size",
                   "adambridge_segment_size"):
            getattr(lib, fn).restype = ctypes.c_int
        lib.adambridge_set_simd_level.argtypes = [ctypes.c_int]
        lib.adambridge_pool_create.restype = ctypes.c_void_p
        lib.adambridge_pool_create.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32]
        lib.adambridge_pool_destroy.restype = None
        lib.adambridge_pool_destroy.argtypes = [ctypes.c_void_p]
        lib.adambridge_multi_apply.restype = ctypes.c_int
        lib.adambridge_multi_apply.argtypes = [ctypes.c_void_p, SegArray, ctypes.POINTER(HParams), ctypes.c_int32,
                                               ctypes.c_int32]
        lib.adambridge_multi_step.restype = ctypes.c_int
        lib.adambridge_multi_step.argtypes = [ctypes.c_void_p, SegArray, ctypes.c_int32, ctypes.c_int32]
        for fn, st in (("adambridge_hparams_size", HParams), ("adambridge_group_size", Group),
                       ("adambridge_segment_size", Segment)):
            if getattr(lib, fn)() != ctypes.sizeof(st):
                raise RuntimeError(f"{fn}: layout mismatch")
        _ref = lib
    return _ref


# ------------------------------------------------------------------ cases

STATE_KEYS = ("p", "p_lo", "m", "v", "m_scale", "v_scale", "out")


@dataclasses.dataclass
class Case:
    """One segment's buffers (numpy, host) and scalars."""
    n: int
    algorithm: int = ADAMW
    mv_dtype: int = DT_BF16
    p_dtype: int = DT_F32
    g_dtype: int = DT_BF16
    out_dtype: int = DT_BF16
    offset: int = 0
    index: int = 0
    step: int = 1
    arrays: dict = dataclasses.field(default_factory=dict)
    # explicit coefficients (multi_apply) or group hyperparameters (multi_step)
    hparams: dict | None = None
    group: dict | None = None

    def copy(self) -> "Case":
        return dataclasses.replace(self, arrays={k: v.copy() for k, v in self.arrays.items()},
                                   hparams=None if self.hparams is None else dict(self.hparams),
                                   group=None if self.group is None else dict(self.group))


def hparams_struct(h: dict) -> HParams:
    return HParams(h["beta1"], h["beta2"], h["one_minus_beta1"], h["one_minus_beta2"], h["decay"],
                   h["step_size"], h["inv_sqrt_bc2"], h["eps"], h["seed"] & 0xFFFFFFFF, int(h["stochastic"]))


def hparams_dict(h: HParams) -> dict:
    return {k: getattr(h, k) for k, _ in HParams._fields_}


def group_struct(g: dict) -> Group:
    return Group(g["lr"], g["beta1"], g["beta2"], g["eps"], g["weight_decay"], g["seed"] & (2**64 - 1),
                 int(g["stochastic"]), 0)


def _addr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def check_sizes(case: Case) -> None:
    """Raise unless every buffer the segment's kernels will touch holds its n elements (FP8 codes:
    whole 128-element blocks, one scale per block).  Run before any implementation -- the C oracle,
    the compiled reference or a GPU launch -- is handed the case."""
    a, n = case.arrays, case.n
    nb = -(-n // FP8_BLOCK)
    lion = case.algorithm == LION
    need = {"p": n, "g": n}
    if case.p_dtype == DT_F24:
        need["p_lo"] = n
    if case.out_dtype != DT_NONE:
        need["out"] = n
    for key in ("m",) + (() if lion else ("v",)):
        if case.mv_dtype == DT_FP8:
            need[key] = nb * FP8_BLOCK
            need[key + "_scale"] = nb
        else:
            need[key] = n
    for key, count in need.items():
        arr = a.get(key)
        if arr is None or arr.size < count:
            raise ValueError(f"case buffer {key!r} holds {None if arr is None else arr.size} elements, "
                             f"the segment needs {count}")


def segment_for(case: Case, group: Group | None = None) -> Segment:
    check_sizes(case)
    a = case.arrays
    return Segment(p=_addr(a.get("p")), p_lo=_addr(a.get("p_lo")), g=_addr(a.get("g")), m=_addr(a.get("m")),
                   v=_addr(a.get("v")), m_scale=_addr(a.get("m_scale")), v_scale=_addr(a.get("v_scale")),
                   out=_addr(a.get("out")), group=ctypes.pointer(group) if group is not None else None,
                   n=case.n, step=case.step, index=case.index, offset=case.offset, g_dtype=case.g_dtype,
                   mv_dtype=case.mv_dtype, out_dtype=case.out_dtype, algorithm=case.algorithm,
                   p_dtype=case.p_dtype)


def run_many(cases: list[Case], impl: str = "oracle", width: int = 16, threads: int = 1,
             in_place: bool = False) -> list[Case]:
    """Update ``cases`` (copies unless ``in_place``) in one multi call of ``impl`` ('oracle' or 'ref').

    Every case carries ``hparams`` (multi_apply) or every case carries ``group`` (multi_step).
    ``width``: the reference's vector width whose scalar tail is reproduced (16 AVX-512, 8 AVX2,
    0 the scalar level).  Raises on a non-zero return code.
    """
    work = cases if in_place else [c.copy() for c in cases]
    if not work:
        return work
    by_group = all(c.group is not None for c in work)
    groups = [group_struct(c.group) if by_group else None for c in work]
    segs = [segment_for(c, g) for c, g in zip(work, groups)]
    arr = (ctypes.POINTER(Segment) * len(segs))(*[ctypes.pointer(s) for s in segs])
    hps = None if by_group else (HParams * len(work))(*[hparams_struct(c.hparams) for c in work])
    if impl == "oracle":
        lib = load_oracle()
        rc = (lib.abo_multi_step(arr, len(segs), width, threads) if by_group
              else lib.abo_multi_apply(arr, hps, len(segs), width, threads))
    elif impl == "ref":
        lib = load_reference()
        level = {v: k for k, v in LEVEL_WIDTH.items()}[width]
        lib.adambridge_set_simd_level(level)
        pool = lib.adambridge_pool_create(threads, None, 0) if threads > 1 else None
        try:
            rc = (lib.adambridge_multi_step(pool, arr, len(segs), threads) if by_group
                  else lib.adambridge_multi_apply(pool, arr, hps, len(segs), threads))
        finally:
            if pool:
                lib.adambridge_pool_destroy(pool)
            lib.adambridge_set_simd_level(-1)
    else:
        raise ValueError(impl)
    if rc != 0:
        raise RuntimeError(f"{impl} multi call returned {rc}")
    return work


def run(case: Case, impl: str = "oracle", width: int = 16, threads: int = 1) -> Case:
    return run_many([case], impl, width, threads)[0]


def hparams_for(case: Case) -> dict:
    """The coefficients the oracle derives from ``case.group`` and ``case.step`` (kernels.c:793-809)."""
    lib = load_oracle()
    g = group_struct(case.group)
    seg = segment_for(case, g)
    h = HParams()
    lib.abo_hparams_for(ctypes.byref(seg), ctypes.byref(h))
    return hparams_dict(h)


# ------------------------------------------------------------ generators

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> BF16 bits, nearest-even with quiet NaN (kernels.c:108-112), vectorised."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = (b + 0x7FFF + ((b >> 16) & 1)).astype(np.uint32)
    r = np.where(nan, b | 0x00400000, r)
    return (r >> 16).astype(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f24_planes(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """float32 -> FP24 (hi, lo) planes, nearest-even (kernels.c:145-150 with sr=0)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7F + ((b >> 8) & 1)) & ~np.uint32(0xFF)).astype(np.uint32)
    r = np.where(nan, b | 0x00400000, r)
    return (r >> 16).astype(np.uint16), ((r >> 8) & 0xFF).astype(np.uint8)


def f24_value(hi: np.ndarray, lo: np.ndarray) -> np.ndarray:
    return ((hi.astype(np.uint32) << 16) | (lo.astype(np.uint32) << 8)).view(np.float32)


def round_values(bits: np.ndarray, kind: str, seed: int | None = None, offset: int = 0) -> np.ndarray:
    """FP32 bit patterns rounded by the C oracle's master / weight rules (abo_round_values): kind 'fp24'
    -> the FP32 bits the FP24 master stores, 'bf16' -> BF16 codes; stochastic with stream ``seed``
    (element i at index offset + i), nearest otherwise."""
    src = np.ascontiguousarray(bits, dtype=np.uint32)
    out = np.empty_like(src)
    load_oracle().abo_round_values(src.ctypes.data, out.ctypes.data, src.size, 0 if kind == "fp24" else 1,
                                   int(seed is not None), 0 if seed is None else seed & 0xFFFFFFFF, offset)
    return out if kind == "fp24" else out.astype(np.uint16)


def fp8_decode_table(role: int) -> np.ndarray:
    lib = load_oracle()
    return np.array([lib.abo_fp8_decode(c, role) for c in range(256)], dtype=np.float32)


def make_case(rng: np.random.Generator, n: int, *, algorithm=ADAMW, mv_dtype=DT_BF16, p_dtype=DT_F32,
              g_dtype=DT_BF16, out_dtype=DT_BF16, offset=0, index=0, step=1, stochastic=True,
              grad_scale=1e-3, special=False, explicit=True, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
              weight_decay=0.01, seed=0) -> Case:
    """A random segment in a plausible mid-training state.

    ``special`` sprinkles zeros, subnormals, infinities and NaNs into every input.
    ``explicit``: carry explicit coefficients (multi_apply) rather than a group (multi_step).
    """
    lion = algorithm == LION
    master = rng.normal(0.0, 0.02, n).astype(np.float32)
    g = (rng.normal(0.0, 1.0, n) * grad_scale).astype(np.float32)
    m = (rng.normal(0.0, 1.0, n) * grad_scale * 0.3).astype(np.float32)
    v = ((rng.normal(0.0, 1.0, n) * grad_scale) ** 2 * rng.uniform(0.2, 2.0, n)).astype(np.float32)
    if special and n:
        pick = lambda frac: rng.random(n) < frac  # noqa: E731
        tiny = np.float32(1e-41)
        for arr in (master, g, m):
            arr[pick(0.02)] = 0.0
            arr[pick(0.01)] = -0.0
            arr[pick(0.01)] = tiny * rng.uniform(-1, 1)
            arr[pick(0.003)] = np.inf
            arr[pick(0.003)] = -np.inf
            arr[pick(0.003)] = np.nan
        v[pick(0.02)] = 0.0
        v[pick(0.01)] = tiny
        v[pick(0.003)] = np.inf
        v[pick(0.003)] = np.nan
        g[pick(0.01)] = 3e38
    arrays: dict[str, np.ndarray] = {}
    if p_dtype == DT_F24:
        arrays["p"], arrays["p_lo"] = f24_planes(master)
    else:
        arrays["p"] = master
    arrays["g"] = bf16_bits(g) if g_dtype == DT_BF16 else g
    if mv_dtype == DT_FP8:
        nb = max(1, -(-n // FP8_BLOCK))
        for key, role, val in (("m", 0, m), ("v", 1, np.sqrt(np.abs(v)))):
            if lion and key == "v":
                continue
            codes = rng.integers(0, 256, nb * FP8_BLOCK, dtype=np.uint8)
            if not special:  # finite codes only
                bad = np.isnan(fp8_decode_table(role)[codes]) | np.isinf(fp8_decode_table(role)[codes])
                codes[bad] = codes[bad] & 0x70
            codes[n:] = 0
            finite = np.abs(val[np.isfinite(val)])
            top = float(finite.max()) if finite.size else 1e-6
            scale = (max(top, 1e-6) / (448.0 if role == 0 else 57344.0)
                     * rng.uniform(0.5, 2.0, nb)).astype(np.float32)
            if special:
                scale[rng.random(nb) < 0.1] = 1.0
            arrays[key] = codes
            arrays[key + "_scale"] = scale
    elif mv_dtype == DT_BF16:
        arrays["m"] = bf16_bits(m)
        if not lion:
            arrays["v"] = bf16_bits(v)
    else:
        arrays["m"] = m
        if not lion:
            arrays["v"] = v
    if out_dtype == DT_BF16:
        arrays["out"] = np.full(n, 0xDEAD, dtype=np.uint16)
    elif out_dtype == DT_F32:
        arrays["out"] = np.full(n, np.nan, dtype=np.float32)
    case = Case(n=n, algorithm=algorithm, mv_dtype=mv_dtype, p_dtype=p_dtype, g_dtype=g_dtype,
                out_dtype=out_dtype, offset=offset, index=index, step=step, arrays=arrays)
    group = {"lr": lr, "beta1": betas[0], "beta2": betas[1], "eps": 0.0 if lion else eps,
             "weight_decay": weight_decay, "seed": seed, "stochastic": int(stochastic)}
    case.group = group
    if explicit:
        case.hparams = hparams_for(case)
        case.group = None
    return case


def outputs_equal(a: Case, b: Case, nan_equiv: bool = False) -> list[str]:
    """Names of state arrays that differ bitwise.

    ``nan_equiv``: any two NaNs count as equal (float32 and BF16 values, FP8 NaN codes).  IEEE 754
    leaves the payload and sign of a NaN result unspecified when NaNs meet or are generated; the
    reference's own bits there depend on its compiler's operand order and on the host ISA's default
    NaN, so NaN-vs-NaN is the parity bar wherever inputs are non-finite.
    """
    bad = []
    for k in STATE_KEYS:
        x, y = a.arrays.get(k), b.arrays.get(k)
        if x is None and y is None:
            continue
        if x is None or y is None or x.shape != y.shape:
            bad.append(k)
            continue
        if x.dtype == np.float32 and nan_equiv:
            xb, yb = x.view(np.uint32), y.view(np.uint32)
            same = (xb == yb) | (np.isnan(x) & np.isnan(y))
        elif x.dtype == np.uint16 and nan_equiv and k in ("p", "m", "v", "out"):
            xf, yf = bf16_value(x), bf16_value(y)
            same = (x == y) | (np.isnan(xf) & np.isnan(yf))
        elif x.dtype == np.uint8 and nan_equiv and k in ("m", "v") and a.mv_dtype == DT_FP8:
            table = fp8_decode_table(0 if k == "m" else 1)
            same = (x == y) | (np.isnan(table[x]) & np.isnan(table[y]))
        else:
            same = x.view(np.uint8).reshape(x.shape[0], -1) == y.view(np.uint8).reshape(y.shape[0], -1) \
                if x.size else np.ones(0, bool)
        if not np.all(same):
            bad.append(k)
    return bad


def threads_default() -> int:
    return max(1, min(16, os.cpu_count() or 1))
