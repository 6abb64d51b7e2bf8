"""Storage formats of the optimizer state, as stateless functions over tensors.

The formats are the reference's (adambridge/precision.py:57-108, 341-480; the
rounding rules of adambridge/csrc/adambridge_kernels.c:100-165, 826-876):

========  ==========================================================  ==========
name      encoding                                                    bytes/elem
========  ==========================================================  ==========
fp32      IEEE single                                                 4
bf16      top 16 bits of the FP32 value, nearest-even or stochastic   2
fp8 m     E4M3FN code of x / s, s = block absmax / 448                1 + 4/128
fp8 v     E5M2 code of sqrt(v) / s, s = block absmax / 57344          1 + 4/128
fp24      top 24 bits of the FP32 value: BF16 plane + one byte plane  3
========  ==========================================================  ==========

FP8 blocks hold 128 consecutive elements and one FP32 scale (1 for an all-zero
block); codes are padded with zeros to whole blocks.  Stochastic rounding adds
the low bits of a counter hash of the element's index to the FP32 bits before
cutting them (kernels.c:120-126, 152-160, 857-876); the index of element i of a
parameter is ``(offset + i) mod 2^32`` and the hash is lowbias32 of the index
xor the stream's 32-bit seed.

On the optimizer's step path every format is encoded and decoded by the HIP
kernels.  What runs here is the work off that path -- initial state,
``set_precision``, checkpoints -- and the functions are written so that a
device tensor is converted by the library's kernels in one pass over HBM --
moments to nearest by ``adambridge_convert``, FP24 masters (both ways) and
bf16 working weights by ``adambridge_convert_plane`` -- and a host tensor by
torch casts and integer operations; both give the kernels' bits
(tests/test_host_cpu.py, tests/test_convert_gpu.py).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

__all__ = [
    "PRECISIONS", "MASTER_PRECISIONS", "FP8_BLOCK", "Fp8Format", "FP8_FORMATS", "canonical_precision",
    "canonical_master_precision", "moment_bytes", "bytes_per_param", "lowbias32", "stream_seed", "counter_hash",
    "round_bits_stochastic", "bf16_encode", "bf16_weight", "fp8_blocks", "fp8_encode", "fp8_decode", "fp24_encode",
    "fp24_round", "fp24_split", "fp24_join", "convert_plane",
]

# Accepted spellings (case-insensitive) -> canonical name: the reference's tables,
# adambridge/precision.py:64-75, since user code passes these strings.
_MOMENT_NAMES = {"fp32": "fp32", "float32": "fp32", "bf16": "bf16", "bf16_moments": "bf16", "bfloat16": "bf16",
                 "fp8": "fp8", "fp8_moments": "fp8"}
_MASTER_NAMES = {"fp32": "fp32", "float32": "fp32", "fp24": "fp24", "float24": "fp24"}
PRECISIONS = ("fp32", "bf16", "fp8")
MASTER_PRECISIONS = ("fp32", "fp24")
FP8_BLOCK = 128

_U32 = 0xFFFFFFFF


@dataclass(frozen=True)
class Fp8Format:
    """The FP8 encoding of one moment role (precision.py:77-82)."""

    role: str
    dtype: torch.dtype
    fmax: float           # largest finite magnitude
    mantissa_bits: int
    sqrt_domain: bool     # v is kept as sqrt(v)


FP8_FORMATS = {
    "m": Fp8Format("m", torch.float8_e4m3fn, 448.0, 3, False),
    "v": Fp8Format("v", torch.float8_e5m2, 57344.0, 2, True),
}


def _lookup(table: dict, name, what: str) -> str:
    key = name.lower() if isinstance(name, str) else None
    if key not in table:
        raise ValueError(f"unknown {what} {name!r}; expected one of {sorted(table)}")
    return table[key]


def canonical_precision(name: str) -> str:
    """'fp32', 'bf16' or 'fp8' for any accepted spelling of a moment precision."""
    return _lookup(_MOMENT_NAMES, name, "precision")


def canonical_master_precision(name: str) -> str:
    """'fp32' or 'fp24' for any accepted spelling of a master precision."""
    return _lookup(_MASTER_NAMES, name, "master precision")


def moment_bytes(precision: str) -> float:
    """Bytes per element of one moment vector (FP8: the code plus its share of the block scale)."""
    p = canonical_precision(precision)
    return 4.0 if p == "fp32" else 2.0 if p == "bf16" else 1.0 + 4.0 / FP8_BLOCK


def bytes_per_param(precision: str, moments: int = 2, master: str = "fp32") -> float:
    """State bytes per parameter: the master plus ``moments`` moment vectors (precision.py:103-108)."""
    master_bytes = 3.0 if canonical_master_precision(master) == "fp24" else 4.0
    return master_bytes + moments * moment_bytes(precision)


# ------------------------------------------------------- rounding streams

def lowbias32(x: int) -> int:
    """The counter hash of kernels.c:100-106 on one 32-bit value."""
    x &= _U32
    x ^= x >> 16
    x = (x * 0x7FEB352D) & _U32
    x ^= x >> 15
    x = (x * 0x846CA68B) & _U32
    return x ^ (x >> 16)


# salts of the second-moment and FP24-master streams (kernels.c:164-165)
_STREAM_SALT = {"v": 0xA511E9B3, "p": 0x6C8E9CF5}


def stream_seed(seed: int, role: str) -> int:
    """The 32-bit rounding stream of ``role`` ('m', 'v' or 'p', the FP24 master) for a step seed:
    the seed itself for m, a hash of it with the role's salt otherwise."""
    seed &= _U32
    return seed if role == "m" else lowbias32(seed ^ _STREAM_SALT[role])


def counter_hash(start: int, n: int, seed: int, device=None) -> torch.Tensor:
    """lowbias32((start + i) mod 2^32 ^ seed) for i < n, as int64 values in [0, 2^32).

    Worked in int64: every product of two values below 2^32 keeps its low 32 bits exact however
    the 64-bit multiply wraps, and the mask brings the result back below 2^32."""
    x = torch.arange(start, start + n, dtype=torch.int64, device=device).bitwise_and_(_U32)
    x.bitwise_xor_(seed & _U32)
    for mult, shift in ((0x7FEB352D, 16), (0x846CA68B, 15)):
        x.bitwise_xor_(x >> shift)
        x.mul_(mult).bitwise_and_(_U32)
    return x.bitwise_xor_(x >> 16)


def _as_u32(x: torch.Tensor) -> torch.Tensor:
    """The FP32 bits of ``x`` as int64 values in [0, 2^32)."""
    return x.detach().reshape(-1).to(torch.float32).contiguous().view(torch.int32).to(torch.int64).bitwise_and_(_U32)


def _from_u32(bits: torch.Tensor) -> torch.Tensor:
    """int64 values in [0, 2^32) -> the FP32 tensor with those bits."""
    return (bits - ((bits >> 31) << 32)).to(torch.int32).view(torch.float32)


def round_bits_stochastic(x: torch.Tensor, dropped: int, start: int, seed: int) -> torch.Tensor:
    """FP32 ``x`` with its low ``dropped`` bits cut after adding the same bits of the rounding stream
    (integer addition on the bits: it moves the magnitude of a sign-magnitude float).  A new flat
    tensor; ``start`` is the stream index of ``x[0]``."""
    low = (1 << dropped) - 1
    bits = _as_u32(x)
    bits += counter_hash(start, bits.numel(), seed, bits.device).bitwise_and_(low)
    return _from_u32(bits.bitwise_and_(_U32 ^ low))


def _device_convert(src: torch.Tensor, dst: torch.Tensor, dst_scale: torch.Tensor | None, n: int, role: str) -> None:
    """Nearest-even encode of ``n`` FP32 values into device buffers by the library's conversion kernel."""
    from . import _hip   # loaded only once a format is encoded on the device

    x = src.detach().reshape(-1)[:n].to(dst.device, torch.float32).contiguous()
    _hip.load().convert(x, None, dst, dst_scale, n, role)


def _on_device(x: torch.Tensor) -> bool:
    """Whether ``x``'s conversions run as the library's plane-conversion kernel (device memory)
    rather than as torch integer operations (host memory)."""
    return x.is_cuda


def _values(x: torch.Tensor) -> torch.Tensor:
    """``x`` flat and contiguous, as float32 unless it is bfloat16 (both are planes the kernel reads)."""
    flat = x.detach().reshape(-1)
    if flat.dtype not in (torch.float32, torch.bfloat16):
        flat = flat.to(torch.float32)
    return flat.contiguous()


def convert_plane(src, dst, n: int, device, offset: int = 0, seed: int | None = None) -> None:
    """``n`` values from plane ``src`` into plane ``dst`` by the library's plane-conversion kernel
    (adambridge_convert_plane) on ``device``'s current stream; planes are ``_hip.Plane`` structs."""
    from . import _hip

    _hip.load().convert_plane(src, dst, n, torch.device(device), offset, seed)


# --------------------------------------------------------------------- BF16

def bf16_encode(x: torch.Tensor, seed: int | None = None, start: int = 0) -> torch.Tensor:
    """FP32 ``x`` as a flat BF16 tensor on x's device: stochastic with stream ``seed``, else
    nearest-even (a NaN becomes 0x7fc0, as torch's cast gives)."""
    flat = x.detach().reshape(-1)
    if seed is not None:
        return round_bits_stochastic(flat, 16, start, seed).to(torch.bfloat16)   # exact: low bits are zero
    if flat.is_cuda:
        out = torch.empty(flat.numel(), dtype=torch.bfloat16, device=flat.device)
        if flat.numel():
            _device_convert(flat, out, None, flat.numel(), "m")
        return out
    return flat.to(torch.bfloat16)


def bf16_weight(x: torch.Tensor) -> torch.Tensor:
    """FP32 ``x`` as the bf16 working weight the kernels write (kernels.c:108-112): nearest-even,
    a NaN kept with its sign and payload and made quiet.  A new flat tensor on x's device (there
    written by the plane-conversion kernel, with no temporaries)."""
    if _on_device(x):
        from . import _hip

        src = _values(x)
        out = torch.empty(src.numel(), dtype=torch.bfloat16, device=src.device)
        if src.numel():
            convert_plane(_hip.plane_of(src), _hip.plane_of(out), src.numel(), src.device)
        return out
    bits = _as_u32(x)
    nan = bits.bitwise_and(0x7FFFFFFF) > 0x7F800000
    rounded = (bits + 0x7FFF + bits.bitwise_right_shift(16).bitwise_and_(1)).bitwise_and_(_U32)
    bits = torch.where(nan, bits.bitwise_or(0x00400000), rounded).bitwise_right_shift_(16)
    return bits.sub_(bits.ge(0x8000).long() << 16).to(torch.int16).view(torch.bfloat16)


# ---------------------------------------------------------------------- FP8

def fp8_blocks(n: int, block: int = FP8_BLOCK) -> int:
    """Blocks holding n elements (at least one)."""
    return max(1, math.ceil(n / block))


def fp8_encode(x: torch.Tensor, role: str, seed: int | None = None, start: int = 0,
               block: int = FP8_BLOCK) -> tuple[torch.Tensor, torch.Tensor]:
    """FP32 ``x`` (n values) -> (codes, scales): codes of ``role``'s format padded with zeros to whole
    blocks, one FP32 scale per block.  ``start`` (a multiple of ``block``) is the element index of
    ``x[0]`` in the rounding stream ``seed``; without a seed the codes are nearest-even.

    Per block: v goes to the sqrt domain after clamping at zero; the scale is absmax / fmax (1 for a
    block whose absmax is zero or NaN); each value is divided by it, stochastically cut when a seed
    is given, clamped to +-fmax and cast to the format."""
    fmt = FP8_FORMATS[role]
    flat = x.detach().reshape(-1).to(torch.float32)
    n = flat.numel()
    nb = fp8_blocks(n, block)
    if seed is None and flat.is_cuda and block == FP8_BLOCK:
        codes = torch.empty(nb * block, dtype=fmt.dtype, device=flat.device)
        scales = torch.empty(nb, dtype=torch.float32, device=flat.device)
        _device_convert(flat, codes, scales, n, role)
        return codes, scales
    values = torch.zeros(nb * block, dtype=torch.float32, device=flat.device)
    values[:n] = flat
    if fmt.sqrt_domain:
        values = values.clamp(min=0).sqrt()
    rows = values.view(nb, block)
    amax = rows.abs().amax(dim=1)
    scales = torch.where(amax > 0, amax / fmt.fmax, torch.ones_like(amax))
    q = (rows / scales[:, None]).reshape(-1)
    if seed is not None:
        q = round_bits_stochastic(q, 23 - fmt.mantissa_bits, start, seed)
    return q.clamp(-fmt.fmax, fmt.fmax).to(fmt.dtype), scales


def fp8_decode(codes: torch.Tensor, scales: torch.Tensor, role: str, n: int) -> torch.Tensor:
    """The first n FP32 values held by block codes and scales (v squared back from the sqrt domain)."""
    nb = scales.numel()
    rows = codes.reshape(-1)[: codes.numel() // nb * nb].view(nb, -1)
    x = rows.to(torch.float32) * scales.reshape(nb, 1).to(torch.float32)
    if FP8_FORMATS[role].sqrt_domain:
        x = x * x
    return x.reshape(-1)[:n]


# --------------------------------------------------------------------- FP24

def fp24_encode(x: torch.Tensor, seed: int | None = None, start: int = 0,
                out: tuple[torch.Tensor, torch.Tensor] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """FP32 ``x`` rounded to its top 24 bits (kernels.c:145-160) and split into the FP24 planes (hi:
    BF16 bits as bfloat16, lo: the next byte as uint8): stochastic with stream ``seed`` (element i
    at stream index ``start + i``), else nearest-even with a NaN kept NaN (quiet bit set).  ``out``:
    contiguous planes to write (new ones otherwise).  On the device one pass of the plane-conversion
    kernel; in host memory torch integer operations."""
    src = _values(x)
    n = src.numel()
    if out is None:
        out = (torch.empty(n, dtype=torch.bfloat16, device=src.device), torch.empty(n, dtype=torch.uint8, device=src.device))
    hi, lo = out
    if _on_device(src):
        from . import _hip

        if src.dtype != torch.float32:   # the FP32 value is what is rounded (a BF16 NaN is quietened too)
            src = src.to(torch.float32)
        if n:
            convert_plane(_hip.plane_of(src), _hip.fp24_plane(hi, lo), n, src.device, start, seed)
        return hi, lo
    h, low = fp24_split(fp24_round(src, seed, start))
    hi.copy_(h)
    lo.copy_(low)
    return hi, lo


def fp24_round(x: torch.Tensor, seed: int | None = None, start: int = 0) -> torch.Tensor:
    """FP32 ``x`` rounded to its top 24 bits (kernels.c:145-160), as a new flat FP32 tensor:
    stochastic with stream ``seed``, else nearest-even with a NaN kept NaN (quiet bit set, its low
    byte kept).  The reference's torch helpers' rule (precision.py:191-204), for the store API's
    functions of that name; the optimizer's own state goes through fp24_encode."""
    if seed is not None:
        return round_bits_stochastic(x, 8, start, seed)
    bits = _as_u32(x)
    nan = torch.isnan(x.detach().reshape(-1))
    rounded = (bits + 0x7F + ((bits >> 8) & 1)).bitwise_and_(_U32 ^ 0xFF)
    return _from_u32(torch.where(nan, bits | 0x00400000, rounded))


def fp24_split(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Planes of FP32 values already rounded to 24 bits: (BF16 bits as bfloat16, next byte as uint8)."""
    if _on_device(x):
        return fp24_encode(x)   # nearest-even leaves a 24-bit value as it is
    bits = _as_u32(x)
    hi = ((bits >> 16) - (((bits >> 31) & 1) << 16)).to(torch.int16).view(torch.bfloat16)
    return hi, ((bits >> 8) & 0xFF).to(torch.uint8)


def fp24_join(hi: torch.Tensor, lo: torch.Tensor) -> torch.Tensor:
    """FP32 values from the two FP24 planes (on the device, one pass of the plane-conversion kernel)."""
    if _on_device(hi):
        from . import _hip

        h, low = hi.reshape(-1).contiguous(), lo.reshape(-1).contiguous()
        out = torch.empty(h.numel(), dtype=torch.float32, device=h.device)
        if h.numel():
            convert_plane(_hip.fp24_plane(h, low), _hip.plane_of(out), h.numel(), h.device)
        return out
    top = hi.reshape(-1).contiguous().view(torch.int16).to(torch.int64).bitwise_and_(0xFFFF)
    return _from_u32((top << 16) | (lo.reshape(-1).to(torch.int64) << 8))
