"""Storage formats of the master weights and the moments, resident in device memory.

Same formats, layouts, names and checkpoint dictionaries as the reference's
``adambridge/precision.py``; the tensors live on the parameter's device (HBM)
instead of host RAM, and the per-step update of every format is done by the
HIP kernel (``libadambridge_hip.so``).  What runs here, with torch ops on the
device, is only the conversion work off the step path: initial encoding,
``set_precision`` and checkpoint loading.

==========  ==================  ====================  ===============
precision   first moment m      second moment v       bytes / param*
==========  ==================  ====================  ===============
fp32        FP32                FP32                  12
bf16        BF16                BF16                  8
fp8         E4M3 + block scale  E5M2 + block scale    ~6.06
==========  ==================  ====================  ===============

\\* with an FP32 master (FP24: one byte less); gradient and weights excluded.

FP8 keeps one FP32 scale per 128 elements (block absmax / format max) and
stores ``sqrt(v)`` rather than ``v`` (precision.py:341-418).  The FP24 master is
the top 24 bits of the FP32 value as two planes, the BF16 bits and the next
byte (precision.py:421-480).
"""

from __future__ import annotations

import math
from abc import ABC, abstractmethod
from typing import Any

import torch

__all__ = [
    "PRECISIONS", "MASTER_PRECISIONS", "FP8_BLOCK", "canonical_precision", "canonical_master_precision",
    "MomentStore", "FP32Store", "BF16Store", "FP8Store", "FP24Store", "make_store", "make_master",
    "store_from_state_dict", "check_master_state", "load_master_", "master_to_fp32", "bytes_per_param",
    "round_to_bf16_stochastic", "round_to_fp8_stochastic", "round_to_fp24_stochastic", "round_to_fp24_nearest_",
    "moment_seed", "random_bits", "PackedState", "PackedMaster", "PackedMoment", "RecordState",
    "RecordMaster", "RecordMoment",
]

# Accepted spellings (precision.py:64-75), case-insensitive.
_ALIASES = {"fp32": "fp32", "float32": "fp32", "bf16": "bf16", "bf16_moments": "bf16", "bfloat16": "bf16",
            "fp8": "fp8", "fp8_moments": "fp8"}
PRECISIONS = ("fp32", "bf16", "fp8")
_MASTER_ALIASES = {"fp32": "fp32", "float32": "fp32", "fp24": "fp24", "float24": "fp24"}
MASTER_PRECISIONS = ("fp32", "fp24")

FP8_BLOCK = 128
# role -> (dtype, max finite value, mantissa bits), precision.py:78-82
_FP8_FORMATS = {
    "m": (torch.float8_e4m3fn, 448.0, 3),
    "v": (torch.float8_e5m2, 57344.0, 2),
}


def canonical_precision(name: str) -> str:
    try:
        return _ALIASES[name.lower()]
    except (KeyError, AttributeError):
        raise ValueError(f"unknown precision {name!r}; expected one of {sorted(_ALIASES)}") from None


def canonical_master_precision(name: str) -> str:
    try:
        return _MASTER_ALIASES[name.lower()]
    except (KeyError, AttributeError):
        raise ValueError(f"unknown master precision {name!r}; expected one of {sorted(_MASTER_ALIASES)}") from None


def bytes_per_param(precision: str, moments: int = 2, master: str = "fp32") -> float:
    """State bytes per parameter: master + ``moments`` moment vectors (precision.py:103-108)."""
    precision = canonical_precision(precision)
    moment = {"fp32": 4.0, "bf16": 2.0, "fp8": 1.0 + 4.0 / FP8_BLOCK}[precision]
    return {"fp32": 4.0, "fp24": 3.0}[canonical_master_precision(master)] + moments * moment


# ----------------------------------------------------- stochastic rounding

def _hash32(x: int) -> int:
    x &= 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x7FEB352D) & 0xFFFFFFFF
    x ^= x >> 15
    x = (x * 0x846CA68B) & 0xFFFFFFFF
    return x ^ (x >> 16)


def moment_seed(seed: int, role: str) -> int:
    """32-bit rounding stream of ``role`` ('m', 'v' or 'p'), as the kernel derives it
    (kernels.c:164-165; precision.py:131-137)."""
    seed &= 0xFFFFFFFF
    if role == "m":
        return seed
    return _hash32(seed ^ (0xA511E9B3 if role == "v" else 0x6C8E9CF5))


def _i32(v: int) -> int:
    v &= 0xFFFFFFFF
    return v - (1 << 32) if v >= 1 << 31 else v


def random_bits(offset: int, n: int, seed: int, device=None) -> torch.Tensor:
    """lowbias32(index ^ seed) for indices offset .. offset+n-1, as int32 bit patterns (precision.py:145-158)."""
    if offset + n <= 1 << 31:
        x = torch.arange(offset, offset + n, dtype=torch.int32, device=device)
    else:
        x = (torch.arange(offset, offset + n, dtype=torch.int64, device=device) & 0xFFFFFFFF).to(torch.int32)
    x.bitwise_xor_(_i32(seed))
    x.bitwise_xor_(x.bitwise_right_shift(16).bitwise_and_(0xFFFF))
    x.mul_(0x7FEB352D)
    x.bitwise_xor_(x.bitwise_right_shift(15).bitwise_and_(0x1FFFF))
    x.mul_(_i32(0x846CA68B))
    x.bitwise_xor_(x.bitwise_right_shift(16).bitwise_and_(0xFFFF))
    return x


def _stochastic_truncate_(x: torch.Tensor, dropped: int, offset: int, seed: int) -> torch.Tensor:
    noise = random_bits(offset, x.numel(), seed, x.device).bitwise_and_((1 << dropped) - 1)
    x.view(torch.int32).add_(noise).bitwise_and_(-(1 << dropped))
    return x


def round_to_bf16_stochastic(x: torch.Tensor, seed: int, offset: int = 0) -> torch.Tensor:
    """FP32 ``x`` (clobbered) stochastically rounded to BF16."""
    return _stochastic_truncate_(x, 16, offset, seed).to(torch.bfloat16)


def round_to_fp8_stochastic(x: torch.Tensor, dtype: torch.dtype, seed: int, offset: int = 0) -> torch.Tensor:
    """Pre-scaled FP32 ``x`` (clobbered) stochastically rounded to ``dtype``."""
    _, fmax, mbits = next(f for f in _FP8_FORMATS.values() if f[0] == dtype)
    _stochastic_truncate_(x, 23 - mbits, offset, seed)
    return x.clamp_(-fmax, fmax).to(dtype)


def round_to_fp24_stochastic(x: torch.Tensor, seed: int, offset: int = 0) -> torch.Tensor:
    return _stochastic_truncate_(x, 8, offset, seed)


def round_to_fp24_nearest_(x: torch.Tensor) -> torch.Tensor:
    """Round FP32 ``x`` in place to its top 24 bits, nearest-even, NaN quietened (kernels.c:145-150)."""
    b = x.view(torch.int32)
    nan = x.isnan()
    quiet = b.bitwise_or(0x00400000)
    b.add_(b.bitwise_right_shift(8).bitwise_and_(1).add_(0x7F)).bitwise_and_(~0xFF)
    b.copy_(torch.where(nan, quiet, b))
    return x


# ------------------------------------------------------------------ stores

class MomentStore(ABC):
    """One flat state vector of one parameter, on ``device``."""

    precision: str

    def __init__(self, numel: int, device=None):
        self.numel = numel
        self.device = torch.device(device) if device is not None else torch.device("cpu")

    @abstractmethod
    def to_fp32(self) -> torch.Tensor: ...

    @abstractmethod
    def write(self, lo: int, hi: int, x: torch.Tensor, seed: int | None = None) -> None:
        """Store FP32 ``x`` (clobbered) into ``[lo, hi)``: stochastic with stream ``seed``, else nearest-even."""

    @property
    @abstractmethod
    def nbytes(self) -> int: ...

    @property
    def native_buffers(self) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(values or codes, block scales or None) in the kernel's layout."""
        raise NotImplementedError

    @abstractmethod
    def state_dict(self) -> dict[str, Any]: ...


class FP32Store(MomentStore):
    precision = "fp32"

    def __init__(self, numel: int, init: torch.Tensor | None = None, device=None):
        super().__init__(numel, device)
        self.data = torch.zeros(numel, dtype=torch.float32, device=self.device)
        if init is not None:
            self.data.copy_(init.detach().reshape(-1))

    @classmethod
    def wrap(cls, data: torch.Tensor) -> "FP32Store":
        """A store over an existing flat FP32 tensor (an FP32 parameter updated in place)."""
        store = cls.__new__(cls)
        MomentStore.__init__(store, data.numel(), data.device)
        store.data = data
        return store

    def write(self, lo, hi, x, seed=None):
        dst = self.data[lo:hi]
        if x.data_ptr() != dst.data_ptr():
            dst.copy_(x)

    def to_fp32(self):
        return self.data.clone()

    @property
    def nbytes(self):
        return self.data.nbytes

    @property
    def native_buffers(self):
        return self.data, None

    def state_dict(self):
        return {"precision": "fp32", "data": self.data}


def _device_encode(x: torch.Tensor, dst: torch.Tensor, dst_scale: torch.Tensor | None, n: int, role: str) -> None:
    """Nearest-even encode of ``n`` values into a device store's buffers with the library's
    conversion kernel (adambridge_convert): the same bits as the torch casts below produce on the
    host, in one pass over HBM."""
    from . import _hip   # the library is needed only once a store lives on the device

    src = x.detach().reshape(-1)[:n].to(dst.device, torch.float32).contiguous()
    _hip.load().convert(src, None, dst, dst_scale, n, role)


class BF16Store(MomentStore):
    """BF16 values, nearest-even from FP32 (torch's rounding: NaN becomes 0x7fc0)."""

    precision = "bf16"

    def __init__(self, numel: int, init: torch.Tensor | None = None, device=None):
        super().__init__(numel, device)
        self.data = torch.zeros(numel, dtype=torch.bfloat16, device=self.device)
        if init is not None:
            self.write(0, numel, init)

    def write(self, lo, hi, x, seed=None):
        if seed is not None:
            self.data[lo:hi].copy_(round_to_bf16_stochastic(x, seed, lo))
        elif self.data.is_cuda:
            _device_encode(x, self.data[lo:hi], None, hi - lo, "m")
        else:
            self.data[lo:hi].copy_(x.detach().reshape(-1))   # torch rounds to nearest even

    def to_fp32(self):
        return self.data.float()

    @property
    def nbytes(self):
        return self.data.nbytes

    @property
    def native_buffers(self):
        return self.data, None

    def state_dict(self):
        return {"precision": "bf16", "data": self.data}


class FP8Store(MomentStore):
    """FP8 codes padded to whole 128-element blocks, one FP32 scale per block.  The
    second moment ('v') is stored as sqrt(v) in E5M2 (precision.py:341-418)."""

    precision = "fp8"

    def __init__(self, numel: int, role: str, init: torch.Tensor | None = None, block: int = FP8_BLOCK,
                 device=None):
        super().__init__(numel, device)
        if role not in _FP8_FORMATS:
            raise ValueError(f"role must be 'm' or 'v', got {role!r}")
        self.role = role
        self.block = block
        self.dtype, self.fmax, _ = _FP8_FORMATS[role]
        self.sqrt_domain = role == "v"
        nblocks = max(1, math.ceil(numel / block))
        self.q = torch.zeros(nblocks * block, dtype=self.dtype, device=self.device)
        self.scale = torch.ones(nblocks, dtype=torch.float32, device=self.device)
        if init is not None:
            self.write(0, numel, init.detach().reshape(-1).to(self.device, torch.float32).clone())

    def read(self, lo: int, hi: int) -> torch.Tensor:
        b0, b1 = lo // self.block, math.ceil(hi / self.block)
        x = self.q[b0 * self.block: b1 * self.block].float().view(-1, self.block)
        x.mul_(self.scale[b0:b1, None])
        if self.sqrt_domain:
            x.square_()
        return x.view(-1)[: hi - lo]

    def write(self, lo, hi, x, seed=None):
        n = hi - lo
        b0, b1 = lo // self.block, math.ceil(hi / self.block)
        if seed is None and self.q.is_cuda and self.block == FP8_BLOCK:
            if lo % self.block:
                raise ValueError("FP8 writes start on a block boundary")
            _device_encode(x, self.q[b0 * self.block: b1 * self.block], self.scale[b0:b1], n, self.role)
            return
        if self.sqrt_domain:
            x = x.clamp_(min=0).sqrt_()
        padded = (b1 - b0) * self.block
        if padded != n:
            x = torch.nn.functional.pad(x, (0, padded - n))
        xb = x.view(-1, self.block)
        amax = xb.abs().amax(dim=1)
        scale = torch.where(amax > 0, amax / self.fmax, torch.ones_like(amax))
        xb.div_(scale[:, None])
        flat = xb.view(-1)
        if seed is not None:
            q = round_to_fp8_stochastic(flat, self.dtype, seed, b0 * self.block)
        else:
            q = flat.clamp_(-self.fmax, self.fmax).to(self.dtype)
        self.q[b0 * self.block: b1 * self.block].copy_(q)
        self.scale[b0:b1].copy_(scale)

    def to_fp32(self):
        return self.read(0, self.numel).clone()

    @property
    def nbytes(self):
        return self.q.nbytes + self.scale.nbytes

    @property
    def native_buffers(self):
        if self.block != FP8_BLOCK:
            raise ValueError("the kernel implements 128-element FP8 blocks only")
        return self.q, self.scale

    def state_dict(self):
        return {"precision": "fp8", "role": self.role, "block": self.block, "q": self.q, "scale": self.scale}


class FP24Store(MomentStore):
    """FP24 master: ``hi`` (bfloat16 = the top 16 bits) and ``lo`` (uint8 = the next 8)."""

    precision = "fp24"
    INIT_CHUNK = 1 << 24

    def __init__(self, numel: int, init: torch.Tensor | None = None, device=None):
        super().__init__(numel, device)
        self.hi = torch.zeros(numel, dtype=torch.bfloat16, device=self.device)
        self.lo = torch.zeros(numel, dtype=torch.uint8, device=self.device)
        if init is not None:
            self.init_from_(init)

    def init_from_(self, src: torch.Tensor) -> None:
        """From any tensor: a BF16 source is exact (lo = 0); anything else rounds to nearest even,
        a chunk at a time (precision.py:441-455)."""
        src = src.detach().reshape(-1)
        if src.dtype == torch.bfloat16:
            self.hi.copy_(src)
            self.lo.zero_()
            return
        for lo in range(0, self.numel, self.INIT_CHUNK):
            hi = min(lo + self.INIT_CHUNK, self.numel)
            self.write(lo, hi, src[lo:hi].to(self.device, torch.float32, copy=True))

    def read(self, lo: int, hi: int) -> torch.Tensor:
        x = self.hi[lo:hi].float()
        x.view(torch.int32).bitwise_or_(self.lo[lo:hi].to(torch.int32).bitwise_left_shift(8))
        return x

    def write(self, lo, hi, x, seed=None):
        if seed is not None:
            round_to_fp24_stochastic(x, seed, lo)
        else:
            round_to_fp24_nearest_(x)
        b = x.view(torch.int32)
        self.hi[lo:hi].view(torch.int16).copy_(b.bitwise_right_shift(16).to(torch.int16))
        self.lo[lo:hi].copy_(b.bitwise_right_shift(8).bitwise_and(0xFF).to(torch.uint8))

    def to_fp32(self):
        return self.read(0, self.numel)

    @property
    def nbytes(self):
        return self.hi.nbytes + self.lo.nbytes

    @property
    def native_buffers(self):
        return self.hi, self.lo

    def state_dict(self):
        return {"precision": "fp24", "hi": self.hi, "lo": self.lo}


class PackedState:
    """FP32 master and BF16 moments of one parameter interleaved in HBM, 16 bytes per pair of
    elements: {p[2k], p[2k+1], m[2k] | m[2k+1] << 16, v[2k] | v[2k+1] << 16} (the kernel's
    ADAMBRIDGE_DT_PACKED layout).  One 16-byte stream instead of three separate ones, which the
    MI355X memory system streams faster.  With ``double_buffer`` two buffers alternate: the
    kernel reads ``current`` and writes ``other``, then :meth:`flip` makes the result current.

    The values are exactly those of an FP32Store master and two BF16Store moments; ``get`` and
    ``set`` convert to and from those flat tensors (checkpoints, ``set_precision``)."""

    def __init__(self, numel: int, init: torch.Tensor | None = None, device=None, double_buffer: bool = False):
        self.numel = numel
        self.device = torch.device(device) if device is not None else torch.device("cpu")
        pairs = max(1, (numel + 1) // 2)
        self.bufs = [torch.zeros(pairs, 4, dtype=torch.int32, device=self.device)]
        if double_buffer:
            self.bufs.append(torch.zeros(pairs, 4, dtype=torch.int32, device=self.device))
        self.cur = 0
        if init is not None:
            self.set("p", init.detach().reshape(-1).to(self.device, torch.float32))

    @property
    def current(self) -> torch.Tensor:
        return self.bufs[self.cur]

    @property
    def other(self) -> torch.Tensor | None:
        return self.bufs[1 - self.cur] if len(self.bufs) == 2 else None

    def flip(self) -> None:
        if len(self.bufs) == 2:
            self.cur = 1 - self.cur

    def _columns(self, role: str) -> torch.Tensor:
        """(pairs, 2) strided view of the role's two values per pair."""
        if role == "p":
            return self.current.view(torch.float32)[:, 0:2]
        col = 4 if role == "m" else 6
        return self.current.view(torch.bfloat16)[:, col:col + 2]

    def get(self, role: str) -> torch.Tensor:
        """Flat contiguous copy: FP32 master (role 'p') or BF16 moment ('m', 'v')."""
        return self._columns(role).reshape(-1)[: self.numel].clone()

    def set(self, role: str, x: torch.Tensor) -> None:
        dst = self._columns(role)
        flat = x.reshape(-1).to(self.device, dst.dtype)
        if flat.numel() != 2 * dst.shape[0]:
            flat = torch.nn.functional.pad(flat, (0, 2 * dst.shape[0] - flat.numel()))
        dst.copy_(flat.view(-1, 2))

    @property
    def nbytes(self) -> int:
        return sum(b.nbytes for b in self.bufs)


class PackedMaster(MomentStore):
    """The FP32 master held in a :class:`PackedState` (precision 'fp32')."""

    precision = "fp32"

    def __init__(self, packed: PackedState):
        super().__init__(packed.numel, packed.device)
        self.packed = packed

    @property
    def data(self) -> torch.Tensor:
        return self.packed.get("p")

    def write(self, lo, hi, x, seed=None):
        if lo != 0 or hi != self.numel:
            raise ValueError("a packed master is written whole")
        self.packed.set("p", x)

    def to_fp32(self):
        return self.packed.get("p")

    @property
    def nbytes(self):
        return self.packed.nbytes // 2   # 8 of every 16 bytes (per buffer)

    def state_dict(self):
        return {"precision": "fp32", "data": self.packed.get("p")}


class PackedMoment(MomentStore):
    """A BF16 moment held in a :class:`PackedState` (precision 'bf16')."""

    precision = "bf16"

    def __init__(self, packed: PackedState, role: str):
        super().__init__(packed.numel, packed.device)
        self.packed = packed
        self.role = role

    @property
    def data(self) -> torch.Tensor:
        return self.packed.get(self.role)

    def write(self, lo, hi, x, seed=None):
        if lo != 0 or hi != self.numel:
            raise ValueError("a packed moment is written whole")
        if seed is not None:
            x = round_to_bf16_stochastic(x, seed, 0)
        self.packed.set(self.role, x)

    def to_fp32(self):
        return self.packed.get(self.role).float()

    @property
    def nbytes(self):
        return self.packed.nbytes // 4   # 4 of every 16 bytes

    def state_dict(self):
        return {"precision": "bf16", "data": self.packed.get(self.role)}


RECORD_BYTES = 768


class RecordState:
    """FP32 master and both FP8 moments of one parameter in one 768-byte record per 128-element
    block (the kernel's ADAMBRIDGE_DT_PACKED_FP8 layout), plus the two block-scale arrays.  In the
    record of block b, lane l's elements 128b + 8l + j (j < 8) hold their master at byte 16l + 4j
    (j < 4) or 256 + 16l + 4(j - 4) (j >= 4), their E4M3 m code at 512 + 16l + j and their E5M2
    code of sqrt(v) at 520 + 16l + j.  The kernel then reads and writes one contiguous stream of
    state instead of three, which keeps its speed the same wherever the buffers land in HBM.

    The values are exactly those of an FP32Store master and two FP8Store moments; ``get`` /
    ``set`` convert the master, ``codes`` / ``set_codes`` the moments' codes."""

    def __init__(self, numel: int, init: torch.Tensor | None = None, device=None):
        self.numel = numel
        self.device = torch.device(device) if device is not None else torch.device("cpu")
        self.blocks = max(1, math.ceil(numel / FP8_BLOCK))
        self.rec = torch.zeros(self.blocks, RECORD_BYTES, dtype=torch.uint8, device=self.device)
        self.scales = {"m": torch.ones(self.blocks, dtype=torch.float32, device=self.device),
                       "v": torch.ones(self.blocks, dtype=torch.float32, device=self.device)}
        if init is not None:
            self.set("p", init.detach().reshape(-1).to(self.device, torch.float32))

    # the kernel's buffer, in the interface of PackedState (one buffer, updated in place)
    @property
    def current(self) -> torch.Tensor:
        return self.rec

    other = None

    def flip(self) -> None:
        pass

    def _master(self) -> torch.Tensor:
        """(blocks, 16, 2, 4) strided FP32 view: [b, l, h, j] is element 128b + 8l + 4h + j."""
        return self.rec[:, :512].view(torch.float32).view(self.blocks, 2, 16, 4).permute(0, 2, 1, 3)

    def _codes(self, role: str) -> torch.Tensor:
        """(blocks, 16, 8) strided uint8 view of the role's codes, element order."""
        lo = 0 if role == "m" else 8
        return self.rec[:, 512:].view(self.blocks, 16, 16)[:, :, lo:lo + 8]

    def get(self, role: str) -> torch.Tensor:
        """Flat contiguous copy of the FP32 master (role 'p')."""
        if role != "p":
            raise ValueError("records hold the master as values and the moments as codes")
        return self._master().reshape(-1)[: self.numel].clone()

    def set(self, role: str, x: torch.Tensor) -> None:
        if role != "p":
            raise ValueError("records hold the master as values and the moments as codes")
        flat = x.reshape(-1).to(self.device, torch.float32)
        if flat.numel() != self.blocks * FP8_BLOCK:
            flat = torch.nn.functional.pad(flat, (0, self.blocks * FP8_BLOCK - flat.numel()))
        self._master().copy_(flat.view(self.blocks, 16, 2, 4))

    def codes(self, role: str) -> torch.Tensor:
        """The role's codes, padded to whole blocks, as a contiguous FP8 tensor (FP8Store.q)."""
        return self._codes(role).reshape(-1).view(_FP8_FORMATS[role][0])

    def set_codes(self, role: str, q: torch.Tensor) -> None:
        self._codes(role).copy_(q.reshape(-1).view(torch.uint8).view(self.blocks, 16, 8))

    @property
    def nbytes(self) -> int:
        return self.rec.nbytes + sum(t.nbytes for t in self.scales.values())


class RecordMaster(MomentStore):
    """The FP32 master held in a :class:`RecordState` (precision 'fp32')."""

    precision = "fp32"

    def __init__(self, records: RecordState):
        super().__init__(records.numel, records.device)
        self.packed = records

    @property
    def data(self) -> torch.Tensor:
        return self.packed.get("p")

    def write(self, lo, hi, x, seed=None):
        if lo != 0 or hi != self.numel:
            raise ValueError("a master in records is written whole")
        self.packed.set("p", x)

    def to_fp32(self):
        return self.packed.get("p")

    @property
    def nbytes(self):
        return 4 * self.numel   # the master values (the last record's unused slots count with m)

    def state_dict(self):
        return {"precision": "fp32", "data": self.packed.get("p")}


class RecordMoment(MomentStore):
    """An FP8 moment held in a :class:`RecordState` (precision 'fp8'): its codes in the records,
    its block scales in the state's scale array for the role."""

    precision = "fp8"
    block = FP8_BLOCK

    def __init__(self, records: RecordState, role: str):
        super().__init__(records.numel, records.device)
        self.packed = records
        self.role = role

    @property
    def q(self) -> torch.Tensor:
        return self.packed.codes(self.role)

    @property
    def scale(self) -> torch.Tensor:
        return self.packed.scales[self.role]

    def _store(self) -> "FP8Store":
        """A separate FP8Store with this moment's codes and scales (a copy)."""
        st = FP8Store(self.numel, self.role, device=self.device)
        st.q.copy_(self.q)
        st.scale.copy_(self.scale)
        return st

    def adopt(self, store: "FP8Store") -> None:
        """Take the codes and scales of a separate FP8Store of the same size and role."""
        if store.block != FP8_BLOCK or store.role != self.role or store.numel != self.numel:
            raise ValueError("records take 128-element FP8 blocks of the same role and size")
        self.packed.set_codes(self.role, store.q)
        self.scale.copy_(store.scale)

    def read(self, lo: int, hi: int) -> torch.Tensor:
        return self._store().read(lo, hi)

    def write(self, lo, hi, x, seed=None):
        if lo != 0 or hi != self.numel:
            raise ValueError("a moment in records is written whole")
        st = FP8Store(self.numel, self.role, device=self.device)
        st.write(0, self.numel, x, seed)
        self.adopt(st)

    def to_fp32(self):
        return self._store().to_fp32()

    @property
    def nbytes(self):
        # 128 code bytes per record and one scale, as a separate FP8Store; m also counts the master
        # slots of the last record past the end, so that master + m + v is the whole RecordState
        pad = self.packed.blocks * 512 - 4 * self.numel if self.role == "m" else 0
        return self.packed.blocks * (FP8_BLOCK + 4) + pad

    def state_dict(self):
        return {"precision": "fp8", "role": self.role, "block": FP8_BLOCK, "q": self.q, "scale": self.scale}


def make_store(precision: str, numel: int, role: str, init: torch.Tensor | None = None, device=None) -> MomentStore:
    precision = canonical_precision(precision)
    if device is None and init is not None:
        device = init.device
    if precision == "fp32":
        return FP32Store(numel, init, device=device)
    if precision == "bf16":
        return BF16Store(numel, init, device=device)
    return FP8Store(numel, role, init, device=device)


def make_master(precision: str, numel: int, init: torch.Tensor | None = None, device=None) -> MomentStore:
    precision = canonical_master_precision(precision)
    if device is None and init is not None:
        device = init.device
    if precision == "fp24":
        return FP24Store(numel, init, device=device)
    return FP32Store(numel, init, device=device)


def _checked(t: Any, numel: int, what: str) -> torch.Tensor:
    """``t`` if it is a tensor of exactly ``numel`` elements (precision.py:534-540)."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"checkpoint {what} is {type(t).__name__}, expected a tensor")
    if t.numel() != numel:
        raise ValueError(f"checkpoint {what} has {t.numel()} elements, expected {numel} (a different model?)")
    return t


def check_master_state(saved: Any, numel: int, what: str) -> None:
    """Validate checkpoint master weights: an FP32 tensor or an fp32/fp24 store dict (precision.py:501-516)."""
    if isinstance(saved, torch.Tensor):
        _checked(saved, numel, what)
        return
    if not isinstance(saved, dict) or saved.get("precision") not in MASTER_PRECISIONS:
        raise ValueError(f"checkpoint {what}: expected a tensor or an fp32/fp24 store, got "
                         f"{saved.get('precision') if isinstance(saved, dict) else type(saved).__name__!r}")
    if saved["precision"] == "fp24":
        if _checked(saved.get("hi"), numel, f"{what} (hi plane)").dtype != torch.bfloat16:
            raise ValueError(f"checkpoint {what}: the hi plane must be bfloat16")
        if _checked(saved.get("lo"), numel, f"{what} (lo plane)").dtype != torch.uint8:
            raise ValueError(f"checkpoint {what}: the lo plane must be uint8")
    else:
        _checked(saved.get("data"), numel, what)


def master_to_fp32(saved: Any, numel: int, device=None) -> torch.Tensor:
    """Checkpoint master weights as a flat FP32 tensor on ``device``."""
    if isinstance(saved, torch.Tensor):
        return saved.detach().reshape(-1).to(device, torch.float32)
    if saved["precision"] == "fp24":
        store = FP24Store(numel, device=device)
        store.hi.copy_(saved["hi"].reshape(-1))
        store.lo.copy_(saved["lo"].reshape(-1))
        return store.to_fp32()
    return saved["data"].detach().reshape(-1).to(device, torch.float32)


def load_master_(store: MomentStore, saved: Any) -> None:
    """Load validated checkpoint master weights into ``store``, converting fp32 <-> fp24."""
    if isinstance(store, FP24Store) and isinstance(saved, dict) and saved.get("precision") == "fp24":
        store.hi.copy_(saved["hi"].reshape(-1))
        store.lo.copy_(saved["lo"].reshape(-1))
        return
    x = master_to_fp32(saved, store.numel, store.device)
    if isinstance(store, FP32Store):
        store.data.copy_(x)
        return
    src = saved if isinstance(saved, torch.Tensor) else saved.get("data")
    if isinstance(src, torch.Tensor) and x.data_ptr() == src.data_ptr():
        x = x.clone()
    store.write(0, store.numel, x)


def store_from_state_dict(state: dict[str, Any], numel: int, role: str, device=None) -> MomentStore:
    """Rebuild a moment store from a checkpoint, validating every field (precision.py:555-575)."""
    if not isinstance(state, dict) or state.get("precision") not in PRECISIONS:
        raise ValueError("checkpoint moment store has unknown precision "
                         f"{state.get('precision') if isinstance(state, dict) else state!r}")
    precision = state["precision"]
    if precision == "fp8":
        saved_role, block = state.get("role", role), state.get("block")
        if saved_role not in _FP8_FORMATS:
            raise ValueError(f"checkpoint FP8 store has unknown role {saved_role!r}")
        if not isinstance(block, int) or isinstance(block, bool) or not 0 < block <= 1 << 20:
            raise ValueError(f"checkpoint FP8 store has invalid block size {block!r}")
        store = FP8Store(numel, saved_role, block=block, device=device)
        store.q.copy_(_checked(state.get("q"), store.q.numel(), "FP8 codes"))
        store.scale.copy_(_checked(state.get("scale"), store.scale.numel(), "FP8 scales"))
        if saved_role != role or block != FP8_BLOCK:
            store = FP8Store(numel, role, init=store.to_fp32(), device=device)
        return store
    store = make_store(precision, numel, role, device=device)
    store.data.copy_(_checked(state.get("data"), numel, f"{precision} moments"))
    return store
