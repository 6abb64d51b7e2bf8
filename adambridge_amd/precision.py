"""Moment and master stores: one flat vector of optimizer state in one storage format.

The reference's store API (adambridge/precision.py: ``make_store``,
``FP8Store``, ``state_dict`` dictionaries, ...) over the stateless codecs of
:mod:`adambridge_amd.formats`.  A store keeps its tensors on one device; on a
GPU they sit in HBM next to the parameter.  The optimizer's fused kernel reads
and writes them in place through :attr:`MomentStore.native_buffers`; the
methods here are for everything off the step path: initial values,
``set_precision``, checkpoints and inspection.

Checkpoint dictionaries are the reference's, key for key, so checkpoints move
between the two implementations:

    fp32 / bf16   {"precision", "data"}
    fp8           {"precision": "fp8", "role", "block", "q", "scale"}
    fp24 master   {"precision": "fp24", "hi", "lo"}
"""

from __future__ import annotations

from typing import Any

import torch

from . import formats as F
from .formats import (FP8_BLOCK, MASTER_PRECISIONS, PRECISIONS, bytes_per_param, canonical_master_precision,
                      canonical_precision)

__all__ = [
    "PRECISIONS", "MASTER_PRECISIONS", "FP8_BLOCK", "canonical_precision", "canonical_master_precision",
    "MomentStore", "FP32Store", "BF16Store", "FP8Store", "FP24Store", "make_store", "make_master",
    "store_from_state_dict", "check_master_state", "load_master_", "master_to_fp32", "bytes_per_param",
    "round_to_bf16_stochastic", "round_to_fp8_stochastic", "round_to_fp24_stochastic", "round_to_fp24_nearest_",
    "moment_seed", "random_bits",
]


# ----------------------------------------------- the reference's rounding helpers

def moment_seed(seed: int, role: str) -> int:
    """32-bit rounding stream of ``role`` ('m', 'v' or 'p', the FP24 master) for a step seed."""
    return F.stream_seed(seed, role)


def random_bits(offset: int, n: int, seed: int, device=None) -> torch.Tensor:
    """The rounding stream's bits for element indices offset .. offset + n - 1, as int32 patterns."""
    h = F.counter_hash(offset, n, seed, device)
    return (h - ((h >> 31) << 32)).to(torch.int32)


def round_to_bf16_stochastic(x: torch.Tensor, seed: int, offset: int = 0) -> torch.Tensor:
    """FP32 ``x`` stochastically rounded to BF16 (``offset``: stream index of x[0])."""
    return F.bf16_encode(x, seed, offset).view(x.shape)


def round_to_fp8_stochastic(x: torch.Tensor, dtype: torch.dtype, seed: int, offset: int = 0) -> torch.Tensor:
    """Pre-scaled FP32 ``x`` stochastically rounded to the FP8 ``dtype``, clamped to its range."""
    fmt = next(f for f in F.FP8_FORMATS.values() if f.dtype == dtype)
    cut = F.round_bits_stochastic(x, 23 - fmt.mantissa_bits, offset, seed)
    return cut.clamp(-fmt.fmax, fmt.fmax).to(dtype).view(x.shape)


def round_to_fp24_stochastic(x: torch.Tensor, seed: int, offset: int = 0) -> torch.Tensor:
    """FP32 ``x`` stochastically rounded in place to its top 24 bits; returns ``x``."""
    return x.copy_(F.fp24_round(x, seed, offset).view(x.shape))


def round_to_fp24_nearest_(x: torch.Tensor) -> torch.Tensor:
    """FP32 ``x`` rounded in place to its top 24 bits, nearest-even, a NaN kept NaN; returns ``x``."""
    return x.copy_(F.fp24_round(x).view(x.shape))


# ---------------------------------------------------------------------- stores

def _home(device, init: torch.Tensor | None) -> torch.device:
    if device is not None:
        return torch.device(device)
    return init.device if init is not None else torch.device("cpu")


def _flat_fp32(x: torch.Tensor, device: torch.device) -> torch.Tensor:
    return x.detach().reshape(-1).to(device=device, dtype=torch.float32)


class MomentStore:
    """A flat vector of ``numel`` values in one format, on ``device``.

    ``write(lo, hi, x, seed)`` stores FP32 ``x`` into ``[lo, hi)`` -- stochastically rounded with
    stream ``seed``, or nearest-even without one; ``read(lo, hi)`` and ``to_fp32()`` decode."""

    precision = ""

    def __init__(self, numel: int, device):
        self.numel = int(numel)
        self.device = torch.device(device)

    def read(self, lo: int, hi: int) -> torch.Tensor:
        return self.to_fp32()[lo:hi]

    def write(self, lo: int, hi: int, x: torch.Tensor, seed: int | None = None) -> None:
        raise NotImplementedError

    def to_fp32(self) -> torch.Tensor:
        raise NotImplementedError

    @property
    def tensors(self) -> tuple[torch.Tensor, ...]:
        """Every tensor the store owns."""
        raise NotImplementedError

    @property
    def nbytes(self) -> int:
        return sum(t.nbytes for t in self.tensors)

    @property
    def native_buffers(self) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(values or codes, second buffer -- FP8 block scales or the FP24 low plane -- or None), the
        buffers the fused kernel takes."""
        raise NotImplementedError

    def state_dict(self) -> dict[str, Any]:
        raise NotImplementedError


class FP32Store(MomentStore):
    precision = "fp32"

    def __init__(self, numel: int, init: torch.Tensor | None = None, device=None):
        super().__init__(numel, _home(device, init))
        self.data = torch.zeros(self.numel, dtype=torch.float32, device=self.device)
        if init is not None:
            self.data.copy_(init.detach().reshape(-1))

    @classmethod
    def wrap(cls, data: torch.Tensor) -> "FP32Store":
        """The store whose values are the flat FP32 tensor ``data`` itself (an FP32 parameter that
        the kernel updates in place)."""
        store = cls(0, device=data.device)
        store.numel, store.data = data.numel(), data
        return store

    def read(self, lo, hi):
        return self.data[lo:hi]

    def write(self, lo, hi, x, seed=None):
        dst = self.data[lo:hi]
        if x.data_ptr() != dst.data_ptr():
            dst.copy_(x.detach().reshape(-1))

    def to_fp32(self):
        return self.data.clone()

    @property
    def tensors(self):
        return (self.data,)

    @property
    def native_buffers(self):
        return self.data, None

    def state_dict(self):
        return {"precision": "fp32", "data": self.data}


class BF16Store(MomentStore):
    precision = "bf16"

    def __init__(self, numel: int, init: torch.Tensor | None = None, device=None):
        super().__init__(numel, _home(device, init))
        self.data = torch.zeros(self.numel, dtype=torch.bfloat16, device=self.device)
        if init is not None:
            self.write(0, self.numel, init)

    def read(self, lo, hi):
        return self.data[lo:hi].float()

    def write(self, lo, hi, x, seed=None):
        self.data[lo:hi].copy_(F.bf16_encode(_flat_fp32(x, self.device), seed, lo))

    def to_fp32(self):
        return self.data.float()

    @property
    def tensors(self):
        return (self.data,)

    @property
    def native_buffers(self):
        return self.data, None

    def state_dict(self):
        return {"precision": "bf16", "data": self.data}


class FP8Store(MomentStore):
    """Block-scaled FP8 codes (``q``, padded to whole blocks) and one FP32 scale per block
    (``scale``); role 'v' keeps sqrt(v).  The fused kernel takes 128-element blocks."""

    precision = "fp8"

    def __init__(self, numel: int, role: str, init: torch.Tensor | None = None, block: int = FP8_BLOCK,
                 device=None):
        super().__init__(numel, _home(device, init))
        if role not in F.FP8_FORMATS:
            raise ValueError(f"role must be 'm' or 'v', got {role!r}")
        self.role, self.block = role, int(block)
        self.format = F.FP8_FORMATS[role]
        self.dtype, self.fmax = self.format.dtype, self.format.fmax
        self.sqrt_domain = self.format.sqrt_domain
        nb = F.fp8_blocks(self.numel, self.block)
        self.q = torch.zeros(nb * self.block, dtype=self.dtype, device=self.device)
        self.scale = torch.ones(nb, dtype=torch.float32, device=self.device)
        if init is not None:
            self.write(0, self.numel, init)

    def _blocks(self, lo: int, hi: int) -> tuple[int, int]:
        return lo // self.block, -(-hi // self.block)

    def read(self, lo, hi):
        b0, b1 = self._blocks(lo, hi)
        codes = self.q[b0 * self.block: b1 * self.block]
        return F.fp8_decode(codes, self.scale[b0:b1], self.role, (b1 - b0) * self.block)[lo - b0 * self.block:
                                                                                          hi - b0 * self.block]

    def write(self, lo, hi, x, seed=None):
        if lo % self.block:
            raise ValueError("FP8 writes start on a block boundary")
        b0 = lo // self.block
        codes, scales = F.fp8_encode(_flat_fp32(x, self.device)[: hi - lo], self.role, seed, lo, self.block)
        self.q[b0 * self.block: b0 * self.block + codes.numel()].copy_(codes)
        self.scale[b0: b0 + scales.numel()].copy_(scales)

    def to_fp32(self):
        return F.fp8_decode(self.q, self.scale, self.role, self.numel).clone()

    @property
    def tensors(self):
        return (self.q, self.scale)

    @property
    def native_buffers(self):
        if self.block != FP8_BLOCK:
            raise ValueError("the kernel implements 128-element FP8 blocks only")
        return self.q, self.scale

    def state_dict(self):
        return {"precision": "fp8", "role": self.role, "block": self.block, "q": self.q, "scale": self.scale}


class FP24Store(MomentStore):
    """The FP24 master: ``hi`` (bfloat16, the top 16 bits) and ``lo`` (uint8, the next 8)."""

    precision = "fp24"
    INIT_CHUNK = 1 << 24   # elements converted at a time from a wider source (bounds the temporaries)

    def __init__(self, numel: int, init: torch.Tensor | None = None, device=None):
        super().__init__(numel, _home(device, init))
        self.hi = torch.zeros(self.numel, dtype=torch.bfloat16, device=self.device)
        self.lo = torch.zeros(self.numel, dtype=torch.uint8, device=self.device)
        if init is not None:
            self.init_from_(init)

    def init_from_(self, src: torch.Tensor) -> None:
        """Planes from ``src``: BF16 bits are exact (low plane zero); other values round to nearest even,
        INIT_CHUNK elements at a time."""
        flat = src.detach().reshape(-1)
        if flat.dtype == torch.bfloat16:
            self.hi.copy_(flat)
            self.lo.zero_()
            return
        if self.device.type == "cuda" and flat.dtype == torch.float32:   # one pass, no temporaries
            self.write(0, self.numel, flat)
            return
        for a in range(0, self.numel, self.INIT_CHUNK):
            b = min(self.numel, a + self.INIT_CHUNK)
            self.write(a, b, flat[a:b])

    def read(self, lo, hi):
        return F.fp24_join(self.hi[lo:hi], self.lo[lo:hi])

    def write(self, lo, hi, x, seed=None):
        F.fp24_encode(_flat_fp32(x, self.device), seed, lo, out=(self.hi[lo:hi], self.lo[lo:hi]))

    def to_fp32(self):
        return self.read(0, self.numel)

    @property
    def tensors(self):
        return (self.hi, self.lo)

    @property
    def native_buffers(self):
        return self.hi, self.lo

    def state_dict(self):
        return {"precision": "fp24", "hi": self.hi, "lo": self.lo}


_MOMENT_STORES = {"fp32": FP32Store, "bf16": BF16Store}


def make_store(precision: str, numel: int, role: str, init: torch.Tensor | None = None, device=None) -> MomentStore:
    """A moment store of ``precision`` for ``role`` ('m' or 'v': which FP8 format)."""
    precision = canonical_precision(precision)
    if precision == "fp8":
        return FP8Store(numel, role, init, device=device)
    return _MOMENT_STORES[precision](numel, init, device=device)


def make_master(precision: str, numel: int, init: torch.Tensor | None = None, device=None) -> MomentStore:
    """A master-weight store, 'fp32' or 'fp24'."""
    precision = canonical_master_precision(precision)
    return (FP24Store if precision == "fp24" else FP32Store)(numel, init, device=device)


# ----------------------------------------------------------------- checkpoints

def _tensor_of(value: Any, numel: int, what: str) -> torch.Tensor:
    """``value`` if it is a tensor of exactly ``numel`` elements; a ValueError naming ``what`` otherwise
    (a checkpoint may come from another model, another version or an untrusted source)."""
    if not isinstance(value, torch.Tensor):
        raise ValueError(f"checkpoint {what} is {type(value).__name__}, expected a tensor")
    if value.numel() != numel:
        raise ValueError(f"checkpoint {what} has {value.numel()} elements, expected {numel} (a different model?)")
    return value


_checked = _tensor_of


def check_master_state(saved: Any, numel: int, what: str) -> None:
    """Raise ValueError unless ``saved`` is checkpoint master weights for ``numel`` elements: an FP32
    tensor, an fp32 store dict or an fp24 store dict with bfloat16 / uint8 planes."""
    if isinstance(saved, torch.Tensor):
        _tensor_of(saved, numel, what)
        return
    kind = saved.get("precision") if isinstance(saved, dict) else None
    if kind not in MASTER_PRECISIONS:
        found = kind if isinstance(saved, dict) else type(saved).__name__
        raise ValueError(f"checkpoint {what}: expected a tensor or an fp32/fp24 store, got {found!r}")
    if kind == "fp32":
        _tensor_of(saved.get("data"), numel, what)
        return
    for plane, dtype in (("hi", torch.bfloat16), ("lo", torch.uint8)):
        if _tensor_of(saved.get(plane), numel, f"{what} ({plane} plane)").dtype != dtype:
            raise ValueError(f"checkpoint {what}: the {plane} plane must be {str(dtype).split('.')[-1]}")


def master_to_fp32(saved: Any, numel: int, device=None) -> torch.Tensor:
    """Validated checkpoint master weights as a flat FP32 tensor on ``device``."""
    if isinstance(saved, dict) and saved.get("precision") == "fp24":   # joined where the values go
        return F.fp24_join(saved["hi"].to(device), saved["lo"].to(device))
    values = saved if isinstance(saved, torch.Tensor) else saved["data"]
    return values.detach().reshape(-1).to(device=device, dtype=torch.float32)


def load_master_(store: MomentStore, saved: Any) -> None:
    """Validated checkpoint master weights into ``store``: planes copied as they are between FP24
    stores, values converted (FP24 rounding to nearest) otherwise."""
    if isinstance(store, FP24Store) and isinstance(saved, dict) and saved.get("precision") == "fp24":
        store.hi.copy_(saved["hi"].reshape(-1))
        store.lo.copy_(saved["lo"].reshape(-1))
        return
    store.write(0, store.numel, master_to_fp32(saved, store.numel, store.device))


def store_from_state_dict(state: Any, numel: int, role: str, device=None) -> MomentStore:
    """A moment store rebuilt from its checkpoint dictionary, every field validated first.  An FP8
    store saved for the other role is decoded in its own format and re-encoded in ``role``'s."""
    kind = state.get("precision") if isinstance(state, dict) else None
    if kind not in PRECISIONS:
        raise ValueError("checkpoint moment store has unknown precision "
                         f"{kind if isinstance(state, dict) else state!r}")
    if kind != "fp8":
        data = _tensor_of(state.get("data"), numel, f"{kind} moments")
        store = make_store(kind, numel, role, device=device)
        store.data.copy_(data.reshape(-1))
        return store
    saved_role, block = state.get("role", role), state.get("block")
    if saved_role not in F.FP8_FORMATS:
        raise ValueError(f"checkpoint FP8 store has unknown role {saved_role!r}")
    if type(block) is not int or not 0 < block <= 1 << 20:
        raise ValueError(f"checkpoint FP8 store has invalid block size {block!r}")
    nb = F.fp8_blocks(numel, block)
    codes = _tensor_of(state.get("q"), nb * block, "FP8 codes")
    scales = _tensor_of(state.get("scale"), nb, "FP8 scales")
    store = FP8Store(numel, saved_role, block=block, device=device)
    store.q.copy_(codes.reshape(-1))
    store.scale.copy_(scales.reshape(-1))
    if saved_role == role:
        return store
    return FP8Store(numel, role, init=store.to_fp32(), device=device)
