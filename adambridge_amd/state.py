"""One parameter's optimizer state in HBM, in the layout the fused kernel streams fastest.

A :class:`ParamState` owns every device buffer of one parameter's state --
master weights, moments, FP8 block scales -- and knows three things about them:

* how the kernel sees them: :meth:`ParamState.bind` fills the state fields of
  the parameter's ``adambridge_segment``;
* what they hold, in the reference's terms: :meth:`ParamState.master_fp32`,
  :meth:`ParamState.moment` (a store of the reference's API), :meth:`ParamState.export`
  (checkpoint entries) and :meth:`ParamState.window` (the separate arrays of an
  element range, for inspection and parity checks);
* how to take values in: :meth:`ParamState.load`.

Layouts (the byte layouts are declared in include/adambridge_hip.h):

==============  =====================================  ======================================
layout          serves                                 bytes of state per element
==============  =====================================  ======================================
separate        anything (the reference's arrays)      master 4 (FP24: 3) + moments
pairs           AdamW, FP32 master, BF16 moments       16 per 2 elements (x2 double-buffered)
fp8-records     AdamW, FP32 master, FP8 moments        768 per 128 + two FP32 scales per 128
fp8-f24-rec.    AdamW, FP24 master, FP8 moments        640 per 128 + two FP32 scales per 128
lion-records    Lion, FP32 master, BF16 moment         1536 per 256 (x2 double-buffered)
lion-f32-rec.   Lion, FP32 master, FP32 moment         2048 per 256 (x2 double-buffered)
lion-fp8-rec.   Lion, FP32 master, FP8 moment          640 per 128 + one FP32 scale per 128
lion-fp8-f24-r. Lion, FP24 master, FP8 moment          512 per 128 + one FP32 scale per 128
f32-records     AdamW, FP32 master, FP32 moments       3072 per 256 (x2 double-buffered)
f24-records     AdamW, FP24 master, BF16 moments       1792 per 256 (x2 double-buffered)
f24-f32-rec.    AdamW, FP24 master, FP32 moments       2816 per 256 (x2 double-buffered)
lion-f24-rec.   Lion, FP24 master, BF16 moment         1280 per 256 (x2 double-buffered)
lion-f24-f32-r. Lion, FP24 master, FP32 moment         1792 per 256 (x2 double-buffered)
==============  =====================================  ======================================

The interleaved layouts turn the master and moment streams into one stream of
state per parameter (measured faster on MI355X, see adambridge_hip.hip).  Values,
roundings and rounding streams are those of the separate arrays, element for
element, so the layout never shows in results or checkpoints.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _hip
from . import formats as F
from .precision import BF16Store, FP8Store, FP24Store, FP32Store, MomentStore, load_master_, make_master, make_store

__all__ = ["ParamState", "SeparateState", "PairState", "AdamRecordState", "LionRecordState", "F32RecordState",
           "F24RecordState", "LionF24RecordState", "AdamF24RecordState", "LionF32RecordState", "LionFP8RecordState", "F24F32RecordState", "LionF24F32RecordState", "LionFP8F24RecordState", "choose_layout", "new_state", "new_states",
           "arena_plan", "arena_memory", "LAYOUTS"]

LAYOUTS = ("separate", "pairs", "fp8-records", "lion-records", "f32-records", "f24-records", "lion-f24-records",
           "fp8-f24-records", "lion-f32-records", "lion-fp8-records", "f24-f32-records",
           "lion-f24-f32-records", "lion-fp8-f24-records")
IN_PLACE = ("fp8-records", "fp8-f24-records", "lion-fp8-records", "lion-fp8-f24-records")   # never double-buffered

# Arenas of at least this many bytes follow an allocate/free of their own size (new_states); None: never.
RECYCLE_MIN_BYTES: int | None = 256 << 20


def choose_layout(algorithm: str, precision: str, master_precision: str, requested: str = "auto",
                  master_is_param: bool = False) -> str:
    """The layout of a parameter's state: the interleaved one for its (algorithm, precision, master
    precision) when there is one and the master is a buffer of the optimizer's own, else 'separate'."""
    if requested == "separate" or master_is_param:
        return "separate"
    if master_precision == "fp24":
        return {("adamw", "bf16"): "f24-records", ("lion", "bf16"): "lion-f24-records",
                ("adamw", "fp8"): "fp8-f24-records", ("adamw", "fp32"): "f24-f32-records",
                ("lion", "fp32"): "lion-f24-f32-records", ("lion", "fp8"): "lion-fp8-f24-records"}.get(
                    (algorithm, precision), "separate")
    return {("adamw", "bf16"): "pairs", ("adamw", "fp8"): "fp8-records", ("adamw", "fp32"): "f32-records",
            ("lion", "bf16"): "lion-records", ("lion", "fp32"): "lion-f32-records",
            ("lion", "fp8"): "lion-fp8-records"}.get((algorithm, precision),
                                                                                        "separate")


class ParamState:
    """Base of the layouts: ``numel`` elements of one parameter on ``device``."""

    layout = ""
    precision = ""            # moment precision
    master_precision = "fp32"
    master_is_param = False   # the master is the FP32 parameter itself, updated in place
    gathers = False           # a checkpoint export builds new tensors (interleaved layouts)

    def __init__(self, numel: int, device, roles: tuple[str, ...]):
        self.numel = int(numel)
        self.device = torch.device(device)
        self.roles = roles    # ('m', 'v') for AdamW, ('m',) for Lion

    # -- the kernel's view ---------------------------------------------------

    def bind(self, seg: _hip.Segment) -> None:
        """Set the state fields of ``seg``: p, p_lo, m, v, m_scale, v_scale, p_dtype, mv_dtype."""
        raise NotImplementedError

    @property
    def alternates(self) -> bool:
        """True if the buffers swap after every update (double buffering): rebind before each launch."""
        return False

    def advance(self) -> None:
        """After a launch: the state just written becomes the current one."""

    # -- contents ----------------------------------------------------------------

    def master_fp32(self) -> torch.Tensor:
        """The master weights as a flat FP32 tensor (a copy unless they are stored as one)."""
        raise NotImplementedError

    def master_plane(self) -> _hip.Plane:
        """Where the master weights lie, as the plane-conversion kernel addresses them
        (adambridge_plane: the separate arrays, or the master column of the interleaved layout)."""
        raise NotImplementedError

    def write_weights(self, param: torch.Tensor) -> None:
        """Write the working weights the masters give (kernels.c:108-112; FP32 parameters take the
        master's value) into ``param`` on the device's current stream: one pass of the
        plane-conversion kernel, no temporaries for a contiguous parameter."""
        dst = param.data
        flat = dst.view(-1) if dst.is_contiguous() else torch.empty(self.numel, dtype=dst.dtype, device=dst.device)
        if self.numel:
            F.convert_plane(self.master_plane(), _hip.plane_of(flat), self.numel, self.device)
        if flat.data_ptr() != dst.data_ptr() or not dst.is_contiguous():
            dst.copy_(flat.view(dst.shape))

    def moment(self, role: str) -> MomentStore:
        """Moment ``role`` as a store of the reference's API (a copy for interleaved layouts)."""
        raise NotImplementedError

    def export_master(self) -> Any:
        """Checkpoint master entry: an FP32 tensor, or an FP24 store dictionary."""
        return self.master_fp32()

    def export(self, host: bool = False) -> dict[str, Any]:
        """This state's checkpoint entries: ``master``, ``exp_avg`` and (AdamW) ``exp_avg_sq``; with
        ``host``, as copies in host memory (what is gathered on the device is freed on return)."""
        out = {"master": self.export_master()}
        for role, key in zip(self.roles, ("exp_avg", "exp_avg_sq")):
            out[key] = self.moment(role).state_dict()
        return _on_host(out) if host else out

    def load(self, master: Any = None, moments: dict[str, MomentStore] | None = None) -> None:
        """Take validated checkpoint master weights (or FP32 values) and moment stores of this state's
        precision; anything left out keeps its value."""
        raise NotImplementedError

    def footprint(self) -> tuple[int, int]:
        """Device bytes held: (master, moments), every buffer counted once."""
        raise NotImplementedError

    def window(self, lo: int, hi: int) -> dict[str, torch.Tensor]:
        """Elements [lo, hi) as the separate arrays the oracle takes: 'p' (FP32, or the FP24 hi plane
        and 'p_lo'), 'm', 'v' (FP32 values, BF16 bits, or FP8 codes with 'm_scale' / 'v_scale' of the
        blocks covering the range; FP8 ranges start on a block boundary)."""
        raise NotImplementedError


def _on_host(entry: Any) -> Any:
    """``entry`` (a tensor, or a checkpoint dictionary of them) with every tensor copied to host memory."""
    if isinstance(entry, torch.Tensor):
        return entry.cpu()
    if isinstance(entry, dict):
        return {k: _on_host(v) for k, v in entry.items()}
    return entry


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _as_master_values(master: Any, numel: int, device) -> torch.Tensor:
    """FP32 values from checkpoint master weights (tensor or store dictionary) or plain values."""
    from .precision import master_to_fp32
    return master_to_fp32(master, numel, device)


def _master_source(master: Any, numel: int, device) -> _hip.Plane:
    """Checkpoint master weights (tensor or store dictionary) or plain values as a device plane the
    plane-conversion kernel reads: FP24 planes, or the values as float32 / bfloat16 (others are
    cast to float32), flat and contiguous on ``device``.  Returns the plane and the tensors that
    hold its memory (to keep alive until the kernel has run)."""
    if isinstance(master, dict) and master.get("precision") == "fp24":
        hi = master["hi"].reshape(-1).to(device).contiguous()
        lo = master["lo"].reshape(-1).to(device).contiguous()
        return _hip.fp24_plane(hi, lo), (hi, lo)
    values = master if isinstance(master, torch.Tensor) else master["data"]
    flat = values.detach().reshape(-1).to(device)
    if flat.dtype not in (torch.float32, torch.bfloat16):
        flat = flat.to(torch.float32)
    flat = flat.contiguous()
    return _hip.plane_of(flat), (flat,)


# ------------------------------------------------------------------- separate

class SeparateState(ParamState):
    """The reference's arrays: a master store (FP32 -- possibly the FP32 parameter itself -- or FP24)
    and one store per moment."""

    layout = "separate"

    def __init__(self, master: MomentStore, moments: dict[str, MomentStore], master_is_param: bool = False):
        super().__init__(master.numel, master.device, tuple(moments))
        self.master = master
        self.stores = dict(moments)
        self.master_is_param = master_is_param   # instance value over the class default
        self.precision = next(iter(moments.values())).precision
        self.master_precision = master.precision

    def bind(self, seg):
        values, low = self.master.native_buffers
        seg.p, seg.p_lo = values.data_ptr(), _ptr(low)
        seg.p_dtype = _hip.MASTER_CODES[self.master_precision]
        m_values, m_scale = self.stores["m"].native_buffers
        seg.m, seg.m_scale = m_values.data_ptr(), _ptr(m_scale)
        seg.v = seg.v_scale = None
        if "v" in self.stores:
            v_values, v_scale = self.stores["v"].native_buffers
            seg.v, seg.v_scale = v_values.data_ptr(), _ptr(v_scale)
        seg.mv_dtype = _hip.MOMENT_CODES[self.precision]

    def master_fp32(self):
        return self.master.data if isinstance(self.master, FP32Store) else self.master.to_fp32()

    def master_plane(self):
        if isinstance(self.master, FP24Store):
            return _hip.fp24_plane(self.master.hi, self.master.lo)
        return _hip.plane_of(self.master.data.view(-1))

    def export_master(self):
        return self.master.data if isinstance(self.master, FP32Store) else self.master.state_dict()

    def moment(self, role):
        return self.stores[role]

    def load(self, master=None, moments=None):
        if master is not None:
            load_master_(self.master, master)
        for role, store in (moments or {}).items():
            if isinstance(store, FP8Store) and store.block != F.FP8_BLOCK:   # the kernel takes 128-blocks
                store = FP8Store(self.numel, role, init=store.to_fp32(), device=self.device)
            self.stores[role] = store if store.device == self.device else _moved(store, self.device)

    def footprint(self):
        master = 0 if self.master_is_param else self.master.nbytes
        return master, sum(s.nbytes for s in self.stores.values())

    def window(self, lo, hi):
        out: dict[str, torch.Tensor] = {}
        if isinstance(self.master, FP24Store):
            out["p"], out["p_lo"] = self.master.hi[lo:hi], self.master.lo[lo:hi]
        else:
            out["p"] = self.master.data[lo:hi]
        for role, store in self.stores.items():
            if isinstance(store, FP8Store):
                b0, b1 = lo // store.block, -(-hi // store.block)
                out[role] = store.q[b0 * store.block: b1 * store.block].view(torch.uint8)
                out[role + "_scale"] = store.scale[b0:b1]
            else:
                out[role] = store.data[lo:hi]
        return out


def _moved(store: MomentStore, device) -> MomentStore:
    """A copy of ``store`` on ``device``."""
    sd = store.state_dict()
    from .precision import store_from_state_dict
    role = getattr(store, "role", "m")
    return store_from_state_dict({k: v.to(device) if isinstance(v, torch.Tensor) else v for k, v in sd.items()},
                                 store.numel, role, device=device)


# ------------------------------------------------------------ interleaved base

class _Interleaved(ParamState):
    """State in one buffer (two when double-buffered): ``current`` is read, ``target`` written."""

    gathers = True

    def export_bytes(self) -> int:
        """Device bytes a checkpoint export of this state gathers (one buffer's worth)."""
        return self.current.nbytes

    def __init__(self, numel, device, roles, buffers: list[torch.Tensor]):
        super().__init__(numel, device, roles)
        self.buffers = buffers
        self.turn = 0

    @property
    def current(self) -> torch.Tensor:
        return self.buffers[self.turn]

    @property
    def target(self) -> torch.Tensor | None:
        return self.buffers[1 - self.turn] if len(self.buffers) == 2 else None

    @property
    def alternates(self):
        return len(self.buffers) == 2

    def advance(self):
        if len(self.buffers) == 2:
            self.turn ^= 1

    def _column(self, role: str) -> torch.Tensor:
        """The strided view of ``role``'s values ('p' the FP32 master, 'm' / 'v' the moments) in
        ``current``, in element order once flattened (padding included)."""
        raise NotImplementedError

    def _padded(self) -> int:
        return self._column("p").numel()

    def _put(self, role: str, values: torch.Tensor) -> None:
        column = self._column(role)
        flat = torch.zeros(column.numel(), dtype=column.dtype, device=self.device)
        flat[: self.numel] = values.reshape(-1)[: self.numel].to(self.device)
        column.copy_(flat.view(column.shape))

    # The master column, the plane-conversion kernel's view of it: (stride in bytes, log2 of the
    # elements per group) of an FP32 master; the FP24-master and FP8-record layouts override master_plane.
    PLANE: tuple[int, int] = (0, 0)

    def master_plane(self):
        stride, log2 = self.PLANE
        return _hip.Plane(self.current.data_ptr(), None, stride, _hip.DT_F32, log2)

    def _load_master(self, master: Any) -> None:
        """Checkpoint master weights or plain values into the master column: on the device one pass
        of the plane-conversion kernel (FP24 rounds to nearest; padding slots keep their bits), in
        host memory a torch copy."""
        if self.device.type != "cuda":
            self._put("p", _as_master_values(master, self.numel, self.device))
            return
        src, keep = _master_source(master, self.numel, self.device)   # keep: alive until enqueued
        if self.numel:
            F.convert_plane(src, self.master_plane(), self.numel, self.device)
        del keep   # memory made on this stream and freed to it: reused only after the copy

    def master_fp32(self):
        if self.device.type != "cuda":
            return self._column("p").reshape(-1)[: self.numel].clone()
        out = torch.empty(self.numel, dtype=torch.float32, device=self.device)
        if self.numel:
            F.convert_plane(self.master_plane(), _hip.plane_of(out), self.numel, self.device)
        return out

    def footprint(self):
        total = sum(b.nbytes for b in self.buffers)
        master = 4 * self.numel * len(self.buffers)
        return master, total - master


class PairState(_Interleaved):
    """AdamW, FP32 master, BF16 moments: 16 bytes per pair of elements {p[2k], p[2k+1], m[2k] | m[2k+1] << 16,
    v[2k] | v[2k+1] << 16} (ADAMBRIDGE_DT_PACKED)."""

    layout = "pairs"
    precision = "bf16"
    PLANE = (16, 1)   # element i's master at 16 (i >> 1) + 4 (i & 1)

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        pairs = max(1, (int(numel) + 1) // 2)
        bufs = [m.view(torch.int32).view(pairs, 4) for m in memory] if memory else \
            [torch.zeros(pairs, 4, dtype=torch.int32, device=device) for _ in range(2 if double_buffer else 1)]
        super().__init__(numel, device, ("m", "v"), bufs)

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return max(1, (int(numel) + 1) // 2) * 16

    def bind(self, seg):
        seg.p, seg.p_lo = self.current.data_ptr(), _ptr(self.target)
        seg.m = seg.v = seg.m_scale = seg.v_scale = None
        seg.p_dtype, seg.mv_dtype = _hip.DT_PACKED, _hip.DT_BF16

    def _column(self, role):
        if role == "p":
            return self.current.view(torch.float32)[:, 0:2]
        k = 4 if role == "m" else 6
        return self.current.view(torch.bfloat16)[:, k:k + 2]

    def moment(self, role):
        store = BF16Store(self.numel, device=self.device)
        store.data.copy_(self._column(role).reshape(-1)[: self.numel])
        return store

    def load(self, master=None, moments=None):
        if master is not None:
            self._load_master(master)
        for role, store in (moments or {}).items():
            self._put(role, _bf16_bits(store, self.device))

    def window(self, lo, hi):
        return {"p": self._column("p").reshape(-1)[lo:hi], "m": self._column("m").reshape(-1)[lo:hi],
                "v": self._column("v").reshape(-1)[lo:hi]}


class LionRecordState(_Interleaved):
    """Lion, FP32 master, BF16 moment: 1536-byte records of 256 elements, the 256 masters then the 256 m
    values, each in element order (ADAMBRIDGE_DT_PACKED_LION)."""

    layout = "lion-records"
    precision = "bf16"
    PLANE = (1536, 8)

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        records = max(1, -(-int(numel) // 256))
        bufs = [m.view(records, 1536) for m in memory] if memory else \
            [torch.zeros(records, 1536, dtype=torch.uint8, device=device) for _ in range(2 if double_buffer else 1)]
        super().__init__(numel, device, ("m",), bufs)

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return max(1, -(-int(numel) // 256)) * 1536

    def bind(self, seg):
        seg.p, seg.p_lo = self.current.data_ptr(), _ptr(self.target)
        seg.m = seg.v = seg.m_scale = seg.v_scale = None
        seg.p_dtype, seg.mv_dtype = _hip.DT_PACKED_LION, _hip.DT_BF16

    def _column(self, role):
        if role == "p":
            return self.current[:, :1024].view(torch.float32)
        return self.current[:, 1024:].view(torch.bfloat16)

    def moment(self, role):
        store = BF16Store(self.numel, device=self.device)
        store.data.copy_(self._column("m").reshape(-1)[: self.numel])
        return store

    def load(self, master=None, moments=None):
        if master is not None:
            self._load_master(master)
        if moments and "m" in moments:
            self._put("m", _bf16_bits(moments["m"], self.device))

    def window(self, lo, hi):
        return {"p": self._column("p").reshape(-1)[lo:hi], "m": self._column("m").reshape(-1)[lo:hi]}


class F32RecordState(_Interleaved):
    """AdamW, FP32 master, FP32 moments: 3072-byte records of 256 elements, the 256 masters, then the
    256 m, then the 256 v values, each in element order (ADAMBRIDGE_DT_PACKED_F32)."""

    layout = "f32-records"
    precision = "fp32"
    PLANE = (3072, 8)

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        records = max(1, -(-int(numel) // 256))
        bufs = [m.view(records, 3072) for m in memory] if memory else \
            [torch.zeros(records, 3072, dtype=torch.uint8, device=device) for _ in range(2 if double_buffer else 1)]
        super().__init__(numel, device, ("m", "v"), bufs)

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return max(1, -(-int(numel) // 256)) * 3072

    def bind(self, seg):
        seg.p, seg.p_lo = self.current.data_ptr(), _ptr(self.target)
        seg.m = seg.v = seg.m_scale = seg.v_scale = None
        seg.p_dtype, seg.mv_dtype = _hip.DT_PACKED_F32, _hip.DT_F32

    def _column(self, role):
        k = {"p": 0, "m": 1, "v": 2}[role]
        return self.current[:, 1024 * k:1024 * (k + 1)].view(torch.float32)

    def moment(self, role):
        return FP32Store(self.numel, init=self._column(role).reshape(-1)[: self.numel], device=self.device)

    def load(self, master=None, moments=None):
        if master is not None:
            self._load_master(master)
        for role, store in (moments or {}).items():
            self._put(role, store.to_fp32().to(self.device))

    def window(self, lo, hi):
        return {r: self._column(r).reshape(-1)[lo:hi] for r in ("p", "m", "v")}


class LionF32RecordState(F32RecordState):
    """Lion, FP32 master, FP32 moment: 2048-byte records of 256 elements, the 256 masters then the 256 m
    values, each in element order (ADAMBRIDGE_DT_PACKED_LION_F32)."""

    layout = "lion-f32-records"
    RECORD = 2048
    PLANE = (2048, 8)

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        records = max(1, -(-int(numel) // 256))
        bufs = [m.view(records, self.RECORD) for m in memory] if memory else \
            [torch.zeros(records, self.RECORD, dtype=torch.uint8, device=device) for _ in range(2 if double_buffer else 1)]
        _Interleaved.__init__(self, numel, device, ("m",), bufs)

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return max(1, -(-int(numel) // 256)) * LionF32RecordState.RECORD

    def bind(self, seg):
        super().bind(seg)
        seg.p_dtype = _hip.DT_PACKED_LION_F32

    def _column(self, role):
        k = {"p": 0, "m": 1}[role]
        return self.current[:, 1024 * k:1024 * (k + 1)].view(torch.float32)

    def window(self, lo, hi):
        return {r: self._column(r).reshape(-1)[lo:hi] for r in ("p", "m")}


class F24RecordState(_Interleaved):
    """AdamW, FP24 master, BF16 moments: 1792-byte records of 256 elements, the 256 master high halves
    (BF16 bits), the 256 master low bytes, the 256 m and the 256 v values (BF16), each in element
    order (ADAMBRIDGE_DT_PACKED_F24)."""

    layout = "f24-records"
    precision = "bf16"
    master_precision = "fp24"

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        records = max(1, -(-int(numel) // 256))
        bufs = [m.view(records, 1792) for m in memory] if memory else \
            [torch.zeros(records, 1792, dtype=torch.uint8, device=device) for _ in range(2 if double_buffer else 1)]
        super().__init__(numel, device, ("m", "v"), bufs)

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return max(1, -(-int(numel) // 256)) * 1792

    def bind(self, seg):
        seg.p, seg.p_lo = self.current.data_ptr(), _ptr(self.target)
        seg.m = seg.v = seg.m_scale = seg.v_scale = None
        seg.p_dtype, seg.mv_dtype = _hip.DT_PACKED_F24, _hip.DT_BF16

    def _column(self, role):
        """'p' the hi plane (BF16 bits), 'lo' the lo plane (uint8), 'm' / 'v' the moments (BF16)."""
        if role == "lo":
            return self.current[:, 512:768]
        k = {"p": 0, "m": 768, "v": 1280}[role]
        return self.current[:, k:k + 512].view(torch.bfloat16)

    RECORD = 1792

    def master_plane(self):
        base = self.current.data_ptr()
        return _hip.Plane(base, base + 512, self.RECORD, _hip.DT_F24, 8)

    def _planes(self) -> FP24Store:
        """The master as an FP24 store (a copy of the two planes)."""
        store = FP24Store(self.numel, device=self.device)
        if self.device.type == "cuda":
            if self.numel:   # bit for bit: FP24 into FP24
                F.convert_plane(self.master_plane(), _hip.fp24_plane(store.hi, store.lo), self.numel, self.device)
            return store
        store.hi.copy_(self._column("p").reshape(-1)[: self.numel])
        store.lo.copy_(self._column("lo").reshape(-1)[: self.numel])
        return store

    def master_fp32(self):
        if self.device.type == "cuda":
            return super().master_fp32()   # one pass: the record's planes expanded to FP32
        return self._planes().to_fp32()

    def export_master(self):
        return self._planes().state_dict()

    def moment(self, role):
        store = BF16Store(self.numel, device=self.device)
        store.data.copy_(self._column(role).reshape(-1)[: self.numel])
        return store

    def load(self, master=None, moments=None):
        if master is not None:
            if self.device.type == "cuda":
                self._load_master(master)   # FP24 planes bit for bit; other values rounded to nearest
            else:
                planes = FP24Store(self.numel, device=self.device)
                load_master_(planes, master)   # FP24 planes as they are; other values rounded to nearest
                self._put("p", planes.hi)
                self._put("lo", planes.lo)
        for role, store in (moments or {}).items():
            self._put(role, _bf16_bits(store, self.device))

    def footprint(self):
        total = sum(b.nbytes for b in self.buffers)
        master = 3 * self.numel * len(self.buffers)
        return master, total - master

    def window(self, lo, hi):
        return {"p": self._column("p").reshape(-1)[lo:hi], "p_lo": self._column("lo").reshape(-1)[lo:hi],
                "m": self._column("m").reshape(-1)[lo:hi], "v": self._column("v").reshape(-1)[lo:hi]}


class F24F32RecordState(F24RecordState):
    """AdamW, FP24 master, FP32 moments: 2816-byte records of 256 elements, the 256 master high halves
    (BF16 bits), the 256 master low bytes, the 256 m and the 256 v values (FP32), each in element
    order (ADAMBRIDGE_DT_PACKED_F24_F32)."""

    layout = "f24-f32-records"
    precision = "fp32"
    RECORD = 2816   # master_plane's record stride too

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        records = max(1, -(-int(numel) // 256))
        bufs = [m.view(records, self.RECORD) for m in memory] if memory else \
            [torch.zeros(records, self.RECORD, dtype=torch.uint8, device=device) for _ in range(2 if double_buffer else 1)]
        _Interleaved.__init__(self, numel, device, ("m", "v"), bufs)

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return max(1, -(-int(numel) // 256)) * F24F32RecordState.RECORD

    def bind(self, seg):
        super().bind(seg)
        seg.p_dtype, seg.mv_dtype = _hip.DT_PACKED_F24_F32, _hip.DT_F32

    def _column(self, role):
        """'p' the hi plane (BF16 bits), 'lo' the lo plane (uint8), 'm' / 'v' the moments (FP32)."""
        if role in ("p", "lo"):
            return super()._column(role)
        k = {"m": 768, "v": 1792}[role]
        return self.current[:, k:k + 1024].view(torch.float32)

    def moment(self, role):
        return FP32Store(self.numel, init=self._column(role).reshape(-1)[: self.numel], device=self.device)

    def load(self, master=None, moments=None):
        super().load(master)
        for role, store in (moments or {}).items():
            self._put(role, store.to_fp32().to(self.device))


class LionF24RecordState(F24RecordState):
    """Lion, FP24 master, BF16 moment: 1280-byte records of 256 elements, the 256 master high halves,
    the 256 low bytes and the 256 m values, each in element order (ADAMBRIDGE_DT_PACKED_LION_F24)."""

    layout = "lion-f24-records"
    RECORD = 1280   # master_plane's record stride too

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        records = max(1, -(-int(numel) // 256))
        bufs = [m.view(records, self.RECORD) for m in memory] if memory else \
            [torch.zeros(records, self.RECORD, dtype=torch.uint8, device=device) for _ in range(2 if double_buffer else 1)]
        _Interleaved.__init__(self, numel, device, ("m",), bufs)

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return max(1, -(-int(numel) // 256)) * LionF24RecordState.RECORD

    def bind(self, seg):
        super().bind(seg)
        seg.p_dtype = _hip.DT_PACKED_LION_F24

    def window(self, lo, hi):
        w = super().window(lo, hi)
        del w["v"]
        return w


class LionF24F32RecordState(LionF24RecordState):
    """Lion, FP24 master, FP32 moment: 1792-byte records of 256 elements, the 256 master high halves,
    the 256 low bytes and the 256 m values (FP32), each in element order
    (ADAMBRIDGE_DT_PACKED_LION_F24_F32)."""

    layout = "lion-f24-f32-records"
    precision = "fp32"
    RECORD = 1792   # master_plane's record stride too

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return max(1, -(-int(numel) // 256)) * LionF24F32RecordState.RECORD

    def bind(self, seg):
        super().bind(seg)
        seg.p_dtype, seg.mv_dtype = _hip.DT_PACKED_LION_F24_F32, _hip.DT_F32

    def _column(self, role):
        """'p' the hi plane (BF16 bits), 'lo' the lo plane (uint8), 'm' the moment (FP32)."""
        if role == "m":
            return self.current[:, 768:1792].view(torch.float32)
        return super()._column(role)

    def moment(self, role):
        return FP32Store(self.numel, init=self._column(role).reshape(-1)[: self.numel], device=self.device)

    def load(self, master=None, moments=None):
        F24RecordState.load(self, master)
        for role, store in (moments or {}).items():
            self._put(role, store.to_fp32().to(self.device))


class AdamRecordState(_Interleaved):
    """AdamW, FP32 master, FP8 moments: one 768-byte record per 128-element block
    (ADAMBRIDGE_DT_PACKED_FP8) -- lane l's elements 8l .. 8l + 7 keep their masters at 16l (first
    four) and 256 + 16l (last four), their m codes at 512 + 16l and v codes at 520 + 16l -- plus an
    FP32 block-scale array per moment.  Updated in place."""

    layout = "fp8-records"
    precision = "fp8"

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        self.blocks = F.fp8_blocks(int(numel))
        rec = memory[0].view(self.blocks, 768) if memory else \
            torch.zeros(self.blocks, 768, dtype=torch.uint8, device=device)
        super().__init__(numel, device, ("m", "v"), [rec])   # updated in place: never double-buffered
        self.scales = {r: torch.ones(self.blocks, dtype=torch.float32, device=device) for r in ("m", "v")}

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return F.fp8_blocks(int(numel)) * 768

    def bind(self, seg):
        seg.p, seg.p_lo, seg.m, seg.v = self.current.data_ptr(), None, None, None
        seg.m_scale, seg.v_scale = self.scales["m"].data_ptr(), self.scales["v"].data_ptr()
        seg.p_dtype, seg.mv_dtype = _hip.DT_PACKED8, _hip.DT_FP8

    def _column(self, role):
        if role == "p":   # [block, lane, half, j] = element 128 block + 8 lane + 4 half + j
            return self.current[:, :512].view(torch.float32).view(self.blocks, 2, 16, 4).permute(0, 2, 1, 3)
        k = 0 if role == "m" else 8
        return self.current[:, 512:].view(self.blocks, 16, 16)[:, :, k:k + 8]

    def master_plane(self):
        return _hip.Plane(self.current.data_ptr(), None, 0, _hip.DT_PACKED8, 0)

    def _codes(self, role: str) -> torch.Tensor:
        return self._column(role).reshape(-1).view(F.FP8_FORMATS[role].dtype)

    def moment(self, role):
        store = FP8Store(self.numel, role, device=self.device)
        store.q.copy_(self._codes(role))
        store.scale.copy_(self.scales[role])
        return store

    def load(self, master=None, moments=None):
        if master is not None:
            self._load_master(master)
        for role, store in (moments or {}).items():
            if not isinstance(store, FP8Store) or store.role != role or store.block != F.FP8_BLOCK:
                store = FP8Store(self.numel, role, init=store.to_fp32(), device=self.device)
            self._column(role).copy_(store.q.to(self.device).view(torch.uint8).view(self.blocks, 16, 8))
            self.scales[role].copy_(store.scale.to(self.device))

    def footprint(self):
        return 4 * self.numel, self.current.nbytes - 4 * self.numel + sum(s.nbytes for s in self.scales.values())

    def export_bytes(self):
        return self.current.nbytes + sum(s.nbytes for s in self.scales.values())

    def window(self, lo, hi):
        b0, b1 = lo // 128, -(-hi // 128)
        out = {"p": self._column("p").reshape(-1)[lo:hi]}
        for role in ("m", "v"):
            out[role] = self._column(role)[b0:b1].reshape(-1)
            out[role + "_scale"] = self.scales[role][b0:b1]
        return out


class AdamF24RecordState(AdamRecordState):
    """AdamW, FP24 master, FP8 moments: one 640-byte record per 128-element block
    (ADAMBRIDGE_DT_PACKED_FP8_F24) -- the block's 128 master high halves (BF16 bits) at 0 and its 128
    low bytes at 256, both in element order, then lane l's m codes at 384 + 16l and v codes at
    392 + 16l -- plus an FP32 block-scale array per moment.  Updated in place."""

    layout = "fp8-f24-records"
    master_precision = "fp24"
    RECORD = 640

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        self.blocks = F.fp8_blocks(int(numel))
        rec = memory[0].view(self.blocks, self.RECORD) if memory else \
            torch.zeros(self.blocks, self.RECORD, dtype=torch.uint8, device=device)
        _Interleaved.__init__(self, numel, device, ("m", "v"), [rec])   # updated in place: never double-buffered
        self.scales = {r: torch.ones(self.blocks, dtype=torch.float32, device=device) for r in ("m", "v")}

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return F.fp8_blocks(int(numel)) * AdamF24RecordState.RECORD

    def bind(self, seg):
        super().bind(seg)
        seg.p_dtype = _hip.DT_PACKED8_F24

    def _column(self, role):
        """'p' the hi plane (BF16 bits), 'lo' the lo plane (uint8), 'm' / 'v' the codes, in element order."""
        if role == "p":
            return self.current[:, :256].view(torch.bfloat16)
        if role == "lo":
            return self.current[:, 256:384]
        k = 0 if role == "m" else 8
        return self.current[:, 384:].view(self.blocks, 16, 16)[:, :, k:k + 8]

    def master_plane(self):
        base = self.current.data_ptr()
        return _hip.Plane(base, base + 256, self.RECORD, _hip.DT_F24, 7)

    def _planes(self) -> FP24Store:
        return F24RecordState._planes(self)

    def master_fp32(self):
        if self.device.type == "cuda":
            return _Interleaved.master_fp32(self)   # one pass: the record's planes expanded to FP32
        return self._planes().to_fp32()

    def export_master(self):
        return self._planes().state_dict()

    def load(self, master=None, moments=None):
        if master is not None and self.device.type != "cuda":
            planes = FP24Store(self.numel, device=self.device)
            load_master_(planes, master)   # FP24 planes as they are; other values rounded to nearest
            self._put("p", planes.hi)
            self._put("lo", planes.lo)
            master = None
        super().load(master, moments)   # on the device: FP24 planes bit for bit, other values to nearest

    def footprint(self):
        return 3 * self.numel, self.current.nbytes - 3 * self.numel + sum(s.nbytes for s in self.scales.values())

    def window(self, lo, hi):
        out = super().window(lo, hi)
        out["p_lo"] = self._column("lo").reshape(-1)[lo:hi]
        return out


class LionFP8RecordState(AdamRecordState):
    """Lion, FP32 master, FP8 moment: one 640-byte record per 128-element block
    (ADAMBRIDGE_DT_PACKED_LION_FP8) -- the masters as in the AdamW FP8 records (lane l's elements
    8l .. 8l + 7 at 16l and 256 + 16l), then the block's 128 m codes in element order at 512 -- plus
    the FP32 m block scales.  Updated in place."""

    layout = "lion-fp8-records"
    RECORD = 640   # master_plane's record stride too

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        self.blocks = F.fp8_blocks(int(numel))
        rec = memory[0].view(self.blocks, self.RECORD) if memory else \
            torch.zeros(self.blocks, self.RECORD, dtype=torch.uint8, device=device)
        _Interleaved.__init__(self, numel, device, ("m",), [rec])   # updated in place: never double-buffered
        self.scales = {"m": torch.ones(self.blocks, dtype=torch.float32, device=device)}

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return F.fp8_blocks(int(numel)) * LionFP8RecordState.RECORD

    def bind(self, seg):
        seg.p, seg.p_lo, seg.m, seg.v = self.current.data_ptr(), None, None, None
        seg.m_scale, seg.v_scale = self.scales["m"].data_ptr(), None
        seg.p_dtype, seg.mv_dtype = _hip.DT_PACKED8_LION, _hip.DT_FP8

    def _column(self, role):
        if role == "p":
            return super()._column("p")
        return self.current[:, 512:].view(self.blocks, 16, 8)   # 'm': element order

    def master_plane(self):
        return _hip.Plane(self.current.data_ptr(), None, self.RECORD, _hip.DT_PACKED8, 0)

    def window(self, lo, hi):
        b0, b1 = lo // 128, -(-hi // 128)
        return {"p": self._column("p").reshape(-1)[lo:hi], "m": self._column("m")[b0:b1].reshape(-1),
                "m_scale": self.scales["m"][b0:b1]}


class LionFP8F24RecordState(AdamF24RecordState):
    """Lion, FP24 master, FP8 moment: one 512-byte record per 128-element block
    (ADAMBRIDGE_DT_PACKED_LION_FP8_F24) -- the block's 128 master high halves at 0 and 128 low bytes at
    256, then its 128 m codes at 384, each in element order -- plus the FP32 m block scales.  Updated
    in place."""

    layout = "lion-fp8-f24-records"
    RECORD = 512   # master_plane's record stride too

    def __init__(self, numel, device, double_buffer: bool = False, memory: list[torch.Tensor] | None = None):
        self.blocks = F.fp8_blocks(int(numel))
        rec = memory[0].view(self.blocks, self.RECORD) if memory else \
            torch.zeros(self.blocks, self.RECORD, dtype=torch.uint8, device=device)
        _Interleaved.__init__(self, numel, device, ("m",), [rec])   # updated in place: never double-buffered
        self.scales = {"m": torch.ones(self.blocks, dtype=torch.float32, device=device)}

    @staticmethod
    def buffer_bytes(numel: int) -> int:
        return F.fp8_blocks(int(numel)) * LionFP8F24RecordState.RECORD

    def bind(self, seg):
        seg.p, seg.p_lo, seg.m, seg.v = self.current.data_ptr(), None, None, None
        seg.m_scale, seg.v_scale = self.scales["m"].data_ptr(), None
        seg.p_dtype, seg.mv_dtype = _hip.DT_PACKED8_LION_F24, _hip.DT_FP8

    def _column(self, role):
        if role == "m":
            return self.current[:, 384:].view(self.blocks, 16, 8)   # element order
        return super()._column(role)

    def window(self, lo, hi):
        b0, b1 = lo // 128, -(-hi // 128)
        return {"p": self._column("p").reshape(-1)[lo:hi], "p_lo": self._column("lo").reshape(-1)[lo:hi],
                "m": self._column("m")[b0:b1].reshape(-1), "m_scale": self.scales["m"][b0:b1]}


def _bf16_bits(store: MomentStore, device) -> torch.Tensor:
    """A moment's values as BF16 (the store's own bits when it is BF16, nearest-even otherwise)."""
    if isinstance(store, BF16Store):
        return store.data.to(device)
    return F.bf16_encode(store.to_fp32().to(device))


# -------------------------------------------------------------------- building

_INTERLEAVED = {"pairs": PairState, "lion-records": LionRecordState, "fp8-records": AdamRecordState,
                "f32-records": F32RecordState, "f24-records": F24RecordState, "lion-f24-records": LionF24RecordState,
                "fp8-f24-records": AdamF24RecordState, "lion-f32-records": LionF32RecordState,
                "lion-fp8-records": LionFP8RecordState, "f24-f32-records": F24F32RecordState,
                "lion-f24-f32-records": LionF24F32RecordState, "lion-fp8-f24-records": LionFP8F24RecordState}
ARENA_ALIGN = 2 << 20
SMALL_ALIGN = 256


def arena_plan(layout: str, sizes: list[int], double_buffer: bool = False) -> tuple[list[list[int]], int]:
    """Byte offsets of each state's buffers in one zeroed arena and the arena's size, for interleaved
    states of ``sizes`` elements.  A buffer of 2 MiB or more starts on a 2 MiB boundary; smaller ones
    (norms, biases) are packed at 256-byte boundaries, so that a model of many small tensors does
    not pay 2 MiB for each."""
    cls = _INTERLEAVED[layout]
    copies = 2 if double_buffer and layout not in IN_PLACE else 1
    offsets, total = [], 0
    for n in sizes:
        nbytes = cls.buffer_bytes(n)
        align = ARENA_ALIGN if nbytes >= ARENA_ALIGN else SMALL_ALIGN
        mine = []
        for _ in range(copies):
            total = -(-total // align) * align
            mine.append(total)
            total += nbytes
        offsets.append(mine)
    return offsets, -(-total // SMALL_ALIGN) * SMALL_ALIGN


def _place(nbytes: int, device, place: bool) -> None:
    """Before allocating ``nbytes`` of state: an allocate/free of that size (see new_states)."""
    if place and RECYCLE_MIN_BYTES is not None and nbytes >= RECYCLE_MIN_BYTES:
        _hip.load().recycle_device_memory(nbytes, torch.device(device))   # placement only: failure is harmless


def new_states(layout: str, algorithm: str, precision: str, master_precision: str, device,
               masters: list[torch.Tensor], double_buffer: bool = False,
               master_params: list[torch.Tensor | None] | None = None, place: bool = True,
               memory: list[list[torch.Tensor]] | None = None) -> list[ParamState]:
    """Fresh states for several parameters on one device: master from ``masters[i]`` (any dtype;
    FP24 rounds to nearest) or, in the separate layout, the FP32 parameter ``master_params[i]`` itself;
    moments zero, FP8 scales one.

    Interleaved states share one arena: a single zeroed allocation, each buffer of 2 MiB or more at
    a 2 MiB-aligned offset and smaller ones packed (arena_plan) -- one allocation instead of one
    per parameter.  The update streams from it as fast as
    from per-parameter allocations (the 7B bf16-moment step built first in a fresh process: 21.43
    ms per launch from the arena, 21.41 from 291 allocations).  State of RECYCLE_MIN_BYTES or more
    (an arena, or the separate layout's stores together) is allocated right after a block of its
    size was allocated from the driver and freed, which places it where the update streams at a
    copy's rate: 20.63 against 21.43 ms for that first build, and 30.13 against 31.49 ms with FP32
    moments in separate arrays (the driver's first placements in a fresh process stream this
    update 3-4% slower; measured on MI355X, cause unknown).  The allocate/free holds no more memory
    than the state; it waits for the device to go idle (the free does), so ``place=False`` skips it
    where that would stall a pipeline.  ``memory``: zeroed buffers of an arena made earlier (arena_memory), one list
    per state, used instead of a new arena (interleaved layouts)."""
    roles = ("m",) if algorithm == "lion" else ("m", "v")
    if layout == "separate":
        # the stores are allocations of their own; the same placement step covers them all at once
        own_master = [not (master_params and master_params[i] is not None) for i in range(len(masters))]
        total = sum(int(t.numel() * ((3 if master_precision == "fp24" else 4) * own + len(roles) * F.moment_bytes(precision)))
                    for t, own in zip(masters, own_master))
        _place(total, device, place)
        out: list[ParamState] = []
        for i, values in enumerate(masters):
            param = master_params[i] if master_params else None
            numel = values.numel()
            if param is not None:
                master = FP32Store.wrap(param.data.view(-1))
            else:
                master = make_master(master_precision, numel, init=values, device=device)
            moments = {r: make_store(precision, numel, r, device=device) for r in roles}
            out.append(SeparateState(master, moments, master_is_param=param is not None))
        return out
    if layout not in _INTERLEAVED:
        raise ValueError(f"unknown state layout {layout!r}; expected one of {LAYOUTS}")
    cls = _INTERLEAVED[layout]
    sizes = [t.numel() for t in masters]
    if memory is None:
        memory = arena_memory(layout, sizes, device, double_buffer, place)
    states = []
    for n, mem, values in zip(sizes, memory, masters):
        state = cls(n, device, double_buffer, memory=mem)
        state.load(master=values.detach().reshape(-1))   # bf16 or fp32, read as it is by the conversion
        states.append(state)
    return states


def arena_memory(layout: str, sizes: list[int], device, double_buffer: bool = False,
                 place: bool = True) -> list[list[torch.Tensor]]:
    """Zeroed device memory for interleaved states of ``sizes`` elements in one arena (placed as in
    new_states unless ``place`` is False): for each state, its buffer (two when double-buffered)."""
    cls = _INTERLEAVED[layout]
    offsets, total = arena_plan(layout, sizes, double_buffer)
    _place(total, device, place)
    arena = torch.zeros(total, dtype=torch.uint8, device=device)
    return [[arena[o: o + cls.buffer_bytes(n)] for o in offs] for n, offs in zip(sizes, offsets)]


def new_state(layout: str, algorithm: str, precision: str, master_precision: str, numel: int, device,
              master_values: torch.Tensor | None = None, master_param: torch.Tensor | None = None,
              double_buffer: bool = False) -> ParamState:
    """One fresh state (see :func:`new_states`); without ``master_values`` the master starts at zero."""
    values = master_values if master_values is not None else torch.zeros(numel, dtype=torch.float32, device=device)
    return new_states(layout, algorithm, precision, master_precision, device, [values], double_buffer,
                      [master_param])[0]
