"""Update engine: optimizer state in HBM, updates launched on HIP streams.

The reference's engine (adambridge/engine.py) moves every gradient to host
RAM, updates it on a CPU thread pool and copies the weights back.  Here all of
that state lives in device memory next to the parameter, and one HIP kernel
launch updates a whole batch of tensors in place:

* ``step()`` (synchronous mode): every parameter with a gradient, in one launch;
* the gradient hook (``attach_hooks``): each parameter is updated on a side
  stream as soon as its gradient is ready, overlapping the rest of the backward
  pass; small parameters are batched into one launch at ``step_sync``;
* ``step_sync`` orders the side stream before the caller's next work with a
  stream wait -- no host synchronisation.

Ordering on the device replaces the reference's host threads and events::

    compute stream        side stream                 write-back stream (delayed mode)
    --------------        -----------                 --------------------------------
    grad ready  -------->  wait `ready`
    (backward goes on)     [wait `written`]  <-------  wait `ready` + previous update: out -> param
                           fused update (one launch)
                           record `done`
    step_sync: wait side (exact) or wait write-back (delayed)

Delayed updates (engine.py:46-69): the update of step t writes the slot's
``out`` buffer; step t+1's hook copies it into the parameter on the
write-back stream (after backward has finished reading the parameter) before
the side stream overwrites ``out`` with update t+1.  The model trains with
weights one step stale; ``flush`` applies everything pending.

The parameter index, the per-slot step counter and the element offset fix the
rounding stream exactly as in the reference, so results do not depend on how
updates are batched.
"""

from __future__ import annotations

import ctypes
import logging
import threading
import time
from dataclasses import dataclass, field

import torch

from . import _hip
from .precision import (FP8_BLOCK, BF16Store, FP8Store, FP32Store, MomentStore, PackedMaster, PackedMoment,
                        PackedState, RecordMaster, RecordMoment, RecordState, make_master,
                        make_store)

__all__ = ["UpdateEngine", "ParamSlot", "SmallGroup", "StepStats"]

log = logging.getLogger("adambridge_amd")
_MASK64 = (1 << 64) - 1


class ParamSlot:
    """Device-side optimizer state of one parameter (reference ParamSlot, engine.py:257-293)."""

    __slots__ = ("index", "param", "group", "numel", "step", "master", "out", "out_view", "m", "v", "submitted",
                 "seg", "seg_ptr", "seg_group", "small", "done_ev", "in_place", "pending_grad", "packed")

    def __init__(self, index: int, param: torch.Tensor, group: dict):
        self.index = index
        self.param = param
        self.group = group
        self.numel = param.numel()
        self.step = 0
        self.master: MomentStore | None = None   # FP32Store (maybe the parameter itself) or FP24Store
        self.out: torch.Tensor | None = None     # own write-back buffer (delayed / deferred write-back)
        self.out_view: torch.Tensor | None = None
        self.m: MomentStore | None = None
        self.v: MomentStore | None = None        # None for Lion
        self.submitted = False
        self.seg: _hip.Segment | None = None     # cached kernel descriptor of the buffers above
        self.seg_ptr = None                      # ctypes pointer to seg
        self.seg_group: _hip.Group | None = None   # the group struct seg.group points at
        self.small: SmallGroup | None = None
        self.done_ev: torch.cuda.Event | None = None   # the last update of this slot has run
        self.in_place = False                    # master is the FP32 parameter itself
        self.pending_grad = None                 # keeps a grad alive until its update is enqueued
        # master + BF16 moments interleaved, or master + FP8 codes in block records (m, v, master view it)
        self.packed: PackedState | RecordState | None = None

    @property
    def initialized(self) -> bool:
        return self.master is not None


class SmallGroup:
    """Small parameters of one device, updated together at step_sync (engine.py:296-337)."""

    def __init__(self, slots: list[ParamSlot]):
        self.slots = slots
        self.device = slots[0].param.device
        for slot in slots:
            slot.small = self


@dataclass
class StepStats:
    """Timing of one optimizer step in seconds (engine.py:340-349, plus the GPU update time).

    ``cpu_update`` and ``per_device_cpu`` are kept for API compatibility and are zero here:
    no host thread updates anything.  With timing enabled (``autotune`` or ``engine.timing``):
    ``gpu_backward`` spans the first to the last gradient-ready event, ``gpu_update`` the side
    stream's first update start to its last update end, and ``exposed_tail`` the last
    gradient-ready event to the end of the last update (what the next forward waits for)."""

    num_updates: int = 0
    gpu_backward: float | None = None
    cpu_update: float = 0.0
    stall: float = 0.0
    per_device_cpu: dict[str, float] = field(default_factory=dict)
    gpu_update: float | None = None
    exposed_tail: float | None = None


class _DeviceStreams:
    def __init__(self, device: torch.device):
        self.device = device
        self.side = torch.cuda.Stream(device)     # default priority (mixed priorities have hung on this pool)
        self.wb = torch.cuda.Stream(device)


class UpdateEngine:
    """Owns the kernel library handle, the streams and the group descriptors."""

    def __init__(self, *, precision: str, algorithm: str = "adamw", stochastic_rounding: bool = True, seed: int = 0,
                 overlap_writeback: bool = True, timing: bool = False, master_precision: str = "fp32",
                 delay_capable: bool = False, state_layout: str = "auto", double_buffer: bool = False):
        if state_layout not in ("auto", "packed", "separate"):
            raise ValueError("state_layout must be 'auto', 'packed' or 'separate'")
        if algorithm not in _hip.ALGORITHMS:
            raise ValueError(f"algorithm must be one of {sorted(_hip.ALGORITHMS)}")
        if master_precision not in _hip.MASTER_CODES:
            raise ValueError(f"master_precision must be one of {sorted(_hip.MASTER_CODES)}")
        self.kernels = _hip.load()
        self.algorithm = algorithm
        self.lion = algorithm == "lion"
        self.precision = precision
        self.master_precision = master_precision
        self.stochastic = stochastic_rounding
        self.seed = seed
        self.overlap_writeback = overlap_writeback
        self.timing = timing
        self.delay = False            # toggled between steps only
        self.delay_capable = delay_capable
        self.state_layout = state_layout
        self.double_buffer = double_buffer
        self._lock = threading.RLock()
        self._streams: dict[torch.device, _DeviceStreams] = {}
        self._groups: dict[int, tuple[dict, _hip.Group]] = {}
        self._owed: dict[ParamSlot, None] = {}     # delayed: `out` holds an update not yet in the parameter
        self._fresh: dict[ParamSlot, None] = {}
        self._deferred: list[ParamSlot] = []       # overlap_writeback=False: copy out -> param at step_sync
        self._num_updates = 0
        self._ready_events: list[torch.cuda.Event] = []
        self._update_events: list[tuple[torch.cuda.Event, torch.cuda.Event]] = []
        self._used: set[torch.device] = set()
        self._grads_kept = False
        self.launch_log: list | None = None   # set to a list to record launch timing events (no host sync)
        self._closed = False

    # ------------------------------------------------------------------ setup

    def streams(self, device: torch.device) -> _DeviceStreams:
        s = self._streams.get(device)
        if s is None:
            with self._lock:
                s = self._streams.get(device)
                if s is None:
                    s = self._streams[device] = _DeviceStreams(device)
        return s

    def _check_param(self, p: torch.Tensor) -> None:
        if not p.is_cuda:
            raise ValueError("adambridge_amd keeps optimizer state in GPU memory and updates it with a HIP kernel: "
                             f"parameters must be on a GPU, got one on {p.device}")
        if p.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"parameters must be float32 or bfloat16 (the kernel's weight formats), got {p.dtype}")

    def initialize(self, slot: ParamSlot) -> None:
        """Lazy state: master = the parameter's current value (FP32, or FP24 rounded to nearest), moments
        zero, FP8 scales one (engine.py:991-1025; precision.py:263-267, 307-311, 365-371)."""
        p = slot.param
        self._check_param(p)
        dev = p.device
        with torch.cuda.device(dev), torch.no_grad():
            src = p.detach().reshape(-1)
            in_place = (p.dtype == torch.float32 and self.master_precision == "fp32" and p.is_contiguous()
                        and not self.delay_capable and self.overlap_writeback)
            if in_place:
                slot.master = FP32Store.wrap(p.data.view(-1))
            else:
                slot.master = make_master(self.master_precision, slot.numel, init=src, device=dev)
            slot.in_place = in_place
            slot.packed = None
            kind = self._packable(slot)
            if kind == "bf16":
                packed = PackedState(slot.numel, init=slot.master.data, device=dev, double_buffer=self.double_buffer)
                self._adopt_packed(slot, packed)
            elif kind == "fp8":
                self._adopt_records(slot, RecordState(slot.numel, init=slot.master.data, device=dev))
            else:
                slot.m = make_store(self.precision, slot.numel, "m", device=dev)
                slot.v = None if self.lion else make_store(self.precision, slot.numel, "v", device=dev)
            needs_out = not in_place and (self.delay_capable or not self.overlap_writeback or not p.is_contiguous())
            slot.out = torch.empty(slot.numel, dtype=p.dtype, device=dev) if needs_out else None
            slot.out_view = slot.out.view(p.shape) if slot.out is not None else None
        slot.seg = None
        slot.seg_ptr = None

    def _packable(self, slot: ParamSlot) -> str | None:
        """Which interleaved layout serves the slot: 'bf16' (pairs, BF16 moments) or 'fp8' (block
        records, FP8 moments), for AdamW with an FP32 master of its own; None for the separate one."""
        if self.state_layout == "separate" or self.lion or self.master_precision != "fp32" or slot.in_place:
            return None
        return self.precision if self.precision in ("bf16", "fp8") else None

    @staticmethod
    def _adopt_packed(slot: ParamSlot, packed: PackedState) -> None:
        slot.packed = packed
        slot.master = PackedMaster(packed)
        slot.m = PackedMoment(packed, "m")
        slot.v = PackedMoment(packed, "v")
        slot.seg = None
        slot.seg_ptr = None

    @staticmethod
    def _adopt_records(slot: ParamSlot, records: RecordState) -> None:
        slot.packed = records
        slot.master = RecordMaster(records)
        slot.m = RecordMoment(records, "m")
        slot.v = RecordMoment(records, "v")
        slot.seg = None
        slot.seg_ptr = None

    def _ensure_out(self, slot: ParamSlot) -> None:
        if slot.out is None and not slot.in_place:
            slot.out = torch.empty(slot.numel, dtype=slot.param.dtype, device=slot.param.device)
            slot.out_view = slot.out.view(slot.param.shape)

    def convert_moments(self, slot: ParamSlot, precision: str) -> None:
        """Re-encode a slot's moments in another precision (between steps); the engine's
        ``precision`` is already the new one."""
        dev = slot.param.device
        with torch.no_grad():
            if slot.packed is not None:   # leave the interleaved layout
                slot.master = FP32Store(slot.numel, init=slot.packed.get("p"), device=dev)
                slot.packed = None
            m = make_store(precision, slot.numel, "m", init=slot.m.to_fp32(), device=dev)
            v = None if slot.v is None else make_store(precision, slot.numel, "v", init=slot.v.to_fp32(), device=dev)
            slot.m, slot.v = m, v
            if self._packable(slot):
                self._pack(slot)
        slot.seg = None
        slot.seg_ptr = None

    def _pack(self, slot: ParamSlot) -> None:
        """Move an FP32 master and BF16 (FP8) moments, separate stores, into the interleaved layout
        (block records)."""
        if self._packable(slot) == "fp8":
            m, v = slot.m, slot.v
            self._adopt_records(slot, RecordState(slot.numel, init=slot.master.to_fp32(), device=slot.param.device))
            slot.m.adopt(m)
            slot.v.adopt(v)
            return
        packed = PackedState(slot.numel, init=slot.master.to_fp32(), device=slot.param.device,
                             double_buffer=self.double_buffer)
        packed.set("m", slot.m.data)
        packed.set("v", slot.v.data)
        self._adopt_packed(slot, packed)

    def replace_moments(self, slot: ParamSlot, m: MomentStore, v: MomentStore | None) -> None:
        if isinstance(slot.packed, PackedState) and isinstance(m, BF16Store) and isinstance(v, BF16Store):
            with torch.no_grad():
                slot.packed.set("m", m.data)
                slot.packed.set("v", v.data)
            return
        if (isinstance(slot.packed, RecordState) and isinstance(m, FP8Store) and isinstance(v, FP8Store)
                and m.block == v.block == FP8_BLOCK):
            with torch.no_grad():
                slot.m.adopt(m)
                slot.v.adopt(v)
            return
        if slot.packed is not None:   # another precision: the slot leaves the interleaved layout
            slot.master = FP32Store(slot.numel, init=slot.packed.get("p"), device=slot.param.device)
            slot.packed = None
        slot.m, slot.v = m, v
        slot.seg = None
        slot.seg_ptr = None

    # ------------------------------------------------------------ descriptors

    def _group_struct(self, group: dict) -> _hip.Group:
        """The group's hyperparameters, refreshed from the dict on every batch so LR schedulers
        apply (engine.py:931-946)."""
        entry = self._groups.get(id(group))
        if entry is None or entry[0] is not group:
            entry = self._groups[id(group)] = (group, _hip.Group())
        g = entry[1]
        beta1, beta2 = group["betas"]
        g.lr = float(group["lr"])
        g.beta1 = float(beta1)
        g.beta2 = float(beta2)
        g.eps = float(group.get("eps", 0.0))
        g.weight_decay = float(group["weight_decay"])
        g.seed = self.seed & _MASK64
        g.stochastic = int(self.stochastic)
        return g

    def _new_segment(self, slot: ParamSlot) -> _hip.Segment:
        """The slot's descriptor: its state buffers, size, index and formats (fixed until the state
        is replaced); the per-update fields are filled by :meth:`_segment`."""
        seg = _hip.Segment()
        if isinstance(slot.packed, RecordState):
            seg.p_dtype = _hip.DT_PACKED8
            seg.m = seg.v = seg.p_lo = None
            seg.m_scale = slot.packed.scales["m"].data_ptr()
            seg.v_scale = slot.packed.scales["v"].data_ptr()
            seg.mv_dtype = _hip.DT_FP8
        elif slot.packed is not None:
            seg.p_dtype = _hip.DT_PACKED
            seg.m = seg.v = seg.m_scale = seg.v_scale = seg.p_lo = None
            seg.mv_dtype = _hip.DT_BF16
        else:
            p_hi, p_lo = slot.master.native_buffers
            seg.p = p_hi.data_ptr()
            seg.p_lo = p_lo.data_ptr() if p_lo is not None else None
            seg.p_dtype = _hip.MASTER_CODES[slot.master.precision]
            m_data, m_scale = slot.m.native_buffers
            seg.m = m_data.data_ptr()
            seg.m_scale = m_scale.data_ptr() if m_scale is not None else None
            if slot.v is not None:
                v_data, v_scale = slot.v.native_buffers
                seg.v = v_data.data_ptr()
                seg.v_scale = v_scale.data_ptr() if v_scale is not None else None
            seg.mv_dtype = _hip.MOMENT_CODES[slot.m.precision]
        seg.n = slot.numel
        seg.index = slot.index
        seg.offset = 0
        seg.algorithm = _hip.ALGORITHMS[self.algorithm]
        slot.seg = seg
        slot.seg_ptr = ctypes.pointer(seg)
        slot.seg_group = None
        return seg

    def _segment(self, slot: ParamSlot, grad: torch.Tensor, out_ptr: int | None, out_dtype: torch.dtype | None,
                 group: _hip.Group):
        """Pointer to the slot's descriptor, filled in for this update: gradient, output, step, group."""
        seg = slot.seg
        if seg is None:
            seg = self._new_segment(slot)
        if slot.packed is not None:   # the buffers alternate when double-buffered
            seg.p = slot.packed.current.data_ptr()
            other = slot.packed.other
            seg.p_lo = other.data_ptr() if other is not None else None
        dt = grad.dtype
        if dt is torch.bfloat16:
            seg.g_dtype = _hip.DT_BF16
        elif dt is torch.float32:
            seg.g_dtype = _hip.DT_F32
        else:
            raise TypeError(f"gradients must be float32 or bfloat16, got {dt}")
        seg.g = grad.data_ptr()
        if out_ptr is None:
            seg.out = None
            seg.out_dtype = _hip.DT_NONE
        else:
            seg.out = out_ptr
            seg.out_dtype = _hip.DT_F32 if out_dtype is torch.float32 else _hip.DT_BF16
        seg.step = slot.step
        if slot.seg_group is not group:
            seg.group = ctypes.pointer(group)
            slot.seg_group = group
        return slot.seg_ptr

    def _target(self, slot: ParamSlot, hooked: bool) -> tuple[int | None, torch.dtype | None]:
        """Where the kernel writes the new working weight: (device address, dtype), or (None, None)."""
        if slot.in_place:
            return None, None                   # the master is the parameter
        p = slot.param
        if self.delay or (hooked and not self.overlap_writeback) or not p.is_contiguous():
            self._ensure_out(slot)
            return slot.out.data_ptr(), slot.out.dtype
        return p.data_ptr(), p.dtype

    # ------------------------------------------------------------ submission

    def update(self, slots: list[ParamSlot], grads: list[torch.Tensor], hooked: bool = False,
               grads_kept: bool = True) -> None:
        """Enqueue one fused update of ``slots`` with ``grads`` (one launch per device).

        Ordered after the work already queued on each device's current stream; runs on the
        device's side stream.  Safe to call from the autograd thread.  ``grads_kept``: the
        caller leaves the gradients attached to the parameters, where later work on the compute
        stream may modify them in place, so even a delayed step orders the compute stream after
        this update."""
        by_dev: dict[torch.device, list[int]] = {}
        for i, slot in enumerate(slots):
            if not slot.initialized:
                self._check_param(slot.param)   # before any device context: CPU tensors get this error
            by_dev.setdefault(slot.param.device, []).append(i)
        for dev, idx in by_dev.items():
            self._update_device(dev, [slots[i] for i in idx], [grads[i] for i in idx], hooked)
            if grads_kept:
                self._grads_kept = True

    def _update_device(self, dev: torch.device, slots: list[ParamSlot], grads: list[torch.Tensor],
                       hooked: bool) -> None:
        st = self.streams(dev)
        with torch.cuda.device(dev):
            current = torch.cuda.current_stream(dev)
            for slot in slots:   # lazy state, built on the compute stream before `ready`
                if not slot.initialized:
                    self.initialize(slot)
            ready = torch.cuda.Event(enable_timing=self.timing)
            ready.record(current)
            if self.timing:
                self._ready_events.append(ready)
            st.side.wait_event(ready)
            if self.delay:
                owed = []
                with self._lock:
                    for slot in slots:
                        if slot in self._owed:
                            owed.append(slot)
                            del self._owed[slot]
                        self._fresh[slot] = None
                if owed:
                    written = self._write_back(dev, owed, ready)
                    st.side.wait_event(written)
            grads = [g if g.is_contiguous() else g.contiguous() for g in grads]
            segs = []
            structs: dict[int, _hip.Group] = {}   # each group's hyperparameters, read once per launch
            try:
                for slot, g in zip(slots, grads):
                    if g.numel() != slot.numel:
                        raise ValueError(f"gradient of parameter {slot.index} has {g.numel()} elements, "
                                         f"expected {slot.numel}")
                    if g.device != dev:
                        raise ValueError(f"gradient of parameter {slot.index} is on {g.device}, parameter on {dev}")
                    gs = structs.get(id(slot.group))
                    if gs is None:
                        gs = structs[id(slot.group)] = self._group_struct(slot.group)
                    slot.step += 1
                    segs.append(self._segment(slot, g, *self._target(slot, hooked), gs))
            except BaseException:
                for slot in slots[:len(segs)]:
                    slot.step -= 1
                raise
            timed = self.timing or self.launch_log is not None
            start = None
            if timed:
                start = torch.cuda.Event(enable_timing=True)
                start.record(st.side)
            self.kernels.set_stream(st.side)
            try:
                self.kernels.multi_step(None, self.kernels.segment_array(segs))
            except BaseException:
                for slot in slots:
                    slot.step -= 1
                raise
            done = torch.cuda.Event(enable_timing=timed)
            done.record(st.side)
            if self.timing:
                self._update_events.append((start, done))
            if self.launch_log is not None:   # (start, end, elements) of every launch, read after a sync
                self.launch_log.append((start, done, sum(s.numel for s in slots)))
            for slot in slots:
                slot.done_ev = done
                if slot.packed is not None:
                    slot.packed.flip()   # the new state is in the other buffer (double-buffered)
                if not self.delay and slot.out is not None and not slot.in_place and \
                        (hooked and not self.overlap_writeback or not slot.param.is_contiguous()):
                    self._deferred.append(slot)
            for g in grads:
                g.record_stream(st.side)
            self._used.add(dev)
            with self._lock:
                self._num_updates += len(slots)

    def _write_back(self, dev: torch.device, slots: list[ParamSlot], ready: torch.cuda.Event | None
                    ) -> torch.cuda.Event:
        """Copy the slots' finished updates from ``out`` into the parameters on the write-back stream,
        after ``ready`` (the compute stream's work so far) and each slot's last update."""
        st = self.streams(dev)
        if ready is None:
            ready = torch.cuda.Event()
            ready.record(torch.cuda.current_stream(dev))
        st.wb.wait_event(ready)
        for ev in {id(s.done_ev): s.done_ev for s in slots if s.done_ev is not None}.values():
            st.wb.wait_event(ev)
        with torch.cuda.stream(st.wb):
            torch._foreach_copy_([s.param.data for s in slots], [s.out_view for s in slots])
        written = torch.cuda.Event()
        written.record(st.wb)
        return written

    # ---------------------------------------------------------- synchronizing

    def _order(self) -> None:
        """The caller's current stream waits for every update (exact mode, or gradients still
        attached to the parameters) or only for the write-backs (delayed mode)."""
        kept, self._grads_kept = self._grads_kept, False
        for dev in self._used:
            st = self.streams(dev)
            current = torch.cuda.current_stream(dev)
            current.wait_stream(st.wb)
            if not self.delay or kept:
                current.wait_stream(st.side)

    def finish_step(self) -> StepStats:
        """Order this step's updates before the caller's next GPU work (engine.py:1219-1253).
        Delayed mode: updates from earlier steps whose parameters got no gradient this step are
        written back now, so no parameter lags by more than one step."""
        t0 = time.perf_counter()
        if self.delay:
            with self._lock:
                left, self._owed, self._fresh = list(self._owed), self._fresh, {}
            self._write_back_slots(left)
        deferred, self._deferred = self._deferred, []
        if deferred:
            self._write_back_slots(deferred)
        self._order()
        stats = StepStats(stall=time.perf_counter() - t0)
        with self._lock:
            stats.num_updates, self._num_updates = self._num_updates, 0
        if self.timing:
            self._fill_timing(stats)
        return stats

    def _fill_timing(self, stats: StepStats) -> None:
        readies, self._ready_events = self._ready_events, []
        updates, self._update_events = self._update_events, []
        if readies:
            readies[-1].synchronize()
        if len(readies) >= 2:
            stats.gpu_backward = readies[0].elapsed_time(readies[-1]) / 1e3
        if updates:
            updates[-1][1].synchronize()
            stats.gpu_update = updates[0][0].elapsed_time(updates[-1][1]) / 1e3
            if readies:
                stats.exposed_tail = max(0.0, readies[-1].elapsed_time(updates[-1][1]) / 1e3)

    def _write_back_slots(self, slots: list[ParamSlot]) -> None:
        by_dev: dict[torch.device, list[ParamSlot]] = {}
        for slot in slots:
            if slot.out_view is not None:
                by_dev.setdefault(slot.param.device, []).append(slot)
        for dev, members in by_dev.items():
            self._write_back(dev, members, None)

    def wait(self) -> None:
        """Block the host until every enqueued update has run."""
        for dev in list(self._used):
            st = self.streams(dev)
            st.side.synchronize()
            st.wb.synchronize()

    def flush(self) -> None:
        """Apply every pending delayed update to the parameters and order them before the
        caller's next work, so it sees the weights an exact optimizer would have produced."""
        with self._lock:
            slots = list({**self._owed, **self._fresh})
            self._owed, self._fresh = {}, {}
        self._write_back_slots(slots)
        deferred, self._deferred = self._deferred, []
        self._write_back_slots(deferred)
        for dev in self._used:
            st = self.streams(dev)
            current = torch.cuda.current_stream(dev)
            current.wait_stream(st.side)
            current.wait_stream(st.wb)

    def discard_pending(self) -> None:
        """Wait for enqueued updates and forget those not yet written to the parameters."""
        self.wait()
        with self._lock:
            self._owed, self._fresh = {}, {}
        self._deferred = []

    def close(self) -> None:
        if self._closed:
            return
        self._closed = True
        try:
            self.wait()
        except Exception:  # noqa: BLE001 -- closing must not raise from a finalizer
            pass
