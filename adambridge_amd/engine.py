"""Update engine: optimizer state in HBM, updates launched on HIP streams.

The reference's engine (adambridge/engine.py) copies every gradient to host
RAM, updates it on a CPU thread pool and copies the weights back.  Here the
state of each parameter is a :class:`~adambridge_amd.state.ParamState` in device
memory and one launch of the fused HIP kernel updates a whole batch of
parameters in place; what is left to the host is ordering and bookkeeping.

Stream order takes the place of the reference's threads.  By default (``update_stream=
"current"``) each update is launched on the stream current where it is submitted -- in a
gradient hook, the stream autograd runs that parameter's backward on -- right after the kernels
that produced its gradient, and before the rest of the backward pass::

    current stream:  ... dW(i) | update(i) | dX(i-1), dW(i-1) | update(i-1) | ... | step_sync
                                                          (buffered weights -> parameters, owed
                                                           delayed weights; nothing to wait for)

An update streams HBM at the rate of a copy, and so do most of the backward kernels beside it;
run side by side the two share the bandwidth at close to 1:1, and the cross-stream events cost
the compute stream time of their own, so the in-order launch is the faster one (c5: the step
0.5-1 ms shorter).  ``update_stream="side"`` keeps the overlapped form::

    compute stream        side stream                 write-back stream
    --------------        -----------                 -----------------
    grad ready  -------->  wait `ready`
    (backward goes on)     fused update (one launch)
                           record `done`  ---------->  [at step_sync: wait `done`; buffered
                                                        weights -> parameters]
    step_sync: current stream waits for both

Delayed updates (``delay``) keep the reference's semantics -- each parameter receives its
updates one step late -- without a buffer of their own: the update writes the parameter's
weight of the master as it was before the update (the previous update's result, flag
ADAMBRIDGE_SEG_OUT_PREVIOUS), so the newest weight stays in the master until the parameter's
next update, or a flush, writes it.

``update`` may be called from the autograd thread (the gradient hooks) and
never waits on the host.  The rounding streams are keyed by (parameter index,
the slot's own step count, element index), as in the reference, so results do
not depend on how updates are batched into launches.
"""

from __future__ import annotations

import ctypes
import threading
import time
import weakref
from dataclasses import dataclass, field

import torch

from . import _hip
from .precision import MomentStore, make_store
from .state import ParamState, arena_memory, choose_layout, new_states

__all__ = ["UpdateEngine", "ParamSlot", "SmallGroup", "StepStats"]

_GRAD_CODES = {torch.bfloat16: _hip.DT_BF16, torch.float32: _hip.DT_F32}


class ParamSlot:
    """One parameter: its index (rounding stream), group, step count, state and kernel descriptor."""

    __slots__ = ("index", "param", "group", "numel", "step", "state", "out", "out_view", "submitted", "seg",
                 "seg_ptr", "bound", "_small", "done_ev", "seg_group", "seg_out")

    def __init__(self, index: int, param: torch.Tensor, group: dict):
        self.index = index
        self.param = param
        self.group = group
        self.numel = param.numel()
        self.step = 0
        self.state: ParamState | None = None
        self.out: torch.Tensor | None = None        # write-back buffer (deferred write-back, strided parameter)
        self.out_view: torch.Tensor | None = None   # the same, shaped like the parameter
        self.submitted = False                      # updated (or queued) in the current step
        self.seg = _hip.Segment(n=self.numel, index=index)
        self.seg_ptr = ctypes.pointer(self.seg)
        self.bound: ParamState | None = None        # the state whose buffers seg points at
        self._small: weakref.ref | None = None
        self.done_ev: torch.cuda.Event | None = None   # recorded after the slot's latest update
        self.seg_group: _hip.Group | None = None    # the group struct seg points at
        self.seg_out: tuple | None = None           # (out, out_dtype, reserved) seg holds

    @property
    def initialized(self) -> bool:
        return self.state is not None

    @property
    def small(self) -> SmallGroup | None:
        """The small-parameter batch this slot is updated in, or None.  Held weakly: the batch holds
        its slots, and a cycle would keep every slot -- its parameter group, hence every parameter,
        and its state, a view of an arena shared with all the others -- alive until the garbage
        collector ran, instead of freeing the HBM when the optimizer is dropped."""
        return None if self._small is None else self._small()

    @small.setter
    def small(self, group: SmallGroup | None) -> None:
        self._small = None if group is None else weakref.ref(group)

    # The moments through the state (copies for interleaved layouts), as the reference's slots expose them.
    @property
    def m(self) -> MomentStore | None:
        return None if self.state is None else self.state.moment("m")

    @property
    def v(self) -> MomentStore | None:
        return None if self.state is None or "v" not in self.state.roles else self.state.moment("v")


class SmallGroup:
    """Parameters under the small-parameter threshold on one device: they get no hook and are updated
    together, in one launch, at step_sync (the reference's SmallGroup, engine.py:296-337)."""

    def __init__(self, slots: list[ParamSlot]):
        self.slots = slots
        self.device = slots[0].param.device
        for slot in slots:
            slot.small = self


@dataclass
class StepStats:
    """Timing of one optimizer step, in seconds (the reference's fields, engine.py:340-349, plus two).

    ``cpu_update`` and ``per_device_cpu`` stay zero: no host thread updates anything.  With timing on
    (``autotune``, or ``UpdateEngine.timing``), from events on the device: ``gpu_backward`` spans the
    first to the last gradient-ready event of the step, ``gpu_update`` the first update's start to the
    last update's end, and ``exposed_tail`` the last gradient-ready event to the last update's end
    (what work after backward waits for)."""

    num_updates: int = 0
    gpu_backward: float | None = None
    cpu_update: float = 0.0
    stall: float = 0.0
    per_device_cpu: dict[str, float] = field(default_factory=dict)
    gpu_update: float | None = None
    exposed_tail: float | None = None


class _Hyper:
    """The ``adambridge_group`` struct of each parameter group, refilled from the group's dict at every
    launch so that learning-rate schedulers and edits to the dict take effect (engine.py:931-946).
    The struct object of a group stays the same, so descriptors keep pointing at it."""

    def __init__(self, seed: int, stochastic: bool):
        self.seed = seed & 0xFFFFFFFFFFFFFFFF
        self.stochastic = int(stochastic)
        self._by_group: dict[int, tuple[dict, _hip.Group]] = {}

    def refresh(self, group: dict) -> _hip.Group:
        held = self._by_group.get(id(group))
        if held is None or held[0] is not group:
            held = self._by_group[id(group)] = (group, _hip.Group())
        struct = held[1]
        b1, b2 = group["betas"]
        struct.__init__(float(group["lr"]), float(b1), float(b2), float(group.get("eps", 0.0)),
                        float(group["weight_decay"]), self.seed, self.stochastic, 0)
        return struct


class _Lanes:
    """A device's two streams besides the caller's, for ``update_stream="side"``: updates run on
    ``side``, copies into the parameters (buffered weights, owed delayed updates) on ``wb`` (both at
    the default priority, made at first use)."""

    def __init__(self, device: torch.device):
        self.device = device
        self._side: torch.cuda.Stream | None = None
        self._wb: torch.cuda.Stream | None = None

    @property
    def side(self) -> torch.cuda.Stream:
        if self._side is None:
            self._side = torch.cuda.Stream(self.device)
        return self._side

    @property
    def wb(self) -> torch.cuda.Stream:
        if self._wb is None:
            self._wb = torch.cuda.Stream(self.device)
        return self._wb


class UpdateEngine:
    """Owns the kernel library handle, the streams, the group structs and the pending write-backs."""

    def __init__(self, *, precision: str, algorithm: str = "adamw", stochastic_rounding: bool = True, seed: int = 0,
                 overlap_writeback: bool = True, timing: bool = False, master_precision: str = "fp32",
                 delay_capable: bool = False, state_layout: str = "auto", double_buffer: bool = False,
                 update_stream: str = "current"):
        if state_layout not in ("auto", "packed", "separate"):
            raise ValueError("state_layout must be 'auto', 'packed' or 'separate'")
        if update_stream not in ("current", "side"):
            raise ValueError("update_stream must be 'current' or 'side'")
        if algorithm not in _hip.ALGORITHMS:
            raise ValueError(f"algorithm must be one of {sorted(_hip.ALGORITHMS)}")
        if master_precision not in _hip.MASTER_CODES:
            raise ValueError(f"master_precision must be one of {sorted(_hip.MASTER_CODES)}")
        self.kernels = _hip.load()
        self.algorithm = algorithm
        self._algo_code = _hip.ALGORITHMS[algorithm]
        self.lion = algorithm == "lion"
        self.precision = precision
        self.master_precision = master_precision
        self.overlap_writeback = overlap_writeback
        self.timing = timing
        self.delay = False              # toggled between steps only
        self.delay_capable = delay_capable
        self.state_layout = state_layout
        self.double_buffer = double_buffer
        self.apart = update_stream == "side"   # updates on a side stream of their own
        self._hyper = _Hyper(seed, stochastic_rounding)
        self._lock = threading.RLock()
        self._lanes: dict[torch.device, _Lanes] = {}
        self._owed: dict[ParamSlot, None] = {}     # delayed: the master holds an update not yet in the parameter
        self._fresh: dict[ParamSlot, None] = {}    # delayed: updated during the current step
        self._deferred: list[ParamSlot] = []       # weights written to `out`, copied in at step_sync
        self._num_updates = 0
        self._ready_events: list[torch.cuda.Event] = []
        self._update_events: list[tuple[torch.cuda.Event, torch.cuda.Event]] = []
        # every stream this engine enqueued work on, by device (what the caller's stream must wait for)
        self._streams: dict[torch.device, dict[int, torch.cuda.Stream]] = {}
        self.launch_log: list | None = None   # a list: (start, end, elements) of every launch, read after a sync
        self.hooked_slots: list[ParamSlot] = []   # the parameters gradient hooks update (set by the optimizer)
        self._reserved: dict[ParamSlot, list[torch.Tensor]] = {}   # arena memory set aside for hooked states
        self._reserved_on: set[torch.device] = set()
        self._closed = False

    # ----------------------------------------------------------------- state

    def lanes(self, device: torch.device) -> _Lanes:
        lanes = self._lanes.get(device)
        if lanes is None:
            with self._lock:
                lanes = self._lanes.setdefault(device, _Lanes(device))
        return lanes

    @staticmethod
    def check_param(p: torch.Tensor) -> None:
        if not p.is_cuda:
            raise ValueError("adambridge_amd keeps optimizer state in GPU memory and updates it with a HIP kernel: "
                             f"parameters must be on a GPU, got one on {p.device}")
        if p.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"parameters must be float32 or bfloat16 (the kernel's weight formats), got {p.dtype}")

    def _master_is_param(self, p: torch.Tensor) -> bool:
        """An FP32 parameter is its own master, updated in place by the kernel, unless updates are
        written elsewhere first (delayed or deferred write-back)."""
        return (p.dtype == torch.float32 and self.master_precision == "fp32" and p.is_contiguous()
                and not self.delay_capable and self.overlap_writeback)

    def layout_for(self, slot: ParamSlot, precision: str | None = None) -> str:
        return choose_layout(self.algorithm, precision or self.precision, self.master_precision,
                             "separate" if self.state_layout == "separate" else "auto",
                             self._master_is_param(slot.param))

    def initialize(self, slots: list[ParamSlot], place: bool = True) -> None:
        """Lazy state for ``slots`` (engine.py:991-1025; precision.py:263-267, 307-311, 365-371): the master
        from each parameter's current value (FP32, or FP24 rounded to nearest), moments zero, FP8
        scales one.  The interleaved states of one device and layout share one arena, placed by an
        allocate/free of its size first unless ``place`` is False (see state.new_states).  Without
        ``place`` (a gradient hook), the first call on a device sets aside one placed arena for the
        interleaved states of every hooked parameter not initialized yet (``hooked_slots``), and each
        state is built on its share when its parameter's first update comes -- one placement, one
        wait for the device, instead of one allocation per parameter where the driver puts it."""
        for slot in slots:
            self.check_param(slot.param)
        todo: dict[tuple[torch.device, str], list[ParamSlot]] = {}
        for slot in slots:
            todo.setdefault((slot.param.device, self.layout_for(slot)), []).append(slot)
        for (device, layout), members in todo.items():
            with torch.cuda.device(device), torch.no_grad():
                if not place:
                    self._reserve(device)
                for group in ([s for s in members if s in self._reserved],
                              [s for s in members if s not in self._reserved]):
                    if not group:
                        continue
                    memory = [self._reserved.pop(s) for s in group] if group[0] in self._reserved else None
                    masters = [s.param.detach().reshape(-1) for s in group]
                    params = [s.param if self._master_is_param(s.param) else None for s in group]
                    states = new_states(layout, self.algorithm, self.precision, self.master_precision, device,
                                        masters, self.double_buffer, params, place, memory)
                    for slot, state in zip(group, states):
                        self._adopt(slot, state)
                        self._ensure_out(slot)

    def _reserve(self, device: torch.device) -> None:
        """Once per device: one placed arena per interleaved layout for the hooked parameters on
        ``device`` that have no state yet (see :meth:`initialize`)."""
        if device in self._reserved_on:
            return
        self._reserved_on.add(device)
        by_layout: dict[str, list[ParamSlot]] = {}
        for slot in self.hooked_slots:
            if slot.initialized or slot in self._reserved or slot.param.device != device:
                continue
            layout = self.layout_for(slot)
            if layout != "separate":
                by_layout.setdefault(layout, []).append(slot)
        for layout, members in by_layout.items():
            memory = arena_memory(layout, [s.numel for s in members], device, self.double_buffer)
            self._reserved.update(zip(members, memory))

    @staticmethod
    def _adopt(slot: ParamSlot, state: ParamState) -> None:
        slot.state = state
        state.bind(slot.seg)
        slot.bound = state

    def rebuild(self, slots: list[ParamSlot], precision: str | None = None, masters: list | None = None,
                moments: list[dict[str, MomentStore] | None] | None = None) -> None:
        """New states for ``slots`` in ``precision`` (default: the engine's), each in the layout that
        serves it -- one arena per device and layout, as :meth:`initialize`.  ``masters[i]``: checkpoint
        master weights for slot i, or None to keep its master (a fresh slot: the parameter's value);
        ``moments[i]``: stores of that precision, or None to re-encode its current moments."""
        precision = precision or self.precision
        masters = masters or [None] * len(slots)
        moments = moments or [None] * len(slots)
        self._reserved.clear()   # set aside for the old precision's layout; set aside again on the next hook
        self._reserved_on.clear()
        groups: dict[tuple[torch.device, str], list[int]] = {}
        for i, slot in enumerate(slots):
            self.check_param(slot.param)
            groups.setdefault((slot.param.device, self.layout_for(slot, precision)), []).append(i)
        for (device, layout), picks in groups.items():
            with torch.cuda.device(device), torch.no_grad():
                values, params, loads = [], [], []
                for i in picks:
                    slot, old = slots[i], slots[i].state
                    param = slot.param if self._master_is_param(slot.param) else None
                    values.append(slot.param.detach().reshape(-1) if param is not None or old is None
                                  else old.master_fp32())
                    params.append(param)
                    held = moments[i]
                    if held is None:
                        held = {r: make_store(precision, slot.numel, r, init=old.moment(r).to_fp32(), device=device)
                                for r in old.roles}
                    loads.append(held)
                states = new_states(layout, self.algorithm, precision, self.master_precision, device, values,
                                    self.double_buffer, params)
                for i, state, held in zip(picks, states, loads):
                    state.load(master=masters[i], moments=held)
                    self._adopt(slots[i], state)
                    self._ensure_out(slots[i])

    def _ensure_out(self, slot: ParamSlot) -> None:
        """The write-back buffer of a slot whose updates go there first (deferred write-back, a
        non-contiguous parameter)."""
        p = slot.param
        wanted = not slot.state.master_is_param and (not self.overlap_writeback or not p.is_contiguous())
        if wanted and slot.out is None:
            slot.out = torch.empty(slot.numel, dtype=p.dtype, device=p.device)
            slot.out_view = slot.out.view(p.shape)

    # ------------------------------------------------------------ descriptors

    def _target(self, slot: ParamSlot, hooked: bool) -> tuple[int | None, torch.dtype | None, bool]:
        """Where the kernel writes the working weight: (device address, dtype, buffered), or (None, None,
        False).  Buffered: the slot's `out`, copied into the parameter at step_sync -- a strided
        parameter, or a hooked update with overlap_writeback=False (exact mode only: a delayed update
        writes the previous weight, which the parameter may take at once)."""
        state = slot.state
        if state.master_is_param:
            return None, None, False            # the master is the parameter
        p = slot.param
        if not p.is_contiguous() or (hooked and not self.overlap_writeback and not self.delay):
            if slot.out is None:
                slot.out = torch.empty(slot.numel, dtype=p.dtype, device=p.device)
                slot.out_view = slot.out.view(p.shape)
            return slot.out.data_ptr(), slot.out.dtype, True
        return p.data_ptr(), p.dtype, False

    def _describe(self, slot: ParamSlot, grad: torch.Tensor, hooked: bool, group: _hip.Group):
        """The slot's descriptor for this update: gradient, output, step, group (state fields bound).
        Returns the descriptor's pointer and whether the weight goes to the slot's buffer."""
        seg = slot.seg
        if slot.bound is not slot.state or slot.state.alternates:
            slot.state.bind(seg)
            slot.bound = slot.state
        seg.offset = 0
        seg.algorithm = self._algo_code
        g_dtype = _GRAD_CODES.get(grad.dtype)
        if g_dtype is None:
            raise TypeError(f"gradients must be float32 or bfloat16, got {grad.dtype}")
        seg.g_dtype = g_dtype
        seg.g = grad.data_ptr()
        out, dtype, buffered = self._target(slot, hooked)
        if self.delay and slot.step == 1:
            # a delayed first update owes the parameter nothing: its weight is the one the master was
            # made from (which an FP24 master holds only rounded)
            out, dtype, buffered = None, None, False
        # fields that rarely change are written only when they do (host time per step with ~300 slots)
        want = (out, _hip.DT_NONE if out is None else _hip.DT_F32 if dtype is torch.float32 else _hip.DT_BF16,
                _hip.SEG_OUT_PREVIOUS if self.delay and out is not None else 0)
        if slot.seg_out != want:
            seg.out, seg.out_dtype, seg.reserved = want
            slot.seg_out = want
        seg.step = slot.step
        if slot.seg_group is not group:
            seg.group = ctypes.pointer(group)
            slot.seg_group = group
        return slot.seg_ptr, buffered

    # ------------------------------------------------------------ submission

    def update(self, slots: list[ParamSlot], grads: list[torch.Tensor], hooked: bool = False) -> None:
        """Enqueue one fused update of ``slots`` with ``grads``, one launch per device, on the device's side
        stream after the work already queued on its current stream (the gradients are kept alive for it
        by ``record_stream``; the caller's stream waits for it at :meth:`finish_step`)."""
        by_device: dict[torch.device, list[int]] = {}
        for i, slot in enumerate(slots):
            if not slot.initialized:
                self.check_param(slot.param)   # before any device context: a CPU tensor gets this error
            by_device.setdefault(slot.param.device, []).append(i)
        for device, picks in by_device.items():
            self._launch(device, [slots[i] for i in picks], [grads[i] for i in picks], hooked)

    def _launch(self, device: torch.device, slots: list[ParamSlot], grads: list[torch.Tensor], hooked: bool) -> None:
        with torch.cuda.device(device):
            current = torch.cuda.current_stream(device)
            stream = self.lanes(device).side if self.apart else current
            for slot, g in zip(slots, grads):
                if g.numel() != slot.numel:
                    raise ValueError(f"gradient of parameter {slot.index} has {g.numel()} elements, "
                                     f"expected {slot.numel}")
                if g.device != device:
                    raise ValueError(f"gradient of parameter {slot.index} is on {g.device}, parameter on {device}")
            # A strided gradient is read from a contiguous copy (logical order), made on the compute
            # stream before the update is ordered after it.
            grads = [g if g.is_contiguous() else g.contiguous() for g in grads]
            fresh = [s for s in slots if not s.initialized]
            if fresh:   # built on the compute stream, before `ready`; a hook does not wait for the device
                self.initialize(fresh, place=not hooked)
            if self.apart or self.timing:
                ready = torch.cuda.Event(enable_timing=self.timing)
                ready.record(current)
                if self.timing:
                    self._ready_events.append(ready)
                if self.apart:
                    stream.wait_event(ready)
            structs: dict[int, _hip.Group] = {}   # each group's hyperparameters, read once per launch
            for slot in slots:
                slot.step += 1
            try:
                ptrs, buffered = [], []
                for slot, g in zip(slots, grads):
                    gs = structs.get(id(slot.group))
                    if gs is None:
                        gs = structs[id(slot.group)] = self._hyper.refresh(slot.group)
                    ptr, into_out = self._describe(slot, g, hooked, gs)
                    ptrs.append(ptr)
                    if into_out:
                        buffered.append(slot)
                arr = self.kernels.segment_array(ptrs)
                self.kernels.set_stream(stream)
                timed = self.timing or self.launch_log is not None
                start = torch.cuda.Event(enable_timing=True) if timed else None
                if start is not None:   # right before the launch: the pair brackets the library call only
                    start.record(stream)
                self.kernels.multi_step(None, arr)
            except BaseException:
                for slot in slots:   # nothing was enqueued: the library validates and plans before launching
                    slot.step -= 1
                raise
            done = None
            if self.apart or timed:
                done = torch.cuda.Event(enable_timing=timed)
                done.record(stream)
            if self.timing:
                self._update_events.append((start, done))
            if self.launch_log is not None:
                self.launch_log.append((start, done, sum(s.numel for s in slots)))
            for slot in slots:   # in stream order, what follows on `stream` needs no event
                slot.done_ev = done if self.apart else None
                slot.state.advance()
            self._deferred += buffered
            if self.delay:   # each update wrote the weight owed from the slot's last one, and owes its own
                with self._lock:
                    for slot in slots:
                        self._owed.pop(slot, None)
                        self._fresh[slot] = None
            for g in grads:   # the gradient is released after this; its memory waits for the update
                g.record_stream(stream)
            with self._lock:
                self._note(device, stream)
                self._num_updates += len(slots)

    def _note(self, device: torch.device, stream: torch.cuda.Stream) -> None:
        self._streams.setdefault(device, {})[stream.cuda_stream] = stream

    def _join(self) -> None:
        """The caller's current stream, on each device, waits for the work this engine enqueued on any
        other stream, and stands for all of it from then on."""
        with self._lock:
            streams = {d: dict(ss) for d, ss in self._streams.items()}
        for device, members in streams.items():
            current = torch.cuda.current_stream(device)
            for key, s in members.items():
                if key != current.cuda_stream:
                    current.wait_stream(s)
            with self._lock:   # streams noted meanwhile (another thread) stay
                held = self._streams[device]
                for key in members:
                    held.pop(key, None)
                held[current.cuda_stream] = current

    def _write_back(self, device: torch.device, slots: list[ParamSlot], ready: torch.cuda.Event | None
                    ) -> torch.cuda.Event | None:
        """Copy the slots' finished updates from ``out`` into the parameters: on the current stream
        after the updates (already ordered there), or with ``update_stream="side"`` on the write-back
        stream after ``ready`` (the compute stream so far) and each slot's latest update; returns the
        event of the copies on the write-back stream (None on the current stream)."""
        if not self.apart:
            with torch.cuda.device(device), torch.no_grad():
                torch._foreach_copy_([s.param.data for s in slots], [s.out_view for s in slots])
                with self._lock:
                    self._note(device, torch.cuda.current_stream(device))
            return None
        lanes = self.lanes(device)
        if ready is None:
            ready = torch.cuda.Event()
            ready.record(torch.cuda.current_stream(device))
        lanes.wb.wait_event(ready)
        for ev in {id(s.done_ev): s.done_ev for s in slots if s.done_ev is not None}.values():
            lanes.wb.wait_event(ev)
        with torch.cuda.stream(lanes.wb):
            torch._foreach_copy_([s.param.data for s in slots], [s.out_view for s in slots])
        written = torch.cuda.Event()
        written.record(lanes.wb)
        with self._lock:
            self._note(device, lanes.wb)
        return written

    def _write_back_all(self, slots: list[ParamSlot]) -> None:
        by_device: dict[torch.device, list[ParamSlot]] = {}
        for slot in slots:
            if slot.out_view is not None:
                by_device.setdefault(slot.param.device, []).append(slot)
        for device, members in by_device.items():
            self._write_back(device, members, None)

    def _weights_from_masters(self, slots: list[ParamSlot]) -> None:
        """Write each slot's newest weight -- its master in the parameter's dtype, as the kernels round
        it -- into the parameter, after the work so far on the current stream (which may still read
        the old weights) and the slot's latest update: on the current stream itself, or with
        ``update_stream="side"`` on the write-back stream.  For delayed updates owed to parameters
        that their next update will not reach in time."""
        by_device: dict[torch.device, list[ParamSlot]] = {}
        for slot in slots:
            if slot.state is not None and not slot.state.master_is_param:
                by_device.setdefault(slot.param.device, []).append(slot)
        for device, members in by_device.items():
            if not self.apart:
                with torch.cuda.device(device), torch.no_grad():
                    for slot in members:   # one conversion pass each, straight into the parameter
                        slot.state.write_weights(slot.param)
                    with self._lock:
                        self._note(device, torch.cuda.current_stream(device))
                continue
            lanes = self.lanes(device)
            with torch.cuda.device(device):
                ready = torch.cuda.Event()
                ready.record(torch.cuda.current_stream(device))
                lanes.wb.wait_event(ready)
                for ev in {id(s.done_ev): s.done_ev for s in members if s.done_ev is not None}.values():
                    lanes.wb.wait_event(ev)
                with torch.cuda.stream(lanes.wb), torch.no_grad():
                    for slot in members:   # one conversion pass each, straight into the parameter
                        slot.state.write_weights(slot.param)
            with self._lock:
                self._note(device, lanes.wb)

    # ---------------------------------------------------------- synchronizing

    def finish_step(self) -> StepStats:
        """Order this step's updates before the caller's next work on each device (engine.py:1219-1253).
        Delayed mode: updates owed from earlier steps whose parameters got no gradient this step are
        written back now, so no parameter lags by more than one step."""
        t0 = time.perf_counter()
        with self._lock:   # owed updates whose parameters got no gradient this step: written now
            left, self._owed, self._fresh = list(self._owed), self._fresh, {}
        if not self.apart:
            self._join()   # updates submitted on other streams (hooks on another stream), before the copies
        self._weights_from_masters(left)
        deferred, self._deferred = self._deferred, []
        self._write_back_all(deferred)
        self._join()   # the updates write the parameters, delayed ones too
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

    def wait(self) -> None:
        """Block the host until every enqueued update and write-back has run."""
        with self._lock:
            streams = [s for ss in self._streams.values() for s in ss.values()]
        for s in streams:
            s.synchronize()

    def flush(self) -> None:
        """Write every pending delayed update into its parameter and order all of it before the caller's
        next work, which then sees the weights an exact optimizer would have produced."""
        if not self.apart:
            self._join()   # updates submitted on other streams, before the copies
        deferred, self._deferred = self._deferred, []
        self._write_back_all(deferred)
        with self._lock:
            pending = list({**self._owed, **self._fresh})
            self._owed, self._fresh = {}, {}
        self._weights_from_masters(pending)
        self._join()

    def discard_pending(self) -> None:
        """Wait for enqueued updates and forget those not yet written into the parameters."""
        self.wait()
        with self._lock:
            self._owed, self._fresh = {}, {}
        self._deferred = []

    def close(self) -> None:
        if self._closed:
            return
        self._closed = True
        self._reserved.clear()
        try:
            self.wait()
        except Exception:  # noqa: BLE001 -- a finalizer must not raise
            pass
