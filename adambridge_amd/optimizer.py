"""AdamBridge / OptiComputeAdamW / LionBridge with the optimizer state in HBM.

The constructor, methods, checkpoint format and error behaviour are the
reference's (adambridge/optimizer.py, cited per method).  The implementation is
built around where the state lives here: each parameter's FP32 (or FP24)
master, moments and FP8 block scales are a
:class:`~adambridge_amd.state.ParamState` in device memory, and one launch of
the fused HIP kernel (libadambridge_hip.so) updates a whole batch of
parameters in a single pass over HBM, writing the new working weights into
``p.data``.

Numerically this is torch.optim.AdamW (decoupled weight decay, bias
correction, the same operation order), or Lion, with the reference kernel's
exact rounding: results are bit-identical to the reference's native CPU kernel
on the same inputs.

The parts:

* ``_Registry`` -- the parameters in index order (the index selects the
  rounding stream), their slots, and the small ones batched at step_sync;
* ``_StepWindow`` -- what the gradient hooks may do in the current step:
  ``no_sync`` nesting, gradient-accumulation micro-batches;
* ``_HookSet`` -- the post-accumulate-grad hooks;
* ``_LaunchPoints`` -- where a backward pass launches the hooked updates: at the
  start of the next hooked module's backward (its GEMMs), not beside the
  elementwise work that follows a weight gradient;
* ``_CheckpointReader`` -- validates a whole checkpoint before anything changes.

Host-side knobs of the reference with nothing to act on here -- NUMA
placement, thread counts, the PyTorch-kernel chunk size, the pinned transfer
ring, the GPU state budget, the CPU thread auto-tuner -- are accepted and
validated as the reference validates them, and otherwise ignored.
"""

from __future__ import annotations

import contextlib
import logging
import weakref
from typing import Any, Callable, Iterable

import torch
import torch._dynamo  # noqa: F401 -- imported here, not by the first torch.compiler.disable() call: that import
#                       keeps the frames on the stack alive, which would pin the optimizer being built

from .engine import ParamSlot, SmallGroup, StepStats, UpdateEngine
from .precision import (_checked, bytes_per_param, canonical_master_precision, canonical_precision,
                        check_master_state, make_store, store_from_state_dict)

__all__ = ["AdamBridge", "LionBridge", "OptiComputeAdamW", "AutoTuneConfig"]

log = logging.getLogger("adambridge_amd")


class AutoTuneConfig:
    """Accepted for API compatibility (reference autotune.py:34-44).  The reference tunes its host
    thread count and steps the moment precision down when the host update outlasts the backward
    pass; on the GPU the update is a bandwidth-bound kernel launch, so nothing is tuned."""

    def __init__(self, warmup_steps: int = 3, window: int = 5, threshold: float = 1.1,
                 min_precision: str = "fp8", tune_threads: bool = True):
        self.warmup_steps = warmup_steps
        self.window = window
        self.threshold = threshold
        self.min_precision = canonical_precision(min_precision)
        self.tune_threads = tune_threads


# ------------------------------------------------------------- validation

def _check_arguments(algorithm: str, lr, betas, eps, weight_decay, delay_warmup_steps, accumulation_steps,
                     chunk_size, transfer_buffer_mb, gpu_state_budget, backend) -> None:
    """The reference's argument checks and messages (optimizer.py:152-170), then this build's own."""
    rules = [
        (0.0 <= lr, f"invalid learning rate: {lr}"),
        (delay_warmup_steps >= 0 and accumulation_steps >= 1,
         "delay_warmup_steps must be >= 0 and accumulation_steps >= 1"),
        (0.0 <= eps, f"invalid epsilon: {eps}"),
        (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0, f"invalid betas: {betas}"),
        (0.0 <= weight_decay, f"invalid weight_decay: {weight_decay}"),
        (chunk_size is None or (chunk_size > 0 and chunk_size % 128 == 0),
         "chunk_size must be a positive multiple of 128"),
        (transfer_buffer_mb is None or transfer_buffer_mb >= 0, "transfer_buffer_mb must be >= 0"),
        (gpu_state_budget is None or gpu_state_budget == "auto"
         or (isinstance(gpu_state_budget, int) and gpu_state_budget >= 0),
         "gpu_state_budget must be None, 'auto' or a number of bytes >= 0"),
        (not gpu_state_budget or algorithm == "adamw", "gpu_state_budget is only available for AdamW"),
        (backend in ("auto", "native", "torch"), "backend must be 'auto', 'native' or 'torch'"),
        (backend != "torch", "backend='torch' is not available: the update runs only as the fused HIP kernel"),
    ]
    for ok, message in rules:
        if not ok:
            raise ValueError(message)


# ------------------------------------------------------------------ parts

class _Registry:
    """Parameters in index order, the slot of each, and the small-parameter batches."""

    def __init__(self):
        self.ordered: list[ParamSlot] = []
        self.by_param: dict[torch.Tensor, ParamSlot] = {}
        self.small: list[SmallGroup] = []

    def register(self, p: torch.Tensor, group: dict) -> ParamSlot:
        if p.is_sparse:
            raise ValueError("AdamBridge does not support sparse parameters")
        slot = ParamSlot(len(self.ordered), p, group)
        self.ordered.append(slot)
        self.by_param[p] = slot
        return slot

    def batch_small(self, threshold: int) -> None:
        """Device parameters under ``threshold`` elements: one batch per device, no hooks."""
        per_device: dict[torch.device, list[ParamSlot]] = {}
        for slot in self.ordered:
            p = slot.param
            if p.is_cuda and p.requires_grad and slot.numel < threshold and slot.small is None:
                per_device.setdefault(p.device, []).append(slot)
        self.small += [SmallGroup(members) for members in per_device.values()]

    def pending(self, *, include_small: bool = True) -> list[ParamSlot]:
        """Slots with a gradient and no update yet in this step."""
        return [s for s in self.ordered if not s.submitted and s.param.grad is not None
                and (include_small or s.small is None)]

    def hook_targets(self, params: Iterable[torch.Tensor] | None = None) -> list[torch.Tensor]:
        """The parameters that get a gradient hook: those of ``params`` (default: every registered one)
        that take gradients and are not updated in a small-parameter batch."""
        slots = self.ordered if params is None else [self.by_param[p] for p in params if p in self.by_param]
        return [s.param for s in slots if s.param.requires_grad and s.small is None]

    def new_step(self) -> None:
        for slot in self.ordered:
            slot.submitted = False


class _StepWindow:
    """What the gradient hooks may do in the current step (optimizer.py:285-304): nothing inside
    ``no_sync``; with gradient accumulation, update only on the window's last backward pass, counted
    by a callback at the end of each backward."""

    def __init__(self, every: int):
        self.every = every
        self.suppressed = 0      # no_sync nesting depth
        self.backwards = 0       # backward passes finished since the last step
        self.counting = False    # an end-of-backward callback is queued
        self.closed = 0          # steps closed without an error

    @contextlib.contextmanager
    def suppress(self):
        """Hooks do nothing inside (nestable)."""
        self.suppressed += 1
        try:
            yield
        finally:
            self.suppressed -= 1

    @contextlib.contextmanager
    def closing(self, registry: _Registry):
        """Close a step: whatever happens inside, the next one starts with no parameter marked as
        updated and no backward pass counted; a step closed without an error is counted."""
        try:
            yield
        finally:
            registry.new_step()
            self.backwards = 0
        self.closed += 1

    def hook_may_update(self) -> bool:
        if self.suppressed:
            return False
        if self.every == 1:
            return True
        if not self.counting:
            self.counting = True
            torch.autograd.Variable._execution_engine.queue_callback(self._backward_finished)
        return self.backwards + 1 >= self.every

    def _backward_finished(self) -> None:
        self.backwards += 1
        self.counting = False


class _HookSet:
    """Post-accumulate-grad hooks calling one method of the optimizer, kept opaque to TorchDynamo so
    that compiled autograd calls it instead of tracing the launches inside (optimizer.py:271-274).
    The hooks reach the optimizer through a weak reference: parameters (which hold their hooks) and
    the optimizer's own attributes then form no cycle, and dropping the last reference to the
    optimizer frees its device state at once, without waiting for the garbage collector."""

    def __init__(self, method: Callable[[torch.Tensor], None]):
        target = weakref.WeakMethod(method)

        def on_grad_ready(p: torch.Tensor) -> None:
            bound = target()
            if bound is not None:
                bound(p)

        self._fn = torch.compiler.disable(on_grad_ready)
        self._handles: list = []
        self.active = False

    def add(self, params: Iterable[torch.Tensor]) -> None:
        self._handles += [p.register_post_accumulate_grad_hook(self._fn) for p in params]

    def clear(self) -> None:
        while self._handles:
            self._handles.pop().remove()
        self.active = False


class _LaunchPoints:
    """Where a backward pass launches the hooked updates it has deferred when they run on a side stream
    (``update_stream="side"``): at the start of the backward of each module that owns hooked
    parameters, and at the end of the pass.

    A parameter's gradient is ready right after its weight-gradient GEMM; what the backward runs next
    is usually elementwise work bound by HBM (an activation's or a norm's backward), which an update
    started then -- itself bound by HBM -- slows by about as much as it saves.  The backward of the
    next module that owns hooked parameters begins with its GEMMs, which read HBM at a third of its
    rate on average, so the update is launched there instead (measured: the elementwise kernels then
    keep their speed, the GEMMs beside the updates slow by about the updates' own time, which is why
    the in-order launch on the current stream is the default): a forward hook on each such module
    registers a hook on the gradient of the module's output, which fires when that gradient is
    computed and before the module's own backward kernels are enqueued.  A forward pass that ran
    under compilation (or without gradients) registers nothing, and its backward launches each
    update at its parameter's hook.  Hooks reach the optimizer through a weak reference, as
    :class:`_HookSet`'s do."""

    def __init__(self, launch: Callable[[], None]):
        target = weakref.WeakMethod(launch)

        def fire(*_grad) -> None:   # a gradient hook: leaves the gradient as it is
            bound = target()
            if bound is not None:
                bound()

        self.fire = torch.compiler.disable(fire)
        self.armed = False          # this step's forward registered launch points
        self._handles: list = []

        def on_forward(module, inputs, output) -> None:
            if torch.compiler.is_compiling() or not torch.is_grad_enabled():
                return
            out = output
            if isinstance(out, (tuple, list)):
                out = next((t for t in out if isinstance(t, torch.Tensor) and t.requires_grad), None)
            if isinstance(out, torch.Tensor) and out.requires_grad:
                out.register_hook(self.fire)
                self.armed = True

        self._on_forward = on_forward

    def add(self, modules: Iterable[torch.nn.Module]) -> None:
        self._handles += [m.register_forward_hook(self._on_forward) for m in modules]

    def clear(self) -> None:
        while self._handles:
            self._handles.pop().remove()
        self.armed = False


class _CheckpointReader:
    """A checkpoint's per-parameter entries, validated as a whole before anything is changed (a
    checkpoint may come from another model, another version or an untrusted source)."""

    def __init__(self, state_dict: dict[str, Any], slots: list[ParamSlot], lion: bool):
        self.entries = {self._index(key, len(slots)): entry for key, entry in state_dict["state"].items()}
        for index, entry in self.entries.items():
            self._validate(index, entry, slots[index].numel, lion)

    @staticmethod
    def _index(key: Any, count: int) -> int:
        """The parameter index a state key names (string keys come back from JSON round trips)."""
        index = int(key) if isinstance(key, str) and key.isdigit() else key
        if type(index) is int and 0 <= index < count:
            return index
        raise ValueError(f"checkpoint state for parameter {index!r}: this optimizer has parameters 0..{count - 1}")

    @staticmethod
    def _validate(index: int, entry: dict[str, Any], numel: int, lion: bool) -> None:
        """Sizes and formats of one entry: its master (tensor or store dictionary), its plain-tensor
        moments (the torch.optim.AdamW layout; store dictionaries are checked when rebuilt), and the
        second moment AdamW needs."""
        if entry.get("master") is not None:
            check_master_state(entry["master"], numel, f"master weights of parameter {index}")
        plain = {k: v for k, v in entry.items() if k in ("exp_avg", "exp_avg_sq") and isinstance(v, torch.Tensor)}
        for key, tensor in plain.items():
            _checked(tensor, numel, f"{key} of parameter {index}")
        if not lion and "exp_avg_sq" not in entry:
            raise ValueError("checkpoint has no exp_avg_sq (saved by LionBridge?); AdamW needs both moments")

    @staticmethod
    def moment(saved: Any, numel: int, role: str, precision: str, device):
        """A saved moment as a store of ``precision``: the torch.optim.AdamW layout (a plain tensor)
        converted, a store dictionary rebuilt and converted if its precision differs."""
        if isinstance(saved, torch.Tensor):
            return make_store(precision, numel, role, init=saved.to(device, torch.float32), device=device)
        store = store_from_state_dict(saved, numel, role, device=device)
        if store.precision == precision:
            return store
        return make_store(precision, numel, role, init=store.to_fp32(), device=device)


# -------------------------------------------------------------- the optimizer

class AdamBridge(torch.optim.Optimizer):
    r"""AdamW whose state lives in GPU memory and is updated by one fused HIP kernel.

    **Synchronous** -- a drop-in replacement for any optimizer::

        loss.backward()
        opt.step()          # one kernel launch updates every parameter with a gradient
        opt.zero_grad()

    **Layer-wise asynchronous** -- each parameter is updated as soon as its gradient is ready::

        opt.attach_hooks(model)
        loss.backward()     # each update is enqueued from the parameter's gradient hook
        opt.step_sync()     # the next forward pass (on the current stream) sees the new weights

    In asynchronous mode gradients are released as soon as their update is
    enqueued (``release_grads=True``).  ``delay_updates=True`` applies each
    update one step late (weights one step stale, as the reference and
    DeepSpeed's delayed parameter update); ``flush()`` applies what is pending.
    The update kernel then writes each parameter the weight of its master from
    before the update, so the stale weights take no memory or copies of their own.

    Args follow the reference (optimizer.py:126-216): ``lr``, ``betas``, ``eps``,
    ``weight_decay`` as in torch.optim.AdamW; ``precision`` 'fp32' | 'bf16' | 'fp8'
    moment storage; ``master_precision`` 'fp32' | 'fp24'; ``stochastic_rounding``;
    ``seed``; ``release_grads``; ``overlap_writeback``; ``small_param_threshold``;
    ``delay_updates``; ``delay_warmup_steps``; ``accumulation_steps``.  Accepted and
    ignored (host-only in the reference): ``numa_aware``, ``num_threads``,
    ``chunk_size``, ``transfer_buffer_mb``, ``gpu_state_budget``, ``autotune``.
    ``backend``: 'auto' or 'native' (both the HIP kernel); 'torch' is refused --
    there is no second implementation to switch to.

    HIP-specific: ``state_layout`` -- 'auto' (default) keeps each parameter's master and
    moments interleaved where a layout for its precision exists (AdamW with BF16 moments:
    16 bytes per pair of elements; AdamW with FP8 moments: one 768-byte record per
    128-element block, block scales apart; Lion with a BF16 moment: one 1536-byte record per
    256 elements), which stream faster from HBM than separate arrays; 'separate' keeps the
    reference's arrays; values, rounding and checkpoints are identical either way.
    ``double_buffer`` -- interleaved BF16 state alternates between two buffers (reads and
    writes go to different memory), at 8 (Lion 6) more bytes per parameter; FP8 records are
    updated in place.
    ``update_stream`` -- 'current' (default): each update runs on the stream current where it is
    enqueued, in order with the backward kernels around it (in a hook, right after the kernels
    that produced its gradient); 'side': on a side stream of the optimizer's own, overlapping
    the rest of the backward pass, each hooked update launched when the next hooked module's
    backward starts (``_LaunchPoints``).  Both give the same bytes.  The update and the
    backward's kernels each stream HBM near its limit, so side by side they share it at close to
    1:1 and the events between the streams cost time of their own: in-order is the faster form
    (the 24-layer 2048/8192 MLP: 0.5-1 ms per step).
    """

    _algorithm = "adamw"

    def __init__(
        self,
        params: Iterable[torch.Tensor] | Iterable[dict[str, Any]],
        lr: float = 1e-3,
        betas: tuple[float, float] = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 1e-2,
        *,
        precision: str = "fp32",
        stochastic_rounding: bool = True,
        backend: str = "auto",
        numa_aware: bool = True,
        num_threads: int | None = None,
        chunk_size: int | None = None,
        release_grads: bool = True,
        overlap_writeback: bool = True,
        autotune: bool | AutoTuneConfig = False,
        seed: int = 0,
        small_param_threshold: int = 65536,
        delay_updates: bool = False,
        delay_warmup_steps: int = 0,
        accumulation_steps: int = 1,
        transfer_buffer_mb: int | None = None,
        gpu_state_budget: int | str | None = None,
        master_precision: str = "fp32",
        state_layout: str = "auto",
        double_buffer: bool = False,
        update_stream: str = "current",
    ):
        _check_arguments(self._algorithm, lr, betas, eps, weight_decay, delay_warmup_steps, accumulation_steps,
                         chunk_size, transfer_buffer_mb, gpu_state_budget, backend)
        self.precision = canonical_precision(precision)
        self.master_precision = canonical_master_precision(master_precision)
        self.gpu_state_budget = gpu_state_budget or None   # every byte of state is on the GPU already
        self.release_grads = release_grads
        self.small_param_threshold = small_param_threshold
        self.accumulation_steps = accumulation_steps
        self.delay_updates = delay_updates
        self.delay_warmup_steps = delay_warmup_steps
        self.last_step_stats: StepStats | None = None
        self._registry = _Registry()
        self._window = _StepWindow(accumulation_steps)
        self._hooks = _HookSet(self._on_grad_ready)
        self._points = _LaunchPoints(self._launch_deferred)
        self._deferred: list[tuple[ParamSlot, torch.Tensor]] = []   # hooked updates waiting for a launch point
        self._end_queued = False     # the current backward pass launches what is left at its end
        self._autotune_log: list[str] = []
        if autotune:
            self._autotune_log.append("autotune: nothing to tune on the GPU (no host threads, one kernel launch)")

        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))

        self._engine = UpdateEngine(
            precision=self.precision, algorithm=self._algorithm, stochastic_rounding=stochastic_rounding,
            seed=seed, overlap_writeback=overlap_writeback, timing=bool(autotune),
            master_precision=self.master_precision, delay_capable=delay_updates, state_layout=state_layout,
            double_buffer=double_buffer, update_stream=update_stream)
        self._engine.delay = delay_updates and delay_warmup_steps == 0
        self._finalizer = weakref.finalize(self, UpdateEngine.close, self._engine)
        self._registry.batch_small(small_param_threshold)

    # Slots in index order and by parameter (names the tests and tools read).
    @property
    def _ordered(self) -> list[ParamSlot]:
        return self._registry.ordered

    @property
    def _slots(self) -> dict[torch.Tensor, ParamSlot]:
        return self._registry.by_param

    @property
    def _small_groups(self) -> list[SmallGroup]:
        return self._registry.small

    # ---------------------------------------------------------------- groups

    def add_param_group(self, param_group: dict[str, Any]) -> None:
        """Every new parameter takes the next index, its rounding stream (optimizer.py:221-237)."""
        super().add_param_group(param_group)
        group = self.param_groups[-1]
        added = [self._registry.register(p, group) for p in group["params"]]
        if self._hooks.active:
            self._hooks.add(s.param for s in added if s.param.requires_grad)

    def _regroup(self) -> None:
        """Point every slot at its group dict again (load_state_dict replaces the dicts)."""
        for group in self.param_groups:
            for p in group["params"]:
                self._registry.by_param[p].group = group

    # ------------------------------------------------------------ async mode

    def attach_hooks(self, model: torch.nn.Module | None = None) -> "AdamBridge":
        """Update each parameter as soon as its gradient is ready (optimizer.py:255-269): the
        parameters of ``model`` (default: all) that require gradients and are not small."""
        if not self._hooks.active:
            targets = self._registry.hook_targets(None if model is None else model.parameters())
            self._hooks.add(targets)
            self._hooks.active = True
            self._engine.hooked_slots = [self._registry.by_param[p] for p in targets]
            if model is not None and self._engine.apart:   # launch points: each owner's backward start
                ids = {id(p) for p in targets}
                self._points.add(m for m in model.modules() if any(id(p) in ids for p in m.parameters(recurse=False)))
        return self

    def detach_hooks(self) -> None:
        self._hooks.clear()
        self._points.clear()

    @property
    def _hooked(self) -> bool:
        return self._hooks.active

    def no_sync(self):
        """Accumulate gradients without updating (every micro-batch but the last): a context manager."""
        return self._window.suppress()

    def _on_grad_ready(self, p: torch.Tensor) -> None:
        """The hook (optimizer.py:291-304): update ``p`` with this gradient, unless the step window says
        otherwise -- launched at the next launch point of this backward pass when its forward
        registered them (_LaunchPoints), else now."""
        if p.grad is None or not self._window.hook_may_update():
            return
        slot = self._registry.by_param[p]
        if not self._points.armed:
            self._submit([slot], [p.grad], hooked=True, release=self.release_grads)
            return
        self._check_submission([slot], [p.grad])
        self._deferred.append((slot, p.grad))
        slot.submitted = True
        if self.release_grads:
            p.grad = None   # the update holds the gradient until it is launched
        if not self._end_queued:   # whatever no later launch point takes is launched when the pass ends
            torch.autograd.Variable._execution_engine.queue_callback(self._end_of_backward)
            self._end_queued = True

    def _launch_deferred(self) -> None:
        """Launch the deferred hooked updates (one launch per device), ordered after the work enqueued
        so far on the current stream."""
        todo, self._deferred = self._deferred, []
        if todo:
            try:
                self._engine.update([s for s, _ in todo], [g for _, g in todo], hooked=True)
            except Exception as exc:
                raise RuntimeError(f"adambridge update failed: {exc}") from exc

    def _end_of_backward(self) -> None:
        self._end_queued = False
        self._points.armed = False   # the next forward registers new launch points
        self._launch_deferred()

    @staticmethod
    def _check_submission(slots: list[ParamSlot], grads: list[torch.Tensor]) -> None:
        if any(s.submitted for s in slots):
            raise RuntimeError(
                "AdamBridge: parameter received a second gradient before step_sync(); "
                "run extra backward passes inside optimizer.no_sync() to accumulate gradients")
        if any(g.is_sparse for g in grads):
            raise RuntimeError("AdamBridge does not support sparse gradients")

    def _submit(self, slots: list[ParamSlot], grads: list[torch.Tensor], hooked: bool, release: bool) -> None:
        """One launch for ``slots`` (optimizer.py:310-321, batched)."""
        self._check_submission(slots, grads)
        try:
            self._engine.update(slots, grads, hooked=hooked)
        except Exception as exc:   # surfaced as the reference surfaces its workers' errors (engine.py:1150-1158)
            raise RuntimeError(f"adambridge update failed: {exc}") from exc
        for slot in slots:
            slot.submitted = True
            if release:
                slot.param.grad = None

    def step_sync(self) -> StepStats:
        """Close the step (optimizer.py:332-355): update what the hooks left -- the small parameters,
        and with gradient accumulation any parameter whose window the step cut short -- then order
        every update before subsequent work on the current stream (a stream wait, not a host wait)."""
        self._launch_deferred()   # normally launched by their backward pass already
        self._points.armed = False
        with self._window.closing(self._registry):
            if not self._window.suppressed:
                self._update_leftovers()
            stats = self._engine.finish_step()
        self.last_step_stats = stats
        if self.delay_updates and self._window.closed >= self.delay_warmup_steps:
            self._engine.delay = True   # the warm-up steps are over (optimizer.py:349-350)
        return stats

    def _update_leftovers(self) -> None:
        """What the hooks did not update: with gradient accumulation, the parameters whose window the
        step cut short; the small parameters, one launch per device."""
        if self.accumulation_steps > 1:
            late = self._registry.pending(include_small=False)
            if late:
                self._submit(late, [s.param.grad for s in late], hooked=False, release=False)
        release = self.release_grads and self._hooks.active
        for batch in self._registry.small:
            live = [s for s in batch.slots if not s.submitted and s.param.grad is not None]
            if live:
                self._submit(live, [s.param.grad for s in live], hooked=self._hooks.active, release=release)

    def flush(self) -> None:
        """Apply every pending (delayed) update to the parameters (optimizer.py:432-436)."""
        self._engine.flush()

    # ------------------------------------------------------------- sync mode

    @torch.no_grad()
    def step(self, closure: Callable[[], torch.Tensor] | None = None):
        """Update every parameter that has a gradient and no update yet this step -- all of them in one
        launch per device -- then :meth:`step_sync` (optimizer.py:440-451)."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        todo = self._registry.pending()
        if todo:
            self._submit(todo, [s.param.grad for s in todo], hooked=False, release=False)
        self.step_sync()
        return loss

    # ------------------------------------------------------------- precision

    def set_precision(self, precision: str) -> None:
        """Re-encode every moment in another precision, between steps (optimizer.py:453-463)."""
        precision = canonical_precision(precision)
        self._engine.wait()
        if precision == self.precision:
            return
        self._engine.rebuild([s for s in self._ordered if s.initialized], precision)
        self._engine.precision = self.precision = precision

    @property
    def autotune_log(self) -> list[str]:
        return list(self._autotune_log)

    def tune_threads(self, numel: int = 1 << 22) -> dict[str, dict[int, float]]:
        """Nothing to tune: the update is one kernel launch per batch (reference optimizer.py:481-487)."""
        return {}

    # ------------------------------------------------------------ inspection

    @property
    def backend(self) -> str:
        """The device code that runs the update, e.g. ``'hip/gfx950'`` (reference: ``'native/<isa>'``)."""
        return self._engine.kernels.backend

    def memory_report(self) -> dict[str, int]:
        """Bytes held by the optimizer, by category (optimizer.py:496-513): ``master``, ``moments``,
        ``staging`` (write-back buffers) and ``reserved`` (arena memory the first gradient hook set
        aside for hooked parameters whose state is not built yet), and their sum ``total``.  Every
        byte is device memory, so ``gpu_state`` -- in the reference the state kept on the GPU apart
        from its host-memory ``total`` -- equals ``total`` here; no host memory is held."""
        master = moments = staging = 0
        for slot in self._ordered:
            if slot.state is None:
                continue
            a, b = slot.state.footprint()
            master, moments = master + a, moments + b
            staging += 0 if slot.out is None else slot.out.nbytes
        reserved = sum(t.nbytes for bufs in self._engine._reserved.values() for t in bufs)
        total = master + moments + staging + reserved
        return {"master": master, "moments": moments, "staging": staging, "reserved": reserved, "total": total,
                "gpu_state": total}

    def expected_bytes_per_param(self) -> float:
        return bytes_per_param(self.precision, 1 if self._algorithm == "lion" else 2, master=self.master_precision)

    def master_params(self) -> list[torch.Tensor | None]:
        """FP32 master copies (``None`` before a parameter's first update; decoded for FP24 and the
        interleaved layouts).  Waits for enqueued updates."""
        self._engine.wait()
        return [None if s.state is None else s.state.master_fp32() for s in self._ordered]

    # ------------------------------------------------------------ checkpoint

    def state_dict(self) -> dict[str, Any]:
        """The reference's checkpoint (optimizer.py:525-544), after applying pending delayed updates so
        that the model's weights match the saved masters.  States in the reference's separate arrays
        are exported as their own device tensors; interleaved states are gathered into the reference's
        arrays, on the device when it has room for all of them, else parameter by parameter into host
        memory (then the device holds one parameter's copy at a time)."""
        self._engine.flush()
        self._engine.wait()
        out = super().state_dict()
        host = self._export_to_host()
        out["state"] = {s.index: {"step": s.step, **s.state.export(host=host and s.state.gathers)}
                        for s in self._ordered if s.state is not None}
        out["adambridge"] = {"precision": self.precision, "master_precision": self.master_precision, "format": 1,
                             "algorithm": self._algorithm}
        return out

    _EXPORT_MARGIN = 1 << 30   # device bytes left free when a checkpoint is gathered on the device

    def _export_to_host(self) -> bool:
        """True if gathering every interleaved state's checkpoint arrays on its device would not fit in
        the memory free there (the driver's free memory plus what torch holds cached and unused)."""
        need: dict[torch.device, int] = {}
        for slot in self._ordered:
            if slot.state is not None and slot.state.gathers:
                need[slot.state.device] = need.get(slot.state.device, 0) + slot.state.export_bytes()
        for device, nbytes in need.items():
            free = torch.cuda.mem_get_info(device)[0]
            free += torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device)
            if nbytes + self._EXPORT_MARGIN > free:
                return True
        return False

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        """An AdamBridge / LionBridge checkpoint, or a torch.optim.AdamW one, moments converted to this
        optimizer's precision (optimizer.py:546-602).  Nothing changes unless all of it is valid."""
        self._engine.discard_pending()
        reader = _CheckpointReader(state_dict, self._ordered, self._algorithm == "lion")
        super().load_state_dict({"state": {}, "param_groups": state_dict["param_groups"]})
        self._regroup()
        keys = (("m", "exp_avg"),) if self._algorithm == "lion" else (("m", "exp_avg"), ("v", "exp_avg_sq"))
        slots, masters, moments = [], [], []
        with torch.no_grad():
            for index, entry in reader.entries.items():
                slot = self._ordered[index]
                slot.step = int(entry["step"])
                slots.append(slot)
                masters.append(entry.get("master"))
                moments.append({role: reader.moment(entry[key], slot.numel, role, self.precision, slot.param.device)
                                for role, key in keys})
        self._engine.rebuild(slots, self.precision, masters, moments)

    def close(self) -> None:
        """Apply pending delayed updates and release the engine (optimizer.py:604-612)."""
        self.detach_hooks()
        if self._finalizer.detach() is None:   # closed before
            return
        try:
            self._engine.flush()
        finally:
            self._engine.close()


OptiComputeAdamW = AdamBridge


class LionBridge(AdamBridge):
    r"""Lion (Chen et al., 2023) with the same HBM state, kernel and pipeline as :class:`AdamBridge`::

        c = beta1 * m + (1 - beta1) * g
        p = p * (1 - lr * weight_decay) - lr * sign(c)
        m = beta2 * m + (1 - beta2) * g

    One moment instead of two.  Every keyword of :class:`AdamBridge` except ``eps``
    applies; the moment is saved as ``exp_avg`` (optimizer.py:628-659).
    """

    _algorithm = "lion"

    def __init__(self, params, lr: float = 1e-4, betas: tuple[float, float] = (0.9, 0.99),
                 weight_decay: float = 0.0, **kwargs):
        if "eps" in kwargs:
            raise TypeError("LionBridge has no eps")
        super().__init__(params, lr=lr, betas=betas, eps=0.0, weight_decay=weight_decay, **kwargs)
