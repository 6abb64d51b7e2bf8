"""AdamBridge / OptiComputeAdamW / LionBridge with the optimizer state in HBM.

Same constructor, methods and checkpoint format as the reference's
``adambridge/optimizer.py`` (cited per method); what differs is where the
state lives and what updates it.  The FP32 (or FP24) master weights, the
moments and the FP8 block scales are device tensors next to each parameter,
and one fused HIP kernel launch (libadambridge_hip.so) updates a whole batch of
parameters in a single pass over HBM, writing the new working weights into
``p.data``.

Numerically this is torch.optim.AdamW (decoupled weight decay, bias
correction, the same operation order) with the reference kernel's exact
rounding: results are bit-identical to the reference's native CPU kernel on
the same inputs (AVX-512 rounding by default, see ``HipKernels.set_simd_level``).

Host-side knobs of the reference that have nothing to act on here -- NUMA
placement, thread counts, PyTorch-kernel chunk size, the pinned transfer ring,
the GPU state budget, the CPU thread auto-tuner -- are accepted and validated
as the reference validates them, and otherwise ignored.
"""

from __future__ import annotations

import contextlib
import logging
import weakref
from typing import Any, Callable, Iterable

import torch

from . import _hip
from .engine import ParamSlot, SmallGroup, StepStats, UpdateEngine
from .precision import (FP32Store, PackedMaster, RecordMaster, _checked, bytes_per_param, canonical_master_precision,
                        canonical_precision, check_master_state, load_master_, make_store, store_from_state_dict)

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


class AdamBridge(torch.optim.Optimizer):
    r"""AdamW whose state lives in GPU memory and is updated by one fused HIP kernel.

    **Synchronous** -- a drop-in replacement for any optimizer::

        loss.backward()
        opt.step()          # one kernel launch updates every parameter with a gradient
        opt.zero_grad()

    **Layer-wise asynchronous** -- each update overlaps the rest of the backward pass::

        opt.attach_hooks(model)
        loss.backward()     # every parameter is updated on a side stream as soon as its gradient is ready
        opt.step_sync()     # the next forward pass (on the current stream) sees the new weights

    In asynchronous mode gradients are released as soon as their update is
    enqueued (``release_grads=True``).  ``delay_updates=True`` applies each
    update one step late (weights one step stale, as the reference and
    DeepSpeed's delayed parameter update); ``flush()`` applies what is pending.

    Args follow the reference (optimizer.py:126-216): ``lr``, ``betas``, ``eps``,
    ``weight_decay`` as in torch.optim.AdamW; ``precision`` 'fp32' | 'bf16' | 'fp8'
    moment storage; ``master_precision`` 'fp32' | 'fp24'; ``stochastic_rounding``;
    ``seed``; ``release_grads``; ``overlap_writeback``; ``small_param_threshold``;
    ``delay_updates``; ``delay_warmup_steps``; ``accumulation_steps``.  Accepted and
    ignored (host-only in the reference): ``numa_aware``, ``num_threads``,
    ``chunk_size``, ``transfer_buffer_mb``, ``gpu_state_budget``, ``autotune``.
    ``backend``: 'auto' or 'native' (both the HIP kernel); 'torch' is refused --
    there is no second implementation to switch to.

    HIP-specific: ``state_layout`` -- 'auto' (default) keeps an FP32 master and BF16
    moments interleaved, 16 bytes per pair of elements, and an FP32 master and FP8
    moments in one 768-byte record per 128-element block (block scales apart), which
    stream faster from HBM than separate arrays; 'separate' keeps the reference's layout;
    values, rounding and checkpoints are identical either way.  ``double_buffer`` -- the
    BF16 interleaved state alternates between two buffers (reads and writes go to
    different memory), at 8 more bytes per parameter; measured at the 7B list it is as
    fast as one buffer (20.8 ms), and 3% faster only where the single buffer landed in
    slow HBM (FP8 records are updated in place).
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
    ):
        # validation as optimizer.py:152-170
        if not 0.0 <= lr:
            raise ValueError(f"invalid learning rate: {lr}")
        if delay_warmup_steps < 0 or accumulation_steps < 1:
            raise ValueError("delay_warmup_steps must be >= 0 and accumulation_steps >= 1")
        if not 0.0 <= eps:
            raise ValueError(f"invalid epsilon: {eps}")
        if not 0.0 <= betas[0] < 1.0 or not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"invalid betas: {betas}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"invalid weight_decay: {weight_decay}")
        if chunk_size is not None and (chunk_size <= 0 or chunk_size % 128):
            raise ValueError("chunk_size must be a positive multiple of 128")
        if transfer_buffer_mb is not None and transfer_buffer_mb < 0:
            raise ValueError("transfer_buffer_mb must be >= 0")
        if not (gpu_state_budget is None or gpu_state_budget == "auto"
                or (isinstance(gpu_state_budget, int) and gpu_state_budget >= 0)):
            raise ValueError("gpu_state_budget must be None, 'auto' or a number of bytes >= 0")
        if gpu_state_budget and self._algorithm != "adamw":
            raise ValueError("gpu_state_budget is only available for AdamW")
        if backend not in ("auto", "native", "torch"):
            raise ValueError("backend must be 'auto', 'native' or 'torch'")
        if backend == "torch":
            raise ValueError("backend='torch' is not available: the update runs only as the fused HIP kernel")
        self.gpu_state_budget = gpu_state_budget or None   # everything is on the GPU already
        self.precision = canonical_precision(precision)
        self.master_precision = canonical_master_precision(master_precision)
        self.release_grads = release_grads
        self.small_param_threshold = small_param_threshold
        self._slots: dict[torch.Tensor, ParamSlot] = {}
        self._ordered: list[ParamSlot] = []
        self._hooks: list[torch.utils.hooks.RemovableHandle] = []
        self._hooked = False
        self._accumulating = 0
        self.accumulation_steps = accumulation_steps
        self._micro = 0
        self._backward_counted = False
        self.delay_updates = delay_updates
        self.delay_warmup_steps = delay_warmup_steps
        self._steps_synced = 0
        self.last_step_stats: StepStats | None = None
        self._autotune = autotune
        self._autotune_log: list[str] = []

        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))

        self._engine = UpdateEngine(
            precision=self.precision, algorithm=self._algorithm, stochastic_rounding=stochastic_rounding,
            seed=seed, overlap_writeback=overlap_writeback, timing=bool(autotune),
            master_precision=self.master_precision, delay_capable=delay_updates, state_layout=state_layout,
            double_buffer=double_buffer)
        self._engine.delay = delay_updates and delay_warmup_steps == 0
        self._finalizer = weakref.finalize(self, UpdateEngine.close, self._engine)
        self._small_groups = self._build_small_groups()
        if autotune:
            self._autotune_log.append("autotune: nothing to tune on the GPU (no host threads, one kernel launch)")

    # ---------------------------------------------------------------- groups

    def add_param_group(self, param_group: dict[str, Any]) -> None:
        """optimizer.py:221-237: every parameter gets the next index (its rounding stream)."""
        super().add_param_group(param_group)
        group = self.param_groups[-1]
        for p in group["params"]:
            if p.is_sparse:
                raise ValueError("AdamBridge does not support sparse parameters")
            slot = ParamSlot(len(self._ordered), p, group)
            self._slots[p] = slot
            self._ordered.append(slot)
            if self._hooked and p.requires_grad:
                self._hooks.append(p.register_post_accumulate_grad_hook(self._hook()))

    def _build_small_groups(self) -> list[SmallGroup]:
        """Small GPU parameters, by device: no hook, one batched launch at step_sync (optimizer.py:239-246)."""
        by_dev: dict[torch.device, list[ParamSlot]] = {}
        for slot in self._ordered:
            p = slot.param
            if p.is_cuda and p.requires_grad and slot.numel < self.small_param_threshold:
                by_dev.setdefault(p.device, []).append(slot)
        return [SmallGroup(slots) for slots in by_dev.values()]

    def _rebind_groups(self) -> None:
        for group in self.param_groups:
            for p in group["params"]:
                self._slots[p].group = group

    # ------------------------------------------------------------ async mode

    def attach_hooks(self, model: torch.nn.Module | None = None) -> "AdamBridge":
        """Update each parameter as soon as its gradient is ready (optimizer.py:255-269)."""
        if self._hooked:
            return self
        wanted = None if model is None else {id(p) for p in model.parameters()}
        hook = self._hook()
        for slot in self._ordered:
            p = slot.param
            if p.requires_grad and slot.small is None and (wanted is None or id(p) in wanted):
                self._hooks.append(p.register_post_accumulate_grad_hook(hook))
        self._hooked = True
        return self

    def _hook(self):
        """Opaque to TorchDynamo, like the reference (optimizer.py:271-274)."""
        return torch.compiler.disable(self._on_grad_ready)

    def detach_hooks(self) -> None:
        for h in self._hooks:
            h.remove()
        self._hooks.clear()
        self._hooked = False

    @contextlib.contextmanager
    def no_sync(self):
        """Accumulate gradients without updating (all but the last micro-batch)."""
        self._accumulating += 1
        try:
            yield
        finally:
            self._accumulating -= 1

    def _on_grad_ready(self, p: torch.Tensor) -> None:
        """optimizer.py:291-304."""
        if self._accumulating or p.grad is None:
            return
        if self.accumulation_steps > 1:
            if not self._backward_counted:
                self._backward_counted = True
                torch.autograd.Variable._execution_engine.queue_callback(self._end_of_backward)
            if self._micro + 1 < self.accumulation_steps:
                return
        self._submit([self._slots[p]], [p.grad], hooked=True, release=self.release_grads)

    def _end_of_backward(self) -> None:
        self._micro += 1
        self._backward_counted = False

    def _submit(self, slots: list[ParamSlot], grads: list[torch.Tensor], hooked: bool, release: bool) -> None:
        """optimizer.py:310-321, batched: one launch for ``slots``."""
        for slot, grad in zip(slots, grads):
            if slot.submitted:
                raise RuntimeError(
                    "AdamBridge: parameter received a second gradient before step_sync(); "
                    "run extra backward passes inside optimizer.no_sync() to accumulate gradients")
            if grad.is_sparse:
                raise RuntimeError("AdamBridge does not support sparse gradients")
        try:
            self._engine.update(slots, grads, hooked=hooked, grads_kept=not release)
        except Exception as exc:   # surfaced like the reference's worker errors (engine.py:1150-1158)
            raise RuntimeError(f"adambridge update failed: {exc}") from exc
        for slot in slots:
            slot.submitted = True
            if release:
                slot.param.grad = None

    def _flush_small(self, release: bool) -> None:
        """The small parameters' updates, one launch per device (optimizer.py:323-330)."""
        for group in self._small_groups:
            live = [s for s in group.slots if not s.submitted and s.param.grad is not None]
            if live:
                self._submit(live, [s.param.grad for s in live], hooked=self._hooked, release=release)

    def step_sync(self) -> StepStats:
        """Update the small parameters and order every update of this step before subsequent
        work on the current stream -- a stream wait, not a host wait.  With delayed updates, only
        the write-backs are ordered (optimizer.py:332-355)."""
        try:
            if not self._accumulating:
                if self.accumulation_steps > 1:
                    self._submit_remaining()  # a window cut short: hooks have not fired
                self._flush_small(release=self.release_grads and self._hooked)
            stats = self._engine.finish_step()
        finally:
            for slot in self._ordered:
                slot.submitted = False
            self._micro = 0
        self.last_step_stats = stats
        self._steps_synced += 1
        if self.delay_updates and self._steps_synced >= self.delay_warmup_steps:
            self._engine.delay = True
        return stats

    def _submit_remaining(self, release: bool = False) -> None:
        todo = [s for s in self._ordered
                if not s.submitted and s.small is None and s.param.grad is not None]
        if todo:
            self._submit(todo, [s.param.grad for s in todo], hooked=False, release=release)

    def flush(self) -> None:
        """Apply every pending (delayed) update to the parameters (optimizer.py:432-436)."""
        self._engine.flush()

    # ------------------------------------------------------------- sync mode

    @torch.no_grad()
    def step(self, closure: Callable[[], torch.Tensor] | None = None):
        """Update every parameter that has a gradient and was not updated by a hook this iteration
        -- all of them in one kernel launch -- then :meth:`step_sync` (optimizer.py:440-451)."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        todo = [s for s in self._ordered if not s.submitted and s.param.grad is not None]
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
        self._engine.precision = precision
        for slot in self._ordered:
            if slot.initialized:
                self._engine.convert_moments(slot, precision)
        self.precision = precision

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
        """Device bytes held by the optimizer, by category (optimizer.py:496-513)."""
        report = {"master": 0, "moments": 0, "staging": 0}
        for slot in self._ordered:
            if not slot.initialized:
                continue
            if not slot.in_place:
                report["master"] += slot.master.nbytes
            report["moments"] += slot.m.nbytes + (slot.v.nbytes if slot.v is not None else 0)
            if slot.out is not None:
                report["staging"] += slot.out.nbytes
        report["total"] = sum(report.values())
        report["gpu_state"] = report["total"]   # all of it is on the GPU
        return report

    def expected_bytes_per_param(self) -> float:
        return bytes_per_param(self.precision, 1 if self._algorithm == "lion" else 2, master=self.master_precision)

    def master_params(self) -> list[torch.Tensor | None]:
        """FP32 master copies (``None`` before a parameter's first update; decoded for FP24 and
        the interleaved layout).  Waits for enqueued updates."""
        self._engine.wait()
        out = []
        for slot in self._ordered:
            if not slot.initialized:
                out.append(None)
            elif isinstance(slot.master, FP32Store):
                out.append(slot.master.data)
            else:
                out.append(slot.master.to_fp32())
        return out

    # ------------------------------------------------------------ checkpoint

    def state_dict(self) -> dict[str, Any]:
        """Applies pending delayed updates first; the reference's layout (optimizer.py:525-544)."""
        self._engine.flush()
        self._engine.wait()
        sd = super().state_dict()
        sd["state"] = {}
        for slot in self._ordered:
            if not slot.initialized:
                continue
            if isinstance(slot.master, (FP32Store, PackedMaster, RecordMaster)):
                master = slot.master.data   # a plain FP32 tensor (interleaved layouts: a contiguous copy)
            else:
                master = slot.master.state_dict()
            st = sd["state"][slot.index] = {"step": slot.step, "master": master, "exp_avg": slot.m.state_dict()}
            if slot.v is not None:
                st["exp_avg_sq"] = slot.v.state_dict()
        sd["adambridge"] = {"precision": self.precision, "master_precision": self.master_precision, "format": 1,
                            "algorithm": self._algorithm}
        return sd

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        """An AdamBridge / LionBridge checkpoint, or a torch.optim.AdamW one (moments converted to this
        optimizer's precision).  Everything is validated before anything changes (optimizer.py:546-602)."""
        self._engine.discard_pending()
        saved = {int(k) if isinstance(k, str) and k.isdigit() else k: v for k, v in state_dict["state"].items()}
        lion = self._algorithm == "lion"
        for index, st in saved.items():
            if isinstance(index, bool) or not isinstance(index, int) or not 0 <= index < len(self._ordered):
                raise ValueError(f"checkpoint state for parameter {index!r}: this optimizer has parameters "
                                 f"0..{len(self._ordered) - 1}")
            numel = self._ordered[index].numel
            if st.get("master") is not None:
                check_master_state(st["master"], numel, f"master weights of parameter {index}")
            for key in ("exp_avg", "exp_avg_sq"):
                if isinstance(st.get(key), torch.Tensor):
                    _checked(st[key], numel, f"{key} of parameter {index}")
            if not lion and "exp_avg_sq" not in st:
                raise ValueError("checkpoint has no exp_avg_sq (saved by LionBridge?); AdamW needs both moments")
        super().load_state_dict({"state": {}, "param_groups": state_dict["param_groups"]})
        self._rebind_groups()
        with torch.no_grad():
            for index, st in saved.items():
                slot = self._ordered[index]
                if not slot.initialized:
                    self._engine.initialize(slot)
                slot.step = int(st["step"])
                if st.get("master") is not None:
                    load_master_(slot.master, st["master"])
                dev = slot.param.device
                self._engine.replace_moments(
                    slot, self._load_store(st["exp_avg"], slot.numel, "m", dev),
                    None if lion else self._load_store(st["exp_avg_sq"], slot.numel, "v", dev))

    def _load_store(self, saved, numel: int, role: str, device):
        if isinstance(saved, torch.Tensor):   # torch.optim.AdamW layout
            return make_store(self.precision, numel, role, init=saved.to(device, torch.float32), device=device)
        store = store_from_state_dict(saved, numel, role, device=device)
        if store.precision != self.precision:
            store = make_store(self.precision, numel, role, init=store.to_fp32(), device=device)
        return store

    def close(self) -> None:
        """Apply pending delayed updates and release the engine (optimizer.py:604-612)."""
        self.detach_hooks()
        if self._finalizer.alive:
            try:
                self._engine.flush()
            finally:
                self._finalizer()


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
