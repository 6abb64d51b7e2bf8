"""The native-kernel module of the reference's API (adambridge/native.py), over the HIP library.

Code written against ``adambridge.native`` finds the same names here:

- ``load()`` / ``available()`` / ``load_error()``;
- ``library_path()`` / ``cache_dir()`` / ``build()`` / ``BuildError``;
- ``StepCoefficients`` (the per-step scalars of ``multi_apply``);
- ``NativeKernels`` (here :class:`adambridge_amd._hip.HipKernels`), ``Group``, ``Segment``.

They work on ``libadambridge_hip.so``, built in-tree for gfx950 by hipcc.

One difference is deliberate. The reference falls back to PyTorch kernels when its library is
missing, and ``ADAMBRIDGE_DISABLE_NATIVE`` selects that fallback. Here there is no second
implementation. ``load()`` still reports a missing library as ``None`` with the reason in
``load_error()``, as the reference does, and ``ADAMBRIDGE_DISABLE_NATIVE`` has no effect. The
optimizer itself raises when the library cannot be loaded.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass
from pathlib import Path

from . import _hip
from . import build as _build

__all__ = ["BuildError", "Group", "Segment", "StepCoefficients", "NativeKernels", "library_path", "cache_dir",
           "build", "load", "available", "load_error"]

Group = _hip.Group
Segment = _hip.Segment
_HParams = _hip.HParams
NativeKernels = _hip.HipKernels


class BuildError(RuntimeError):
    """The library could not be compiled (reference native.py:54-56)."""


def library_path() -> Path:
    """Where the library is loaded from: next to this package (reference native.py:172-174)."""
    return _hip.LIB_PATH


def cache_dir() -> Path:
    """The directory holding the built library (the reference keeps a per-user build cache;
    this build compiles in-tree)."""
    return _hip.LIB_PATH.parent


def build(force: bool = False, verbose: bool = False) -> Path:
    """Compile the library with hipcc for gfx950 (reference native.py:209-241).  It always
    recompiles, so ``force`` changes nothing."""
    try:
        return _build.build(verbose=verbose)
    except (RuntimeError, OSError) as exc:
        raise BuildError(str(exc)) from exc


@dataclass
class StepCoefficients:
    """Per-step scalars for ``multi_apply`` (reference native.py:243-270), in double precision
    like the reference's (the library's own ``multi_step`` derives them in C++, identically)."""

    beta1: float
    beta2: float
    decay: float
    step_size: float
    inv_sqrt_bc2: float
    eps: float

    @classmethod
    def for_step(cls, lr: float, beta1: float, beta2: float, eps: float, weight_decay: float,
                 step: int) -> "StepCoefficients":
        bc1 = 1.0 - beta1 ** step
        bc2 = 1.0 - beta2 ** step
        return cls(beta1=beta1, beta2=beta2, decay=1.0 - lr * weight_decay, step_size=lr / bc1,
                   inv_sqrt_bc2=1.0 / bc2 ** 0.5, eps=eps)

    @classmethod
    def for_lion(cls, lr: float, beta1: float, beta2: float, weight_decay: float) -> "StepCoefficients":
        """No bias correction: the step is ``lr * sign(c)``."""
        return cls(beta1=beta1, beta2=beta2, decay=1.0 - lr * weight_decay, step_size=lr, inv_sqrt_bc2=1.0, eps=0.0)


_lock = threading.Lock()
_load_error: str | None = None


def load(build_if_missing: bool = True) -> NativeKernels | None:
    """The loaded library (built first if it is missing and ``build_if_missing``); ``None`` if it
    cannot be had, with the reason in :func:`load_error` (reference native.py:443-461)."""
    global _load_error
    with _lock:
        try:
            if not library_path().exists():
                if not build_if_missing:
                    return None
                build()
            kernels = _hip.load()
            _load_error = None
            return kernels
        except (RuntimeError, OSError) as exc:
            _load_error = str(exc)
            return None


def available() -> bool:
    return load() is not None


def load_error() -> str | None:
    return _load_error
