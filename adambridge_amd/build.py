"""Build libadambridge_hip.so (gfx950) in-tree with hipcc.

    python -m adambridge_amd.build

Flags: -O3; -ffp-contract=off (products and sums round separately except where
the source writes an FMA, as the reference's kernels do); HIP's default
correctly rounded FP32 division and sqrt and kept denormals (no fast-math);
packed FP32 instructions disabled for device code.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = PKG / "csrc" / "adambridge_hip.hip"
DEPS = [SRC, PKG / "csrc" / "abh_device.hpp", PKG / "csrc" / "abh_host.inc", ROOT / "include" / "adambridge_hip.h"]
LIB = PKG / "libadambridge_hip.so"
ARCH = os.environ.get("ADAMBRIDGE_HIP_ARCH", "gfx950")


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def command(out: Path = LIB) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-ffp-contract=off", "-fno-fast-math", "-fvisibility=hidden",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wall", "-Wno-unused-result",
            f"-I{ROOT / 'include'}", str(SRC), "-o", str(out)]


def build(verbose: bool = False) -> Path:
    """Compile the library (always; a stale library is never reused)."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
