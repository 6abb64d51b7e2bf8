"""The C ABI from a plain C11 program (tests/c_client/abi_client.c), no Python in between.

CPU: the header compiles as C11 under -Wall -Wextra -Werror, the struct sizes hold at compile
time, and the program links against the in-tree library and gets the reference's argument
codes (kernels.c:1537-1553) without touching a device.

GPU: the program built by build() (tests/c_client/Makefile) allocates device buffers with
hipMalloc, creates a pool bound to its own HIP stream, and calls adambridge_multi_step for three
steps over three segments at once: AdamW with BF16 moments and a scalar tail; AdamW with FP8
moments, an FP24 master and stochastic rounding at element offset 384; Lion with zero
gradients.  Then one adambridge_multi_apply with explicit coefficients, and one
adambridge_fused_adamw on the first tensor at an element offset.  After every call every buffer
must equal, byte for byte, the same update computed by the CPU oracle (oracle/liboracle.so) on
host copies, and a call with one invalid segment must change nothing.
"""

import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CLIENT_DIR = ROOT / "tests" / "c_client"
CLIENT = CLIENT_DIR / "abi_client"
LIB = ROOT / "adambridge_amd" / "libadambridge_hip.so"
ORACLE = ROOT / "oracle" / "liboracle.so"


def test_c_client_compiles_and_checks_arguments(tmp_path):
    assert LIB.exists(), "libadambridge_hip.so is not built: run __graft_entry__.build()"
    exe = tmp_path / "abi_client"
    build = subprocess.run(["make", "-s", "-B", "-C", str(CLIENT_DIR), f"OUT={exe}"], capture_output=True, text=True)
    if build.returncode != 0:
        pytest.fail(build.stdout + build.stderr)
    run = subprocess.run([str(exe), "abi"], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "PASSED (0 failures)" in run.stdout


@pytest.mark.gpu
def test_c_client_updates_match_oracle():
    assert CLIENT.exists(), "tests/c_client/abi_client is not built: run __graft_entry__.build()"
    assert ORACLE.exists(), "oracle/liboracle.so is not built: run __graft_entry__.build()"
    print(f"running {CLIENT} gpu {ORACLE}", flush=True)
    run = subprocess.run([str(CLIENT), "gpu", str(ORACLE)], capture_output=True, text=True, timeout=120)
    print(run.stdout, flush=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.count("identical to the oracle") == 5   # 3 x multi_step, multi_apply, fused_adamw
