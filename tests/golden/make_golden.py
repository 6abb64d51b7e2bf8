"""Write the golden vectors in this directory from the reference kernel.

The reference's fused update (adambridge/csrc/adambridge_kernels.c) is compiled
from its own source by oracle/Makefile into oracle/_ref/libadambridge_ref.so;
this script drives its exported C entry points (adambridge_multi_apply and
adambridge_multi_step, kernels.c:1611-1641) on seeded inputs covering every
branch of the hot path and stores inputs and outputs:

    vectors.npz   arrays, keys "c<i>.<phase>.<name>" (phase: in, out, or g<k> for
                  the gradient of step k of a multi-step case)
    vectors.json  per-case scalars (dtypes, n, offset, index, step, coefficients
                  or group, the SIMD width whose tail the case pins, steps)

Run in the container that holds the reference tree:

    make -C oracle && python tests/golden/make_golden.py

The reference's storage layouts and its C ABI are the only things relied on;
no reference Python is imported.  The width recorded per case is the vector
width of the ISA the reference ran at (set with adambridge_set_simd_level):
16 = AVX-512, 8 = AVX2, 0 = its scalar level.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent


def specs():
    """(description, kwargs for make_case, width, steps) in a fixed order."""
    out = []
    # every storage/algorithm combination at an odd size with a tail, SR on, bf16 grads and out
    for algo in (O.ADAMW, O.LION):
        for mv in (O.DT_F32, O.DT_BF16, O.DT_FP8):
            for pt in (O.DT_F32, O.DT_F24):
                for sr in (True, False):
                    out.append((f"algo{algo} mv{mv} p{pt} sr{int(sr)}",
                                dict(n=1000 + 37, algorithm=algo, mv_dtype=mv, p_dtype=pt, stochastic=sr), 16, 1))
    # grad / out dtypes
    for gt in (O.DT_F32, O.DT_BF16):
        for ot in (O.DT_NONE, O.DT_F32, O.DT_BF16):
            for mv in (O.DT_F32, O.DT_BF16, O.DT_FP8):
                out.append((f"g{gt} out{ot} mv{mv}", dict(n=300, g_dtype=gt, out_dtype=ot, mv_dtype=mv), 16, 1))
    # sizes around the vector width and the FP8 block
    for n in (1, 15, 16, 17, 127, 128, 129, 255, 257):
        for mv in (O.DT_BF16, O.DT_FP8):
            out.append((f"n{n} mv{mv}", dict(n=n, mv_dtype=mv), 16, 1))
    # other ISAs' tails
    for width in (8, 0):
        for mv in (O.DT_F32, O.DT_BF16, O.DT_FP8):
            out.append((f"width{width} mv{mv}", dict(n=517, mv_dtype=mv), width, 1))
    # element offsets (chunks of a parameter) incl. the 32-bit index wrap, and large param indices
    out.append(("offset wrap bf16", dict(n=700, offset=2**32 - 300, index=12345), 16, 1))
    out.append(("offset chunk fp8", dict(n=700, mv_dtype=O.DT_FP8, offset=128 * 1000, index=7), 16, 1))
    out.append(("offset chunk fp24", dict(n=700, p_dtype=O.DT_F24, offset=2**24, index=3), 16, 1))
    # non-finite and subnormal inputs
    for algo in (O.ADAMW, O.LION):
        for mv in (O.DT_F32, O.DT_BF16, O.DT_FP8):
            out.append((f"special algo{algo} mv{mv}",
                        dict(n=1500, algorithm=algo, mv_dtype=mv, special=True, p_dtype=O.DT_F24 if mv == O.DT_FP8
                             else O.DT_F32), 16, 1))
    # coefficients derived by the kernel from a group and the step (multi_step), several steps in a row
    for mv, algo in ((O.DT_F32, O.ADAMW), (O.DT_BF16, O.ADAMW), (O.DT_FP8, O.ADAMW), (O.DT_BF16, O.LION)):
        out.append((f"multistep algo{algo} mv{mv}",
                    dict(n=1031, mv_dtype=mv, algorithm=algo, explicit=False, index=5, lr=2e-3,
                         weight_decay=0.1 if algo == O.LION else 0.01, betas=(0.9, 0.99 if algo == O.LION else 0.999),
                         seed=42), 16, 6))
    return out


def main():
    if not O.reference_available():
        raise SystemExit("oracle/_ref/libadambridge_ref.so is missing: run `make -C oracle` with the reference tree")
    rng = np.random.default_rng(20261201)
    arrays: dict[str, np.ndarray] = {}
    meta = []
    for i, (desc, kw, width, steps) in enumerate(specs()):
        case = O.make_case(rng, **kw)
        entry = {"desc": desc, "n": case.n, "algorithm": case.algorithm, "mv_dtype": case.mv_dtype,
                 "p_dtype": case.p_dtype, "g_dtype": case.g_dtype, "out_dtype": case.out_dtype,
                 "offset": case.offset, "index": case.index, "step": case.step, "width": width,
                 "steps": steps, "special": bool(kw.get("special", False)),
                 "hparams": case.hparams, "group": case.group}
        for k, a in case.arrays.items():
            if k != "g":
                arrays[f"c{i}.in.{k}"] = a
        state = case
        for k in range(steps):
            if k > 0:  # a fresh gradient for every later step
                g = (rng.normal(0.0, 1.0, case.n) * 1e-3).astype(np.float32)
                state.arrays["g"] = O.bf16_bits(g) if case.g_dtype == O.DT_BF16 else g
            arrays[f"c{i}.g{k}"] = state.arrays["g"].copy()
            state = O.run(state, "ref", width)
            state.step += 1
        for k, a in state.arrays.items():
            if k != "g":
                arrays[f"c{i}.out.{k}"] = a
        meta.append(entry)
    np.savez_compressed(OUT / "vectors.npz", **arrays)
    (OUT / "vectors.json").write_text(json.dumps(meta, indent=1))
    size = (OUT / "vectors.npz").stat().st_size
    print(f"wrote {len(meta)} cases, vectors.npz {size / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
