"""Run oracle ``Case``s through the HIP library (test helper).

The case's numpy arrays are copied to device tensors, one multi_apply (or
multi_step) call of libadambridge_hip.so updates them on the current stream,
and the results come back as a new Case for comparison with the oracle.
"""

from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np
import torch

from oracle import oracle as O

from adambridge_amd import _hip

GOLDEN = Path(__file__).resolve().parent / "golden"
WIDTH_LEVEL = {16: "avx512", 8: "avx2", 0: "scalar"}


def to_device(a: np.ndarray, device="cuda") -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).to(device)
    return torch.from_numpy(a.copy()).to(device)


def from_device(t: torch.Tensor, like: np.ndarray) -> np.ndarray:
    return t.cpu().numpy().view(like.dtype).reshape(like.shape)


def hip_segment(case: O.Case, tensors: dict, group: _hip.Group | None) -> _hip.Segment:
    ptr = lambda k: tensors[k].data_ptr() if k in tensors else None  # noqa: E731
    return _hip.Segment(p=ptr("p"), p_lo=ptr("p_lo"), g=ptr("g"), m=ptr("m"), v=ptr("v"), m_scale=ptr("m_scale"),
                        v_scale=ptr("v_scale"), out=ptr("out"),
                        group=ctypes.pointer(group) if group is not None else None, n=case.n, step=case.step,
                        index=case.index, offset=case.offset, g_dtype=case.g_dtype, mv_dtype=case.mv_dtype,
                        out_dtype=case.out_dtype, algorithm=case.algorithm, p_dtype=case.p_dtype)


class Prepared:
    """Device copies of cases, their segments and coefficients, ready for one library call."""

    def __init__(self, cases: list[O.Case], tensors_hook=None, seg_flags: int = 0):
        self.work = [c.copy() for c in cases]
        for c in self.work:
            O.check_sizes(c)   # every buffer covers what the launch will touch, before anything runs
        self.dev = [{k: to_device(a) for k, a in c.arrays.items()} for c in self.work]
        if tensors_hook is not None:
            for i, t in enumerate(self.dev):
                tensors_hook(i, t)
        self.by_group = all(c.group is not None for c in self.work)
        self.groups = [_hip.Group(**{k: c.group[k] for k in ("lr", "beta1", "beta2", "eps", "weight_decay")},
                                  seed=c.group["seed"] & (2**64 - 1), stochastic=int(c.group["stochastic"]))
                       if self.by_group else None for c in self.work]
        self.segs = [hip_segment(c, t, g) for c, t, g in zip(self.work, self.dev, self.groups)]
        for seg in self.segs:
            seg.reserved = seg_flags
        self.arr = _hip.load().segment_array([ctypes.pointer(s) for s in self.segs])
        self.hps = None if self.by_group else [
            _hip.HParams(**{k: c.hparams[k] for k, _ in _hip.HParams._fields_}) for c in self.work]

    def call(self, pool: int | None = None) -> None:
        """multi_step (cases with groups) or multi_apply, on the current stream."""
        kernels = _hip.load()
        kernels.set_stream(torch.cuda.current_stream())
        if self.by_group:
            kernels.multi_step(pool, self.arr)
        else:
            kernels.multi_apply(pool, self.arr, self.hps)

    def collect(self) -> list[O.Case]:
        """The device state copied back into the cases (after a synchronisation)."""
        out = [c.copy() for c in self.work]
        for c, t in zip(out, self.dev):
            for k in list(c.arrays):
                if k in t:
                    c.arrays[k] = from_device(t[k], c.arrays[k])
        return out


def run_hip(cases: list[O.Case], width: int = 16, pool: int | None = None,
            tensors_hook=None, seg_flags: int = 0) -> list[O.Case]:
    """Update copies of ``cases`` in one call of the HIP library; returns them.

    ``tensors_hook(i, tensors)`` may replace device tensors before the call (misalignment tests);
    ``seg_flags`` goes into every segment's ``reserved`` field."""
    prep = Prepared(cases, tensors_hook, seg_flags)
    kernels = _hip.load()
    kernels.set_simd_level(WIDTH_LEVEL[width])
    try:
        prep.call(pool)
        torch.cuda.synchronize()
    finally:
        kernels.set_simd_level(None)
    return prep.collect()


def golden_cases():
    """(meta, input Case, gradients per step, expected Case) for every golden vector."""
    meta = json.loads((GOLDEN / "vectors.json").read_text())
    data = np.load(GOLDEN / "vectors.npz")
    out = []
    for i, m in enumerate(meta):
        arrays = {k.split(".", 2)[2]: data[k] for k in data.files if k.startswith(f"c{i}.in.")}
        expect = {k.split(".", 2)[2]: data[k] for k in data.files if k.startswith(f"c{i}.out.")}
        grads = [data[f"c{i}.g{k}"] for k in range(m["steps"])]
        case = O.Case(n=m["n"], algorithm=m["algorithm"], mv_dtype=m["mv_dtype"], p_dtype=m["p_dtype"],
                      g_dtype=m["g_dtype"], out_dtype=m["out_dtype"], offset=m["offset"], index=m["index"],
                      step=m["step"], arrays=arrays, hparams=m["hparams"], group=m["group"])
        exp = case.copy()
        exp.arrays = expect
        out.append((m, case, grads, exp))
    return out


def run_steps(case: O.Case, grads: list, runner, width: int) -> O.Case:
    """Apply len(grads) consecutive updates with ``runner(cases, width) -> cases``."""
    state = case.copy()
    for g in grads:
        state.arrays["g"] = g.copy()
        state = runner([state], width)[0]
        state.step += 1
    return state


def pack_state(case: O.Case) -> np.ndarray:
    """Separate FP32 master + BF16 moments -> the interleaved layout (pairs x 4 uint32)."""
    n = case.n
    pairs = max(1, (n + 1) // 2)
    out = np.zeros((pairs, 4), np.uint32)
    p = np.zeros(2 * pairs, np.uint32)
    p[:n] = case.arrays["p"].view(np.uint32)
    m = np.zeros(2 * pairs, np.uint32)
    m[:n] = case.arrays["m"]
    v = np.zeros(2 * pairs, np.uint32)
    v[:n] = case.arrays["v"]
    out[:, 0], out[:, 1] = p[0::2], p[1::2]
    out[:, 2] = m[0::2] | (m[1::2] << 16)
    out[:, 3] = v[0::2] | (v[1::2] << 16)
    return out


def unpack_state(case: O.Case, state: np.ndarray) -> None:
    """The interleaved layout -> the case's separate arrays (in place)."""
    n = case.n
    p = np.empty(2 * state.shape[0], np.uint32)
    p[0::2], p[1::2] = state[:, 0], state[:, 1]
    m = np.empty(2 * state.shape[0], np.uint32)
    m[0::2], m[1::2] = state[:, 2] & 0xFFFF, state[:, 2] >> 16
    v = np.empty(2 * state.shape[0], np.uint32)
    v[0::2], v[1::2] = state[:, 3] & 0xFFFF, state[:, 3] >> 16
    case.arrays["p"] = p[:n].view(np.float32).copy()
    case.arrays["m"] = m[:n].astype(np.uint16)
    case.arrays["v"] = v[:n].astype(np.uint16)


def run_hip_packed(cases: list[O.Case], width: int = 16, double_buffer: bool = False,
                   misalign_g: bool = False, seg_flags: int = 0) -> list[O.Case]:
    """Like run_hip for AdamW / FP32 master / BF16 moment cases, through the interleaved layout
    (ADAMBRIDGE_DT_PACKED): pack on the host, one call, unpack the result."""
    kernels = _hip.load()
    work = [c.copy() for c in cases]
    keep, segs = [], []
    by_group = all(c.group is not None for c in work)
    groups = []
    for c in work:
        assert c.algorithm == O.ADAMW and c.mv_dtype == O.DT_BF16 and c.p_dtype == O.DT_F32
        O.check_sizes(c)
        state = torch.from_numpy(pack_state(c).view(np.int32)).cuda()
        dst = torch.full_like(state, -1) if double_buffer else None
        g = to_device(c.arrays["g"])
        if misalign_g:
            buf = torch.empty(g.numel() + 1, dtype=g.dtype, device=g.device)
            buf[1:].copy_(g)
            keep.append(buf)
            g = buf[1:]
        out = to_device(c.arrays["out"]) if "out" in c.arrays else None
        keep += [state, dst, g, out]
        grp = None
        if by_group:
            grp = _hip.Group(**{k: c.group[k] for k in ("lr", "beta1", "beta2", "eps", "weight_decay")},
                             seed=c.group["seed"] & (2**64 - 1), stochastic=int(c.group["stochastic"]))
        groups.append(grp)
        segs.append(_hip.Segment(p=state.data_ptr(), p_lo=dst.data_ptr() if dst is not None else None,
                                 g=g.data_ptr(), m=None, v=None, out=out.data_ptr() if out is not None else None,
                                 group=ctypes.pointer(grp) if grp is not None else None, n=c.n, step=c.step,
                                 index=c.index, offset=c.offset, g_dtype=c.g_dtype, mv_dtype=O.DT_BF16,
                                 out_dtype=c.out_dtype, algorithm=0, p_dtype=_hip.DT_PACKED, reserved=seg_flags))
    arr = kernels.segment_array([ctypes.pointer(s) for s in segs])
    kernels.set_simd_level(WIDTH_LEVEL[width])
    try:
        kernels.set_stream(torch.cuda.current_stream())
        if by_group:
            kernels.multi_step(None, arr)
        else:
            hps = [_hip.HParams(**{k: c.hparams[k] for k, _ in _hip.HParams._fields_}) for c in work]
            kernels.multi_apply(None, arr, hps)
        torch.cuda.synchronize()
    finally:
        kernels.set_simd_level(None)
    it = iter(keep)
    for c in work:
        if misalign_g:
            next(it)
        state, dst, g, out = next(it), next(it), next(it), next(it)
        result = (dst if dst is not None else state).cpu().numpy().view(np.uint32)
        unpack_state(c, result)
        if out is not None:
            c.arrays["out"] = from_device(out, c.arrays["out"])
    return work


def pack_records(case: O.Case) -> np.ndarray:
    """Separate FP32 master + FP8 codes -> ADAMBRIDGE_DT_PACKED_FP8 records (blocks x 768 bytes):
    per block, lane l's elements 8l .. 8l + 7 have their master at 16l (first four) and 256 + 16l
    (last four), their m codes at 512 + 16l and v codes at 520 + 16l."""
    n = case.n
    nb = max(1, -(-n // 128))
    p = np.zeros(nb * 128, np.uint32)
    p[:n] = case.arrays["p"].view(np.uint32)
    rec = np.zeros((nb, 768), np.uint8)
    rec[:, :512] = p.reshape(nb, 16, 2, 4).transpose(0, 2, 1, 3).reshape(nb, 128).view(np.uint8)
    codes = np.zeros((nb, 16, 16), np.uint8)
    for key, lo in (("m", 0), ("v", 8)):
        c = np.zeros(nb * 128, np.uint8)
        src = case.arrays[key]
        c[:min(src.size, nb * 128)] = src[:nb * 128]
        codes[:, :, lo:lo + 8] = c.reshape(nb, 16, 8)
    rec[:, 512:] = codes.reshape(nb, 256)
    return rec


def unpack_records(case: O.Case, rec: np.ndarray) -> None:
    """ADAMBRIDGE_DT_PACKED_FP8 records -> the case's separate master and code arrays (in place)."""
    n, nb = case.n, rec.shape[0]
    p = np.ascontiguousarray(rec[:, :512]).view(np.uint32).reshape(nb, 2, 16, 4).transpose(0, 2, 1, 3).reshape(-1)
    case.arrays["p"] = p[:n].view(np.float32).copy()
    codes = np.ascontiguousarray(rec[:, 512:]).reshape(nb, 16, 16)
    for key, lo in (("m", 0), ("v", 8)):
        size = case.arrays[key].size
        case.arrays[key] = codes[:, :, lo:lo + 8].reshape(-1)[:size].copy()


def pack_f8f24_records(case: O.Case) -> np.ndarray:
    """Separate FP24 master planes + FP8 codes -> ADAMBRIDGE_DT_PACKED_FP8_F24 records (blocks x 640
    bytes): per block, the 128 high halves (bytes 0 .. 255) and the 128 low bytes (256 .. 383) in
    element order, then lane l's m codes at 384 + 16l and v codes at 392 + 16l.  Padding masters
    are set to a fixed pattern so that a test can see the kernel leave them unchanged."""
    n = case.n
    nb = max(1, -(-n // 128))
    hi = np.full(nb * 128, 0xA5A5, np.uint16)
    hi[:n] = case.arrays["p"].view(np.uint16)
    lo = np.full(nb * 128, 0x5A, np.uint8)
    lo[:n] = case.arrays["p_lo"]
    rec = np.zeros((nb, 640), np.uint8)
    rec[:, :256] = hi.reshape(nb, 128).view(np.uint8)
    rec[:, 256:384] = lo.reshape(nb, 128)
    codes = np.zeros((nb, 16, 16), np.uint8)
    for key, k in (("m", 0), ("v", 8)):
        c = np.zeros(nb * 128, np.uint8)
        src = case.arrays[key]
        c[:min(src.size, nb * 128)] = src[:nb * 128]
        codes[:, :, k:k + 8] = c.reshape(nb, 16, 8)
    rec[:, 384:] = codes.reshape(nb, 256)
    return rec


def unpack_f8f24_records(case: O.Case, rec: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """ADAMBRIDGE_DT_PACKED_FP8_F24 records -> the case's separate master planes and codes (in place);
    returns the padding masters' (high halves, low bytes) past n."""
    n, nb = case.n, rec.shape[0]
    hi = np.ascontiguousarray(rec[:, :256]).view(np.uint16).reshape(-1)
    lo = np.ascontiguousarray(rec[:, 256:384]).reshape(-1)
    case.arrays["p"] = hi[:n].view(case.arrays["p"].dtype).copy()
    case.arrays["p_lo"] = lo[:n].copy()
    codes = np.ascontiguousarray(rec[:, 384:]).reshape(nb, 16, 16)
    for key, k in (("m", 0), ("v", 8)):
        size = case.arrays[key].size
        case.arrays[key] = codes[:, :, k:k + 8].reshape(-1)[:size].copy()
    return hi[n:].copy(), lo[n:].copy()


def pack_lion8_records(case: O.Case) -> np.ndarray:
    """Separate FP32 master + FP8 m codes -> ADAMBRIDGE_DT_PACKED_LION_FP8 records (blocks x 640
    bytes): per block the masters as in pack_records (bytes 0 .. 511), then the 128 m codes in
    element order.  Padding masters are set to a fixed pattern so that a test can see the kernel
    leave them unchanged."""
    n = case.n
    nb = max(1, -(-n // 128))
    p = np.full(nb * 128, 0x7F8A5A5A, np.uint32)   # a NaN pattern: any arithmetic on it would show
    p[:n] = case.arrays["p"].view(np.uint32)
    rec = np.zeros((nb, 640), np.uint8)
    rec[:, :512] = p.reshape(nb, 16, 2, 4).transpose(0, 2, 1, 3).reshape(nb, 128).view(np.uint8)
    c = np.zeros(nb * 128, np.uint8)
    src = case.arrays["m"]
    c[:min(src.size, nb * 128)] = src[:nb * 128]
    rec[:, 512:] = c.reshape(nb, 128)
    return rec


def pack_lion8f24_records(case: O.Case) -> np.ndarray:
    """Separate FP24 master planes + FP8 m codes -> ADAMBRIDGE_DT_PACKED_LION_FP8_F24 records (blocks x
    512 bytes): the planes as in pack_f8f24_records, then the 128 m codes in element order."""
    n = case.n
    nb = max(1, -(-n // 128))
    hi = np.full(nb * 128, 0xA5A5, np.uint16)
    hi[:n] = case.arrays["p"].view(np.uint16)
    lo = np.full(nb * 128, 0x5A, np.uint8)
    lo[:n] = case.arrays["p_lo"]
    c = np.zeros(nb * 128, np.uint8)
    src = case.arrays["m"]
    c[:min(src.size, nb * 128)] = src[:nb * 128]
    rec = np.zeros((nb, 512), np.uint8)
    rec[:, :256] = hi.reshape(nb, 128).view(np.uint8)
    rec[:, 256:384] = lo.reshape(nb, 128)
    rec[:, 384:] = c.reshape(nb, 128)
    return rec


def unpack_lion8f24_records(case: O.Case, rec: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """ADAMBRIDGE_DT_PACKED_LION_FP8_F24 records -> the case's master planes and m codes (in place);
    returns the padding masters' (high halves, low bytes) past n."""
    n, nb = case.n, rec.shape[0]
    hi = np.ascontiguousarray(rec[:, :256]).view(np.uint16).reshape(-1)
    lo = np.ascontiguousarray(rec[:, 256:384]).reshape(-1)
    case.arrays["p"] = hi[:n].view(case.arrays["p"].dtype).copy()
    case.arrays["p_lo"] = lo[:n].copy()
    size = case.arrays["m"].size
    case.arrays["m"] = np.ascontiguousarray(rec[:, 384:]).reshape(-1)[:size].copy()
    return hi[n:].copy(), lo[n:].copy()


def unpack_lion8_records(case: O.Case, rec: np.ndarray) -> np.ndarray:
    """ADAMBRIDGE_DT_PACKED_LION_FP8 records -> the case's separate master and m codes (in place);
    returns the padding masters' bits past n."""
    n, nb = case.n, rec.shape[0]
    p = np.ascontiguousarray(rec[:, :512]).view(np.uint32).reshape(nb, 2, 16, 4).transpose(0, 2, 1, 3).reshape(-1)
    case.arrays["p"] = p[:n].view(np.float32).copy()
    size = case.arrays["m"].size
    case.arrays["m"] = np.ascontiguousarray(rec[:, 512:]).reshape(-1)[:size].copy()
    return p[n:].copy()


def run_hip_records(cases: list[O.Case], width: int = 16, misalign_g: bool = False,
                    seg_flags: int = 0, padding: list | None = None) -> list[O.Case]:
    """Like run_hip for FP8 moment cases, through the block-record layouts: AdamW with an FP32 master
    (ADAMBRIDGE_DT_PACKED_FP8) or an FP24 master (ADAMBRIDGE_DT_PACKED_FP8_F24), by the case's
    p_dtype, and Lion with an FP32 or FP24 master (ADAMBRIDGE_DT_PACKED_LION_FP8, _LION_FP8_F24).  Pack
    on the host, one call, unpack the result; ``padding`` receives each FP24 or Lion case's padding
    masters after the call."""
    kernels = _hip.load()
    work = [c.copy() for c in cases]
    keep, segs = [], []
    by_group = all(c.group is not None for c in work)
    for c in work:
        lion = c.algorithm == O.LION
        assert c.mv_dtype == O.DT_FP8 and c.p_dtype in (O.DT_F32, O.DT_F24)
        O.check_sizes(c)
        f24 = c.p_dtype == O.DT_F24
        pack = {(True, True): pack_lion8f24_records, (True, False): pack_lion8_records,
                (False, True): pack_f8f24_records, (False, False): pack_records}[(lion, f24)]
        rec = torch.from_numpy(pack(c)).cuda()
        g = to_device(c.arrays["g"])
        if misalign_g:
            buf = torch.empty(g.numel() + 1, dtype=g.dtype, device=g.device)
            buf[1:].copy_(g)
            keep.append(buf)
            g = buf[1:]
        ms = to_device(c.arrays["m_scale"])
        vs = None if lion else to_device(c.arrays["v_scale"])
        out = to_device(c.arrays["out"]) if "out" in c.arrays else None
        grp = None
        if by_group:
            grp = _hip.Group(**{k: c.group[k] for k in ("lr", "beta1", "beta2", "eps", "weight_decay")},
                             seed=c.group["seed"] & (2**64 - 1), stochastic=int(c.group["stochastic"]))
        keep += [rec, g, ms, vs, out, grp]
        segs.append(_hip.Segment(p=rec.data_ptr(), p_lo=None, g=g.data_ptr(), m=None, v=None,
                                 m_scale=ms.data_ptr(), v_scale=vs.data_ptr() if vs is not None else None,
                                 out=out.data_ptr() if out is not None else None,
                                 group=ctypes.pointer(grp) if grp is not None else None, n=c.n, step=c.step,
                                 index=c.index, offset=c.offset, g_dtype=c.g_dtype, mv_dtype=O.DT_FP8,
                                 out_dtype=c.out_dtype, algorithm=c.algorithm,
                                 p_dtype={(True, True): _hip.DT_PACKED8_LION_F24, (True, False): _hip.DT_PACKED8_LION,
                                          (False, True): _hip.DT_PACKED8_F24, (False, False): _hip.DT_PACKED8}[(lion, f24)],
                                 reserved=seg_flags))
    arr = kernels.segment_array([ctypes.pointer(s) for s in segs])
    kernels.set_simd_level(WIDTH_LEVEL[width])
    try:
        kernels.set_stream(torch.cuda.current_stream())
        if by_group:
            kernels.multi_step(None, arr)
        else:
            hps = [_hip.HParams(**{k: c.hparams[k] for k, _ in _hip.HParams._fields_}) for c in work]
            kernels.multi_apply(None, arr, hps)
        torch.cuda.synchronize()
    finally:
        kernels.set_simd_level(None)
    it = iter(keep)
    for c in work:
        if misalign_g:
            next(it)
        rec, g, ms, vs, out, grp = (next(it) for _ in range(6))
        if c.algorithm == O.LION:
            unpack = unpack_lion8f24_records if c.p_dtype == O.DT_F24 else unpack_lion8_records
            pad = unpack(c, rec.cpu().numpy())
            if padding is not None:
                padding.append(pad)
        elif c.p_dtype == O.DT_F24:
            pad = unpack_f8f24_records(c, rec.cpu().numpy())
            if padding is not None:
                padding.append(pad)
        else:
            unpack_records(c, rec.cpu().numpy())
        c.arrays["m_scale"] = from_device(ms, c.arrays["m_scale"])
        if vs is not None:
            c.arrays["v_scale"] = from_device(vs, c.arrays["v_scale"])
        if out is not None:
            c.arrays["out"] = from_device(out, c.arrays["out"])
    return work


def pack_lion_records(case: O.Case) -> np.ndarray:
    """Separate FP32 master + BF16 m -> ADAMBRIDGE_DT_PACKED_LION records (records x 1536 bytes): per
    256 elements, the 256 masters then the 256 m values, each in element order.  Padding slots are
    set to a fixed pattern so that a test can see the kernel leave them unchanged."""
    n = case.n
    nr = max(1, -(-n // 256))
    p = np.full(nr * 256, 0x7FA5A5A5, np.uint32)   # a NaN pattern: any arithmetic on it would show
    p[:n] = case.arrays["p"].view(np.uint32)
    m = np.full(nr * 256, 0xA5A5, np.uint16)
    m[:n] = case.arrays["m"]
    rec = np.zeros((nr, 1536), np.uint8)
    rec[:, :1024] = p.reshape(nr, 256).view(np.uint8)
    rec[:, 1024:] = m.reshape(nr, 256).view(np.uint8)
    return rec


def unpack_lion_records(case: O.Case, rec: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """ADAMBRIDGE_DT_PACKED_LION records -> the case's separate master and m (in place); returns
    the padding slots' (master bits, m bits) past n."""
    n = case.n
    p = np.ascontiguousarray(rec[:, :1024]).view(np.uint32).reshape(-1)
    m = np.ascontiguousarray(rec[:, 1024:]).view(np.uint16).reshape(-1)
    case.arrays["p"] = p[:n].view(np.float32).copy()
    case.arrays["m"] = m[:n].copy()
    return p[n:].copy(), m[n:].copy()


def run_hip_lion_records(cases: list[O.Case], width: int = 16, double_buffer: bool = False,
                         misalign_g: int = 0, padding: list | None = None, seg_flags: int = 0) -> list[O.Case]:
    """Like run_hip for Lion / FP32 master / BF16 moment cases, through the record layout
    (ADAMBRIDGE_DT_PACKED_LION): pack on the host, one call, unpack the result.  ``misalign_g``
    elements shift the gradient off its allocation's alignment; ``padding`` receives each case's
    padding slots after the call."""
    kernels = _hip.load()
    work = [c.copy() for c in cases]
    keep, segs = [], []
    by_group = all(c.group is not None for c in work)
    for c in work:
        assert c.algorithm == O.LION and c.mv_dtype == O.DT_BF16 and c.p_dtype == O.DT_F32
        O.check_sizes(c)
        rec = torch.from_numpy(pack_lion_records(c)).cuda()
        dst = torch.full_like(rec, 0x5A) if double_buffer else None
        g = to_device(c.arrays["g"])
        if misalign_g:
            shift = int(misalign_g)
            buf = torch.empty(g.numel() + shift, dtype=g.dtype, device=g.device)
            buf[shift:].copy_(g)
            keep.append(buf)
            g = buf[shift:]
        out = to_device(c.arrays["out"]) if "out" in c.arrays else None
        grp = None
        if by_group:
            grp = _hip.Group(**{k: c.group[k] for k in ("lr", "beta1", "beta2", "eps", "weight_decay")},
                             seed=c.group["seed"] & (2**64 - 1), stochastic=int(c.group["stochastic"]))
        keep.append((rec, dst, g, out, grp))
        segs.append(_hip.Segment(p=rec.data_ptr(), p_lo=dst.data_ptr() if dst is not None else None,
                                 g=g.data_ptr(), m=None, v=None, out=out.data_ptr() if out is not None else None,
                                 group=ctypes.pointer(grp) if grp is not None else None, n=c.n, step=c.step,
                                 index=c.index, offset=c.offset, g_dtype=c.g_dtype, mv_dtype=O.DT_BF16,
                                 out_dtype=c.out_dtype, algorithm=O.LION, p_dtype=_hip.DT_PACKED_LION,
                                 reserved=seg_flags))
    arr = kernels.segment_array([ctypes.pointer(s) for s in segs])
    kernels.set_simd_level(WIDTH_LEVEL[width])
    try:
        kernels.set_stream(torch.cuda.current_stream())
        if by_group:
            kernels.multi_step(None, arr)
        else:
            hps = [_hip.HParams(**{k: c.hparams[k] for k, _ in _hip.HParams._fields_}) for c in work]
            kernels.multi_apply(None, arr, hps)
        torch.cuda.synchronize()
    finally:
        kernels.set_simd_level(None)
    entries = [e for e in keep if isinstance(e, tuple)]
    for c, (rec, dst, g, out, grp) in zip(work, entries):
        pad = unpack_lion_records(c, (dst if dst is not None else rec).cpu().numpy())
        if padding is not None:
            padding.append(pad)
        if out is not None:
            c.arrays["out"] = from_device(out, c.arrays["out"])
    return work


def _f32_record_keys(case: O.Case) -> tuple[str, ...]:
    return ("p", "m") if case.algorithm == O.LION else ("p", "m", "v")


def pack_f32_records(case: O.Case) -> np.ndarray:
    """Separate FP32 master, m and v -> ADAMBRIDGE_DT_PACKED_F32 records (records x 3072 bytes): per
    256 elements, the 256 masters, the 256 m, the 256 v, each in element order; for a Lion case
    ADAMBRIDGE_DT_PACKED_LION_F32 records (records x 2048 bytes: masters, then m).  Padding slots
    hold a fixed NaN pattern so that a test can see the kernel leave them unchanged."""
    n = case.n
    nr = max(1, -(-n // 256))
    keys = _f32_record_keys(case)
    rec = np.zeros((nr, len(keys), 256), np.uint32)
    for k, key in enumerate(keys):
        col = np.full(nr * 256, 0x7FA5A5A5 + k, np.uint32)
        col[:n] = case.arrays[key].view(np.uint32)
        rec[:, k, :] = col.reshape(nr, 256)
    return rec.reshape(nr, 256 * len(keys)).view(np.uint8).reshape(nr, 1024 * len(keys))


def unpack_f32_records(case: O.Case, rec: np.ndarray) -> list[np.ndarray]:
    """FP32 records (ADAMBRIDGE_DT_PACKED_F32, or _LION_F32 for a Lion case) -> the case's separate
    master and moments (in place); returns the padding slots (bits) past n of each."""
    n = case.n
    keys = _f32_record_keys(case)
    cols = np.ascontiguousarray(rec).view(np.uint32).reshape(-1, len(keys), 256)
    pads = []
    for k, key in enumerate(keys):
        col = cols[:, k, :].reshape(-1)
        case.arrays[key] = col[:n].view(np.float32).copy()
        pads.append(col[n:].copy())
    return pads


# FP24-master record columns: key, byte range, element type, padding fill
F24_COLUMNS = (("p", (0, 512), np.uint16, 0x7FA5), ("p_lo", (512, 768), np.uint8, 0xA5),
               ("m", (768, 1280), np.uint16, 0x7FA6), ("v", (1280, 1792), np.uint16, 0x7FA7))
# with FP32 moments (ADAMBRIDGE_DT_PACKED_F24_F32, 2816-byte records)
F24_F32_COLUMNS = F24_COLUMNS[:2] + (("m", (768, 1792), np.uint32, 0x7FA6A6A6),
                                     ("v", (1792, 2816), np.uint32, 0x7FA7A7A7))


def _f24_columns(case: O.Case):
    """The case's FP24-master record columns and record size."""
    if case.mv_dtype == O.DT_F32:   # Lion: ADAMBRIDGE_DT_PACKED_LION_F24_F32, no v
        return (F24_F32_COLUMNS[:3], 1792) if case.algorithm == O.LION else (F24_F32_COLUMNS, 2816)
    if case.algorithm == O.LION:   # ADAMBRIDGE_DT_PACKED_LION_F24: no v
        return F24_COLUMNS[:3], 1280
    return F24_COLUMNS, 1792


def pack_f24_records(case: O.Case) -> np.ndarray:
    """Separate FP24 master planes, BF16 m and v -> ADAMBRIDGE_DT_PACKED_F24 records (records x 1792
    bytes): per 256 elements, the 256 hi halves, the 256 lo bytes, the 256 m, the 256 v, each in
    element order (FP32 moments: ADAMBRIDGE_DT_PACKED_F24_F32, 2816 bytes; Lion:
    ADAMBRIDGE_DT_PACKED_LION_F24, 1280 bytes, no v).  Padding slots hold fixed patterns so that a
    test can see the kernel leave them unchanged."""
    n = case.n
    nr = max(1, -(-n // 256))
    columns, size = _f24_columns(case)
    rec = np.zeros((nr, size), np.uint8)
    for key, (a, b), dt, fill in columns:
        col = np.full(nr * 256, fill, dt)
        col[:n] = case.arrays[key].view(dt)
        rec[:, a:b] = col.reshape(nr, 256).view(np.uint8).reshape(nr, b - a)
    return rec


def unpack_f24_records(case: O.Case, rec: np.ndarray) -> list[np.ndarray]:
    """ADAMBRIDGE_DT_PACKED_F24 records -> the case's separate planes, m and v (in place); returns
    the padding slots past n of each."""
    n = case.n
    columns, size = _f24_columns(case)
    rec = np.ascontiguousarray(rec).reshape(-1, size)
    pads = []
    for key, (a, b), dt, _ in columns:
        col = np.ascontiguousarray(rec[:, a:b]).view(dt).reshape(-1)
        case.arrays[key] = col[:n].view(case.arrays[key].dtype).copy()
        pads.append(col[n:].copy())
    return pads


# record kind -> (p_dtype code, moment dtype, master dtype, pack, unpack, algorithm)
_RECORDS = {"f32": (_hip.DT_PACKED_F32, O.DT_F32, O.DT_F32, pack_f32_records, unpack_f32_records, O.ADAMW),
            "f24": (_hip.DT_PACKED_F24, O.DT_BF16, O.DT_F24, pack_f24_records, unpack_f24_records, O.ADAMW),
            "lion-f24": (_hip.DT_PACKED_LION_F24, O.DT_BF16, O.DT_F24, pack_f24_records, unpack_f24_records,
                         O.LION),
            "lion-f32": (_hip.DT_PACKED_LION_F32, O.DT_F32, O.DT_F32, pack_f32_records, unpack_f32_records,
                         O.LION),
            "f24-f32": (_hip.DT_PACKED_F24_F32, O.DT_F32, O.DT_F24, pack_f24_records, unpack_f24_records, O.ADAMW),
            "lion-f24-f32": (_hip.DT_PACKED_LION_F24_F32, O.DT_F32, O.DT_F24, pack_f24_records, unpack_f24_records,
                             O.LION)}


def run_hip_lion_f32_records(cases: list[O.Case], width: int = 16, **kw) -> list[O.Case]:
    """run_hip for Lion / FP32 master / FP32 moment cases through ADAMBRIDGE_DT_PACKED_LION_F32."""
    return run_hip_f32_records(cases, width, kind="lion-f32", **kw)


def run_hip_f24_records(cases: list[O.Case], width: int = 16, **kw) -> list[O.Case]:
    """run_hip through FP24-master records: ADAMBRIDGE_DT_PACKED_F24 (AdamW, BF16 moments),
    ADAMBRIDGE_DT_PACKED_F24_F32 (AdamW, FP32 moments) or, for Lion cases,
    ADAMBRIDGE_DT_PACKED_LION_F24 (BF16 moment) and ADAMBRIDGE_DT_PACKED_LION_F24_F32 (FP32 moment)."""
    kinds = {("lion-" if c.algorithm == O.LION else "") + ("f24-f32" if c.mv_dtype == O.DT_F32 else "f24") for c in cases}
    assert len(kinds) == 1
    return run_hip_f32_records(cases, width, kind=kinds.pop(), **kw)


def run_hip_f32_records(cases: list[O.Case], width: int = 16, double_buffer: bool = False,
                        misalign_g: int = 0, padding: list | None = None, seg_flags: int = 0,
                        kind: str = "f32") -> list[O.Case]:
    """Like run_hip for AdamW cases through a record layout: FP32 master and FP32 moments
    (ADAMBRIDGE_DT_PACKED_F32, ``kind`` 'f32'), or FP24 master and BF16 moments
    (ADAMBRIDGE_DT_PACKED_F24, 'f24'): pack on the host, one call, unpack the result.
    ``misalign_g`` elements shift the gradient off its allocation's alignment; ``padding`` receives
    each case's padding slots after the call."""
    p_code, mv_dt, pt, pack, unpack, algo = _RECORDS[kind]
    kernels = _hip.load()
    work = [c.copy() for c in cases]
    entries, segs = [], []
    by_group = all(c.group is not None for c in work)
    for c in work:
        assert c.algorithm == algo and c.mv_dtype == mv_dt and c.p_dtype == pt
        O.check_sizes(c)
        rec = torch.from_numpy(pack(c)).cuda()
        dst = torch.full_like(rec, 0x5A) if double_buffer else None
        g = to_device(c.arrays["g"])
        keep = []
        if misalign_g:
            buf = torch.empty(g.numel() + int(misalign_g), dtype=g.dtype, device=g.device)
            buf[int(misalign_g):].copy_(g)
            keep.append(buf)
            g = buf[int(misalign_g):]
        out = to_device(c.arrays["out"]) if "out" in c.arrays else None
        grp = None
        if by_group:
            grp = _hip.Group(**{k: c.group[k] for k in ("lr", "beta1", "beta2", "eps", "weight_decay")},
                             seed=c.group["seed"] & (2**64 - 1), stochastic=int(c.group["stochastic"]))
        entries.append((rec, dst, g, out, grp, keep))
        segs.append(_hip.Segment(p=rec.data_ptr(), p_lo=dst.data_ptr() if dst is not None else None,
                                 g=g.data_ptr(), m=None, v=None, out=out.data_ptr() if out is not None else None,
                                 group=ctypes.pointer(grp) if grp is not None else None, n=c.n, step=c.step,
                                 index=c.index, offset=c.offset, g_dtype=c.g_dtype, mv_dtype=mv_dt,
                                 out_dtype=c.out_dtype, algorithm=algo, p_dtype=p_code,
                                 reserved=seg_flags))
    arr = kernels.segment_array([ctypes.pointer(s) for s in segs])
    kernels.set_simd_level(WIDTH_LEVEL[width])
    try:
        kernels.set_stream(torch.cuda.current_stream())
        if by_group:
            kernels.multi_step(None, arr)
        else:
            hps = [_hip.HParams(**{k: c.hparams[k] for k, _ in _hip.HParams._fields_}) for c in work]
            kernels.multi_apply(None, arr, hps)
        torch.cuda.synchronize()
    finally:
        kernels.set_simd_level(None)
    for c, (rec, dst, g, out, grp, keep) in zip(work, entries):
        pad = unpack(c, (dst if dst is not None else rec).cpu().numpy())
        if padding is not None:
            padding.append(pad)
        if out is not None:
            c.arrays["out"] = from_device(out, c.arrays["out"])
    return work

