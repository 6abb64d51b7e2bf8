"""Optimizer behaviour the reference's suite checks, on the device (reference tests/test_cuda.py,
test_hardening.py, test_lion.py, test_gpu_state.py), plus chunked segments through the C ABI."""

import copy
import ctypes

import pytest
import torch

import adambridge_amd as ab
from adambridge_amd import _hip
from adambridge_amd import precision as P
from conftest import max_param_diff
from test_optimizer_gpu import TinyLM, lm_loss

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _trained(**kw):
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, small_param_threshold=2000, **kw)
    for k in range(3):
        lm_loss(model, k).backward()
        opt.step()
        opt.zero_grad()
    return model, opt


def test_checkpoint_string_indices_still_load():
    model, opt = _trained()
    sd = opt.state_dict()
    sd = {**sd, "state": {str(k): v for k, v in sd["state"].items()}}
    other = ab.AdamBridge(copy.deepcopy(model).parameters(), lr=3e-3, small_param_threshold=2000)
    other.load_state_dict(sd)
    for a, b in zip(opt.master_params(), other.master_params()):
        assert torch.equal(a, b)
    opt.close()
    other.close()


@pytest.mark.parametrize("precision,moment_bytes", [("fp32", 4), ("bf16", 2)])
def test_lion_keeps_one_moment_in_memory_and_checkpoint(precision, moment_bytes):
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    opt = ab.LionBridge(model.parameters(), lr=1e-3, precision=precision, state_layout="separate")
    for k in range(2):
        lm_loss(model, k).backward()
        opt.step()
        opt.zero_grad()
    n = sum(p.numel() for p in model.parameters())
    assert opt.memory_report()["moments"] == moment_bytes * n
    assert opt.expected_bytes_per_param() == 4.0 + moment_bytes
    assert ab.bytes_per_param(precision, moments=1) == 4.0 + moment_bytes
    sd = opt.state_dict()
    assert sd["adambridge"]["algorithm"] == "lion"
    assert all("exp_avg" in st and "exp_avg_sq" not in st for st in sd["state"].values())
    assert all(s.v is None for s in opt._ordered)
    opt.close()


def test_device_fp8_stores_keep_small_second_moments_and_convert_roles():
    """The device stores (conversion kernel) keep small v in the sqrt domain and re-encode a store
    saved under the other role, as the host stores do."""
    v = torch.full((128,), 1e-12)
    v[0] = 1.0
    out = P.make_store("fp8", 128, "v", init=v, device=DEV).to_fp32()
    assert abs(out[0].item() - 1.0) < 0.3 and (out[1:] > 0).all()
    x = torch.rand(256, generator=torch.Generator().manual_seed(6)) * 1e-3
    saved = P.make_store("fp8", 256, "m", init=x, device=DEV)
    loaded = P.store_from_state_dict(saved.state_dict(), 256, "v", device=DEV)
    want = P.make_store("fp8", 256, "v", init=saved.to_fp32(), device=DEV)
    assert torch.equal(loaded.to_fp32(), want.to_fp32())


@pytest.mark.parametrize("precision", ["fp32", "bf16", "fp8"])
def test_chunked_segments_match_the_whole_tensor(precision):
    """One tensor updated as three segments at 128-aligned offsets (pointers into the same
    buffers) gives the bytes of one whole-tensor segment (reference tests/test_cuda.py:88-104)."""
    k = _hip.load()
    n = 10_000 + 5
    gen = torch.Generator(device=DEV).manual_seed(2)
    p0 = torch.randn(n, device=DEV, generator=gen) * 0.02
    g = (torch.randn(n, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
    nb = -(-n // 128)
    if precision == "fp8":
        mk = lambda role: (torch.zeros(nb * 128, dtype=torch.uint8, device=DEV),  # noqa: E731
                           torch.ones(nb, device=DEV))
    else:
        dt = torch.float32 if precision == "fp32" else torch.bfloat16
        mk = lambda role: ((torch.randn(n, device=DEV, generator=gen) * 1e-4).to(dt), None)  # noqa: E731
    m0, ms0 = mk("m")
    v0, vs0 = mk("v")
    if precision != "fp8":
        v0 = v0.abs()
    group = _hip.Group(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, seed=7, stochastic=1)
    mv = {"fp32": _hip.DT_F32, "bf16": _hip.DT_BF16, "fp8": _hip.DT_FP8}[precision]
    esz = {"fp32": 4, "bf16": 2, "fp8": 1}[precision]

    def run(bounds):
        p, m, v = p0.clone(), m0.clone(), v0.clone()
        ms, vs = (ms0.clone(), vs0.clone()) if precision == "fp8" else (None, None)
        out = torch.empty(n, dtype=torch.bfloat16, device=DEV)
        segs = []
        for lo, hi in bounds:
            segs.append(_hip.Segment(
                p=p.data_ptr() + 4 * lo, g=g.data_ptr() + 2 * lo, m=m.data_ptr() + esz * lo,
                v=v.data_ptr() + esz * lo, m_scale=ms.data_ptr() + 4 * (lo // 128) if ms is not None else None,
                v_scale=vs.data_ptr() + 4 * (lo // 128) if vs is not None else None, out=out.data_ptr() + 2 * lo,
                group=ctypes.pointer(group), n=hi - lo, step=3, index=11, offset=lo, g_dtype=_hip.DT_BF16,
                mv_dtype=mv, out_dtype=_hip.DT_BF16, algorithm=0, p_dtype=_hip.DT_F32))
        k.set_stream(torch.cuda.current_stream())
        k.multi_step(None, k.segment_array([ctypes.pointer(s) for s in segs]))
        torch.cuda.synchronize()
        return [t for t in (p, m, v, ms, vs, out) if t is not None]

    whole = run([(0, n)])
    chunked = run([(0, 1280), (1280, 6400), (6400, n)])
    for a, b in zip(whole, chunked):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_small_parameter_without_grad_is_not_updated():
    """A batched small parameter whose gradient never arrives keeps its value at step_sync
    (reference tests/test_cuda.py:253-272)."""
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    frozen = model.blocks[0][0].bias   # a small parameter of the batched group
    opt = ab.AdamBridge(model.parameters(), lr=1e-2, small_param_threshold=2000).attach_hooks(model)
    before = frozen.detach().clone()
    frozen.requires_grad_(False)
    for k in range(2):
        lm_loss(model, k).backward()
        opt.step_sync()
    assert torch.equal(frozen.detach(), before)
    assert not opt._slots[frozen].initialized
    opt.close()


def test_autotune_runs_and_records_its_decisions():
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, autotune=True)
    for k in range(3):
        lm_loss(model, k).backward()
        opt.step()
        opt.zero_grad()
    log = opt.autotune_log
    assert log and all(isinstance(line, str) for line in log)
    opt.close()


@pytest.mark.parametrize("budget", [0, "half", "all", "auto"])
def test_gpu_state_budget_values_train_like_torch_adamw(budget):
    """Every budget keeps all state in HBM here; training matches torch AdamW as the reference's
    does at every budget (reference tests/test_gpu_state.py:36-64)."""
    torch.manual_seed(0)
    base = TinyLM().to(DEV)
    total = sum(p.numel() for p in base.parameters()) * 18
    value = {"half": total // 2, "all": total * 2}.get(budget, budget)
    model, ref = copy.deepcopy(base), copy.deepcopy(base)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, small_param_threshold=2000, gpu_state_budget=value)
    opt.attach_hooks(model)
    torch_opt = torch.optim.AdamW(ref.parameters(), lr=3e-3)
    for k in range(6):
        lm_loss(model, k).backward()
        opt.step_sync()
        torch_opt.zero_grad()
        lm_loss(ref, k).backward()
        torch_opt.step()
    torch.cuda.synchronize()
    assert max_param_diff(ref, model) < 1e-5
    report = opt.memory_report()
    assert report["gpu_state"] == report["total"]
    opt.close()
