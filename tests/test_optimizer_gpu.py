"""AdamBridge / LionBridge on the GPU: the reference's behavioural suite
(tests/test_optimizer.py, test_lion.py, test_master24.py, test_cuda.py) on
parameters in HBM, plus end-to-end bit-exactness of the API path against the
oracle (parameter index, step counting, lazy state and seeds included).
"""

import copy
import io

import numpy as np
import pytest
import torch

import adambridge_amd as ab
from conftest import max_param_diff, tiny_mlp
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def train(model, opt, steps, seed=1, batch=16, hooks=False):
    torch.manual_seed(seed)
    losses = []
    for _ in range(steps):
        x = torch.randn(batch, 48, device=DEV, dtype=next(model.parameters()).dtype)
        opt.zero_grad()
        loss = model(x).float().pow(2).mean()
        loss.backward()
        if hooks:
            opt.step_sync()
        else:
            opt.step()
        losses.append(loss.item())
    return losses


class RefLion(torch.optim.Optimizer):
    """Lion as published: p -= lr * (sign(b1 m + (1-b1) g) + wd p); m = b2 m + (1-b2) g."""

    def __init__(self, params, lr=1e-4, betas=(0.9, 0.99), weight_decay=0.0):
        super().__init__(params, dict(lr=lr, betas=betas, weight_decay=weight_decay))

    @torch.no_grad()
    def step(self):
        for group in self.param_groups:
            b1, b2 = group["betas"]
            for p in group["params"]:
                if p.grad is None:
                    continue
                m = self.state[p].setdefault("m", torch.zeros_like(p))
                c = m * b1 + p.grad * (1 - b1)
                p.mul_(1 - group["lr"] * group["weight_decay"]).add_(c.sign(), alpha=-group["lr"])
                m.mul_(b2).add_(p.grad, alpha=1 - b2)


class TinyLM(torch.nn.Module):
    """Embedding + blocks + tied head (reference tests/test_cuda.py:15-31)."""

    def __init__(self, vocab=97, dim=64, layers=4):
        super().__init__()
        self.emb = torch.nn.Embedding(vocab, dim)
        self.blocks = torch.nn.ModuleList(
            torch.nn.Sequential(torch.nn.LayerNorm(dim), torch.nn.Linear(dim, 4 * dim), torch.nn.GELU(),
                                torch.nn.Linear(4 * dim, dim)) for _ in range(layers))
        self.norm = torch.nn.LayerNorm(dim)

    def forward(self, tokens):
        h = self.emb(tokens)
        for blk in self.blocks:
            h = h + blk(h)
        return self.norm(h) @ self.emb.weight.t()


def lm_loss(model, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    tokens = torch.randint(0, 97, (8, 33), device=DEV, generator=g)
    logits = model(tokens[:, :-1])
    return torch.nn.functional.cross_entropy(logits.float().reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1))


# ------------------------------------------------------- against torch AdamW

def test_matches_torch_adamw_with_groups_and_scheduler():
    """reference test_optimizer.py:27-51, FP32 parameters on the GPU."""
    ref_model = tiny_mlp(device=DEV)
    model = copy.deepcopy(ref_model)

    def groups(m):
        return [{"params": [m[0].weight, m[3].weight], "weight_decay": 0.1},
                {"params": [m[0].bias, m[2].weight, m[2].bias, m[3].bias], "weight_decay": 0.0, "lr": 3e-3}]

    ref = torch.optim.AdamW(groups(ref_model), lr=1e-2, betas=(0.8, 0.99))
    opt = ab.AdamBridge(groups(model), lr=1e-2, betas=(0.8, 0.99))
    sched_ref = torch.optim.lr_scheduler.StepLR(ref, step_size=3, gamma=0.5)
    sched = torch.optim.lr_scheduler.StepLR(opt, step_size=3, gamma=0.5)
    torch.manual_seed(1)
    for _ in range(10):
        x = torch.randn(16, 48, device=DEV)
        for m, o, s in ((ref_model, ref, sched_ref), (model, opt, sched)):
            o.zero_grad()
            m(x).pow(2).mean().backward()
            o.step()
            s.step()
    assert max_param_diff(ref_model, model) < 1e-6
    assert opt.backend == "hip/gfx950"
    opt.close()


def test_sync_step_with_clipping():
    """clip_grad_norm_ before step() is seen: grads are read at step (reference test_cuda.py:273-287)."""
    torch.manual_seed(0)
    ref_model = TinyLM().to(DEV)
    model = copy.deepcopy(ref_model)
    ref = torch.optim.AdamW(ref_model.parameters(), lr=3e-3)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3)
    for step in range(5):
        for m, o in ((ref_model, ref), (model, opt)):
            o.zero_grad()
            lm_loss(m, step).backward()
            torch.nn.utils.clip_grad_norm_(m.parameters(), 0.1)
            o.step()
    assert max_param_diff(ref_model, model) < 1e-5
    opt.close()


@pytest.mark.parametrize("overlap", [True, False])
def test_async_hooks_match_torch_adamw(overlap):
    """reference test_cuda.py:41-62."""
    torch.manual_seed(0)
    ref_model = TinyLM().to(DEV)
    model = copy.deepcopy(ref_model)
    ref = torch.optim.AdamW(ref_model.parameters(), lr=3e-3)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, overlap_writeback=overlap).attach_hooks(model)
    for step in range(8):
        ref.zero_grad()
        lm_loss(ref_model, step).backward()
        ref.step()
        opt.zero_grad()
        lm_loss(model, step).backward()
        assert all(p.grad is None for p in model.parameters() if p.numel() >= opt.small_param_threshold)
        stats = opt.step_sync()
        assert all(p.grad is None for p in model.parameters())
        assert stats.num_updates == len(list(model.parameters()))
    assert max_param_diff(ref_model, model) < 1e-5
    opt.close()


@pytest.mark.parametrize("threshold", [0, 2000, 10**9])
def test_hooked_and_grouped_parameters_match_torch_adamw(threshold):
    """reference test_cuda.py:65-83."""
    torch.manual_seed(0)
    ref_model = TinyLM().to(DEV)
    model = copy.deepcopy(ref_model)
    ref = torch.optim.AdamW(ref_model.parameters(), lr=3e-3)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, small_param_threshold=threshold).attach_hooks(model)
    for step in range(6):
        ref.zero_grad()
        lm_loss(ref_model, step).backward()
        ref.step()
        lm_loss(model, step).backward()
        opt.step_sync()
    assert max_param_diff(ref_model, model) < 1e-5
    opt.close()


@pytest.mark.parametrize("mode", ["step", "hooks", "hooks-deferred", "delayed"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_strided_parameters_update_like_contiguous_ones(dtype, mode):
    """A parameter stored transposed, whose gradient autograd lays out the same way, gets the updates of
    a contiguous parameter holding the same values, bit for bit: the update reads the gradient in
    logical order from a contiguous copy made before the update is ordered after the compute stream,
    writes the new weights to a buffer of its own and copies them into the strided parameter."""
    torch.manual_seed(0)
    base = [torch.randn(48, 300, device=DEV).to(dtype), torch.randn(300, device=DEV).to(dtype)]
    flat = [torch.nn.Parameter(base[0].clone()), torch.nn.Parameter(base[1].clone())]
    strided = [torch.nn.Parameter(base[0].t().contiguous().t()), torch.nn.Parameter(base[1].clone())]
    assert not strided[0].is_contiguous() and torch.equal(strided[0], flat[0])
    kw = dict(lr=1e-2, weight_decay=0.1, small_param_threshold=0, overlap_writeback=mode != "hooks-deferred",
              delay_updates=mode == "delayed", delay_warmup_steps=1)
    opts = [ab.AdamBridge(ps, **kw) for ps in (flat, strided)]
    hooked = mode != "step"
    if hooked:
        for opt in opts:
            opt.attach_hooks()
    gen = torch.Generator(device=DEV).manual_seed(1)
    for step in range(6):
        x = torch.randn(64, 48, device=DEV, generator=gen).to(dtype)
        for ps, opt in zip((flat, strided), opts):
            opt.zero_grad(set_to_none=True)
            # the same GEMM for both (contiguous operands); the strided parameter's gradient is then
            # laid out like the parameter by autograd
            (x @ ps[0].contiguous() + ps[1]).float().pow(2).mean().backward()
            if hooked:
                opt.step_sync()
            else:
                assert ps is flat or not ps[0].grad.is_contiguous()
                opt.step()
    for opt in opts:
        opt.close()
    for a, b in zip(flat, strided):
        assert torch.equal(a, b)
    assert not torch.equal(flat[0], base[0])


def _stale_reference(model, steps, make_opt, warmup, micro=1):
    """Losses and final weights of an optimizer whose updates reach the model one step late after
    ``warmup`` exact steps (reference test_cuda.py:129-152); with ``micro`` > 1, each step
    accumulates the gradients of ``micro`` backward passes (seeds 10 k + j) on the same weights."""
    master = copy.deepcopy(model).float()
    ref = make_opt(master.parameters())
    snapshots = [[p.detach().clone() for p in master.parameters()]]
    losses = []
    for k in range(1, steps + 1):
        lag = k - 1 if k <= warmup + 1 else k - 2
        with torch.no_grad():
            for p, w in zip(model.parameters(), snapshots[lag]):
                p.copy_(w)
        model.zero_grad()
        for j in range(micro):
            loss = lm_loss(model, k if micro == 1 else 10 * k + j)
            loss.backward()
            losses.append(loss.item())
        for p, q in zip(master.parameters(), model.parameters()):
            p.grad = q.grad.float()
        ref.step()
        snapshots.append([p.detach().clone() for p in master.parameters()])
    return losses, snapshots[-1]


@pytest.mark.parametrize("warmup", [0, 3])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_delayed_updates_match_one_step_stale_adamw(warmup, precision):
    """reference test_cuda.py:155-177."""
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    want_losses, want = _stale_reference(copy.deepcopy(model), 10, lambda ps: torch.optim.AdamW(ps, lr=3e-3), warmup)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, precision=precision, delay_updates=True,
                        delay_warmup_steps=warmup, small_param_threshold=2000).attach_hooks(model)
    assert any(s.small is not None for s in opt._ordered) and any(s.small is None for s in opt._ordered)
    losses = []
    for k in range(1, 11):
        loss = lm_loss(model, k)
        loss.backward()
        opt.step_sync()
        losses.append(loss.item())
    opt.flush()
    tol = 1e-4 if precision == "fp32" else 2e-2
    assert max(abs(a - b) for a, b in zip(losses, want_losses)) < tol
    assert max((p - w).abs().max().item() for p, w in zip(model.parameters(), want)) < (
        1e-5 if precision == "fp32" else 1e-2)
    opt.close()


@pytest.mark.parametrize("warmup", [0, 2])
def test_delayed_updates_with_accumulation_match_stale_accumulated_adamw(warmup):
    """Delayed updates with accumulation_steps=2 and batched small parameters (reference
    tests/test_gpu_state.py:99-114, which checks only that the weights stay finite): the weights
    follow AdamW on the accumulated gradients, one step stale after the warm-up steps."""
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    want_losses, want = _stale_reference(copy.deepcopy(model), 6, lambda ps: torch.optim.AdamW(ps, lr=3e-3), warmup,
                                         micro=2)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, delay_updates=True, delay_warmup_steps=warmup,
                        accumulation_steps=2, small_param_threshold=2000).attach_hooks(model)
    assert any(s.small is not None for s in opt._ordered) and any(s.small is None for s in opt._ordered)
    losses = []
    for k in range(1, 7):
        for j in range(2):
            loss = lm_loss(model, 10 * k + j)
            loss.backward()
            losses.append(loss.item())
        opt.step_sync()
    opt.flush()
    assert max(abs(a - b) for a, b in zip(losses, want_losses)) < 1e-4
    assert max((p - w).abs().max().item() for p, w in zip(model.parameters(), want)) < 1e-5
    opt.close()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("kind", ["adamw-bf16", "adamw-fp8", "adamw-fp32", "adamw-bf16-fp24", "lion-bf16"])
def test_delayed_weights_are_the_exact_weights_one_step_late(kind, dtype):
    """With gradients that do not depend on the weights, a delayed optimizer's parameters after step
    k are, bit for bit, an exact optimizer's after step k - 1 -- a parameter that gets no gradient
    at a step included -- its masters equal the exact ones at every step, and flush() brings the
    parameters level (the update writes the weight from before it; the newest waits in the master)."""
    algo, precision, *rest = kind.split("-")
    master = rest[0] if rest else "fp32"
    cls = ab.LionBridge if algo == "lion" else ab.AdamBridge
    torch.manual_seed(0)
    shapes = [(300, 70), (1001,), (64, 64), (5,)]
    base = [torch.randn(s, device=DEV).mul_(0.02).to(dtype) for s in shapes]
    exact_ps = [torch.nn.Parameter(t.clone()) for t in base]
    delayed_ps = [torch.nn.Parameter(t.clone()) for t in base]
    kw = dict(lr=1e-2, weight_decay=0.1, precision=precision, master_precision=master, small_param_threshold=0)
    exact = cls(exact_ps, **kw)
    delayed = cls(delayed_ps, delay_updates=True, delay_warmup_steps=0, **kw)
    history = [[p.detach().clone() for p in exact_ps]]
    gen = torch.Generator(device=DEV).manual_seed(5)
    for k in range(1, 6):
        grads = [torch.randn(s, device=DEV, generator=gen).mul_(1e-2).to(dtype) for s in shapes]
        skip = 2 if k == 3 else None   # parameter 2 gets no gradient at step 3
        for ps, opt in ((exact_ps, exact), (delayed_ps, delayed)):
            for i, (p, g) in enumerate(zip(ps, grads)):
                p.grad = None if i == skip else g.clone()
            opt.step()
        history.append([p.detach().clone() for p in exact_ps])
        for i, (got, want) in enumerate(zip(delayed_ps, history[k - 1])):
            assert torch.equal(got, want), f"step {k}: parameter {i} is not the exact weight of step {k - 1}"
        for a, b in zip(exact.master_params(), delayed.master_params()):
            assert torch.equal(a, b)
    assert not torch.equal(history[-1][0], history[-2][0])
    delayed.flush()
    torch.cuda.synchronize()
    for got, want in zip(delayed_ps, exact_ps):
        assert torch.equal(got, want)
    exact.close()
    delayed.close()


def test_delayed_updates_state_dict_close_and_unused_params():
    """reference test_cuda.py:180-209."""
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    opt = ab.AdamBridge(model.parameters(), lr=1e-2, delay_updates=True, small_param_threshold=0).attach_hooks(model)
    head = model.blocks[-1][3].weight
    for k in range(3):
        lm_loss(model, k).backward()
        opt.step_sync()
    before = head.detach().clone()
    head.requires_grad_(False)
    lm_loss(model, 3).backward()
    opt.step_sync()
    torch.cuda.synchronize()
    assert not torch.equal(head, before)
    assert torch.equal(head.detach().reshape(-1), opt._slots[head].state.master_fp32())
    head.requires_grad_(True)
    lm_loss(model, 4).backward()
    opt.step_sync()
    opt.state_dict()
    torch.cuda.synchronize()
    for p, master in zip(model.parameters(), opt.master_params()):
        assert torch.equal(p.detach().reshape(-1), master)
    lm_loss(model, 5).backward()
    opt.step_sync()
    opt.close()
    torch.cuda.synchronize()
    for p, master in zip(model.parameters(), opt.master_params()):
        assert torch.equal(p.detach().reshape(-1), master)


@pytest.mark.parametrize("delay", [False, True])
def test_lion_hooks_match_reference(delay):
    """reference test_cuda.py:212-232."""
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    want_losses, want = _stale_reference(copy.deepcopy(model), 6, lambda ps: RefLion(ps, lr=1e-3, weight_decay=0.1),
                                         warmup=10**9 if not delay else 0)
    opt = ab.LionBridge(model.parameters(), lr=1e-3, weight_decay=0.1, delay_updates=delay).attach_hooks(model)
    losses = []
    for k in range(1, 7):
        loss = lm_loss(model, k)
        loss.backward()
        opt.step_sync()
        losses.append(loss.item())
    opt.flush()
    assert max(abs(a - b) for a, b in zip(losses, want_losses)) < 1e-5
    assert max((p - w).abs().max().item() for p, w in zip(model.parameters(), want)) < 1e-6
    assert all(s.v is None for s in opt._ordered)
    opt.close()


def test_lion_matches_reference_with_groups():
    """reference test_lion.py:46-60."""
    ref_model = tiny_mlp(device=DEV)
    model = copy.deepcopy(ref_model)

    def groups(m):
        return [{"params": [m[0].weight, m[3].weight], "weight_decay": 0.5},
                {"params": [m[0].bias, m[2].weight, m[2].bias, m[3].bias], "lr": 3e-4}]

    ref = RefLion(groups(ref_model), lr=1e-3, betas=(0.9, 0.99), weight_decay=0.0)
    opt = ab.LionBridge(groups(model), lr=1e-3, betas=(0.9, 0.99))
    train(ref_model, ref, 10)
    train(model, opt, 10)
    assert max_param_diff(ref_model, model) < 1e-6
    n = sum(p.numel() for p in model.parameters())
    assert opt.memory_report()["moments"] == 4 * n
    assert opt.expected_bytes_per_param() == 8.0
    sd = opt.state_dict()
    assert sd["adambridge"]["algorithm"] == "lion"
    assert all("exp_avg" in st and "exp_avg_sq" not in st for st in sd["state"].values())
    opt.close()


def test_lion_no_eps():
    with pytest.raises(TypeError):
        ab.LionBridge(tiny_mlp(device=DEV).parameters(), eps=1e-8)


@pytest.mark.parametrize("layout,precision", [("auto", "bf16"), ("auto", "fp32"), ("auto", "fp8"), ("separate", "bf16"),
                                              ("separate", "fp32"), ("separate", "fp8")])
def test_lion_state_dict_resume_is_exact(layout, precision):
    """reference test_lion.py:102-124: a Lion checkpoint resumed into a fresh optimizer continues bit
    for bit (bf16 parameters, so the master is a buffer of its own; 'auto' keeps a BF16, FP32 or FP8
    moment in Lion records, whose checkpoint holds the reference's separate arrays); AdamBridge
    refuses it."""
    kw = dict(lr=1e-3, precision=precision, state_layout=layout, seed=3)
    model = tiny_mlp(device=DEV, dtype=torch.bfloat16)
    opt = ab.LionBridge(model.parameters(), **kw)
    train(model, opt, 3)
    want = {"bf16": "lion-records", "fp32": "lion-f32-records", "fp8": "lion-fp8-records"}[precision] \
        if layout == "auto" else "separate"
    assert {s.state.layout for s in opt._ordered} == {want}
    buf = io.BytesIO()
    torch.save({"model": model.state_dict(), "opt": opt.state_dict()}, buf)
    train(model, opt, 4, seed=7)
    expected = [p.detach().clone() for p in model.parameters()]
    masters = opt.master_params()

    buf.seek(0)
    ckpt = torch.load(buf, weights_only=True)
    model2 = tiny_mlp(seed=5, device=DEV, dtype=torch.bfloat16)
    model2.load_state_dict(ckpt["model"])
    opt2 = ab.LionBridge(model2.parameters(), **kw)
    opt2.load_state_dict(ckpt["opt"])
    train(model2, opt2, 4, seed=7)
    assert all(torch.equal(a, b) for a, b in zip(expected, model2.parameters()))
    assert all(torch.equal(a, b) for a, b in zip(masters, opt2.master_params()))

    adam = ab.AdamBridge(tiny_mlp(device=DEV).parameters())
    with pytest.raises(ValueError, match="exp_avg_sq"):
        adam.load_state_dict(ckpt["opt"])
    for o in (opt, opt2, adam):
        o.close()


@pytest.mark.parametrize("precision", ["bf16", "fp8"])
def test_lion_low_precision_moment_trains_like_fp32(precision):
    """reference test_lion.py:65-74: a BF16 or FP8 moment trains as the FP32 one does."""
    results = {}
    for p in ("fp32", precision):
        model = tiny_mlp(device=DEV)
        opt = ab.LionBridge(model.parameters(), lr=3e-4, precision=p)
        results[p] = train(model, opt, 60)
        opt.close()
    assert results[precision][-1] < 0.5 * results[precision][0]
    assert abs(results[precision][-1] - results["fp32"][-1]) < 0.1 * results["fp32"][0]


@pytest.mark.parametrize("window", [3, 2])
def test_accumulation_steps_match_accumulated_adamw(window):
    """reference test_lion.py:132-153 (AdamW with accumulation_steps)."""
    ref_model = tiny_mlp(device=DEV)
    model = copy.deepcopy(ref_model)
    ref = torch.optim.AdamW(ref_model.parameters(), lr=1e-2)
    opt = ab.AdamBridge(model.parameters(), lr=1e-2, accumulation_steps=3, small_param_threshold=0).attach_hooks(model)
    torch.manual_seed(1)
    for _ in range(4):
        xs = [torch.randn(8, 48, device=DEV) for _ in range(window)]
        ref.zero_grad()
        for x in xs:
            (ref_model(x).pow(2).mean() / window).backward()
        ref.step()
        for x in xs:
            (model(x).pow(2).mean() / window).backward()
        opt.step_sync()
        opt.zero_grad()
    assert max_param_diff(ref_model, model) < 1e-6
    opt.close()


def test_gradient_accumulation_with_no_sync():
    """reference test_cuda.py:311-330."""
    torch.manual_seed(0)
    ref_model = TinyLM().to(DEV)
    model = copy.deepcopy(ref_model)
    ref = torch.optim.AdamW(ref_model.parameters(), lr=3e-3)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3).attach_hooks(model)
    for step in range(3):
        ref.zero_grad()
        for micro in range(3):
            (lm_loss(ref_model, 10 * step + micro) / 3).backward()
        ref.step()
        for micro in range(3):
            if micro < 2:
                with opt.no_sync():
                    (lm_loss(model, 10 * step + micro) / 3).backward()
            else:
                (lm_loss(model, 10 * step + micro) / 3).backward()
        opt.step_sync()
    assert max_param_diff(ref_model, model) < 1e-5
    opt.close()


def test_bf16_params_keep_fp32_master():
    """reference test_cuda.py:290-308: bf16 weights are the RNE of the stored master."""
    torch.manual_seed(0)
    model = TinyLM().to(DEV).to(torch.bfloat16)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, precision="bf16").attach_hooks(model)
    losses = []
    for step in range(30):
        loss = lm_loss(model, step % 4)
        loss.backward()
        opt.step_sync()
        losses.append(loss.item())
    assert losses[-1] < losses[0] - 0.5
    for p, master in zip(model.parameters(), opt.master_params()):
        assert p.dtype == torch.bfloat16 and master.dtype == torch.float32
        assert torch.equal(p.reshape(-1), master.to(torch.bfloat16))
    rep = opt.memory_report()
    n = sum(p.numel() for p in model.parameters())
    assert rep["master"] == 4 * n and rep["moments"] == 4 * n
    opt.close()


def test_weights_visible_to_next_forward_without_host_sync():
    """reference test_cuda.py:333-348: step_sync orders the update on the current stream."""
    torch.manual_seed(0)
    model = tiny_mlp(device=DEV)
    opt = ab.AdamBridge(model.parameters(), lr=0.5).attach_hooks(model)
    x = torch.randn(4, 48, device=DEV)
    model(x).sum().backward()
    opt.step_sync()
    after = [p.clone() for p in model.parameters()]
    torch.cuda.synchronize()
    for p, q in zip(model.parameters(), after):
        assert torch.equal(p, q)
    opt.close()


def test_params_without_grad_are_skipped():
    """reference test_optimizer.py:77-85."""
    model = tiny_mlp(device=DEV)
    frozen = model[0].weight.detach().clone()
    model[0].weight.requires_grad_(False)
    opt = ab.AdamBridge(model.parameters(), lr=1e-2)
    train(model, opt, 2)
    assert torch.equal(model[0].weight, frozen)
    assert opt.master_params()[0] is None
    opt.close()


@pytest.mark.parametrize("hooks", [False, True])
def test_param_group_added_after_steps_trains_like_torch_adamw(hooks):
    """add_param_group between steps (reference optimizer.py:225-237): the new parameters take the
    next indices and their own hyperparameters, and are hooked when hooks are attached."""
    ref_model = tiny_mlp(device=DEV)
    model = copy.deepcopy(ref_model)

    def first(m):
        return [m[0].weight, m[0].bias]

    def second(m):
        return {"params": [m[2].weight, m[2].bias, m[3].weight, m[3].bias], "lr": 3e-3, "weight_decay": 0.1}

    ref = torch.optim.AdamW(first(ref_model), lr=1e-2, weight_decay=0.0)
    opt = ab.AdamBridge(first(model), lr=1e-2, weight_decay=0.0, small_param_threshold=0)
    if hooks:
        opt.attach_hooks()
    torch.manual_seed(1)
    for step in range(6):
        if step == 2:
            ref.add_param_group(second(ref_model))
            opt.add_param_group(second(model))
            assert [s.index for s in opt._ordered] == list(range(6))
        x = torch.randn(16, 48, device=DEV)
        for m, o in ((ref_model, ref), (model, opt)):
            o.zero_grad(set_to_none=True)
            m(x).pow(2).mean().backward()
            if o is opt and hooks:
                if step >= 2:   # the added parameters were updated by their hooks
                    assert model[3].weight.grad is None
                o.step_sync()
            else:
                o.step()
    assert max_param_diff(ref_model, model) < 1e-6
    opt.close()


@pytest.mark.parametrize("precision", ["fp32", "bf16", "fp8"])
@pytest.mark.parametrize("hooks", [False, True])
def test_empty_parameters_beside_others(precision, hooks):
    """A parameter with no elements (an empty bias, a zero-width embedding) takes part in every step,
    checkpoint and rebuild without touching memory, and the others train as torch AdamW does."""
    torch.manual_seed(0)
    shapes = [(64, 48), (0,), (48,), (0, 16)]
    params = [torch.nn.Parameter(torch.randn(s, device=DEV) * 0.1) for s in shapes]
    ref_params = [torch.nn.Parameter(p.detach().clone()) for p in params]
    opt = ab.AdamBridge(params, lr=1e-2, precision=precision, small_param_threshold=0)
    ref = torch.optim.AdamW(ref_params, lr=1e-2)
    if hooks:
        opt.attach_hooks()
    for step in range(4):
        grads = [torch.randn(s, device=DEV) * 1e-2 for s in shapes]
        for ps, o in ((params, opt), (ref_params, ref)):
            o.zero_grad(set_to_none=True)
            for p, g in zip(ps, grads):
                p.grad = g.clone()
            if o is opt and hooks:
                o.step_sync()   # gradients set by hand fire no hook: step_sync updates none of them
                o.step()
            else:
                o.step()
    tol = 1e-6 if precision == "fp32" else 5e-2
    for p, r in zip(params, ref_params):
        assert p.shape == r.shape
        assert p.numel() == 0 or (p - r).abs().max().item() < tol
    sd = opt.state_dict()
    assert sd["state"][1]["master"].numel() == 0
    other = ab.AdamBridge([torch.nn.Parameter(torch.zeros(s, device=DEV)) for s in shapes], lr=1e-2,
                          precision=precision, small_param_threshold=0)
    other.load_state_dict(sd)
    opt.set_precision("bf16" if precision != "bf16" else "fp32")
    opt.close()
    other.close()


@pytest.mark.parametrize("precision", ["bf16", "fp8", "fp32"])
def test_hooked_states_share_one_arena_and_stay_lazy(precision):
    """The first hook sets aside one arena for every hooked parameter's interleaved state; each state
    is still built at its parameter's first update, from the value the parameter holds then (a
    parameter without a gradient in the first step, changed before its first update), and the
    results equal, bit for bit, those of the same steps through step()."""
    results = []
    for hooks in (True, False):
        torch.manual_seed(0)
        model = TinyLM().to(DEV).to(torch.bfloat16)
        opt = ab.AdamBridge(model.parameters(), lr=3e-3, precision=precision, small_param_threshold=2000)
        if hooks:
            opt.attach_hooks(model)
        head = model.blocks[-1][3].weight
        head.requires_grad_(False)   # no gradient in the first step
        lm_loss(model, 0).backward()
        opt.step() if not hooks else opt.step_sync()
        slot = opt._slots[head]
        assert not slot.initialized
        if hooks:
            hooked = [s for s in opt._ordered if s.small is None and s.initialized]
            assert len({s.state.current.untyped_storage().data_ptr() for s in hooked}) == 1
            assert slot in opt._engine._reserved
        with torch.no_grad():
            head.mul_(0.5)           # changed before its first update
        head.requires_grad_(True)
        for step in range(1, 4):
            opt.zero_grad(set_to_none=True)
            lm_loss(model, step).backward()
            opt.step() if not hooks else opt.step_sync()
        if hooks:
            assert slot.state.current.untyped_storage().data_ptr() == hooked[0].state.current.untyped_storage().data_ptr()
            assert not opt._engine._reserved
        results.append(([p.detach().clone() for p in model.parameters()], [m.clone() for m in opt.master_params()]))
        opt.close()
    for xs, ys in zip(*results):
        assert all(torch.equal(x, y) for x, y in zip(xs, ys))


def test_weights_loaded_after_construction_are_respected():
    """reference test_optimizer.py:141-150: lazy master."""
    model = tiny_mlp(seed=0, device=DEV)
    opt = ab.AdamBridge(model.parameters(), lr=0.0, weight_decay=0.0)
    pretrained = tiny_mlp(seed=42, device=DEV)
    model.load_state_dict(pretrained.state_dict())
    train(model, opt, 1)
    assert max_param_diff(model, pretrained) == 0
    opt.close()


@pytest.mark.parametrize("precision", ["fp32", "bf16", "fp8"])
def test_state_dict_resume_is_exact(precision):
    """reference test_optimizer.py:88-118 (bf16 parameters so the master is a separate buffer)."""
    torch.manual_seed(0)
    base = tiny_mlp(device=DEV, dtype=torch.bfloat16)
    a = copy.deepcopy(base)
    opt_a = ab.AdamBridge(a.parameters(), lr=1e-2, precision=precision, seed=7)
    train(a, opt_a, 6, seed=3)
    b = copy.deepcopy(base)
    opt_b = ab.AdamBridge(b.parameters(), lr=1e-2, precision=precision, seed=7)
    train(b, opt_b, 3, seed=3)
    buf = io.BytesIO()
    torch.save({"model": b.state_dict(), "opt": opt_b.state_dict()}, buf)
    buf.seek(0)
    ckpt = torch.load(buf, weights_only=True)
    c = tiny_mlp(seed=123, device=DEV, dtype=torch.bfloat16)
    opt_c = ab.AdamBridge(c.parameters(), lr=1e-2, precision=precision, seed=7)
    c.load_state_dict(ckpt["model"])
    opt_c.load_state_dict(ckpt["opt"])
    torch.manual_seed(3)
    for _ in range(3):
        torch.randn(16, 48, device=DEV, dtype=torch.bfloat16)
    for _ in range(3):
        x = torch.randn(16, 48, device=DEV, dtype=torch.bfloat16)
        opt_c.zero_grad()
        c(x).float().pow(2).mean().backward()
        opt_c.step()
    assert max_param_diff(a, c) == 0
    for x, y in zip(opt_a.master_params(), opt_c.master_params()):
        assert torch.equal(x, y)
    for o in (opt_a, opt_b, opt_c):
        o.close()


@pytest.mark.parametrize("prec", ["fp32", "fp8"])
def test_load_torch_adamw_checkpoint(prec):
    """reference test_optimizer.py:121-138."""
    ref_model = tiny_mlp(device=DEV)
    ref = torch.optim.AdamW(ref_model.parameters(), lr=1e-2)
    train(ref_model, ref, 3)
    model = copy.deepcopy(ref_model)
    opt = ab.AdamBridge(model.parameters(), lr=1e-2, precision=prec)
    opt.load_state_dict(ref.state_dict())
    for slot, p in zip(opt._ordered, ref_model.parameters()):
        assert slot.step == 3 and slot.m.precision == prec
        m_ref = ref.state[p]["exp_avg"].reshape(-1)
        tol = 1e-7 if prec == "fp32" else 0.07 * m_ref.abs().max().item()
        assert (slot.m.to_fp32() - m_ref).abs().max().item() <= tol
    train(ref_model, ref, 3, seed=5)
    train(model, opt, 3, seed=5)
    assert max_param_diff(ref_model, model) < (1e-6 if prec == "fp32" else 1e-2)
    opt.close()


@pytest.mark.parametrize("hooks", [False, True])
def test_set_precision_mid_training(hooks):
    """reference test_optimizer.py:153-166."""
    model = tiny_mlp(device=DEV)
    opt = ab.AdamBridge(model.parameters(), lr=1e-2)
    if hooks:
        opt.attach_hooks(model)
    train(model, opt, 2, hooks=hooks)
    m_before = [s.m.to_fp32() for s in opt._ordered]
    opt.set_precision("bf16_moments")
    for s, m in zip(opt._ordered, m_before):
        assert s.m.precision == "bf16"
        torch.testing.assert_close(s.m.to_fp32(), m, rtol=2**-8, atol=0)
    train(model, opt, 2, hooks=hooks)
    opt.close()


@pytest.mark.parametrize("prec", ["bf16", "fp8"])
def test_low_precision_moments_converge_like_fp32(prec):
    """reference test_optimizer.py:169-191."""
    torch.manual_seed(0)
    w_true = torch.randn(64, 16, device=DEV)
    x_all = torch.randn(2048, 64, device=DEV)
    y_all = x_all @ w_true + 0.01 * torch.randn(2048, 16, device=DEV)

    def run(precision):
        torch.manual_seed(1)
        lin = torch.nn.Linear(64, 16).to(DEV)
        opt = ab.AdamBridge(lin.parameters(), lr=1e-2, weight_decay=0.0, precision=precision)
        for _ in range(1200):
            idx = torch.randint(0, 2048, (64,), device=DEV)
            opt.zero_grad()
            (lin(x_all[idx]) - y_all[idx]).pow(2).mean().backward()
            opt.step()
        opt.close()
        return (lin(x_all) - y_all).pow(2).mean().item()

    base, low = run("fp32"), run(prec)
    assert base < 2e-4
    assert low < 1.2 * base


def test_double_backward_without_no_sync_raises():
    """reference test_optimizer.py:194-202."""
    model = tiny_mlp(device=DEV)
    opt = ab.AdamBridge(model.parameters(), release_grads=False, small_param_threshold=0).attach_hooks(model)
    x = torch.randn(4, 48, device=DEV)
    model(x).sum().backward()
    with pytest.raises(RuntimeError, match="no_sync"):
        model(x).sum().backward()
    opt.step_sync()
    opt.close()


def test_hooks_match_step():
    """reference test_optimizer.py:205-214: same bytes whichever way the update is driven."""
    a, b = tiny_mlp(device=DEV), tiny_mlp(device=DEV)
    opt_a = ab.AdamBridge(a.parameters(), lr=1e-2)
    opt_b = ab.AdamBridge(b.parameters(), lr=1e-2).attach_hooks(b)
    train(a, opt_a, 4)
    train(b, opt_b, 4, hooks=True)
    assert max_param_diff(a, b) == 0
    assert all(p.grad is None for p in b.parameters())
    opt_a.close()
    opt_b.close()


@pytest.mark.parametrize("delay", [False, True])
@pytest.mark.parametrize("overlap", [True, False])
def test_update_streams_give_the_same_bytes(delay, overlap):
    """Updates in order on the current stream (the default) and on a side stream give the same bytes
    as plain step() calls, hooked or not, with buffered write-backs (overlap_writeback=False) and
    delayed updates, and the next forward pass reads the new weights without a host wait."""
    torch.manual_seed(0)
    base = TinyLM(layers=2).to(DEV).to(torch.bfloat16)
    models = {k: copy.deepcopy(base) for k in ("ref", "current", "side", "current-step", "side-step")}
    kw = dict(lr=3e-3, weight_decay=0.01, precision="bf16", small_param_threshold=2000, delay_updates=delay,
              overlap_writeback=overlap)
    opts = {k: ab.AdamBridge(m.parameters(), update_stream=k.split("-")[0] if k != "ref" else "current", **kw)
            for k, m in models.items()}
    for k in ("current", "side"):
        opts[k].attach_hooks(models[k])
    assert opts["side"]._points._handles and not opts["current"]._points._handles
    losses = {k: [] for k in models}
    for step in range(5):
        for k, m in models.items():
            loss = lm_loss(m, step)
            losses[k].append(loss.detach())
            loss.backward()
            if k in ("current", "side"):
                opts[k].step_sync()
            else:
                opts[k].step()
                opts[k].zero_grad(set_to_none=True)
    for k in models:
        opts[k].flush()
    torch.cuda.synchronize()
    for k, m in models.items():
        assert all(torch.equal(a, b) for a, b in zip(models["ref"].parameters(), m.parameters())), k
        assert all(torch.equal(a, b) for a, b in zip(losses["ref"], losses[k])), k
    for opt in opts.values():
        opt.close()


class _TwoStreamMLP(torch.nn.Module):
    """A model whose first layer runs on a stream of its own: its backward, and so its gradient
    hooks, run there too (autograd runs each backward op on its forward op's stream)."""

    stream: torch.cuda.Stream   # set after the copies (a stream is not copyable)

    def __init__(self):
        super().__init__()
        self.a = torch.nn.Linear(48, 256)
        self.b = torch.nn.Linear(256, 48)

    def forward(self, x):
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            h = torch.nn.functional.gelu(self.a(x))
        torch.cuda.current_stream().wait_stream(self.stream)
        h.record_stream(torch.cuda.current_stream())
        return self.b(h)


def test_hooks_on_another_stream_are_ordered_before_step_sync():
    """A gradient hook that fires on another stream enqueues its in-order update there; step_sync() on
    the default stream orders it before the work that follows, and the results equal step()'s."""
    torch.manual_seed(0)
    other = torch.cuda.Stream()
    base = _TwoStreamMLP().to(DEV).to(torch.bfloat16)
    ref_model, model = copy.deepcopy(base), copy.deepcopy(base)
    ref_model.stream = model.stream = other
    kw = dict(lr=3e-3, precision="bf16", small_param_threshold=0)
    ref = ab.AdamBridge(ref_model.parameters(), **kw)
    opt = ab.AdamBridge(model.parameters(), **kw).attach_hooks(model)
    seen = []
    model.a.weight.register_post_accumulate_grad_hook(
        lambda p: seen.append(torch.cuda.current_stream().cuda_stream))
    for step in range(4):
        x = torch.randn(64, 48, device=DEV, generator=torch.Generator(device=DEV).manual_seed(step),
                        dtype=torch.bfloat16)
        ref_model(x).float().pow(2).mean().backward()
        ref.step()
        ref.zero_grad(set_to_none=True)
        model(x).float().pow(2).mean().backward()
        opt.step_sync()   # on the default stream
        snap = [p.detach().clone() for p in model.parameters()]   # read on the default stream at once
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(ref_model.parameters(), snap)), f"step {step}"
    assert seen and all(s == other.cuda_stream for s in seen)   # the hook did fire on the other stream
    ref.close()
    opt.close()


def test_update_stream_is_validated():
    p = torch.nn.Parameter(torch.zeros(4, device=DEV))
    with pytest.raises(ValueError, match="update_stream"):
        ab.AdamBridge([p], update_stream="other")


def test_errors_surface_in_step():
    """reference test_optimizer.py:217-224: a bad group fails the step with a RuntimeError."""
    model = tiny_mlp(device=DEV)
    opt = ab.AdamBridge(model.parameters())
    model(torch.randn(2, 48, device=DEV)).sum().backward()
    opt.param_groups[0]["betas"] = None
    with pytest.raises(RuntimeError, match="update failed"):
        opt.step()
    opt.close()


def test_cpu_parameters_are_refused():
    model = tiny_mlp()
    opt = ab.AdamBridge(model.parameters())
    model(torch.randn(2, 48)).sum().backward()
    with pytest.raises(RuntimeError, match="update failed"):
        opt.step()
    opt.close()


# ------------------------------------------------------------------ FP24

def _bf16_model(seed=0):
    return tiny_mlp(seed, dtype=torch.bfloat16, device=DEV)


def _same_grad_train(pairs, steps, hooks=False):
    """Every optimizer gets the same gradients (reference test_master24.py:22-37)."""
    g = torch.Generator().manual_seed(1)
    for _ in range(steps):
        grads = [(torch.randn(p.shape, generator=g) * 0.1).to(device=DEV, dtype=torch.bfloat16)
                 for p in pairs[0][0].parameters()]
        for model, opt in pairs:
            sum((p * grad).sum() for p, grad in zip(model.parameters(), grads)).backward()
            if hooks:
                opt.step_sync()
            else:
                opt.step()
                opt.zero_grad(set_to_none=True)


@pytest.mark.parametrize("hooks", [False, True])
@pytest.mark.parametrize("precision", ["fp32", "fp8"])
def test_fp24_master_tracks_the_fp32_master(precision, hooks):
    """reference test_master24.py:40-54 and 116-129."""
    a, b = _bf16_model(), _bf16_model()
    kw = dict(lr=1e-2, weight_decay=0.0, small_param_threshold=0, precision=precision)
    opt_a, opt_b = ab.AdamBridge(a.parameters(), **kw), ab.AdamBridge(b.parameters(), master_precision="fp24", **kw)
    if hooks:
        opt_a.attach_hooks(a)
        opt_b.attach_hooks(b)
    assert opt_b.expected_bytes_per_param() == opt_a.expected_bytes_per_param() - 1
    _same_grad_train([(a, opt_a), (b, opt_b)], 20, hooks=hooks)
    for ma, mb in zip(opt_a.master_params(), opt_b.master_params()):
        assert ((ma - mb).abs() <= ma.abs() * 1e-3 + 1e-5).all()
    assert max_param_diff(a, b) <= 2**-7
    n = sum(p.numel() for p in b.parameters())
    assert opt_b.memory_report()["master"] == 3 * n
    assert opt_a.memory_report()["master"] == 4 * n
    opt_a.close()
    opt_b.close()


def test_fp24_checkpoints_round_trip_and_convert():
    """reference test_master24.py:67-95."""
    kw = dict(lr=1e-2, weight_decay=0.0, small_param_threshold=0, precision="bf16")
    model = _bf16_model()
    opt = ab.AdamBridge(model.parameters(), master_precision="fp24", **kw)
    _same_grad_train([(model, opt)], 3)
    sd = opt.state_dict()
    assert sd["adambridge"]["master_precision"] == "fp24"
    saved = sd["state"][0]["master"]
    assert saved["precision"] == "fp24" and saved["hi"].dtype == torch.bfloat16 and saved["lo"].dtype == torch.uint8
    masters = [m.clone() for m in opt.master_params()]

    def loaded(master_precision, state):
        other = ab.AdamBridge(_bf16_model(1).parameters(), master_precision=master_precision, **kw)
        other.load_state_dict(state)
        return other

    same = loaded("fp24", sd)
    as32 = loaded("fp32", sd)
    back = loaded("fp24", as32.state_dict())
    for other in (same, as32, back):
        for x, y in zip(masters, other.master_params()):
            assert torch.equal(x, y)
        assert other._ordered[0].step == 3
        other.close()
    opt.close()


def test_bad_checkpoints_are_rejected_whole():
    """reference test_master24.py:98-113 and test_lion.py:117-121."""
    kw = dict(lr=1e-2, small_param_threshold=0)
    model = _bf16_model()
    opt = ab.AdamBridge(model.parameters(), master_precision="fp24", **kw)
    _same_grad_train([(model, opt)], 1)
    sd = opt.state_dict()
    n = sd["state"][0]["master"]["hi"].numel()
    for bad_master in ({"precision": "fp24", "hi": torch.zeros(1, dtype=torch.bfloat16),
                        "lo": torch.zeros(n, dtype=torch.uint8)},
                       {"precision": "fp24", "hi": torch.zeros(n, dtype=torch.bfloat16),
                        "lo": torch.zeros(n, dtype=torch.int8)},
                       {"precision": "fp16", "hi": torch.zeros(n, dtype=torch.bfloat16)}):
        bad = {**sd, "state": {**sd["state"], 0: {**sd["state"][0], "master": bad_master}}}
        other = ab.AdamBridge(_bf16_model(1).parameters(), master_precision="fp24", **kw)
        with pytest.raises(ValueError):
            other.load_state_dict(bad)
        other.load_state_dict(sd)
        other.close()
    opt.close()


def test_adamw_refuses_a_lion_checkpoint():
    model = _bf16_model()
    lion = ab.LionBridge(model.parameters(), lr=1e-3)
    train(model, lion, 2)
    sd = lion.state_dict()
    adam = ab.AdamBridge(_bf16_model().parameters())
    with pytest.raises(ValueError, match="exp_avg_sq"):
        adam.load_state_dict(sd)
    lion.close()
    adam.close()


# ------------------------------------------- end to end against the oracle

def _oracle_state_after(params_bf16, grads_seq, precision, master, lr, wd, betas, seed, lion=False):
    """Run the same updates through the oracle's multi_step: the API must give the same bytes."""
    mv = {"fp32": O.DT_F32, "bf16": O.DT_BF16, "fp8": O.DT_FP8}[precision]
    cases = []
    for k, p in enumerate(params_bf16):
        n = p.numel()
        x = p.detach().float().reshape(-1).cpu().numpy()
        arrays = {}
        if master == "fp24":
            arrays["p"], arrays["p_lo"] = O.f24_planes(x)
        else:
            arrays["p"] = x.copy()
        if mv == O.DT_FP8:
            nb = -(-n // 128)
            arrays["m"] = np.zeros(nb * 128, np.uint8)
            arrays["m_scale"] = np.ones(nb, np.float32)
            if not lion:
                arrays["v"] = np.zeros(nb * 128, np.uint8)
                arrays["v_scale"] = np.ones(nb, np.float32)
        else:
            dt = np.float32 if mv == O.DT_F32 else np.uint16
            arrays["m"] = np.zeros(n, dt)
            if not lion:
                arrays["v"] = np.zeros(n, dt)
        arrays["out"] = np.zeros(n, np.uint16)
        cases.append(O.Case(n=n, algorithm=O.LION if lion else O.ADAMW, mv_dtype=mv,
                            p_dtype=O.DT_F24 if master == "fp24" else O.DT_F32, g_dtype=O.DT_BF16,
                            out_dtype=O.DT_BF16, offset=0, index=k, step=1, arrays=arrays,
                            group={"lr": lr, "beta1": betas[0], "beta2": betas[1], "eps": 0.0 if lion else 1e-8,
                                   "weight_decay": wd, "seed": seed, "stochastic": 1}))
    for t, grads in enumerate(grads_seq):
        for c, g in zip(cases, grads):
            c.arrays["g"] = g.reshape(-1).cpu().view(torch.int16).numpy().view(np.uint16).copy()
            c.step = t + 1
        O.run_many(cases, "oracle", 16, in_place=True)
    return cases


@pytest.mark.parametrize("precision,master,lion", [("bf16", "fp32", False), ("fp32", "fp32", False),
                                                   ("fp8", "fp24", False), ("bf16", "fp24", True), ("bf16", "fp24", False),
                                                   ("fp8", "fp32", True), ("fp8", "fp32", False)])
@pytest.mark.parametrize("hooks", [False, True])
def test_api_updates_are_bit_exact_against_the_oracle(precision, master, lion, hooks):
    """AdamBridge/LionBridge on bf16 parameters (sync step or per-parameter hooks plus a batched
    small group) give the exact bytes of the reference kernel run on the same gradients with the
    same parameter indices and step numbers."""
    torch.manual_seed(0)
    shapes = [(300, 257), (4099,), (64, 64), (17,), (1000, 130)]
    params = [torch.nn.Parameter((torch.randn(s, device=DEV) * 0.02).to(torch.bfloat16)) for s in shapes]
    init = [p.detach().clone() for p in params]
    lr, wd, betas, seed = (1e-3, 0.1, (0.9, 0.99), 5) if lion else (2e-3, 0.01, (0.9, 0.999), 5)
    cls = ab.LionBridge if lion else ab.AdamBridge
    opt = cls(params, lr=lr, betas=betas, weight_decay=wd, precision=precision, master_precision=master, seed=seed,
              small_param_threshold=5000)
    g = torch.Generator(device=DEV).manual_seed(3)
    grads_seq = [[(torch.randn(s, device=DEV, generator=g) * 1e-2).to(torch.bfloat16) for s in shapes]
                 for _ in range(4)]
    if hooks:
        opt.attach_hooks()
    for grads in grads_seq:
        if hooks:
            # autograd delivers the gradient: loss = sum(p * g) has d/dp = g exactly
            sum((p * gr).float().sum() for p, gr in zip(params, grads)).backward()
            opt.step_sync()
        else:
            for p, gr in zip(params, grads):
                p.grad = gr.clone()
            opt.step()
    torch.cuda.synchronize()
    want = _oracle_state_after(init, grads_seq, precision, master, lr, wd, betas, seed, lion)
    for k, (p, c) in enumerate(zip(params, want)):
        slot = opt._ordered[k]
        assert slot.step == 4
        got_p = p.detach().reshape(-1).cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got_p, c.arrays["out"]), f"param {k} weights"
        m_data = (slot.m.q if hasattr(slot.m, "q") else slot.m.data).detach().cpu()
        want_m = c.arrays["m"]
        assert np.array_equal(m_data.view(torch.uint8).numpy().view(want_m.dtype).reshape(want_m.shape), want_m), \
            f"param {k} m"
        if master == "fp24":
            planes = slot.state.window(0, slot.numel)   # separate arrays or FP24-master records
            hi, lo = planes["p"].contiguous(), planes["p_lo"].contiguous()
            assert np.array_equal(hi.cpu().view(torch.int16).numpy().view(np.uint16), c.arrays["p"])
            assert np.array_equal(lo.cpu().numpy(), c.arrays["p_lo"])
        else:
            assert np.array_equal(slot.state.master_fp32().cpu().numpy().view(np.uint32), c.arrays["p"].view(np.uint32))
    opt.close()


@pytest.mark.parametrize("precision", ["bf16", "fp8"])
def test_back_to_back_table_launches_reuse_staging_slots(precision):
    """24 steps of 20 parameters with no host synchronisation between them: every launch carries
    its descriptors in a device table (more than 7 segments), so the 16 staging slots are reused
    while earlier launches may still be queued, and the uploads run on the queue's copy stream.
    The final state equals the oracle's after the same 24 steps."""
    torch.manual_seed(1)
    shapes = [(97 + 13 * k, 31 + k) for k in range(20)]
    params = [torch.nn.Parameter((torch.randn(s, device=DEV) * 0.02).to(torch.bfloat16)) for s in shapes]
    init = [p.detach().clone() for p in params]
    lr, wd, betas, seed = 2e-3, 0.01, (0.9, 0.999), 9
    opt = ab.AdamBridge(params, lr=lr, betas=betas, weight_decay=wd, precision=precision, seed=seed,
                        small_param_threshold=0)
    g = torch.Generator(device=DEV).manual_seed(5)
    grads_seq = [[(torch.randn(s, device=DEV, generator=g) * 1e-2).to(torch.bfloat16) for s in shapes]
                 for _ in range(24)]
    log = []
    opt._engine.launch_log = log
    for grads in grads_seq:
        for p, gr in zip(params, grads):
            p.grad = gr
        opt.step()
    torch.cuda.synchronize()
    assert len(log) == 24 and all(e == sum(p.numel() for p in params) for _, _, e in log)
    want = _oracle_state_after(init, grads_seq, precision, "fp32", lr, wd, betas, seed)
    for k, (p, c) in enumerate(zip(params, want)):
        slot = opt._ordered[k]
        assert slot.step == 24
        got_p = p.detach().reshape(-1).cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got_p, c.arrays["out"]), f"param {k} weights"
        assert np.array_equal(slot.state.master_fp32().cpu().numpy().view(np.uint32), c.arrays["p"].view(np.uint32))
        m_data = (slot.m.q if hasattr(slot.m, "q") else slot.m.data).detach().cpu()
        assert np.array_equal(m_data.view(torch.uint8).numpy().view(c.arrays["m"].dtype).reshape(-1),
                              c.arrays["m"].reshape(-1)), f"param {k} m"
    opt.close()


def test_multi_tensor_launch_count():
    """step() updates every parameter in one kernel launch."""
    model = TinyLM().to(DEV).to(torch.bfloat16)
    opt = ab.AdamBridge(model.parameters(), lr=1e-3, precision="bf16")
    log = []
    opt._engine.launch_log = log
    lm_loss(model, 0).backward()
    opt.step()
    torch.cuda.synchronize()
    assert len(log) == 1 and log[0][2] == sum(p.numel() for p in model.parameters())
    opt.close()


@pytest.mark.parametrize("precision", ["bf16", "fp8", "fp32", "bf16-fp24"])
@pytest.mark.parametrize("hooks", [False, True])
def test_state_layouts_give_identical_bytes(hooks, precision):
    """The interleaved layouts (default: BF16 pairs, FP8 block records, FP32 records, FP24-master
    records), the separate layout and the double-buffered interleaved layout produce the same
    weights, masters and moments (FP8: codes and scales), step after step."""
    precision, _, master = precision.partition("-")
    results = []
    for kw in (dict(state_layout="separate"), dict(), dict(double_buffer=True)):
        torch.manual_seed(0)
        model = TinyLM().to(DEV).to(torch.bfloat16)
        opt = ab.AdamBridge(model.parameters(), lr=3e-3, precision=precision, small_param_threshold=2000,
                            master_precision=master or "fp32", **kw)
        if hooks:
            opt.attach_hooks(model)
        assert any(s.initialized and s.state.layout != "separate" for s in opt._ordered) or "state_layout" in kw or not opt._ordered[0].initialized
        for step in range(4):
            lm_loss(model, step).backward()
            if hooks:
                opt.step_sync()
            else:
                opt.step()
                opt.zero_grad()
        if "state_layout" not in kw:
            assert all(s.state.layout != "separate" for s in opt._ordered)
        codes = ([s.m.q.view(torch.uint8) for s in opt._ordered] + [s.v.q.view(torch.uint8) for s in opt._ordered]
                 + [s.m.scale.clone() for s in opt._ordered] + [s.v.scale.clone() for s in opt._ordered]
                 if precision == "fp8" else [])
        results.append(([p.detach().clone() for p in model.parameters()], [m.clone() for m in opt.master_params()],
                        [s.m.to_fp32() for s in opt._ordered], [s.v.to_fp32() for s in opt._ordered], codes))
        opt.close()
    for other in results[1:]:
        for xs, ys in zip(results[0], other):
            assert all(torch.equal(x, y) for x, y in zip(xs, ys))


@pytest.mark.parametrize("algo,precision", [("adamw", "bf16"), ("adamw", "fp8"), ("lion", "bf16"),
                                            ("adamw", "fp32"), ("adamw", "bf16-fp24"), ("lion", "bf16-fp24")])
def test_interleaved_checkpoint_gathered_on_host_when_the_device_is_short(algo, precision):
    """Interleaved states (BF16 pairs, FP8 records, Lion records, FP32 records, FP24-master records)
    are gathered into the reference's checkpoint arrays on the device when it has room, else into
    host memory parameter by parameter; either checkpoint loads into a fresh optimizer with
    identical masters and moments."""
    precision, _, master = precision.partition("-")
    torch.manual_seed(0)
    model = TinyLM().to(DEV).to(torch.bfloat16)
    cls = ab.LionBridge if algo == "lion" else ab.AdamBridge
    opt = cls(model.parameters(), lr=3e-3, precision=precision, master_precision=master or "fp32")
    for step in range(3):
        lm_loss(model, step).backward()
        opt.step()
        opt.zero_grad()
    assert all(s.state.gathers for s in opt._ordered)

    def tensors(entry):
        if isinstance(entry, torch.Tensor):
            return [entry]
        return [t for v in entry.values() for t in tensors(v)] if isinstance(entry, dict) else []

    on_device = opt.state_dict()
    opt._EXPORT_MARGIN = 1 << 62   # as if the device had no room left
    on_host = opt.state_dict()
    assert all(t.is_cuda for e in on_device["state"].values() for t in tensors(e))
    assert all(not t.is_cuda for e in on_host["state"].values() for t in tensors(e))
    buf = io.BytesIO()
    torch.save(on_host, buf)
    buf.seek(0)
    saved = torch.load(buf, weights_only=True)
    masters = opt.master_params()
    moments = [(s.m.to_fp32(), None if s.v is None else s.v.to_fp32()) for s in opt._ordered]
    for sd in (on_device, saved):
        other = cls(TinyLM().to(DEV).to(torch.bfloat16).parameters(), lr=3e-3, precision=precision,
                    master_precision=master or "fp32")
        other.load_state_dict(sd)
        assert all(torch.equal(x, y) for x, y in zip(masters, other.master_params()))
        for (m, v), s in zip(moments, other._ordered):
            assert torch.equal(m, s.m.to_fp32()) and (v is None or torch.equal(v, s.v.to_fp32()))
            assert s.step == 3
        other.close()
    opt.close()


@pytest.mark.parametrize("precision", ["bf16", "fp8"])
def test_packed_state_checkpoint_and_set_precision(precision):
    """Checkpoints of the interleaved layouts are the reference format and load into either layout;
    set_precision leaves and re-enters the interleaved layout: the values survive the exit exactly
    and come back as the new precision's encoding of them."""
    torch.manual_seed(0)
    model = TinyLM().to(DEV).to(torch.bfloat16)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, precision=precision)
    for step in range(3):
        lm_loss(model, step).backward()
        opt.step()
        opt.zero_grad()
    sd = opt.state_dict()
    st = sd["state"][0]
    assert isinstance(st["master"], torch.Tensor) and st["master"].dtype == torch.float32
    if precision == "bf16":
        assert st["exp_avg"]["precision"] == "bf16" and st["exp_avg"]["data"].dtype == torch.bfloat16
    else:
        assert st["exp_avg"]["precision"] == "fp8" and st["exp_avg"]["q"].dtype == torch.float8_e4m3fn
        assert st["exp_avg_sq"]["q"].dtype == torch.float8_e5m2 and st["exp_avg_sq"]["scale"].dtype == torch.float32
        n = opt._ordered[0].numel
        assert st["exp_avg"]["q"].numel() == -(-n // 128) * 128 and st["exp_avg"]["scale"].numel() == -(-n // 128)
    masters = [m.clone() for m in opt.master_params()]
    for layout in ("separate", "auto"):
        other = ab.AdamBridge(TinyLM().to(DEV).to(torch.bfloat16).parameters(), lr=3e-3, precision=precision,
                              state_layout=layout)
        other.load_state_dict(sd)
        for x, y in zip(masters, other.master_params()):
            assert torch.equal(x, y)
        for a, b in zip(opt._ordered, other._ordered):
            assert torch.equal(a.m.to_fp32(), b.m.to_fp32()) and torch.equal(a.v.to_fp32(), b.v.to_fp32())
        other.close()
    m_before = [s.m.to_fp32() for s in opt._ordered]
    opt.set_precision("fp32")
    assert all(s.state.layout == "f32-records" for s in opt._ordered)   # bf16 parameters: FP32 records
    for s, m in zip(opt._ordered, m_before):
        assert torch.equal(s.m.to_fp32(), m)
    opt.set_precision(precision)
    assert all(s.state.layout != "separate" for s in opt._ordered)
    from adambridge_amd import precision as P
    for s, m in zip(opt._ordered, m_before):
        assert torch.equal(s.m.to_fp32(), P.make_store(precision, s.numel, "m", init=m, device=DEV).to_fp32())
    for x, y in zip(masters, opt.master_params()):
        assert torch.equal(x, y)
    opt.close()


# ------------------------------------------------------- randomized schedules

def _schedule(seed, steps):
    """A seeded sequence of (event, micro-batches): how each step is driven, and whether a checkpoint
    reload into a new optimizer or a change of moment precision comes first."""
    rng = np.random.default_rng(seed)
    events = []
    for _ in range(steps):
        before = rng.choice(["none", "none", "reload", "precision"])
        events.append((str(before), str(rng.choice(["step", "hooks"])), int(rng.integers(1, 4)),
                       str(rng.choice(["fp32", "bf16", "fp8"]))))
    return events


@pytest.mark.parametrize("lion", [False, True])
@pytest.mark.parametrize("master", ["fp32", "fp24"])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_schedules_match_plain_steps(seed, master, lion):
    """Any mix of plain steps, hooked steps, accumulation over no_sync() micro-batches, checkpoint
    reloads (through torch.save/load) into a new optimizer, and moment precision changes gives the
    same bytes -- weights, masters, moments -- as plain step() calls on the same gradients with the
    same precision changes (reference optimizer.py:291-355, 453-463, 525-602)."""
    cls = ab.LionBridge if lion else ab.AdamBridge
    kw = dict(lr=2e-3, weight_decay=0.01, master_precision=master, small_param_threshold=2000)
    if not lion:
        kw["eps"] = 1e-8

    def make(model, precision):
        return cls(model.parameters(), precision=precision, **kw)

    torch.manual_seed(seed)
    ref_model = TinyLM(layers=2).to(DEV).to(torch.bfloat16)
    model = copy.deepcopy(ref_model)
    precision = "bf16"
    ref, opt = make(ref_model, precision), make(model, precision)
    hooked = False
    g = torch.Generator().manual_seed(100 + seed)
    for step, (before, mode, micros, target) in enumerate(_schedule(seed, 12)):
        if before == "reload":
            buf = io.BytesIO()
            torch.save(opt.state_dict(), buf)
            opt.close()
            buf.seek(0)
            opt = make(model, precision)
            opt.load_state_dict(torch.load(buf, weights_only=True))
            hooked = False
        elif before == "precision" and target != precision:
            precision = target
            ref.set_precision(precision)
            opt.set_precision(precision)
            assert ref.precision == opt.precision == precision
        grads = [[(torch.randn(p.shape, generator=g) * 0.05).to(device=DEV, dtype=torch.bfloat16)
                  for p in ref_model.parameters()] for _ in range(micros)]
        for gs in grads:
            sum((p * x).sum() for p, x in zip(ref_model.parameters(), gs)).backward()
        ref.step()
        ref.zero_grad(set_to_none=True)
        if mode == "hooks" and not hooked:
            opt.attach_hooks(model)
        elif mode == "step" and hooked:
            opt.detach_hooks()
        hooked = mode == "hooks"
        for i, gs in enumerate(grads):
            loss = sum((p * x).sum() for p, x in zip(model.parameters(), gs))
            if hooked and i < micros - 1:
                with opt.no_sync():
                    loss.backward()
            else:
                loss.backward()
        if hooked:
            opt.step_sync()
        else:
            opt.step()
            opt.zero_grad(set_to_none=True)
        assert all(torch.equal(a, b) for a, b in zip(ref_model.parameters(), model.parameters())), \
            f"weights differ after step {step} ({before}, {mode}, {micros} micro-batches, {precision})"
    assert all(torch.equal(a, b) for a, b in zip(ref.master_params(), opt.master_params()))
    for a, b in zip(ref._ordered, opt._ordered):
        assert a.step == b.step
        assert torch.equal(a.m.to_fp32(), b.m.to_fp32())
        if not lion:
            assert torch.equal(a.v.to_fp32(), b.v.to_fp32())
    ref.close()
    opt.close()
