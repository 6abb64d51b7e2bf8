"""AdamBridge inside other training loops (GPU): an unmodified Hugging Face Trainer, and models
under torch.compile with the gradient hooks attached (reference tests/test_hf_trainer.py:15-47,
tests/test_compile.py:20-99).

The hook is wrapped in ``torch.compiler.disable``, so Dynamo and compiled autograd call it as an
opaque function; the update it launches is the same HIP kernel launch as in eager mode.  Not
covered: ``mode="reduce-overhead"`` (graph capture of the backward pass while hooks enqueue work on
another stream).
"""

import copy
import tempfile

import pytest
import torch

import adambridge_amd as ab
from conftest import max_param_diff
from test_optimizer_gpu import DEV, TinyLM, _stale_reference, lm_loss

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


# ------------------------------------------------------------ Hugging Face Trainer

def _train_with_trainer(make_opt, accumulation: int):
    torch.manual_seed(0)
    cfg = transformers.LlamaConfig(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    model = transformers.LlamaForCausalLM(cfg).to(DEV)
    g = torch.Generator().manual_seed(0)
    data = [{"input_ids": ids, "labels": ids} for ids in torch.randint(0, 128, (32, 16), generator=g)]
    with tempfile.TemporaryDirectory() as tmp:
        args = transformers.TrainingArguments(
            output_dir=tmp, per_device_train_batch_size=4, gradient_accumulation_steps=accumulation, max_steps=4,
            learning_rate=1e-3, lr_scheduler_type="constant", weight_decay=0.0, max_grad_norm=0.0, report_to=[],
            logging_strategy="no", save_strategy="no", seed=0, data_seed=0, dataloader_pin_memory=False,
            disable_tqdm=True)
        opt = make_opt(model, accumulation)
        transformers.Trainer(model=model, args=args, train_dataset=data, optimizers=(opt, None)).train()
    if isinstance(opt, ab.AdamBridge):
        opt.close()
    return model


@pytest.mark.parametrize("accumulation", [1, 2])
@pytest.mark.parametrize("delay", [False, True])
def test_hf_trainer_matches_torch_adamw(accumulation, delay):
    ref = _train_with_trainer(lambda m, a: torch.optim.AdamW(m.parameters(), lr=1e-3, weight_decay=0.0),
                              accumulation)
    model = _train_with_trainer(
        lambda m, a: ab.AdamBridge(m.parameters(), lr=1e-3, weight_decay=0.0, delay_updates=delay,
                                   accumulation_steps=a).attach_hooks(m), accumulation)
    # delayed updates train with weights one step stale by design: the same model, loosely
    assert max_param_diff(ref, model) < (5e-3 if delay else 1e-5)


# ------------------------------------------------------------------ torch.compile

@pytest.fixture
def fresh_dynamo():
    torch._dynamo.reset()
    yield
    torch._dynamo.reset()


def _per_block(model):
    for blk in model.blocks:
        blk.compile()
    return model


# The reference's modes (tests/test_compile.py:23-28).  reduce-overhead replays the model's forward and
# backward as HIP graphs; the optimizer's hooks run eagerly between those replays (the hook is
# opaque to Dynamo and the post-accumulate-grad hooks fire outside the compiled backward), so no
# launch of the optimizer is captured.
COMPILERS = {
    "whole-model": lambda m: torch.compile(m),
    "reduce-overhead": lambda m: torch.compile(m, mode="reduce-overhead"),
    "max-autotune": lambda m: torch.compile(m, mode="max-autotune"),
    "per-block": _per_block,
}


def _reference(model, steps=6):
    ref_model = copy.deepcopy(model)
    ref = torch.optim.AdamW(ref_model.parameters(), lr=3e-3)
    for step in range(steps):
        ref.zero_grad()
        lm_loss(ref_model, step).backward()
        ref.step()
    return ref_model


def _train_hooked(fwd, opt, steps=6, compiled_autograd=False):
    for step in range(steps):
        loss = lm_loss(fwd, step)
        if compiled_autograd:
            with torch._dynamo.compiled_autograd._enable(torch.compile):
                loss.backward()
        else:
            loss.backward()
        opt.step_sync()


@pytest.mark.parametrize("how", list(COMPILERS))
def test_compiled_model_with_hooks_matches_torch_adamw(how, fresh_dynamo):
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    ref_model = _reference(model)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, small_param_threshold=0).attach_hooks(model)
    _train_hooked(COMPILERS[how](model), opt)
    assert max_param_diff(ref_model, model) < 1e-5
    opt.close()


def test_compiled_autograd_calls_the_hook_opaquely(fresh_dynamo):
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    ref_model = _reference(model)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3).attach_hooks(model)
    _train_hooked(torch.compile(model), opt, compiled_autograd=True)
    assert max_param_diff(ref_model, model) < 1e-5
    opt.close()


@pytest.mark.parametrize("how", ["per-block", "reduce-overhead"])
def test_delayed_updates_under_compile(how, fresh_dynamo):
    """Delayed updates (one-step-stale weights) under per-block compile and under HIP-graph replay of
    the model (reference tests/test_compile.py:82-99)."""
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    want_losses, want = _stale_reference(copy.deepcopy(model), 8, lambda ps: torch.optim.AdamW(ps, lr=3e-3), 0)
    opt = ab.AdamBridge(model.parameters(), lr=3e-3, delay_updates=True).attach_hooks(model)
    fwd = COMPILERS[how](model)
    losses = []
    for k in range(1, 9):
        loss = lm_loss(fwd, k)
        loss.backward()
        opt.step_sync()
        losses.append(loss.item())
    opt.flush()
    assert max(abs(a - b) for a, b in zip(losses, want_losses)) < 1e-3
    assert max((p - w).abs().max().item() for p, w in zip(model.parameters(), want)) < 1e-5
    opt.close()
