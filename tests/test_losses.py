"""causal_lm_loss: value and gradients of the Hugging Face causal-LM loss, computed a slice of
positions at a time (reference tests/test_losses.py:43-65).  Plain PyTorch, CPU."""

import pytest
import torch

import adambridge_amd as ab

transformers = pytest.importorskip("transformers")

VOCAB = 256


def _model(seed=0, hidden=64, tied=True):
    torch.manual_seed(seed)
    cfg = transformers.Qwen2Config(vocab_size=VOCAB, hidden_size=hidden, intermediate_size=2 * hidden,
                                   num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                                   max_position_embeddings=256, tie_word_embeddings=tied)
    return transformers.Qwen2ForCausalLM(cfg)


def _ids(shape, seed=1):
    return torch.randint(0, VOCAB, shape, generator=torch.Generator().manual_seed(seed))


def _hf(model, ids, labels):
    loss = model(input_ids=ids, labels=labels).loss
    loss.backward()
    grads = [p.grad.clone() for p in model.parameters()]
    model.zero_grad(set_to_none=True)
    return loss.detach(), grads


def _sliced(model, ids, labels, chunk):
    hidden = model.model(input_ids=ids).last_hidden_state
    loss = ab.causal_lm_loss(hidden, model.lm_head, labels, chunk_tokens=chunk)
    loss.backward()
    grads = [p.grad.clone() for p in model.parameters()]
    model.zero_grad(set_to_none=True)
    return loss.detach(), grads


@pytest.mark.parametrize("chunk", [1, 7, 64, 10_000])
@pytest.mark.parametrize("tied", [True, False])
def test_matches_the_hugging_face_loss_and_gradients(chunk, tied):
    model = _model(tied=tied)
    ids = _ids((3, 40))
    want, want_g = _hf(model, ids, ids)
    got, got_g = _sliced(model, ids, ids, chunk)
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-6)
    for a, b in zip(got_g, want_g):
        assert torch.allclose(a, b, rtol=1e-4, atol=1e-6)


def test_ignore_index_and_no_grad():
    model = _model()
    ids = _ids((2, 33))
    labels = ids.clone()
    labels[0, 5:20] = -100
    labels[1, -3:] = -100
    want, _ = _hf(model, ids, labels)
    with torch.no_grad():
        hidden = model.model(input_ids=ids).last_hidden_state
        got = ab.causal_lm_loss(hidden, model.lm_head, labels, chunk_tokens=5)
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-6)
    # every target ignored: zero, not NaN
    with torch.no_grad():
        empty = ab.causal_lm_loss(hidden, model.lm_head, torch.full_like(ids, -100))
    assert empty.item() == 0.0


def test_argument_checks():
    h = torch.zeros(2, 3, 4)
    head = torch.nn.Linear(4, 5)
    with pytest.raises(ValueError):
        ab.causal_lm_loss(h[0], head, torch.zeros(2, 3, dtype=torch.long))
    with pytest.raises(ValueError):
        ab.causal_lm_loss(h, head, torch.zeros(2, 4, dtype=torch.long))
    for bad in (0, -1, 1.5, True):
        with pytest.raises(ValueError):
            ab.causal_lm_loss(h, head, torch.zeros(2, 3, dtype=torch.long), chunk_tokens=bad)
