"""Next-token cross-entropy without the full logits tensor (the reference's adambridge/losses.py API).

The output projection of a large-vocabulary model turns [batch, seq, hidden] activations into
[batch, seq, vocab] logits -- gigabytes in FP32 for a 150k vocabulary -- which training then
keeps for the backward pass.  ``causal_lm_loss`` projects a slice of positions at a time and,
with gradients enabled, recomputes each slice's logits in the backward pass instead of keeping
them, so at most one slice of logits exists at once.  Plain PyTorch: this is off the optimizer's
path and runs wherever the model runs.
"""

from __future__ import annotations

from typing import Callable

import torch
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

__all__ = ["causal_lm_loss"]


def _slice_loss_sum(h: torch.Tensor, target: torch.Tensor, project: Callable[[torch.Tensor], torch.Tensor],
                    ignore_index: int) -> torch.Tensor:
    """Summed cross-entropy of one slice, logits upcast to FP32."""
    logits = project(h).float()
    return F.cross_entropy(logits, target, ignore_index=ignore_index, reduction="sum")


def causal_lm_loss(hidden_states: torch.Tensor, lm_head: Callable[[torch.Tensor], torch.Tensor],
                   labels: torch.Tensor, *, chunk_tokens: int = 1024, ignore_index: int = -100) -> torch.Tensor:
    """Mean next-token cross-entropy of ``lm_head(hidden_states)`` against ``labels``, evaluated
    ``chunk_tokens`` positions at a time (reference adambridge/losses.py:27-70).

    Position ``t`` is scored against ``labels[:, t + 1]`` (the last position of each sequence has
    no target); the mean runs over positions whose target is not ``ignore_index`` -- the Hugging
    Face causal-LM loss.  ``hidden_states``: ``[batch, seq, hidden]``; ``lm_head``: a module or
    function mapping ``[n, hidden]`` to ``[n, vocab]``; ``labels``: ``[batch, seq]`` token ids.
    With gradients enabled, each slice runs under non-reentrant ``torch.utils.checkpoint``.
    """
    if hidden_states.dim() != 3:
        raise ValueError(f"hidden_states must be [batch, seq, hidden], got shape {tuple(hidden_states.shape)}")
    if tuple(labels.shape) != tuple(hidden_states.shape[:2]):
        raise ValueError(f"labels must be [batch, seq] = {tuple(hidden_states.shape[:2])}, got {tuple(labels.shape)}")
    if isinstance(chunk_tokens, bool) or not isinstance(chunk_tokens, int) or chunk_tokens < 1:
        raise ValueError("chunk_tokens must be a positive int")
    b, s, d = hidden_states.shape
    h = hidden_states.reshape(b * s, d)
    # targets: each sequence shifted left by one, its last position ignored
    targets = torch.full((b, s), ignore_index, dtype=labels.dtype, device=labels.device)
    targets[:, :-1] = labels[:, 1:]
    targets = targets.reshape(-1).to(h.device)
    n_scored = (targets != ignore_index).sum()
    recompute = torch.is_grad_enabled() and h.requires_grad
    total = h.new_zeros((), dtype=torch.float32)
    for h_part, t_part in zip(torch.split(h, chunk_tokens), torch.split(targets, chunk_tokens)):
        if recompute:
            total = total + checkpoint(_slice_loss_sum, h_part, t_part, lm_head, ignore_index, use_reentrant=False)
        else:
            total = total + _slice_loss_sum(h_part, t_part, lm_head, ignore_index)
    return total / n_scored.clamp(min=1)
