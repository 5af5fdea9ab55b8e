"""Logprobs from hidden states and the output weight, restated on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Follows
ChunkedDistributedHiddenStatesToLogprobs at TP=1 (reference
nemo_rl/distributed/model_utils.py:2576-2745) and
from_parallel_hidden_states_to_logprobs (model_utils.py:2541-2569).

The reference's logits are the output of a matmul in the inputs' dtype: an
fp32 sum of products, rounded once to that dtype.  Here the sum is taken
exactly (float64) and rounded once to the dtype (``logits_bf16``); a GPU's fp32
sum of the same products can land on the other side of a rounding boundary, so
individual logits may differ by one ulp of the dtype.  The backward follows the reference in float64
from those logits: ``grad_input = (onehot - softmax) * g`` (model_utils.py:2682-2700),
``dH = grad_input . W`` (2701-2703), ``dW = sum over chunks of H^T . grad_input``
(2704-2716).
"""

from __future__ import annotations

from typing import Optional

import torch

from oracle.logprob import _masks


def logits_bf16(hidden: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """[S, B, H] x [V, H] -> [B, S, V] float32 holding the exact products rounded once to
    the inputs' dtype (the reference's matmul output dtype: bf16, fp16 or fp32)."""
    x = torch.matmul(hidden.double(), weight.double().t())  # [S, B, V]
    return x.to(hidden.dtype).float().transpose(0, 1).contiguous()


def hidden_state_logprobs(
    hidden: torch.Tensor,
    target: torch.Tensor,
    weight: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    chunk_size: Optional[int] = None,
) -> torch.Tensor:
    """ChunkedDistributedHiddenStatesToLogprobs.forward: [B, S] fp32 (target already rolled).

    Per chunk of sequence positions (reference model_utils.py:2608-2630): logits
    in fp32, then _compute_distributed_selected_logprobs (max, shifted gather,
    exp-sum, subtract log).
    """
    target_mask, masked_target = _masks(target, vocab_start, vocab_end)
    S = hidden.shape[0]
    cs = S if chunk_size is None else chunk_size
    outs = []
    for c0 in range(0, S, cs):
        c1 = min(S, c0 + cs)
        x = logits_bf16(hidden[c0:c1], weight)  # [B, c, V] fp32
        m = torch.amax(x, dim=-1, keepdim=True)
        shifted = x - m
        sel = torch.gather(shifted, -1, masked_target[:, c0:c1].unsqueeze(-1)).squeeze(-1)
        s = shifted.exp().sum(-1, keepdim=True)
        lp = sel - s.log().squeeze(-1)
        outs.append(lp.masked_fill(target_mask[:, c0:c1], 0.0))
    return torch.cat(outs, dim=1)


def hidden_state_logprob_grads(
    hidden: torch.Tensor,
    target: torch.Tensor,
    weight: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    grad_output: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Float64 (dH [S, B, H], dW [V, H], grad_input [B, S, V]) of the backward.

    grad_input = (onehot(t) * ~mask - exp(log_softmax(x))) * g (reference
    model_utils.py:2682-2700); dH = grad_input . W (2701-2703), transposed back to
    sequence-first (2717-2719); dW = sum_{b,s} grad_input^T . H (2704-2716).
    """
    target_mask, masked_target = _masks(target, vocab_start, vocab_end)
    x = logits_bf16(hidden, weight).double()  # [B, S, V]
    V = weight.shape[0]
    logp = x - x.amax(-1, keepdim=True)
    logp = logp - logp.exp().sum(-1, keepdim=True).log()
    p = logp.exp()
    chosen = torch.nn.functional.one_hot(masked_target, num_classes=V).double()
    chosen = chosen * (~target_mask).unsqueeze(-1).double()
    gi = (chosen - p) * grad_output.double().unsqueeze(-1)  # [B, S, V]
    dh = torch.matmul(gi, weight.double())  # [B, S, H]
    dw = torch.einsum("bsv,bsh->vh", gi, hidden.double().transpose(0, 1))
    return dh.transpose(0, 1).contiguous(), dw, gi


def next_token_hidden_state_logprobs(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    chunk_size: Optional[int] = None,
) -> torch.Tensor:
    """from_parallel_hidden_states_to_logprobs: roll targets by -1, drop the last column."""
    rolled = target.roll(shifts=-1, dims=-1)
    return hidden_state_logprobs(hidden, rolled, weight, vocab_start, vocab_end, chunk_size)[:, :-1]
