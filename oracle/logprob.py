"""Selected-token logprobs and their gradient, restated on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

from __future__ import annotations

from typing import Optional

import torch


def _masks(target: torch.Tensor, vocab_start: int, vocab_end: int):
    # reference model_utils.py:250-254: out-of-range targets are masked to index 0
    target_mask = (target < vocab_start) | (target >= vocab_end)
    masked_target = target - vocab_start
    masked_target = masked_target.masked_fill(target_mask, 0)
    return target_mask, masked_target


def selected_logprobs(
    logits: torch.Tensor,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    chunk_size: Optional[int] = None,
) -> torch.Tensor:
    """[B, S, V] logits, [B, S] targets -> [B, S] fp32 logprobs.

    Restates ChunkedDistributedLogprob.forward (reference model_utils.py:240-290)
    with _compute_distributed_selected_logprobs (model_utils.py:87-135) at TP=1:
    per sequence chunk, upcast to fp32, subtract the row max, gather the
    target, exponentiate and sum, subtract log(sum); zero masked targets.
    """
    target_mask, masked_target = _masks(target, vocab_start, vocab_end)
    S = logits.shape[1]
    cs = S if chunk_size is None else chunk_size
    outs = []
    for c0 in range(0, S, cs):
        c1 = min(S, c0 + cs)
        x = logits[:, c0:c1].to(torch.float32)
        m = torch.amax(x, dim=-1, keepdim=True)
        shifted = x - m
        sel = torch.gather(shifted, -1, masked_target[:, c0:c1].unsqueeze(-1)).squeeze(-1)
        s = shifted.exp().sum(-1, keepdim=True).float()
        lp = sel - s.log().squeeze(-1)
        lp = lp.masked_fill(target_mask[:, c0:c1], 0.0)
        outs.append(lp)
    return torch.cat(outs, dim=1)


def selected_logprobs_grad(
    logits: torch.Tensor,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    grad_output: torch.Tensor,
    chunk_size: Optional[int] = None,
    out_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """Gradient w.r.t. the logits, in the logits dtype (or ``out_dtype``).

    Restates ChunkedDistributedLogprob.backward (reference model_utils.py:293-349):
    per chunk, fp32 log-softmax recomputed as (x - max) - log(sum exp(x - max))
    (model_utils.py:38-72), p = exp(.), grad = (onehot - p) * g, copied into
    a tensor of the logits dtype.
    """
    target_mask, masked_target = _masks(target, vocab_start, vocab_end)
    B, S, V = logits.shape
    cs = S if chunk_size is None else chunk_size
    grad = torch.zeros(logits.shape, dtype=out_dtype or logits.dtype)
    for c0 in range(0, S, cs):
        c1 = min(S, c0 + cs)
        x = logits[:, c0:c1].to(torch.float32)
        m = torch.amax(x, dim=-1, keepdim=True)
        xs = x - m
        lsm = xs - xs.exp().sum(-1, keepdim=True).float().log()
        p = lsm.exp()
        chosen = (~target_mask[:, c0:c1]).unsqueeze(-1) * torch.nn.functional.one_hot(
            masked_target[:, c0:c1], num_classes=V
        )
        g = (chosen.float() - p) * grad_output[:, c0:c1].unsqueeze(-1).float()
        grad[:, c0:c1] = g.to(grad.dtype)
    return grad


def next_token_logprobs(
    logits: torch.Tensor, input_ids: torch.Tensor, chunk_size: Optional[int] = None
) -> torch.Tensor:
    """from_parallel_logits_to_logprobs at TP=CP=1 (reference model_utils.py:967-1062).

    Targets are rolled by -1, the whole [B, S] is computed, the last column dropped.
    """
    V = logits.shape[-1]
    target = input_ids.roll(shifts=-1, dims=-1)
    pad = logits.shape[1] - target.shape[1]
    if pad > 0:
        target = torch.nn.functional.pad(target, (0, pad), value=0)
    lp = selected_logprobs(logits, target, 0, V, chunk_size)
    if pad > 0:
        lp = lp[:, :-pad]
    return lp[:, :-1]


def next_token_logprobs_grad(
    logits: torch.Tensor,
    input_ids: torch.Tensor,
    grad_output: torch.Tensor,
    chunk_size: Optional[int] = None,
    out_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """Gradient of next_token_logprobs: the last row's upstream gradient is zero."""
    V = logits.shape[-1]
    target = input_ids.roll(shifts=-1, dims=-1)
    g = torch.zeros(target.shape, dtype=torch.float32)
    g[:, : grad_output.shape[1]] = grad_output.float()
    return selected_logprobs_grad(logits, target, 0, V, g, chunk_size, out_dtype)


def closed_form_logprobs_f64(logits: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """log_softmax(x)[t] in float64 (the baseline the reference tests use,
    tests/unit/distributed/test_distributed_logprob.py:38-45)."""
    return torch.log_softmax(logits.double(), dim=-1).gather(-1, target.unsqueeze(-1)).squeeze(-1)


def pack_targets(input_ids_packed: torch.Tensor, cu_seqlens: list[int]) -> torch.Tensor:
    """Per-sequence roll by -1 inside packed boundaries (reference model_utils.py:1116-1139)."""
    t = input_ids_packed.reshape(-1)
    out = torch.zeros_like(t)
    for i in range(len(cu_seqlens) - 1):
        a, b = cu_seqlens[i], cu_seqlens[i + 1]
        out[a:b] = t[a:b].roll(shifts=-1, dims=0)
    return out.unsqueeze(0)


def unpack_logprobs(probs: torch.Tensor, cu_seqlens: list[int], unpacked_seqlen: int) -> torch.Tensor:
    """Drop the last position of each sequence and unpack (reference model_utils.py:1211-1231)."""
    probs = probs.reshape(-1)
    n = len(cu_seqlens) - 1
    out = torch.zeros((n, unpacked_seqlen - 1), dtype=probs.dtype)
    for i in range(n):
        a, b = cu_seqlens[i], cu_seqlens[i + 1]
        if b - a > 0:
            seq = probs[a : b - 1]
            k = min(seq.shape[0], unpacked_seqlen - 1)
            if k > 0:
                out[i, :k] = seq[:k]
    return out


def pack_input_ids(
    input_ids: torch.Tensor, cu_seqlens_q: list[int], cu_seqlens_q_padded: list[int], roll_shift: int = 0
) -> torch.Tensor:
    """[B, S, ...] -> [1, T_padded, ...] (reference loss/utils.py:355-408 at CP = 1).

    Each sequence is zero-padded to its padded length, its first
    min(actual_len, S) tokens copied, optionally rolled, and placed at its
    padded start.
    """
    B = input_ids.shape[0]
    tail = tuple(input_ids.shape[2:])
    packed = torch.zeros((cu_seqlens_q_padded[-1], *tail), dtype=input_ids.dtype)
    for i in range(B):
        actual = cu_seqlens_q[i + 1] - cu_seqlens_q[i]
        padded = cu_seqlens_q_padded[i + 1] - cu_seqlens_q_padded[i]
        seq = torch.zeros((padded, *tail), dtype=input_ids.dtype)
        n = min(actual, input_ids.shape[1])
        seq[:n] = input_ids[i, :n]
        if roll_shift != 0:
            seq = seq.roll(shifts=roll_shift, dims=0)
        packed[cu_seqlens_q_padded[i] : cu_seqlens_q_padded[i] + padded] = seq
    return packed.unsqueeze(0)
