"""Logprobs at K ids per row, and the student/teacher divergences, restated on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

from __future__ import annotations

from typing import Optional

import torch


def _log_softmax_fp32(x: torch.Tensor) -> torch.Tensor:
    """(x - max) - log(sum exp(x - max)) in fp32 (reference model_utils.py:38-72 at TP=1)."""
    x = x.to(torch.float32)
    m = torch.amax(x, dim=-1, keepdim=True)
    z = x - m
    s = z.exp().sum(-1, keepdim=True).float()
    return z - s.log()


def gather_logprobs(
    logits: torch.Tensor,
    indices: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    chunk_size: Optional[int] = None,
) -> torch.Tensor:
    """[B, S, V] logits, [B, S, K] ids -> [B, S, K] fp32 (ChunkedDistributedGatherLogprob.forward,
    reference model_utils.py:703-748): per sequence chunk, fp32 log-softmax, gather at the
    clamped local ids, times the in-range mask."""
    B, S, V = logits.shape
    cs = S if chunk_size is None else chunk_size
    outs = []
    for s0 in range(0, S, cs):
        s1 = min(S, s0 + cs)
        lp = _log_softmax_fp32(logits[:, s0:s1])
        gi = indices[:, s0:s1]
        in_range = (gi >= vocab_start) & (gi < vocab_end)
        li = (gi - vocab_start).clamp(min=0, max=V - 1)
        vals = torch.gather(lp, -1, li)
        outs.append(vals * in_range.to(vals.dtype))
    return torch.cat(outs, dim=1)


def gather_logprobs_grad(
    logits: torch.Tensor,
    indices: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    grad_output: torch.Tensor,
    chunk_size: Optional[int] = None,
    out_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """ChunkedDistributedGatherLogprob.backward (reference model_utils.py:750-805): fp32
    grad = -softmax * sum_k g_k, then scatter_add of the in-range g_k at the ids; the fp32
    result is rounded to the logits dtype (what autograd does with it)."""
    B, S, V = logits.shape
    cs = S if chunk_size is None else chunk_size
    grad = torch.zeros((B, S, V), dtype=torch.float32)
    for s0 in range(0, S, cs):
        s1 = min(S, s0 + cs)
        p = _log_softmax_fp32(logits[:, s0:s1]).exp()
        gi = indices[:, s0:s1]
        in_range = (gi >= vocab_start) & (gi < vocab_end)
        li = (gi - vocab_start).clamp(min=0, max=V - 1)
        go = grad_output[:, s0:s1].float()
        chunk = grad[:, s0:s1]
        chunk.copy_(p.neg().mul_(go.sum(dim=-1, keepdim=True)))
        chunk.scatter_add_(2, li, go * in_range.to(go.dtype))
    return grad.to(out_dtype or logits.dtype)


def divergence(
    kind: str,
    student: torch.Tensor,
    teacher: Optional[torch.Tensor],
    chunk_size: Optional[int] = None,
) -> torch.Tensor:
    """Per-row sum_v p_s(v) * w(v), fp32 [B, S] (reference model_utils.py:2377-2434);
    w = log p_s (entropy), -log p_t (cross entropy), log p_s - log p_t (reverse KL)."""
    S = student.shape[1]
    cs = S if chunk_size is None else chunk_size
    outs = []
    for s0 in range(0, S, cs):
        s1 = min(S, s0 + cs)
        ls = _log_softmax_fp32(student[:, s0:s1])
        lt = None if teacher is None else _log_softmax_fp32(teacher[:, s0:s1])
        outs.append((ls.exp() * _weight(kind, ls, lt)).sum(dim=-1))
    return torch.cat(outs, dim=1)


def divergence_grad(
    kind: str,
    student: torch.Tensor,
    teacher: Optional[torch.Tensor],
    grad_output: torch.Tensor,
    chunk_size: Optional[int] = None,
) -> torch.Tensor:
    """(p_s * (w - L)) * g in fp32, copied into the logits dtype
    (reference model_utils.py:2437-2499)."""
    S = student.shape[1]
    cs = S if chunk_size is None else chunk_size
    grad = torch.empty_like(student)
    for s0 in range(0, S, cs):
        s1 = min(S, s0 + cs)
        ls = _log_softmax_fp32(student[:, s0:s1])
        lt = None if teacher is None else _log_softmax_fp32(teacher[:, s0:s1])
        w = _weight(kind, ls, lt)
        p = ls.exp()
        red = (p * w).sum(dim=-1)
        grad[:, s0:s1].copy_(p.mul_(w - red.unsqueeze(-1)).mul_(grad_output[:, s0:s1].float().unsqueeze(-1)))
    return grad


def _weight(kind: str, ls: torch.Tensor, lt: Optional[torch.Tensor]) -> torch.Tensor:
    # reference model_utils.py:2354-2374
    if kind == "entropy":
        return ls
    if kind == "cross_entropy":
        return -lt
    if kind == "reverse_kl":
        return ls - lt
    raise ValueError(kind)


def divergence_f64(kind: str, student: torch.Tensor, teacher: Optional[torch.Tensor]) -> torch.Tensor:
    """Closed forms in float64: sum p log p, -sum p log q, KL(p || q)."""
    ls = torch.log_softmax(student.double(), dim=-1)
    p = ls.exp()
    if kind == "entropy":
        return (p * ls).sum(-1)
    lt = torch.log_softmax(teacher.double(), dim=-1)
    if kind == "cross_entropy":
        return -(p * lt).sum(-1)
    return (p * (ls - lt)).sum(-1)


def vocab_topk(logits: torch.Tensor, k: int, vocab_start: int = 0):
    """(values fp32, global ids) of the k largest logits per row, descending, equal values
    by ascending position (distributed_vocab_topk at TP=1, reference model_utils.py:1867-1935,
    is torch.topk of the fp32 logits plus the vocabulary offset; the tie order is this build's
    choice, a stable descending sort)."""
    x = logits.float()
    vals, idx = torch.sort(x, dim=-1, descending=True, stable=True)
    return vals[..., :k].contiguous(), idx[..., :k] + vocab_start
