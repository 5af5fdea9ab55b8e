"""Other reductions over the vocabulary: logprobs at K ids per row, the
student/teacher entropy, cross entropy and reverse KL, and the top-k export.

Drop-ins, with a vocab group of size 1, for these names of
``nemo_rl.distributed.model_utils``:

* ``ChunkedDistributedGatherLogprob`` and ``get_policy_logprobs_at_sampler_topk``
  (reference model_utils.py:691-805, 1723-1865), the score-centering inputs;
* ``ChunkedDistributedEntropy``, ``ChunkedDistributedCrossEntropyToFixedLogits``
  and ``ChunkedDistributedReverseKLToFixedLogits`` (model_utils.py:2199-2538);
* ``distributed_vocab_topk`` (model_utils.py:1867-1935), the teacher top-k export.

Each forward is one streaming pass over the logits row (both rows for the
teacher divergences) in a gfx950 kernel; each backward is one read and one write
per row.  ``chunk_size`` is validated and kept in the signatures but does not
change results, since every row is independent.
"""

from __future__ import annotations

from typing import Any, Optional

import torch

from rl_amd import _C
from rl_amd.distributed.early_backward import POLICY

__all__ = [
    "ChunkedDistributedCrossEntropyToFixedLogits",
    "ChunkedDistributedEntropy",
    "ChunkedDistributedGatherLogprob",
    "ChunkedDistributedReverseKLToFixedLogits",
    "distributed_vocab_topk",
    "get_policy_logprobs_at_sampler_topk",
    "next_token_and_sampler_topk_logprobs",
]


def _single_rank(group: Optional[Any]) -> None:
    from rl_amd.distributed.model_utils import _require_single_rank

    _require_single_rank(group)


def _chunk(chunk_size: Optional[int]) -> None:
    if chunk_size is not None and int(chunk_size) <= 0:
        raise ValueError("chunk_size must be positive")


def _unit_stride(x: torch.Tensor) -> torch.Tensor:
    return x if x.stride(-1) == 1 else x.contiguous()


class ChunkedDistributedGatherLogprob(torch.autograd.Function):
    """Log-softmax at given ids: ``[B, S, V]`` logits, ``[B, S, K]`` ids -> ``[B, S, K]`` fp32.

    Reference: model_utils.py:691-805.  Ids outside
    ``[vocab_start_index, vocab_end_index)`` give 0.  The backward is
    ``-softmax * sum_k g_k`` plus ``g_k`` at each in-range id, in the logits dtype.
    """

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        vocab_parallel_logits: torch.Tensor,
        global_indices: torch.Tensor,
        vocab_start_index: int,
        vocab_end_index: int,
        chunk_size: int,
        tp_group: Optional[Any],
        inference_only: bool = False,
    ) -> torch.Tensor:
        _single_rank(tp_group)
        _chunk(chunk_size)
        logits = vocab_parallel_logits
        if logits.dim() != 3:
            raise ValueError(f"expected logits of shape [B, S, V], got {tuple(logits.shape)}")
        logits = _unit_stride(logits)
        B, S, _ = logits.shape
        if global_indices.dim() != 3 or tuple(global_indices.shape[:2]) != (B, S):
            raise ValueError(
                f"indices shape {tuple(global_indices.shape)} does not match logits rows {(B, S)}"
            )
        idx = global_indices if global_indices.dtype == torch.int64 else global_indices.long()
        K = idx.shape[2]
        out = torch.empty((B, S, K), dtype=torch.float32, device=logits.device)
        stats = None
        if not inference_only:
            stats = torch.empty((B, S, 2), dtype=torch.float32, device=logits.device)
        _C.gather_logprob_fwd(logits, idx, vocab_start_index, vocab_end_index, out, stats)
        if not inference_only:
            ctx.save_for_backward(logits, idx, stats)
            ctx.vocab = (int(vocab_start_index), int(vocab_end_index))
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):  # type: ignore[override]
        (grad_output,) = grad_outputs
        logits, idx, stats = ctx.saved_tensors
        vs, ve = ctx.vocab
        if idx.shape[2] == 0:
            return torch.zeros_like(logits), None, None, None, None, None, None
        if grad_output.dtype != torch.float32:
            grad_output = grad_output.float()
        early = getattr(ctx, "early", None)
        if early is not None:
            # launched by launch_early_backward: check it against the real gradient
            ctx.early = None
            grad_input, grad_used = early
            POLICY.checked(
                _C.gather_logprob_bwd_recheck(logits, idx, vs, ve, stats, grad_output, grad_used, grad_input))
            return grad_input, None, None, None, None, None, None
        grad_input = torch.empty_like(logits)
        _C.gather_logprob_bwd(logits, idx, vs, ve, stats, grad_output, grad_input)
        return grad_input, None, None, None, None, None, None


def get_policy_logprobs_at_sampler_topk(
    sampler_topk_token_ids: torch.Tensor,
    next_token_logits: torch.Tensor,
    vocab_parallel_rank: Optional[int] = None,
    vocab_parallel_group: Optional[Any] = None,
    context_parallel_group: Optional[Any] = None,
    chunk_size: Optional[int] = None,
    cp_sharder: Optional[Any] = None,
    cu_seqlens_q: Optional[Any] = None,
    cu_seqlens_q_padded: Optional[Any] = None,
    packed_sampler_topk_token_ids: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Next-token log-probs ``[B, S - 1, k]`` at the sampler's top-k ids (reference model_utils.py:1723-1865).

    ``sampler_topk_token_ids`` ``[B, S, k]`` is token-aligned (row t holds the
    ids ranked when token t was drawn), so it is rolled by one to line up with
    the logits.  With packed boundaries, ``packed_sampler_topk_token_ids``
    ``[1, T, k]`` holds the caller-packed, next-token-aligned ids and each
    sequence is unpacked into its own row.
    """
    from rl_amd.distributed.model_utils import _group_size, _is_dtensor

    if cp_sharder is not None or _is_dtensor(next_token_logits):
        raise NotImplementedError(
            "score centering supports the Megatron vocab-parallel and single-device paths"
        )
    if (cu_seqlens_q is None) != (cu_seqlens_q_padded is None):
        raise ValueError("Both packed sequence boundary tuples must be supplied together")
    _single_rank(vocab_parallel_group)
    if _group_size(context_parallel_group) != 1:
        raise NotImplementedError("context parallelism is not supported (CP = 1)")
    if chunk_size is None:
        chunk_size = int(next_token_logits.shape[1])
    dev = next_token_logits.device
    if cu_seqlens_q is not None:
        if packed_sampler_topk_token_ids is None:
            raise ValueError("Packed sampler IDs must be prepared by the loss caller")
        targets = packed_sampler_topk_token_ids.to(device=dev, dtype=torch.long)
    else:
        ids = sampler_topk_token_ids.to(device=dev, dtype=torch.long)
        width = next_token_logits.shape[1]
        if ids.shape[1] > width:
            raise ValueError("Sampler top-k sequence is longer than trainer next_token_logits")
        pad = ids.new_zeros(ids.shape[0], width - ids.shape[1], ids.shape[-1])
        targets = torch.cat([ids, pad], dim=1).roll(-1, dims=1)

    V = next_token_logits.shape[-1]
    rank = 0 if vocab_parallel_rank is None else int(vocab_parallel_rank)
    head = ChunkedDistributedGatherLogprob.apply(
        next_token_logits, targets, rank * V, (rank + 1) * V, chunk_size, vocab_parallel_group,
        False,
    )
    S_ids = sampler_topk_token_ids.shape[1]
    if cu_seqlens_q is None:
        return head[:, : S_ids - 1]

    rows = []
    k = sampler_topk_token_ids.shape[-1]
    for i in range(len(cu_seqlens_q) - 1):
        start = int(cu_seqlens_q_padded[i])
        end = int(cu_seqlens_q_padded[i + 1])
        row = head[:, start:end]
        w = min(end - start - 1, S_ids - 1)
        row = row[:, :w]
        rows.append(torch.cat([row, row.new_zeros(1, S_ids - 1 - w, k)], dim=1))
    return torch.cat(rows, dim=0)


def next_token_and_sampler_topk_logprobs(
    input_ids: torch.Tensor,
    sampler_topk_token_ids: torch.Tensor,
    next_token_logits: torch.Tensor,
    vocab_parallel_rank: Optional[int] = None,
    vocab_parallel_group: Optional[Any] = None,
    chunk_size: Optional[int] = None,
) -> Optional[tuple[torch.Tensor, torch.Tensor]]:
    """``(next_token_logprobs [B, S-1], policy_logprobs_at_sampler_topk [B, S-1, k])`` in one pass.

    The next-token target is one more id per row, so both inputs of a
    score-centering loss come from a single K+1-id gather over the logits
    (one read of each row) and a single backward that writes the summed
    gradient (one read + one write), instead of two forward passes, two
    backward passes and autograd's sum of the two logits gradients.  Values
    equal those of get_next_token_logprobs_from_logits and
    get_policy_logprobs_at_sampler_topk; the gradient is their sum rounded once
    to the logits dtype (the reference rounds each and then adds).  Returns
    None when the shapes call for the separate paths (ids shorter than the
    logits).
    """
    from rl_amd.distributed.model_utils import _check_chunk_size, _check_logits

    _single_rank(vocab_parallel_group)
    _check_chunk_size(chunk_size)
    logits = _check_logits(next_token_logits)
    B, S, V = logits.shape
    if (input_ids.dim() != 2 or tuple(input_ids.shape) != (B, S) or sampler_topk_token_ids.dim() != 3
            or tuple(sampler_topk_token_ids.shape[:2]) != (B, S)):
        return None
    dev = logits.device
    ids = torch.cat([input_ids.to(device=dev, dtype=torch.long).unsqueeze(-1),
                     sampler_topk_token_ids.to(device=dev, dtype=torch.long)], dim=-1)
    ids = ids.roll(-1, dims=1)  # row s holds the ids of position s + 1
    rank = 0 if vocab_parallel_rank is None else int(vocab_parallel_rank)
    out = ChunkedDistributedGatherLogprob.apply(
        logits, ids, rank * V, (rank + 1) * V, chunk_size if chunk_size is not None else S,
        vocab_parallel_group, False,
    )
    curr, plog = out[:, : S - 1, 0], out[:, : S - 1, 1:]
    if out.grad_fn is not None:
        # both views come from one gather node: launch_early_backward can start
        # its backward once the loss knows the gradients of both
        curr._mirl_gather_node = plog._mirl_gather_node = out.grad_fn
    return curr, plog


@torch.no_grad()
def distributed_vocab_topk(
    vocab_parallel_logits: torch.Tensor,
    k: int,
    tp_group: Optional[Any],
    *,
    vocab_start_index: int,
    vocab_end_index: int,
    chunk_size: Optional[int] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k values ``[B, S, k]`` (fp32) and global token ids ``[B, S, k]`` (reference model_utils.py:1867-1935).

    One streaming kernel pass per row for k <= 1024 (group of size 1: no
    candidate exchange); larger k select the exact cut by radix selection and
    sort the k entries in the kernel.  Values are the exact logits, descending;
    equal values are ordered by ascending id.  ``k`` is clamped to the
    vocabulary size as in the reference.
    """
    assert vocab_end_index > vocab_start_index
    _single_rank(tp_group)
    _chunk(chunk_size)
    logits = _unit_stride(vocab_parallel_logits)
    if logits.dim() != 3:
        raise ValueError(f"expected logits of shape [B, S, V_local], got {tuple(logits.shape)}")
    V = logits.shape[-1]
    k_eff = int(min(k, max(1, V)))
    return _C.vocab_topk(logits, k_eff, int(vocab_start_index))


def _validate_student_teacher_logits(
    student: torch.Tensor, teacher: Optional[torch.Tensor]
) -> None:
    """Same checks and messages as the reference (model_utils.py:2520-2538)."""
    if student.ndim != 3:
        raise ValueError(
            "Student logits must be rank 3 [B, S, V_local]; got " f"{tuple(student.shape)}."
        )
    if teacher is not None and student.shape != teacher.shape:
        raise ValueError(
            "Student and teacher logits must share the same [B, S, V_local] shape; "
            f"got {tuple(student.shape)} and {tuple(teacher.shape)}."
        )


class ChunkedDistributedEntropy(torch.autograd.Function):
    """``sum_v p_v log p_v`` per row, ``[B, S]`` fp32 (reference model_utils.py:2199-2241)."""

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        vocab_parallel_logits: torch.Tensor,
        chunk_size: int,
        tp_group: Optional[Any],
        inference_only: bool = False,
    ) -> torch.Tensor:
        return _divergence(ctx, "entropy", vocab_parallel_logits, None, chunk_size, tp_group,
                           inference_only)

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):  # type: ignore[override]
        return _divergence_backward(ctx, grad_outputs[0]), None, None, None


class ChunkedDistributedCrossEntropyToFixedLogits(torch.autograd.Function):
    """``-sum_v p_student log p_teacher`` per row (reference model_utils.py:2244-2297); teacher fixed."""

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        student_vocab_parallel_logits: torch.Tensor,
        teacher_vocab_parallel_logits: torch.Tensor,
        chunk_size: int,
        tp_group: Optional[Any],
        inference_only: bool = False,
    ) -> torch.Tensor:
        return _divergence(ctx, "cross_entropy", student_vocab_parallel_logits,
                           teacher_vocab_parallel_logits, chunk_size, tp_group, inference_only)

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):  # type: ignore[override]
        return _divergence_backward(ctx, grad_outputs[0]), None, None, None, None


class ChunkedDistributedReverseKLToFixedLogits(torch.autograd.Function):
    """``sum_v p_student (log p_student - log p_teacher)`` per row (reference model_utils.py:2300-2351)."""

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        student_vocab_parallel_logits: torch.Tensor,
        teacher_vocab_parallel_logits: torch.Tensor,
        chunk_size: int,
        tp_group: Optional[Any],
        inference_only: bool = False,
    ) -> torch.Tensor:
        return _divergence(ctx, "reverse_kl", student_vocab_parallel_logits,
                           teacher_vocab_parallel_logits, chunk_size, tp_group, inference_only)

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):  # type: ignore[override]
        return _divergence_backward(ctx, grad_outputs[0]), None, None, None, None


def _divergence(
    ctx: Any,
    kind: str,
    student: torch.Tensor,
    teacher: Optional[torch.Tensor],
    chunk_size: int,
    tp_group: Optional[Any],
    inference_only: bool,
) -> torch.Tensor:
    _single_rank(tp_group)
    _chunk(chunk_size)
    _validate_student_teacher_logits(student, teacher)
    student = _unit_stride(student)
    if teacher is not None:
        teacher = _unit_stride(teacher.detach())
        if teacher.dtype != student.dtype:
            teacher = teacher.to(student.dtype)
    B, S, _ = student.shape
    out = torch.empty((B, S), dtype=torch.float32, device=student.device)
    stats = None
    if not inference_only:
        stats = torch.empty((B, S, 4), dtype=torch.float32, device=student.device)
    _C.divergence_fwd(kind, student, teacher, out, stats)
    if not inference_only:
        if teacher is None:
            ctx.save_for_backward(student, out, stats)
        else:
            ctx.save_for_backward(student, out, stats, teacher)
        ctx.kind = kind
    return out


def _divergence_backward(ctx: Any, grad_output: torch.Tensor) -> torch.Tensor:
    saved = ctx.saved_tensors
    if not saved:
        raise RuntimeError("backward through a divergence computed with inference_only=True")
    student, out, stats = saved[:3]
    teacher = saved[3] if len(saved) > 3 else None
    if grad_output.dtype != torch.float32:
        grad_output = grad_output.float()
    grad_input = torch.empty_like(student)
    _C.divergence_bwd(ctx.kind, student, teacher, out, stats, grad_output, grad_input)
    return grad_input
