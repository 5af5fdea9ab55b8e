"""Token log-probabilities from logits: drop-in for ``nemo_rl.distributed.model_utils``.

The autograd Functions and helpers keep the reference's names, call
signatures, tensor layouts and dtypes; the arithmetic runs in the gfx950
kernels of ``libmirl.so``:

* forward: one pass over each logits row (online log-sum-exp with the target
  gather fused in), fp32 output, no [B, S, V] temporaries;
* backward: one read + one write per row, ``(onehot - softmax) * g`` in the
  logits dtype; rows whose upstream gradient is zero are written without
  being read.

Scope: the vocab-parallel group must be ``None`` or of size 1 (one GPU owns
the whole vocabulary); larger groups raise ``NotImplementedError``.  No
collective is ever issued.  ``chunk_size`` is validated and kept in the
signature, but it never changes results: every row is independent.
"""

from __future__ import annotations

from typing import Any, Optional

import numpy as np
import torch

from rl_amd import _C
from rl_amd.distributed.early_backward import POLICY, set_early_backward
from rl_amd.algorithms.logits_sampling_utils import (
    TrainingSamplingParams,
    need_top_k_or_top_p_filtering,
)

__all__ = [
    "ChunkedDistributedCrossEntropyToFixedLogits",
    "ChunkedDistributedEntropy",
    "ChunkedDistributedGatherLogprob",
    "ChunkedDistributedHiddenStatesToLogprobs",
    "ChunkedDistributedLogprob",
    "ChunkedDistributedLogprobWithSampling",
    "ChunkedDistributedReverseKLToFixedLogits",
    "DistributedLogprob",
    "distributed_vocab_topk",
    "DistributedLogprobWithSampling",
    "from_parallel_hidden_states_to_logprobs",
    "from_parallel_logits_to_logprobs",
    "from_parallel_logits_to_logprobs_packed_sequences",
    "get_next_token_logprobs_from_logits",
    "get_policy_logprobs_at_sampler_topk",
    "set_early_backward",
]

_VOCAB_REDUCTIONS = (
    "ChunkedDistributedGatherLogprob",
    "get_policy_logprobs_at_sampler_topk",
    "ChunkedDistributedEntropy",
    "ChunkedDistributedCrossEntropyToFixedLogits",
    "ChunkedDistributedReverseKLToFixedLogits",
    "distributed_vocab_topk",
)


def __getattr__(name: str):
    # the filtered autograd Functions live with the filter kernels' bindings,
    # the hidden-state path with the fused LM-head kernels' bindings, the
    # K-id gather and the divergences in vocab_reductions
    if name in ("DistributedLogprobWithSampling", "ChunkedDistributedLogprobWithSampling"):
        from rl_amd.distributed import sampling

        return getattr(sampling, name)
    if name in ("ChunkedDistributedHiddenStatesToLogprobs", "from_parallel_hidden_states_to_logprobs"):
        from rl_amd.distributed import linear_ce

        return getattr(linear_ce, name)
    if name in _VOCAB_REDUCTIONS:
        from rl_amd.distributed import vocab_reductions

        return getattr(vocab_reductions, name)
    raise AttributeError(name)


def _group_size(group: Optional[Any]) -> int:
    if group is None:
        return 1
    try:
        return torch.distributed.get_world_size(group)
    except (RuntimeError, ValueError):
        return 1
    except (AttributeError, TypeError) as e:
        raise TypeError(
            f"expected a torch.distributed ProcessGroup or None, got {type(group).__name__}"
        ) from e


def _require_single_rank(*groups: Optional[Any]) -> None:
    for g in groups:
        if _group_size(g) != 1:
            raise NotImplementedError(
                "rl_amd computes logprobs with the whole vocabulary on one GPU; "
                f"process groups of size {_group_size(g)} are not supported"
            )


def _check_logits(logits: torch.Tensor) -> torch.Tensor:
    if logits.dim() != 3:
        raise ValueError(f"expected logits of shape [B, S, V], got {tuple(logits.shape)}")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    return logits


def _check_chunk_size(chunk_size: Optional[int]) -> None:
    if chunk_size is not None and int(chunk_size) <= 0:
        raise ValueError("logprob_chunk_size must be positive")


class _RowLogprob(torch.autograd.Function):
    """Selected-token logprobs of rows ``0..R-1`` of ``logits`` (R = target.shape[1]).

    forward:  [B, S, V] logits, [B, R] int64 targets -> [B, R] fp32.
    backward: [B, R] fp32 -> [B, S, V] in the logits dtype (rows >= R are zero).
    """

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        logits: torch.Tensor,
        target: torch.Tensor,
        vocab_start_index: int,
        vocab_end_index: int,
        inference_only: bool,
        reuse_logits_storage: bool,
    ) -> torch.Tensor:
        B, R = target.shape
        out = torch.empty((B, R), dtype=torch.float32, device=logits.device)
        stats = None
        if not inference_only:
            stats = torch.empty((B, R, 2), dtype=torch.float32, device=logits.device)
        _C.logprob_fwd(logits, target, vocab_start_index, vocab_end_index, out, stats)
        if not inference_only:
            ctx.save_for_backward(logits, target, stats)
            ctx.vocab = (int(vocab_start_index), int(vocab_end_index))
            ctx.reuse_logits_storage = bool(reuse_logits_storage)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):  # type: ignore[override]
        (grad_output,) = grad_outputs
        logits, target, stats = ctx.saved_tensors
        vs, ve = ctx.vocab
        if grad_output.dtype != torch.float32:
            grad_output = grad_output.float()
        early = getattr(ctx, "early", None)
        if early is not None:
            # launched by launch_early_backward: check it against the real gradient
            ctx.early = None
            grad_input, grad_used = early
            POLICY.checked(
                _C.logprob_bwd_recheck(logits, target, vs, ve, stats, grad_output, grad_used, grad_input))
            return grad_input, None, None, None, None, None
        reuse = ctx.reuse_logits_storage and not logits.is_leaf
        grad_input = logits if reuse else torch.empty_like(logits)
        _C.logprob_bwd(logits, target, vs, ve, stats, grad_output, grad_input)
        return grad_input, None, None, None, None, None


def launch_early_backward_pair(
    curr: torch.Tensor, grad_curr: torch.Tensor, plog: torch.Tensor, grad_plog: torch.Tensor
) -> bool:
    """launch_early_backward for the next-token and sampler top-k logprobs of one K+1-id
    gather (``next_token_and_sampler_topk_logprobs``): the gather's upstream gradient is
    assembled the way autograd assembles it from the two views (each view's gradient
    scattered into zeros, the two added), its backward is launched, and the gather's
    backward later checks it against the real one on the device."""
    node = getattr(curr, "_mirl_gather_node", None)
    if node is None or getattr(plog, "_mirl_gather_node", None) is not node:
        return False
    if getattr(node, "early", None) is not None:
        return False
    if not POLICY.should_launch():
        return False
    if grad_curr.dtype != torch.float32 or grad_plog.dtype != torch.float32:
        return False
    logits, idx, stats = node.saved_tensors
    B, S, K1 = idx.shape
    if (tuple(curr.shape) != (B, S - 1) or tuple(plog.shape) != (B, S - 1, K1 - 1)
            or tuple(grad_curr.shape) != tuple(curr.shape) or tuple(grad_plog.shape) != tuple(plog.shape)):
        return False
    g_a = torch.zeros((B, S, K1), dtype=torch.float32, device=logits.device)
    g_a[:, : S - 1, 0] = POLICY.hinted(grad_curr)
    g_b = torch.zeros_like(g_a)
    g_b[:, : S - 1, 1:] = POLICY.hinted(grad_plog)
    g = g_a + g_b
    grad_input = torch.empty_like(logits)
    vs, ve = node.vocab
    _C.gather_logprob_bwd(logits, idx, vs, ve, stats, g, grad_input)
    node.early = (grad_input, g)
    return True


def launch_early_backward(logprobs: torch.Tensor, grad: torch.Tensor) -> bool:
    """Start the logits backward of ``logprobs`` for the upstream gradient ``grad`` now.

    For a consumer (the ClippedPG loss) that knows d(loss)/d(logprobs) in closed
    form before autograd runs: the backward kernel is enqueued right away, ahead
    of the host-side synchronisation on the loss's metrics and of autograd's own
    bookkeeping, so the GPU does not wait for them.  When autograd later calls
    the backward, a device-side check compares its real upstream gradient with
    ``grad`` bit for bit and recomputes only if they differ (a scaled loss, a
    second consumer of the logprobs), so results never depend on the guess.
    Applies to logprobs produced directly by this module's row kernel and to
    their unpacking from packed sequences; returns whether the backward was
    started.  set_early_backward chooses when it is (by default it is not
    started again for a while after a check found a different gradient) and the
    loss scale the caller applies, which ``grad`` is multiplied by first.
    """
    fn = logprobs.grad_fn
    if grad.dtype != torch.float32 or tuple(grad.shape) != tuple(logprobs.shape):
        return False
    if isinstance(fn, _UnpackRows._backward_cls):
        # packed sequences: the row kernel's upstream gradient is the unpacking's
        # backward of `grad` (the same kernel autograd will run on the real one)
        src = getattr(fn, "src", None)
        if src is None:
            return False
        (bounds,) = fn.saved_tensors
        return _launch_early_on_node(
            src, (1, fn.n_rows),
            lambda: _C.unpack_rows_bwd(POLICY.hinted(grad), bounds, fn.n_rows).view(1, -1))
    return _launch_early_on_node(fn, tuple(grad.shape), lambda: POLICY.hinted(grad))


def _launch_early_on_node(fn: Any, grad_shape: tuple, make_grad) -> bool:
    """launch_early_backward for the autograd node of a row-kernel output; ``make_grad()``
    forms the node's upstream gradient (shape ``grad_shape``), only once the launch is on."""
    if not isinstance(fn, _RowLogprob._backward_cls):
        return False
    if getattr(fn, "early", None) is not None or getattr(fn, "reuse_logits_storage", True):
        return False
    logits, target, stats = fn.saved_tensors
    if tuple(grad_shape) != tuple(target.shape):
        return False
    if not POLICY.should_launch():
        return False
    grad = make_grad().contiguous()
    grad_input = torch.empty_like(logits)
    vs, ve = fn.vocab
    _C.logprob_bwd(logits, target, vs, ve, stats, grad, grad_input)
    fn.early = (grad_input, grad)
    return True


class DistributedLogprob(torch.autograd.Function):
    """Drop-in for ``DistributedLogprob`` (reference model_utils.py:138-225), group size 1.

    Returns [B, S] fp32 selected-token logprobs (0 where the target lies
    outside ``[vocab_start_index, vocab_end_index)``).  Unlike the reference it
    saves only the logits and an 8-byte per-row statistic for backward, not an
    fp32 softmax of the whole tensor.
    """

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        vocab_parallel_logits: torch.Tensor,
        target: torch.Tensor,
        vocab_start_index: int,
        vocab_end_index: int,
        group: Optional[Any],
        inference_only: bool = False,
    ) -> torch.Tensor:
        _require_single_rank(group)
        logits = _check_logits(vocab_parallel_logits)
        out, stats = _forward_rows(logits, target, vocab_start_index, vocab_end_index, inference_only)
        if not inference_only:
            ctx.save_for_backward(logits, target, stats)
            ctx.vocab = (int(vocab_start_index), int(vocab_end_index))
            ctx.reuse_logits_storage = False
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):  # type: ignore[override]
        grad = _backward_rows(ctx, grad_outputs[0])
        return grad, None, None, None, None, None


class ChunkedDistributedLogprob(torch.autograd.Function):
    """Drop-in for ``ChunkedDistributedLogprob`` (reference model_utils.py:228-349), group size 1.

    ``chunk_size`` is accepted for signature compatibility; the kernels stream
    rows independently, so the result is identical for every chunk size.
    ``reuse_logits_storage`` writes the gradient into the logits' own storage
    when the logits are not a leaf, as in the reference.
    """

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        vocab_parallel_logits: torch.Tensor,
        target: torch.Tensor,
        vocab_start_index: int,
        vocab_end_index: int,
        chunk_size: int,
        tp_group: Optional[Any],
        inference_only: bool = False,
        reuse_logits_storage: bool = False,
    ) -> torch.Tensor:
        _require_single_rank(tp_group)
        _check_chunk_size(chunk_size)
        logits = _check_logits(vocab_parallel_logits)
        out, stats = _forward_rows(logits, target, vocab_start_index, vocab_end_index, inference_only)
        if not inference_only:
            ctx.save_for_backward(logits, target, stats)
            ctx.vocab = (int(vocab_start_index), int(vocab_end_index))
            ctx.reuse_logits_storage = bool(reuse_logits_storage)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):  # type: ignore[override]
        grad = _backward_rows(ctx, grad_outputs[0])
        return grad, None, None, None, None, None, None, None


def _row_logprobs(
    logits: torch.Tensor,
    target: torch.Tensor,
    vocab_start_index: int,
    vocab_end_index: int,
    inference_only: bool,
    reuse_logits_storage: bool,
) -> torch.Tensor:
    """``_RowLogprob`` when autograd will record the call, else the forward kernel alone.

    With ``inference_only`` (nothing is saved for a backward, as in the
    reference) or when no gradient can flow, the autograd Function and the
    per-row statistics are skipped; the logprobs are the same.
    """
    if inference_only or not (logits.requires_grad and torch.is_grad_enabled()):
        out = torch.empty(target.shape, dtype=torch.float32, device=logits.device)
        _C.logprob_fwd(logits, target, vocab_start_index, vocab_end_index, out, None)
        return out
    return _RowLogprob.apply(
        logits, target, vocab_start_index, vocab_end_index, False, reuse_logits_storage
    )


def _forward_rows(
    logits: torch.Tensor,
    target: torch.Tensor,
    vocab_start_index: int,
    vocab_end_index: int,
    inference_only: bool,
) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
    B, S, _ = logits.shape
    if tuple(target.shape) != (B, S):
        raise ValueError(
            f"target shape {tuple(target.shape)} does not match logits rows {(B, S)}"
        )
    if target.dtype != torch.int64:
        target = target.long()
    out = torch.empty((B, S), dtype=torch.float32, device=logits.device)
    stats = None if inference_only else torch.empty((B, S, 2), dtype=torch.float32, device=logits.device)
    _C.logprob_fwd(logits, target, vocab_start_index, vocab_end_index, out, stats)
    return out, stats


def _backward_rows(ctx: Any, grad_output: torch.Tensor) -> torch.Tensor:
    logits, target, stats = ctx.saved_tensors
    vs, ve = ctx.vocab
    if target.dtype != torch.int64:
        target = target.long()
    if grad_output.dtype != torch.float32:
        grad_output = grad_output.float()
    reuse = ctx.reuse_logits_storage and not logits.is_leaf
    grad_input = logits if reuse else torch.empty_like(logits)
    _C.logprob_bwd(logits, target, vs, ve, stats, grad_output, grad_input)
    return grad_input


def _next_token_targets(target: torch.Tensor, n_logit_rows: int) -> torch.Tensor:
    """Targets of rows 0..S_t-2: ``target[:, 1:]`` (reference rolls by -1, then drops the last)."""
    if target.dim() != 2:
        raise ValueError(f"expected target of shape [B, S], got {tuple(target.shape)}")
    if target.shape[1] > n_logit_rows:
        raise ValueError(
            f"target length {target.shape[1]} exceeds the {n_logit_rows} logits rows"
        )
    if target.dtype != torch.int64:
        target = target.long()
    return target[:, 1:]


def from_parallel_logits_to_logprobs(
    vocab_parallel_logits: torch.Tensor,
    target: torch.Tensor,
    vocab_start_index: int,
    vocab_end_index: int,
    tp_group: Optional[Any],
    inference_only: bool = False,
    cp_group: Optional[Any] = None,
    chunk_size: Optional[int] = None,
    sampling_params: Optional[TrainingSamplingParams] = None,
) -> torch.Tensor:
    """Next-token logprobs ``[B, S-1]`` (fp32) from ``[B, S, V]`` logits and ``[B, S]`` targets.

    Drop-in for reference model_utils.py:967-1062 with TP = CP = 1.  Row s of
    the result is the logprob of ``target[:, s+1]`` under ``logits[:, s]``.
    Only the S-1 rows that survive the reference's final ``[:, :-1]`` slice
    are computed; the backward writes zeros for the last row.  With
    ``sampling_params`` the filter decides top-p in the logits' own dtype, as
    the reference's DistributedLogprobWithSampling does on this tensor.
    """
    return _next_token_logprobs(vocab_parallel_logits, target, vocab_start_index,
                                vocab_end_index, tp_group, inference_only, cp_group, chunk_size,
                                sampling_params, None)


def _next_token_logprobs(logits, target, vocab_start_index, vocab_end_index, tp_group,
                         inference_only, cp_group, chunk_size, sampling_params, decision_dtype):
    _require_single_rank(tp_group, cp_group)
    _check_chunk_size(chunk_size)
    logits = _check_logits(logits)
    if need_top_k_or_top_p_filtering(sampling_params):
        from rl_amd.distributed.sampling import filtered_next_token_logprobs

        return filtered_next_token_logprobs(
            logits,
            target,
            sampling_params.top_k,  # type: ignore[union-attr]
            sampling_params.top_p,  # type: ignore[union-attr]
            inference_only=inference_only,
            decision_dtype=decision_dtype,
        )
    tgt = _next_token_targets(target, logits.shape[1])
    return _row_logprobs(logits, tgt, vocab_start_index, vocab_end_index, inference_only, False)


def from_parallel_logits_to_logprobs_packed_sequences(
    vocab_parallel_logits: torch.Tensor,
    target: torch.Tensor,
    cu_seqlens_padded: Any,
    unpacked_seqlen: int,
    vocab_start_index: int,
    vocab_end_index: int,
    group: Optional[Any],
    inference_only: bool = False,
    cp_group: Optional[Any] = None,
    chunk_size: Optional[int] = None,
    sampling_params: Optional[TrainingSamplingParams] = None,
    target_is_pre_rolled: bool = False,
    return_packed_layout: bool = False,
    reuse_logits_storage: bool = False,
) -> torch.Tensor:
    """Logprobs of packed sequences (reference model_utils.py:1065-1231), CP = TP = 1.

    ``vocab_parallel_logits`` is ``[1, T, V]``; ``cu_seqlens_padded`` holds the
    ``B + 1`` sequence boundaries (host integers).  The reference's host loops
    over sequences (target roll, unpacking to ``[B, unpacked_seqlen - 1]``)
    become one gfx950 kernel each over the uploaded boundaries
    (``mirl_packed_roll_targets``, ``mirl_unpack_rows_fwd``); the unpacking's
    backward is the inverse kernel (``mirl_unpack_rows_bwd``).  With
    ``sampling_params`` the filter decides top-p in the logits' own dtype, as
    the reference's DistributedLogprobWithSampling does on this tensor.
    """
    return _packed_sequence_logprobs(
        vocab_parallel_logits, target, cu_seqlens_padded, unpacked_seqlen, vocab_start_index,
        vocab_end_index, group, inference_only, cp_group, chunk_size, sampling_params,
        target_is_pre_rolled, return_packed_layout, reuse_logits_storage, None,
    )


def _packed_sequence_logprobs(vocab_parallel_logits, target, cu_seqlens_padded, unpacked_seqlen,
                              vocab_start_index, vocab_end_index, group, inference_only, cp_group,
                              chunk_size, sampling_params, target_is_pre_rolled,
                              return_packed_layout, reuse_logits_storage, decision_dtype):
    _require_single_rank(group, cp_group)
    _check_chunk_size(chunk_size)
    logits = _check_logits(vocab_parallel_logits)
    if logits.shape[0] != 1:
        raise ValueError(f"packed logits must have batch 1, got {tuple(logits.shape)}")
    bounds = [int(x) for x in cu_seqlens_padded]
    if len(bounds) < 1 or any(b1 < b0 for b0, b1 in zip(bounds, bounds[1:])) or bounds[0] < 0:
        raise ValueError(f"cu_seqlens_padded must be nondecreasing and nonnegative, got {bounds}")
    dev = logits.device
    bdev = _host_ints_to_device(bounds, dev)
    tgt = target.reshape(1, -1)
    if tgt.dtype != torch.int64:
        tgt = tgt.long()
    if not target_is_pre_rolled:
        if bounds[-1] > tgt.shape[1]:
            raise ValueError(
                f"cu_seqlens_padded ends at {bounds[-1]} but the packed target has {tgt.shape[1]} tokens"
            )
        tgt = _C.packed_roll_targets(tgt.reshape(-1).contiguous(), bdev).unsqueeze(0)
    if need_top_k_or_top_p_filtering(sampling_params):
        from rl_amd.distributed.sampling import filtered_row_logprobs

        probs = filtered_row_logprobs(
            logits, tgt, sampling_params.top_k, sampling_params.top_p,  # type: ignore[union-attr]
            inference_only=inference_only, decision_dtype=decision_dtype,
        )
    else:
        probs = _row_logprobs(
            logits, tgt, vocab_start_index, vocab_end_index, inference_only,
            reuse_logits_storage and chunk_size is not None,
        )
    rows = probs
    probs = probs.squeeze(0)
    if return_packed_layout:
        return probs[:-1].unsqueeze(0)
    if bounds[-1] > probs.shape[0]:
        raise ValueError(
            f"cu_seqlens_padded ends at {bounds[-1]} but only {probs.shape[0]} packed rows were computed"
        )
    out_cols = max(int(unpacked_seqlen) - 1, 0)
    out = _UnpackRows.apply(probs, bdev, out_cols)
    if out.grad_fn is not None:
        out.grad_fn.src = rows.grad_fn  # for launch_early_backward
    return out


def _gather_or_zero(x: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """``x[index]`` along dim 0, where ``index == x.shape[0]`` reads a zero."""
    pad = x.new_zeros((1, *x.shape[1:]))
    return torch.cat([x, pad]).index_select(0, index)


class _UnpackRows(torch.autograd.Function):
    """``[T]`` packed fp32 rows -> ``[B, C]`` by the sequence boundaries; backward is the inverse."""

    @staticmethod
    def forward(ctx: Any, probs: torch.Tensor, bounds: torch.Tensor, cols: int) -> torch.Tensor:  # type: ignore[override]
        ctx.save_for_backward(bounds)
        ctx.n_rows = probs.shape[0]
        return _C.unpack_rows_fwd(probs.contiguous(), bounds, cols)

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):  # type: ignore[override]
        (bounds,) = ctx.saved_tensors
        return _C.unpack_rows_bwd(grad_outputs[0], bounds, ctx.n_rows), None, None


def _is_dtensor(t: torch.Tensor) -> bool:
    try:
        from torch.distributed.tensor import DTensor
    except ImportError:  # torch built without distributed
        return False
    return isinstance(t, DTensor)


def _host_ints_to_device(values: Any, dev: torch.device) -> torch.Tensor:
    """int64 tensor of host integers on ``dev``, staged through pinned memory so
    that the copy is queued on the stream instead of blocking the host."""
    if isinstance(values, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(values, dtype=np.int64))
    else:
        t = torch.tensor(values, dtype=torch.int64)
    if dev.type != "cuda":
        return t.to(dev)
    return t.pin_memory().to(dev, non_blocking=True)


def get_next_token_logprobs_from_logits(
    input_ids: torch.Tensor,
    next_token_logits: torch.Tensor,
    vocab_parallel_rank: Optional[int] = None,
    vocab_parallel_group: Optional[Any] = None,
    context_parallel_group: Optional[Any] = None,
    sampling_params: Optional[TrainingSamplingParams] = None,
    chunk_size: Optional[int] = None,
    cp_sharder: Optional[Any] = None,
) -> torch.Tensor:
    """Next-token logprobs ``[B, S-1]`` (reference model_utils.py:1624-1720).

    With or without a (size-1) vocab group the same kernels run; the
    reference's fp32 upcast of the logits is implicit (the kernels read the
    logits dtype and accumulate in fp32), and its gradient cast back to the
    logits dtype is what the backward writes.
    """
    if cp_sharder is not None:
        raise NotImplementedError("context-parallel sharders are not supported (CP = 1)")
    if _is_dtensor(next_token_logits):
        raise NotImplementedError("DTensor logits are not supported (single GPU)")
    _require_single_rank(vocab_parallel_group, context_parallel_group)
    if vocab_parallel_group is not None:
        assert vocab_parallel_rank is not None, (
            "vocab_parallel_rank must be provided when vocab_parallel_group is provided"
        )
    use_chunking = (
        vocab_parallel_group is not None
        and chunk_size is not None
        and not need_top_k_or_top_p_filtering(sampling_params)
    )
    V = next_token_logits.shape[-1]
    # the reference upcasts to fp32 here (model_utils.py:1660-1666), so the
    # filter decides top-p in fp32; the kernels read the logits dtype directly
    logprobs = _next_token_logprobs(
        next_token_logits, input_ids, 0, V, None, False, None,
        chunk_size if use_chunking else None, sampling_params, torch.float32,
    )
    if logprobs.shape[1] == input_ids.shape[1] - 1:
        return logprobs  # the slice below would be the whole tensor
    return logprobs[:, : input_ids.shape[1] - 1]
