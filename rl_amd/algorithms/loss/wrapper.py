"""Sequence-packing loss wrappers: drop-in for ``nemo_rl.algorithms.loss.wrapper``
(reference wrapper.py:49-249 and :409-440).

* ``SequencePackingLossWrapper`` runs input preparation and the loss once per
  packed sequence and sums the losses; metrics are summed except the
  per-sequence extrema (``_SEQ_METRIC_MIN`` / ``_SEQ_METRIC_MAX``), which are
  reduced by min/max with the +-inf sentinels of empty sequences skipped.
* ``SequencePackingFusionLossWrapper`` calls a packed preparation function
  (``prepare_packed_loss_input``) once on the whole packed row and the loss
  once on the result.
* ``wrap_loss_fn_with_input_preparation`` is the unpacked one-call path.
"""

from __future__ import annotations

import functools
import math
from typing import Any, Callable, Optional

import torch

from rl_amd.algorithms.loss.interfaces import LossFunction
from rl_amd.algorithms.loss.utils import CpuIntTuple

# Metrics combined across the sequences of one packed row by extremum, not sum.
_SEQ_METRIC_MIN: frozenset[str] = frozenset(
    {"probs_ratio_min", "probs_ratio_clamped_min", "opd_full_reverse_kl_min"}
)
_SEQ_METRIC_MAX: frozenset[str] = frozenset(
    {
        "probs_ratio_max",
        "probs_ratio_clamped_max",
        "opd_full_reverse_kl_max",
        "opd_full_decomposition_error",
    }
)


def _scalar(v: Any) -> Any:
    return v.item() if isinstance(v, torch.Tensor) and v.ndim == 0 else v


def _combine_metric(acc: dict[str, Any], k: str, v: Any) -> None:
    if k not in acc:
        acc[k] = math.inf if k in _SEQ_METRIC_MIN else -math.inf if k in _SEQ_METRIC_MAX else 0
    val = _scalar(v)
    if k in _SEQ_METRIC_MIN:
        if not math.isinf(val):
            acc[k] = min(acc[k], val)
    elif k in _SEQ_METRIC_MAX:
        if not math.isinf(val):
            acc[k] = max(acc[k], val)
    else:
        acc[k] += val


class SequencePackingLossWrapper:
    """Per-sequence loss over a packed row (reference wrapper.py:49-182)."""

    def __init__(
        self,
        loss_fn: LossFunction,
        prepare_fn: Callable[..., Any],
        cu_seqlens_q: CpuIntTuple,
        cu_seqlens_q_padded: Optional[CpuIntTuple] = None,
        vocab_parallel_rank: Optional[int] = None,
        vocab_parallel_group: Optional[Any] = None,
        context_parallel_group: Optional[Any] = None,
    ):
        self.loss_fn = loss_fn
        self.prepare_fn = prepare_fn
        self.cu_seqlens_q = cu_seqlens_q
        self.cu_seqlens_q_padded = (
            cu_seqlens_q_padded if cu_seqlens_q_padded is not None else cu_seqlens_q
        )
        self.vocab_parallel_rank = vocab_parallel_rank
        self.vocab_parallel_group = vocab_parallel_group
        self.context_parallel_group = context_parallel_group

    def __call__(
        self,
        next_token_logits: torch.Tensor,
        data: Any,
        global_valid_seqs: Optional[torch.Tensor],
        global_valid_toks: Optional[torch.Tensor],
    ) -> tuple[torch.Tensor, dict[str, Any]]:
        """Sum of per-sequence losses; sequence i reads logits rows ``[padded_start_i, padded_end_i)``."""
        from rl_amd.algorithms.loss.loss_functions import ClippedPGLossFn
        from rl_amd.distributed.model_utils import _require_single_rank

        _require_single_rank(self.context_parallel_group)
        cu, cu_pad = self.cu_seqlens_q, self.cu_seqlens_q_padded
        lengths = [b - a for a, b in zip(cu[:-1], cu[1:])]
        fused_logprobs = getattr(self.loss_fn, "use_fused_linear_logprobs", False)
        # The fused ClippedPG loss keeps each sequence's metrics on the device;
        # they are fetched with one copy after the loop and combined in the
        # same sequence order (the reference synchronises once per sequence).
        on_device = isinstance(self.loss_fn, ClippedPGLossFn)
        seq_metrics: list = []
        early: list = []
        loss_accum: Any = 0
        metrics_accum: dict[str, Any] = {}
        packed_kw = self._packed_prepare_kwargs(next_token_logits, data, lengths) if on_device else None
        if packed_kw is not None:
            return self._per_sequence_losses_from_one_pass(
                next_token_logits, data, global_valid_seqs, global_valid_toks, lengths, packed_kw
            )
        for i, (start, end) in enumerate(zip(cu_pad[:-1], cu_pad[1:])):
            seq_data = {}
            for k, v in data.slice(i, i + 1).items():
                if isinstance(v, torch.Tensor) and v.ndim > 1 and v.shape[1] > 1:
                    seq_data[k] = v[:, : lengths[i]]
                else:
                    seq_data[k] = v
            if fused_logprobs:
                # precomputed logprobs can be one row shorter than the padded boundaries
                logits_i = next_token_logits[:, start : min(end, next_token_logits.shape[1])]
            else:
                logits_i = next_token_logits.narrow(1, start, end - start)
            loss_input, seq_data = self.prepare_fn(
                logits=logits_i,
                data=seq_data,
                loss_fn=self.loss_fn,
                vocab_parallel_rank=self.vocab_parallel_rank,
                vocab_parallel_group=self.vocab_parallel_group,
                context_parallel_group=self.context_parallel_group,
            )
            if on_device:
                loss, mvec, e = self.loss_fn._loss_on_device(
                    data=seq_data,
                    global_valid_seqs=global_valid_seqs,
                    global_valid_toks=global_valid_toks,
                    **loss_input,
                )
                seq_metrics.append(mvec)
                if e is not None:
                    early.append(e)
                loss_accum = loss_accum + loss
                continue
            loss, metrics = self.loss_fn(
                data=seq_data,
                global_valid_seqs=global_valid_seqs,
                global_valid_toks=global_valid_toks,
                **loss_input,
            )
            loss_accum = loss_accum + loss
            for k, v in metrics.items():
                _combine_metric(metrics_accum, k, v)
        if seq_metrics:
            from rl_amd import _C
            from rl_amd.distributed.model_utils import launch_early_backward

            fetch = _C.start_fetch(torch.stack(seq_metrics))
            # each sequence's loss enters the sum with weight 1: its logits
            # backward can start behind the copy (checked again in the backward)
            for e in early:
                if len(e) == 2:
                    launch_early_backward(*e)
            values = _C.finish_fetch(fetch)
            m = seq_metrics[0].numel()
            for i in range(len(seq_metrics)):
                for k, v in self.loss_fn.metrics_from_values(values[i * m : (i + 1) * m]).items():
                    _combine_metric(metrics_accum, k, v)
        return loss_accum, metrics_accum


    def _packed_prepare_kwargs(self, logits: torch.Tensor, data: Any, lengths: list) -> Optional[dict]:
        """Options for ``prepare_packed_loss_input`` when ``prepare_fn`` is ``prepare_loss_input``
        (or a partial of it with options the packed preparation shares); None otherwise."""
        from rl_amd.algorithms.loss.loss_input import prepare_loss_input

        fn, kw = self.prepare_fn, {}
        if isinstance(fn, functools.partial):
            if fn.args:
                return None
            fn, kw = fn.func, dict(fn.keywords)
        if fn is not prepare_loss_input or not set(kw) <= {"sampling_params", "chunk_size"}:
            return None
        if getattr(self.loss_fn, "use_fused_linear_logprobs", False) or "cu_seqlens" in data:
            return None
        if (not isinstance(logits, torch.Tensor) or logits.device.type != "cuda" or logits.dim() != 3
                or logits.shape[0] != 1 or logits.shape[1] < self.cu_seqlens_q_padded[-1]):
            return None
        ids = data["input_ids"]
        if ids.dim() != 2 or len(lengths) != ids.shape[0] or min(lengths, default=0) < 2:
            return None
        if any(b < a for a, b in zip(self.cu_seqlens_q_padded[:-1], self.cu_seqlens_q_padded[1:])):
            return None
        return kw

    def _per_sequence_losses_from_one_pass(
        self,
        logits: torch.Tensor,
        data: Any,
        global_valid_seqs: Optional[torch.Tensor],
        global_valid_toks: Optional[torch.Tensor],
        lengths: list,
        packed_kw: dict,
    ) -> tuple[torch.Tensor, dict[str, Any]]:
        """The per-sequence losses with the logprobs of every sequence from one pass.

        A sequence's next-token logprobs depend only on its own logits rows, so
        they are computed for the whole packed row at once
        (``prepare_packed_loss_input``: one logprob kernel forward and, under
        autograd, one backward over the packed logits) and then cut per
        sequence, where the reference narrows the logits per sequence and
        autograd materialises a logits-sized gradient for each.  The loss and
        its metrics are still computed per sequence and combined in sequence
        order; the metrics of all sequences come back with one copy.
        """
        from rl_amd import _C
        from rl_amd.algorithms.loss.loss_input import _prepare_packed
        from rl_amd.distributed.batched_data_dict import BatchedDataDict

        batch = BatchedDataDict(dict(data.items()))
        loss_input, prepared = _prepare_packed(
            logits, batch, self.loss_fn, self.cu_seqlens_q, self.cu_seqlens_q_padded,
            self.vocab_parallel_rank, self.vocab_parallel_group, self.context_parallel_group,
            packed_kw.get("sampling_params"), packed_kw.get("chunk_size"), False,
        )
        # tensors the preparation produced per next-token position ([B, S-1, ...])
        per_position = {"curr_logprobs_unfiltered"}
        loss_accum: Any = 0
        seq_metrics = []
        for i, L in enumerate(lengths):
            li = {k: (v[i : i + 1, : L - 1] if isinstance(v, torch.Tensor) else v) for k, v in loss_input.items()}
            sd = {}
            for k, v in prepared.slice(i, i + 1).items():
                if isinstance(v, torch.Tensor) and v.ndim > 1 and v.shape[1] > 1:
                    sd[k] = v[:, : L - 1] if k in per_position else v[:, :L]
                else:
                    sd[k] = v
            loss, mvec, _ = self.loss_fn._loss_on_device(
                data=sd, global_valid_seqs=global_valid_seqs, global_valid_toks=global_valid_toks, **li
            )
            loss_accum = loss_accum + loss
            seq_metrics.append(mvec)
        values = _C.wait_and_fetch(torch.stack(seq_metrics))
        m = seq_metrics[0].numel()
        metrics_accum: dict[str, Any] = {}
        for i in range(len(seq_metrics)):
            for k, v in self.loss_fn.metrics_from_values(values[i * m : (i + 1) * m]).items():
                _combine_metric(metrics_accum, k, v)
        return loss_accum, metrics_accum


class SequencePackingFusionLossWrapper:
    """One preparation call and one loss call for all packed sequences (reference wrapper.py:185-249).

    ``prepare_fn`` is ``prepare_packed_loss_input``; the result equals the
    per-sequence wrapper's (same logprobs, one loss over the whole batch).
    """

    def __init__(
        self,
        loss_fn: LossFunction,
        prepare_fn: Callable[..., Any],
        cu_seqlens_q: CpuIntTuple,
        cu_seqlens_q_padded: Optional[CpuIntTuple] = None,
        vocab_parallel_rank: Optional[int] = None,
        vocab_parallel_group: Optional[Any] = None,
        context_parallel_group: Optional[Any] = None,
    ):
        self.loss_fn = loss_fn
        self.prepare_fn = prepare_fn
        self.cu_seqlens_q = cu_seqlens_q
        self.cu_seqlens_q_padded = (
            cu_seqlens_q_padded if cu_seqlens_q_padded is not None else cu_seqlens_q
        )
        self.vocab_parallel_rank = vocab_parallel_rank
        self.vocab_parallel_group = vocab_parallel_group
        self.context_parallel_group = context_parallel_group

    def __call__(
        self,
        next_token_logits: torch.Tensor,
        data: Any,
        global_valid_seqs: Optional[torch.Tensor],
        global_valid_toks: Optional[torch.Tensor],
    ) -> tuple[torch.Tensor, dict[str, Any]]:
        loss_input, prepared = self.prepare_fn(
            logits=next_token_logits,
            data=data,
            loss_fn=self.loss_fn,
            cu_seqlens_q=self.cu_seqlens_q,
            cu_seqlens_q_padded=self.cu_seqlens_q_padded,
            vocab_parallel_rank=self.vocab_parallel_rank,
            vocab_parallel_group=self.vocab_parallel_group,
            context_parallel_group=self.context_parallel_group,
        )
        return self.loss_fn(
            data=prepared,
            global_valid_seqs=global_valid_seqs,
            global_valid_toks=global_valid_toks,
            **loss_input,
        )


def wrap_loss_fn_with_input_preparation(
    next_token_logits: torch.Tensor,
    data: Any,
    global_valid_seqs: Optional[torch.Tensor],
    global_valid_toks: Optional[torch.Tensor],
    loss_fn: LossFunction,
    prepare_fn: Callable[..., Any],
    vocab_parallel_rank: Optional[int] = None,
    vocab_parallel_group: Optional[Any] = None,
    context_parallel_group: Optional[Any] = None,
) -> tuple[torch.Tensor, dict[str, Any]]:
    """Prepare the loss input, then call the loss (reference wrapper.py:409-440)."""
    loss_input, data = prepare_fn(
        logits=next_token_logits,
        data=data,
        loss_fn=loss_fn,
        vocab_parallel_rank=vocab_parallel_rank,
        vocab_parallel_group=vocab_parallel_group,
        context_parallel_group=context_parallel_group,
    )
    return loss_fn(
        data=data,
        global_valid_seqs=global_valid_seqs,
        global_valid_toks=global_valid_toks,
        **loss_input,
    )
