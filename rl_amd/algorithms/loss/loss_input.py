"""Loss-input preparation: drop-in for the LOGIT/LOGPROB branches of
``nemo_rl.algorithms.loss.loss_input`` (reference loss_input.py:215-322 and :468-634).

``prepare_loss_input`` turns ``[B, S, V]`` logits into the ``[B, S-1]``
next-token logprobs the loss consumes; ``prepare_packed_loss_input`` does the
same for one packed row ``[1, T, V]`` in a single kernel pass over all
sequences.  When top-k/top-p filtering is on and the loss carries a KL penalty,
a second, unfiltered pass fills ``data["curr_logprobs_unfiltered"]`` and the
support mask ``~isneginf(logprobs)`` is passed to the loss, as in the reference.

The reference upcasts the logits to fp32 before the (unchunked) logprob call;
the kernels read the logits in their own dtype and accumulate in fp32, which
gives the same values (the upcast is exact) and the same gradient (the fp32
gradient rounded to the logits dtype) without materialising an fp32 copy.
"""

from __future__ import annotations

from typing import Any, Optional

import torch

from rl_amd.algorithms.logits_sampling_utils import (
    TrainingSamplingParams,
    need_top_k_or_top_p_filtering,
)
from rl_amd.algorithms.loss.interfaces import LossFunction, LossInputType
from rl_amd.algorithms.loss.utils import CpuIntTuple, _pack_input_ids
from rl_amd.distributed.model_utils import (
    _group_size,
    _packed_sequence_logprobs,
    get_next_token_logprobs_from_logits,
)
from rl_amd.distributed.model_utils import _is_dtensor
from rl_amd.distributed.vocab_reductions import (
    get_policy_logprobs_at_sampler_topk,
    next_token_and_sampler_topk_logprobs,
)


def _unsupported(what: str) -> NotImplementedError:
    return NotImplementedError(f"{what} is not supported by the rl_amd logprob path")


def _validate_score_centering_data(data: Any) -> None:
    """Reject missing sampler inputs before computing trainer logprobs (reference loss_input.py:53-66)."""
    missing = [
        key for key in ("sampler_topk_token_ids", "sampler_topk_logprobs") if key not in data
    ]
    if missing:
        raise ValueError(
            f"Score centering requires {', '.join(missing)}: use SingleController "
            "with NeMo Gym + vLLM, token_capture.enabled=true and "
            "policy.generation.top_logprobs > 0."
        )


def prepare_loss_input(
    logits: torch.Tensor,
    data: Any,
    loss_fn: LossFunction,
    vocab_parallel_rank: Optional[int] = None,
    vocab_parallel_group: Optional[Any] = None,
    context_parallel_group: Optional[Any] = None,
    sampling_params: Optional[TrainingSamplingParams] = None,
    d2t: Optional[torch.Tensor] = None,
    chunk_size: Optional[int] = None,
    cp_sharder: Optional[Any] = None,
    teacher_output_layer_weight_by_index: Optional[dict[int, torch.Tensor]] = None,
) -> tuple[dict[str, Any], Any]:
    """``(loss_input, data)`` for ``loss_fn`` (reference loss_input.py:215-322).

    LOGIT passes the logits through; LOGPROB computes next-token logprobs
    (filtered when ``sampling_params`` asks for it) and, for a loss with
    ``score_centering``, the log-probs at the sampler's top-k ids.  The other
    input types (OPD, distillation, draft) are outside this path and raise.
    """
    if getattr(loss_fn, "score_centering", False):
        _validate_score_centering_data(data)
    if loss_fn.input_type == LossInputType.LOGIT:
        return {"logits": logits}, data
    if loss_fn.input_type != LossInputType.LOGPROB:
        if loss_fn.input_type in tuple(LossInputType):
            raise _unsupported(f"loss input type {loss_fn.input_type}")
        raise ValueError(f"Unknown loss function input type: {loss_fn.input_type}")

    score_centering = getattr(loss_fn, "score_centering", False)
    fused_linear = getattr(loss_fn, "use_fused_linear_logprobs", False)
    both = None
    if (score_centering and not fused_linear and cp_sharder is None
            and not need_top_k_or_top_p_filtering(sampling_params)
            and not _is_dtensor(logits) and _group_size(context_parallel_group) == 1):
        # next-token and sampler top-k logprobs from one pass over the logits
        both = next_token_and_sampler_topk_logprobs(
            data["input_ids"], data["sampler_topk_token_ids"], logits,
            vocab_parallel_rank=vocab_parallel_rank, vocab_parallel_group=vocab_parallel_group,
            chunk_size=chunk_size,
        )
    if both is not None:
        logprobs = both[0]
    elif fused_linear:
        # the logits argument already holds next-token logprobs [B, >= S-1]
        logprobs = logits.to(torch.float32)[:, : data["input_ids"].shape[1] - 1]
    else:
        logprobs = get_next_token_logprobs_from_logits(
            input_ids=data["input_ids"],
            next_token_logits=logits,
            vocab_parallel_rank=vocab_parallel_rank,
            vocab_parallel_group=vocab_parallel_group,
            context_parallel_group=context_parallel_group,
            sampling_params=sampling_params,
            chunk_size=chunk_size,
            cp_sharder=cp_sharder,
        )

    filtering = need_top_k_or_top_p_filtering(sampling_params)
    if filtering and getattr(loss_fn, "reference_policy_kl_penalty", 0) != 0:
        data["curr_logprobs_unfiltered"] = get_next_token_logprobs_from_logits(
            input_ids=data["input_ids"],
            next_token_logits=logits,
            vocab_parallel_rank=vocab_parallel_rank,
            vocab_parallel_group=vocab_parallel_group,
            context_parallel_group=context_parallel_group,
            sampling_params=None,
            chunk_size=None,
            cp_sharder=cp_sharder,
        )

    loss_input: dict[str, Any] = {"next_token_logprobs": logprobs}
    if filtering:
        loss_input["policy_support_mask"] = ~torch.isneginf(logprobs)
    if both is not None:
        loss_input["policy_logprobs_at_sampler_topk"] = both[1]
    elif score_centering:
        loss_input["policy_logprobs_at_sampler_topk"] = get_policy_logprobs_at_sampler_topk(
            sampler_topk_token_ids=data["sampler_topk_token_ids"],
            next_token_logits=logits,
            vocab_parallel_rank=vocab_parallel_rank,
            vocab_parallel_group=vocab_parallel_group,
            context_parallel_group=context_parallel_group,
            chunk_size=chunk_size,
            cp_sharder=cp_sharder,
        )
    return loss_input, data


def prepare_packed_loss_input(
    logits: torch.Tensor,
    data: Any,
    loss_fn: LossFunction,
    cu_seqlens_q: CpuIntTuple,
    cu_seqlens_q_padded: CpuIntTuple,
    vocab_parallel_rank: Optional[int] = None,
    vocab_parallel_group: Optional[Any] = None,
    context_parallel_group: Optional[Any] = None,
    sampling_params: Optional[TrainingSamplingParams] = None,
    chunk_size: Optional[int] = None,
    reuse_logits_storage: bool = False,
) -> tuple[dict[str, Any], Any]:
    """``(loss_input, data)`` from packed logits ``[1, T, V]`` in one pass (reference loss_input.py:468-634).

    ``data`` holds the unpacked ``[B, S]`` batch; the targets are packed with a
    per-sequence roll inside ``cu_seqlens_q_padded`` and the logprobs come back
    unpacked to ``[B, S-1]``.  When ``data`` carries ``cu_seqlens`` the inputs
    are already one packed row and the physical ``[1, T-1]`` layout is kept.
    """
    if loss_fn.input_type != LossInputType.LOGPROB:
        raise ValueError(
            f"prepare_packed_loss_input only supports LossInputType.LOGPROB, "
            f"got {loss_fn.input_type}. Use SequencePackingLossWrapper with "
            f"prepare_loss_input for other types."
        )
    assert vocab_parallel_group is not None, (
        "prepare_packed_loss_input requires vocab_parallel_group (Megatron TP)."
    )
    assert vocab_parallel_rank is not None, (
        "vocab_parallel_rank must be provided with vocab_parallel_group."
    )
    return _prepare_packed(
        logits, data, loss_fn, cu_seqlens_q, cu_seqlens_q_padded, vocab_parallel_rank,
        vocab_parallel_group, context_parallel_group, sampling_params, chunk_size,
        reuse_logits_storage,
    )


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
    """Packed-sequence logprobs as prepare_packed_loss_input takes them: the
    reference hands over the logits upcast to fp32 whenever it filters
    (loss_input.py:556-560), so top-p is decided in fp32 here; the kernels read
    the logits in their own dtype instead of an fp32 copy."""
    return _packed_sequence_logprobs(
        vocab_parallel_logits, target, cu_seqlens_padded, unpacked_seqlen, vocab_start_index,
        vocab_end_index, group, inference_only, cp_group, chunk_size, sampling_params,
        target_is_pre_rolled, return_packed_layout, reuse_logits_storage, torch.float32,
    )


def _prepare_packed(
    logits: torch.Tensor,
    data: Any,
    loss_fn: LossFunction,
    cu_seqlens_q: CpuIntTuple,
    cu_seqlens_q_padded: CpuIntTuple,
    vocab_parallel_rank: Optional[int],
    vocab_parallel_group: Optional[Any],
    context_parallel_group: Optional[Any],
    sampling_params: Optional[TrainingSamplingParams],
    chunk_size: Optional[int],
    reuse_logits_storage: bool,
) -> tuple[dict[str, Any], Any]:
    """prepare_packed_loss_input without its Megatron-only argument checks (a missing
    vocab group is the single-device case: rank 0, the whole vocabulary)."""
    if vocab_parallel_rank is None:
        vocab_parallel_rank = 0
    if getattr(loss_fn, "score_centering", False):
        _validate_score_centering_data(data)
    cp_size = _group_size(context_parallel_group)
    if cp_size != 1:
        raise _unsupported("context parallelism")

    input_ids = data["input_ids"]
    unpacked_seqlen = input_ids.shape[1]
    prepacked = "cu_seqlens" in data
    if prepacked:
        packed_targets = input_ids
    else:
        packed_targets = _pack_input_ids(
            input_ids, cu_seqlens_q, cu_seqlens_q_padded, cp_rank=0, cp_size=1, roll_shift=-1
        )

    filtering = need_top_k_or_top_p_filtering(sampling_params)
    use_chunking = chunk_size is not None and not filtering
    V = logits.shape[-1]

    def logprobs_of(params: Optional[TrainingSamplingParams], reuse: bool) -> torch.Tensor:
        return from_parallel_logits_to_logprobs_packed_sequences(
            logits,
            packed_targets,
            cu_seqlens_q_padded,
            unpacked_seqlen,
            vocab_start_index=vocab_parallel_rank * V,
            vocab_end_index=(vocab_parallel_rank + 1) * V,
            group=vocab_parallel_group,
            inference_only=False,
            cp_group=context_parallel_group,
            sampling_params=params,
            chunk_size=chunk_size if use_chunking else None,
            target_is_pre_rolled=not prepacked,
            return_packed_layout=prepacked,
            reuse_logits_storage=reuse,
        )

    logprobs = logprobs_of(sampling_params, reuse_logits_storage and use_chunking)
    if filtering and getattr(loss_fn, "reference_policy_kl_penalty", 0) != 0:
        data["curr_logprobs_unfiltered"] = logprobs_of(None, False)

    loss_input: dict[str, Any] = {"next_token_logprobs": logprobs}
    if filtering:
        loss_input["policy_support_mask"] = ~torch.isneginf(logprobs)
    if getattr(loss_fn, "score_centering", False):
        sampler_ids = data["sampler_topk_token_ids"]
        packed_sampler_ids = _pack_input_ids(
            sampler_ids.to(logits.device), cu_seqlens_q, cu_seqlens_q_padded, cp_rank=0,
            cp_size=1, roll_shift=-1,
        )
        loss_input["policy_logprobs_at_sampler_topk"] = get_policy_logprobs_at_sampler_topk(
            sampler_topk_token_ids=sampler_ids,
            next_token_logits=logits,
            vocab_parallel_rank=vocab_parallel_rank,
            vocab_parallel_group=vocab_parallel_group,
            context_parallel_group=context_parallel_group,
            chunk_size=chunk_size,
            cu_seqlens_q=cu_seqlens_q,
            cu_seqlens_q_padded=cu_seqlens_q_padded,
            packed_sampler_topk_token_ids=packed_sampler_ids,
        )
    return loss_input, data
