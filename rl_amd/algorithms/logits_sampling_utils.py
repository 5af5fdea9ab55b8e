"""Training-side top-k / top-p filtering: drop-in for ``nemo_rl.algorithms.logits_sampling_utils``.

``TrainingSamplingParams`` and the predicates keep the reference's semantics
(reference logits_sampling_utils.py:29-66).  ``apply_top_k_top_p`` runs the
gfx950 selection kernel (``rl_amd.distributed.sampling``) and keeps the
reference's autograd contract: gradients outside the kept set are zero.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

# Rows per chunk of the reference's sort-based filter (reference :26).  The
# kernels here do not sort the vocabulary, so the value is accepted and ignored.
TOP_K_TOP_P_CHUNK_SIZE: int = 256


@dataclass
class TrainingSamplingParams:
    """Sampling parameters mirrored from generation (reference :29-44).

    top_k: None or <= 0 disables top-k; top_p: 1.0 disables top-p;
    temperature is applied by the caller (``apply_temperature_scaling``).
    """

    top_k: int | None = None
    top_p: float = 1.0
    temperature: float = 1.0


def _need_top_k_filtering(top_k: int | None) -> bool:
    return top_k is not None and top_k > 0


def _need_top_p_filtering(top_p: float | None) -> bool:
    return top_p is not None and top_p != 1.0


def need_top_k_or_top_p_filtering(sampling_params: Optional[TrainingSamplingParams]) -> bool:
    """True iff top-k (k > 0) or top-p (p != 1) filtering is requested (reference :57-66)."""
    if sampling_params is None:
        return False
    return _need_top_k_filtering(sampling_params.top_k) or _need_top_p_filtering(
        sampling_params.top_p
    )


def apply_top_k_top_p(
    logits: torch.Tensor,
    top_k: int | None,
    top_p: float,
    chunk_size: int | None = TOP_K_TOP_P_CHUNK_SIZE,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Mask logits outside the top-k / top-p set to -inf (reference :256-287).

    Returns ``(filtered_logits, keep_mask)``, or ``(logits, None)`` when no
    filtering is requested.  Ties at the k-th value are all kept; top-p keeps
    the shortest suffix of the ascending (stable) order whose cumulative
    probability exceeds ``1 - top_p``, and always the maximum.

    Top-p is decided in the tensor's own dtype, as the reference's op
    sequence does on an un-upcast tensor (logits_sampling_utils.py:189-191):
    for bf16/fp16 the probabilities are rounded to the dtype and their
    cumulative sum is rounded to it at every step; fp32 tensors (what the
    production callers pass after their upcast) decide in fp32.  The top-k
    set does not depend on the dtype.  The filtered logits keep the input
    dtype.
    """
    if not _need_top_k_filtering(top_k) and not _need_top_p_filtering(top_p):
        return logits, None
    from rl_amd.distributed.sampling import apply_top_k_top_p_kernel

    return apply_top_k_top_p_kernel(logits, top_k, top_p)


def need_temperature_scaling(sampling_params: Optional[TrainingSamplingParams]) -> bool:
    """Whether apply_temperature_scaling will mutate the logits in place
    (reference nemo_rl/models/automodel/train.py:241-245)."""
    return sampling_params is not None and sampling_params.temperature != 1.0


def apply_temperature_scaling(
    logits: torch.Tensor, sampling_params: Optional[TrainingSamplingParams]
) -> torch.Tensor:
    """``logits.div_(sampling_params.temperature)`` in place, in the logits dtype
    (reference nemo_rl/models/automodel/train.py:248-262,
    nemo_rl/models/megatron/train.py:280-294); a no-op for None or T == 1.

    The division runs on the gfx950 temperature kernel with the arithmetic of
    torch's GPU ``div_`` by a Python scalar (the product with ``fl32(1.0 / T)``,
    rounded to the logits dtype) and is recorded for autograd; its backward is
    the same product applied to the gradient.  When the filtered logprobs of
    this package are the only consumer of the scaled logits, that backward is
    folded into their own gradient write, unless the scaled tensor retains its
    gradient (``retain_grad``).  A caller that asks ``autograd.grad`` for the
    scaled tensor itself turns the fold off first
    (``rl_amd.distributed.sampling.set_temperature_fold(False)``).
    """
    if need_temperature_scaling(sampling_params):
        from rl_amd.distributed.sampling import temperature_scale_

        return temperature_scale_(logits, sampling_params.temperature)  # type: ignore[union-attr]
    return logits
