"""Loss-function interfaces: drop-in for ``nemo_rl.algorithms.loss.interfaces`` (reference :23-115)."""

from __future__ import annotations

import enum
from typing import Any, Mapping, Protocol

import torch


class LossType(enum.Enum):
    TOKEN_LEVEL = "token_level"
    SEQUENCE_LEVEL = "sequence_level"


class MetricNormalizer(enum.Enum):
    """Global denominator a returned metric was normalized by."""

    TOKENS = "tokens"
    SEQUENCES = "sequences"
    NONE = "none"


class LossInputType(enum.Enum):
    LOGIT = "logit"
    LOGPROB = "logprob"
    OPD_FULL = "opd_full"
    DISTILLATION = "distillation"
    DISTILLATION_CROSS_TOKENIZER = "distillation_cross_tokenizer"
    DRAFT = "draft"


class LossFunction(Protocol):
    """A loss maps (data, global normalisers, loss inputs) to (scalar loss, metrics)."""

    loss_type: LossType
    input_type: LossInputType

    def __call__(
        self,
        data: Mapping[str, Any],
        global_valid_seqs: torch.Tensor,
        global_valid_toks: torch.Tensor,
        **kwargs: Any,
    ) -> tuple[torch.Tensor, dict[str, Any]]: ...
