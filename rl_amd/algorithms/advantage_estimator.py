"""GRPO advantage estimator: drop-in for the GRPO part of ``nemo_rl.algorithms.advantage_estimator``.

``GRPOAdvantageEstimator.compute_advantage`` runs the group-statistics kernel
(one thread per sample) and returns the advantages broadcast to the token mask
shape, as the reference does (reference advantage_estimator.py:94-145).
"""

from __future__ import annotations

from typing import Any, Literal

import torch
from pydantic import BaseModel, Field
from typing_extensions import Annotated

from rl_amd.algorithms.utils import _to_device_inputs
from rl_amd import _C


class AdvEstimatorConfig(BaseModel, extra="allow"):
    """Advantage-estimator configuration (reference advantage_estimator.py:60-77)."""

    name: Literal["grpo", "gdpo", "opd", "reinforce_plus_plus"] = "grpo"
    normalize_rewards: bool = True
    use_leave_one_out_baseline: bool = True
    reward_weights: list[float] | None = None
    minus_baseline: bool = True
    proximal_teacher_alpha: Annotated[float, Field(gt=0.0, le=1.0)] = 1.0
    subtract_global_baseline: bool = False


class GRPOAdvantageEstimator:
    """GRPO group-relative advantages: ``(r - baseline) / (std + 1e-6)`` per prompt group."""

    def __init__(self, estimator_config: AdvEstimatorConfig, loss_config: Any = None):
        self.use_leave_one_out_baseline = estimator_config.use_leave_one_out_baseline
        self.normalize_rewards = estimator_config.normalize_rewards

    def compute_advantage(self, prompt_ids, rewards, mask, valid_mask=None, **kwargs):
        """Advantages ``[B, S]`` (a broadcast view of one value per sample).

        prompt_ids: [B, k] group keys; rewards: [B]; mask: [B, S] (shape only);
        valid_mask: optional [B], 0 excludes a sample from its group's statistics.
        CPU inputs are computed on the current GPU and returned on their device.
        """
        p, r, v = _to_device_inputs(prompt_ids, rewards, valid_mask)
        adv, _, _, _ = _C.grpo_advantage(
            p, r, v, self.use_leave_one_out_baseline, self.normalize_rewards
        )
        adv = adv.to(device=rewards.device, dtype=rewards.dtype)
        return adv.unsqueeze(-1).expand(mask.shape)
