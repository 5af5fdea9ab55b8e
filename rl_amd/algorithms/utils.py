"""Loss math helpers: drop-in for the hot-path subset of ``nemo_rl.algorithms.utils``.

``calculate_kl`` and ``masked_mean`` are the reference's one-line tensor
formulas (reference utils.py:56-115, :294-306), kept as plain tensor code for
callers that use them directly; ``ClippedPGLossFn`` does not call them — its
kernel fuses the same arithmetic.  ``calculate_baseline_and_std_per_prompt``
runs the GRPO group-statistics kernel.  ``mask_filtered_logprobs_outside_tokens``
and ``compute_seq_logprob_errors`` run token-level kernels (seq_errors.hip).
"""

from __future__ import annotations

from typing import Any, Optional

import torch

from rl_amd import _C


def calculate_kl(
    logprobs: torch.Tensor,
    logprobs_reference: torch.Tensor,
    kl_type: str = "k3",
    input_clamp_value: float | None = 20.0,
    output_clamp_value: float | None = 10.0,
    importance_sampling_weights: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-token KL estimate (k1 / k2 / k3, Schulman 2020) with optional clamps and IS weights."""
    logr = logprobs_reference - logprobs
    if input_clamp_value is not None:
        logr_clamped = logr.clamp(min=-input_clamp_value, max=input_clamp_value)
        if importance_sampling_weights is not None:
            importance_sampling_weights = torch.where(
                logr == logr_clamped,
                importance_sampling_weights,
                importance_sampling_weights.detach(),
            )
        logr = logr_clamped
    if kl_type == "k1":
        kl = -logr
    elif kl_type == "k2":
        kl = torch.square(logr) / 2
    elif kl_type == "k3":
        kl = torch.exp(logr) - 1 - logr
    else:
        raise ValueError(f"Invalid KL type: {kl_type}")
    if importance_sampling_weights is not None:
        kl = importance_sampling_weights * kl
    if output_clamp_value is not None:
        kl = kl.clamp(min=-output_clamp_value, max=output_clamp_value)
    return kl


def masked_mean(
    values: torch.Tensor,
    mask: torch.Tensor,
    dim: Optional[int] = None,
    global_normalization_factor: Optional[torch.Tensor | float] = None,
):
    """``sum(values * mask, dim) / (N + 1e-8)`` with N = sum(mask) or the global factor."""
    normalization_factor = (
        torch.sum(mask, dim=dim) if global_normalization_factor is None else global_normalization_factor
    )
    return torch.sum(values * mask, dim=dim) / (normalization_factor + 1e-8)


class _MaskOutsideTokens(torch.autograd.Function):
    """where(mask, logprobs, 0) on the select kernel; backward where(mask, g, 0) on the same."""

    @staticmethod
    def forward(ctx: Any, logprobs: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:  # type: ignore[override]
        ctx.save_for_backward(mask)
        return _C.mask_outside_tokens(logprobs, mask)

    @staticmethod
    def backward(ctx: Any, grad: torch.Tensor):  # type: ignore[override]
        (mask,) = ctx.saved_tensors
        return _C.mask_outside_tokens(grad, mask), None


def mask_filtered_logprobs_outside_tokens(logprobs: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """Zero filtered logprobs outside ``mask`` (reference utils.py:309-326).

    ``where(mask.bool(), logprobs, 0.0)``: tokens outside the valid-token mask
    (prompt, padding) get 0 instead of the -inf the filter may have given them;
    valid tokens keep -inf.  Returns a new tensor of ``logprobs``' dtype (the
    kernel copies the selected values bit for bit, so fp64 stays exact) and keeps
    autograd: the gradient is ``where(mask, g, 0)``, as for the reference's ``where``.
    """
    if torch.is_grad_enabled() and logprobs.requires_grad:
        return _MaskOutsideTokens.apply(logprobs, mask)
    return _C.mask_outside_tokens(logprobs, mask)


@torch.no_grad()
def compute_seq_logprob_errors(
    *,
    policy_logprobs: torch.Tensor,
    generation_logprobs: torch.Tensor,
    token_mask: torch.Tensor,
    sample_mask: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Mean multiplicative absolute logprob error and validity per sequence (reference utils.py:273-291).

    Inputs are aligned to predicted tokens; with ``w = token_mask * sample_mask[:, None]``,
    ``errors = sum(exp(|gen - pol| * w) * w) / max(sum(w), 1)`` over masked-in tokens and
    ``valid = sum(w) > 0``.  A non-finite logprob on a valid token makes its sequence's error
    non-finite.  Logprobs are computed on in fp32 (others are widened first).
    """
    return _C.seq_logprob_errors(policy_logprobs.to(torch.float32), generation_logprobs.to(torch.float32),
                                 token_mask, sample_mask)


def _to_device_inputs(prompts, rewards, valid_mask):
    if rewards.is_cuda:
        dev = rewards.device
    elif torch.cuda.is_available():
        dev = torch.device("cuda", torch.cuda.current_device())
    else:
        raise _C.MirlError("the GRPO advantage kernel needs a ROCm GPU; none is available")
    p = prompts
    if p.dim() == 1:
        p = p.unsqueeze(1)
    p = p.to(device=dev, dtype=torch.int64).contiguous()
    r = rewards.to(device=dev, dtype=torch.float32).contiguous()
    v = None if valid_mask is None else valid_mask.to(device=dev, dtype=torch.float32).contiguous()
    return p, r, v


def calculate_baseline_and_std_per_prompt(
    prompts: torch.Tensor,
    rewards: torch.Tensor,
    valid_mask: torch.Tensor,
    leave_one_out_baseline: bool = True,
    std_rewards: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-sample group baseline, std and trivial-group flag (reference utils.py:118-234).

    Runs on the GPU; CPU inputs are copied to the current device and the
    results copied back.  ``std_rewards`` (DAPO) replaces the rewards in the
    spread statistics and the trivial-group test only.
    """
    p, r, v = _to_device_inputs(prompts, rewards, valid_mask)
    q = None
    if std_rewards is not None and std_rewards is not rewards:
        q = std_rewards.to(device=r.device, dtype=torch.float32).contiguous()
    _, base, std, trivial = _C.grpo_advantage(
        p, r, v, leave_one_out_baseline, True, want_stats=True, std_rewards=q
    )
    out_dev = rewards.device
    return (
        base.to(device=out_dev, dtype=rewards.dtype),
        std.to(device=out_dev, dtype=rewards.dtype),
        trivial.to(out_dev),
    )
