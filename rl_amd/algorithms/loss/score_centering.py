"""Score-centering correction: drop-in for ``nemo_rl.algorithms.loss.score_centering``.

``compute_score_centering_term`` returns the per-token term
``sum_k sg(c_k) * log p_k`` and the sampler head mass (reference
score_centering.py:22-129), computed by one gfx950 kernel over the tokens; its
backward multiplies the saved coefficients ``c_k`` by the upstream gradient.
``ClippedPGLossFn`` does not call it: its fused kernel applies the same per-token
arithmetic inline.
"""

from __future__ import annotations

from typing import Any, Optional

import torch

from rl_amd import _C

__all__ = ["compute_score_centering_term"]


class _ScoreCenteringTerm(torch.autograd.Function):
    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        plog: torch.Tensor,
        qlog: torch.Tensor,
        mode: str,
        bounds: Optional[tuple],
        outer: Optional[float],
        token_mask: torch.Tensor,
        advantages: Optional[torch.Tensor],
    ):
        B, L, _ = plog.shape
        coef = torch.empty(plog.shape, dtype=plog.dtype, device=plog.device)
        term = torch.empty((B, L), dtype=plog.dtype, device=plog.device)
        head = torch.empty((B, L), dtype=plog.dtype, device=plog.device)
        args = _C.score_centering_args(mode, bounds, outer, plog, qlog, coef)
        _C.score_centering_term(args, plog.dtype, token_mask, advantages, term, head)
        ctx.save_for_backward(coef)
        ctx.mark_non_differentiable(head)
        return term, head

    @staticmethod
    def backward(ctx: Any, grad_term: torch.Tensor, grad_head: torch.Tensor):  # type: ignore[override]
        (coef,) = ctx.saved_tensors
        return coef * grad_term.unsqueeze(-1), None, None, None, None, None, None


def compute_score_centering_term(
    policy_logprobs_at_sampler_topk: torch.Tensor,
    *,
    sampler_topk_logprobs: torch.Tensor,
    importance_sampling_mode: str,
    is_bounds: tuple[float, float] | None,
    token_mask: torch.Tensor,
    adaptive_ppo_clip_advantages: torch.Tensor | None = None,
    adaptive_ppo_clip_outer_bound: float | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token ``sum_v sg(c_v) * log p_v`` ``[B, S]`` and the sampler head mass ``[B, S]``.

    Same arguments, modes (``off``, ``is``, ``tis``, ``icepop``,
    ``adaptive-ppo-clip``) and masking as the reference; both outputs are 0
    where ``token_mask`` is 0.
    """
    if importance_sampling_mode not in _C.SC_MODES:
        raise ValueError(
            f"Unsupported score-centering IS mode {importance_sampling_mode!r}"
        )
    if importance_sampling_mode in ("tis", "icepop", "adaptive-ppo-clip"):
        assert is_bounds is not None
    if importance_sampling_mode == "adaptive-ppo-clip":
        assert adaptive_ppo_clip_advantages is not None
        assert adaptive_ppo_clip_outer_bound is not None
    plog = policy_logprobs_at_sampler_topk
    if plog.dim() != 3:
        raise ValueError(f"expected [B, S, k] log-probs, got {tuple(plog.shape)}")
    if tuple(sampler_topk_logprobs.shape) != tuple(plog.shape):
        raise ValueError(
            f"sampler_topk_logprobs shape {tuple(sampler_topk_logprobs.shape)} does not match "
            f"{tuple(plog.shape)}"
        )
    if tuple(token_mask.shape) != tuple(plog.shape[:2]):
        raise ValueError(f"token_mask shape {tuple(token_mask.shape)} does not match {tuple(plog.shape[:2])}")
    if (importance_sampling_mode == "adaptive-ppo-clip"
            and tuple(adaptive_ppo_clip_advantages.shape) != tuple(plog.shape[:2])):
        raise ValueError("adaptive_ppo_clip_advantages must be [B, S]")
    dtype = plog.dtype if plog.dtype in (torch.float32, torch.float64) else torch.float32
    if plog.dtype != dtype:
        plog = plog.to(dtype)
    qlog = sampler_topk_logprobs.detach().to(device=plog.device, dtype=dtype)
    tm = token_mask.to(device=plog.device, dtype=dtype)
    adv = None
    if importance_sampling_mode == "adaptive-ppo-clip":
        adv = adaptive_ppo_clip_advantages.detach().to(device=plog.device, dtype=dtype)
    term, head = _ScoreCenteringTerm.apply(
        plog, qlog, importance_sampling_mode, is_bounds, adaptive_ppo_clip_outer_bound, tm, adv
    )
    return term, head
