"""Score-centering term restated with PyTorch autograd on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Follows
compute_score_centering_term (reference nemo_rl/algorithms/loss/score_centering.py:22-129)
and adaptive_ppo_clip_kept_mask (nemo_rl/algorithms/loss/clipped_pg.py:38-50).
"""

from __future__ import annotations

import torch


def adaptive_ppo_clip_kept_mask(w, *, advantages, lower_bound, upper_bound, outer_bound):
    """reference clipped_pg.py:38-50"""
    return (
        (w <= outer_bound)
        & ((advantages >= 0) | (w >= lower_bound))
        & ((advantages <= 0) | (w <= upper_bound))
    )


def score_centering_term(
    plog: torch.Tensor,
    *,
    sampler_topk_logprobs: torch.Tensor,
    importance_sampling_mode: str,
    is_bounds,
    token_mask: torch.Tensor,
    adaptive_ppo_clip_advantages=None,
    adaptive_ppo_clip_outer_bound=None,
):
    """(term [B, S], head_mass [B, S]); term carries the gradient to plog."""
    active = token_mask.bool()
    p_log = torch.where(active.unsqueeze(-1), plog, 0.0)
    q_log = torch.where(active.unsqueeze(-1), sampler_topk_logprobs.detach(), 0.0)
    p = p_log.detach().exp()
    q = q_log.exp()
    head_mass = q.sum(-1)
    rho = (1.0 - head_mass).clamp(min=0.0) / (1.0 - p.sum(-1)).clamp(min=1e-6)
    mode = importance_sampling_mode
    if mode == "off":
        mass, alpha = q, rho
    elif mode == "is":
        mass, alpha = p, torch.ones_like(rho)
    elif mode == "tis":
        lo, hi = is_bounds
        mass = torch.minimum(torch.maximum(p, lo * q), hi * q)
        alpha = torch.minimum(torch.maximum(torch.ones_like(rho), lo * rho), hi * rho)
    elif mode == "icepop":
        lo, hi = is_bounds
        ratio = (p_log.detach() - q_log).exp()
        mass = torch.where((ratio >= lo) & (ratio <= hi), p, 0.0)
        tail = rho.reciprocal()
        alpha = ((tail >= lo) & (tail <= hi)).to(p.dtype)
    elif mode == "adaptive-ppo-clip":
        lo, hi = is_bounds
        adv = adaptive_ppo_clip_advantages
        ratio = (p_log.detach() - q_log).exp()
        kept = adaptive_ppo_clip_kept_mask(ratio, advantages=adv.unsqueeze(-1), lower_bound=lo,
                                           upper_bound=hi, outer_bound=adaptive_ppo_clip_outer_bound)
        mass = torch.where(kept, p, 0.0)
        alpha = adaptive_ppo_clip_kept_mask(rho.reciprocal(), advantages=adv, lower_bound=lo,
                                            upper_bound=hi,
                                            outer_bound=adaptive_ppo_clip_outer_bound).to(p.dtype)
    else:
        raise ValueError(f"Unsupported score-centering IS mode {mode!r}")
    coef = mass - alpha.unsqueeze(-1) * p
    term = (coef.detach() * p_log).sum(-1)
    return torch.where(active, term, 0.0), torch.where(active, head_mass, 0.0)
