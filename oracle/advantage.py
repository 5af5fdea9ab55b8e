"""GRPO group baseline / std / advantages restated on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Follows
calculate_baseline_and_std_per_prompt (reference nemo_rl/algorithms/utils.py:118-234)
and GRPOAdvantageEstimator.compute_advantage
(reference nemo_rl/algorithms/advantage_estimator.py:106-145).
"""

from __future__ import annotations

import torch


def baseline_and_std_per_prompt(prompts, rewards, valid_mask, leave_one_out_baseline=True, std_rewards=None):
    """Returns (baseline, std, is_trivial) per sample, fp32 matmul formulation of the reference.

    ``std_rewards`` (reference utils.py:161-162, 190-203) replaces the rewards in the
    spread (std) and in the trivial-group test; the baseline stays on ``rewards``.
    """
    q_all = rewards if std_rewards is None else std_rewards
    baseline = torch.zeros_like(rewards)
    std = torch.zeros_like(rewards)
    trivial = torch.ones_like(rewards, dtype=torch.bool)
    for key in torch.unique(prompts, dim=0):
        idx = torch.arange(len(prompts))[(prompts == key).all(1)]
        n = len(idx)
        M = (1 - torch.eye(n)) if leave_one_out_baseline else torch.ones((n, n))
        v = valid_mask[idx]
        if v.sum() <= 1:
            baseline[idx] = rewards[idx]
            continue
        nv = v.float().sum() - int(leave_one_out_baseline)
        b = torch.matmul(M, rewards[idx] * v) / nv
        q = q_all[idx]
        bq = b if std_rewards is None else torch.matmul(M, q * v) / nv
        sq = torch.matmul(M, torch.pow(q, 2) * v) / nv
        comp = M.bool() & v.bool().unsqueeze(0)
        rr = q.unsqueeze(0).expand(n, -1)
        cmin = rr.masked_fill(~comp, torch.inf).amin(dim=1)
        cmax = rr.masked_fill(~comp, -torch.inf).amax(dim=1)
        baseline[idx] = b
        trivial[idx] = cmin == cmax
        std[idx] = ((sq - bq.square()) * (nv / (nv - 1))).sqrt().nan_to_num(0)
    return baseline, std, trivial


def grpo_advantages(prompt_ids, rewards, mask, valid_mask=None, leave_one_out=True, normalize=True):
    """[B, S] advantages broadcast over the mask shape."""
    v = torch.ones_like(rewards) if valid_mask is None else valid_mask.float()
    baseline, std, trivial = baseline_and_std_per_prompt(prompt_ids, rewards, v, leave_one_out)
    adv = (rewards - baseline).unsqueeze(-1)
    if normalize:
        nm = (std > 0) & ~trivial
        adv[nm] = adv[nm] / (std.unsqueeze(-1)[nm] + 1e-6)
    return adv.expand(mask.shape)
