"""Token-level post-processing of logprobs restated as scalar loops on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Follows
mask_filtered_logprobs_outside_tokens (reference nemo_rl/algorithms/utils.py:309-326):
where(mask.bool(), logprobs, 0.0), and compute_seq_logprob_errors (reference
nemo_rl/algorithms/utils.py:273-291): per sequence, with w = token_mask * sample_mask
(fp32 product), sum(exp(where(w != 0, |gen - pol|, 0) * w) * w) / max(sum(w), 1) and
valid = sum(w) > 0.  Sums are accumulated in float64 and rounded once to fp32.
Pinned by hand-derived known answers in tests/test_oracle_token_metrics.py.
"""

from __future__ import annotations

import math

import torch


def mask_outside_tokens(logprobs: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    lp = logprobs.detach().cpu()
    m = mask.detach().cpu().expand(lp.shape)
    out = torch.empty_like(lp)
    flat_lp, flat_m, flat_o = lp.reshape(-1), m.reshape(-1), out.view(-1)
    for i in range(flat_lp.numel()):
        flat_o[i] = flat_lp[i] if bool(flat_m[i]) else 0.0
    return out


def seq_logprob_errors(policy, generation, token_mask, sample_mask):
    pol = policy.detach().cpu().float()
    gen = generation.detach().cpu().float()
    tm = token_mask.detach().cpu().float()
    sm = sample_mask.detach().cpu().float()
    B, S = pol.shape
    errors = torch.empty(B, dtype=torch.float32)
    valid = torch.empty(B, dtype=torch.bool)
    for b in range(B):
        cnt = 0.0
        acc = 0.0
        for s in range(S):
            w = float(torch.tensor(float(tm[b, s])) * torch.tensor(float(sm[b])))  # fp32 product
            cnt += w
            e = abs(float(gen[b, s]) - float(pol[b, s])) if w != 0.0 else 0.0
            if math.isnan(e * w):
                acc = float("nan")
            else:
                acc += math.exp(e * w) * w if e * w < 700.0 else float("inf")
        errors[b] = acc / max(cnt, 1.0)
        valid[b] = cnt > 0.0
    return errors, valid
