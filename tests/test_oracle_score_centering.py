"""The score-centering oracle, pinned by the reference tests' full-distribution identities (CPU).

The checks follow tests/unit/algorithms/test_score_centering.py:90-256: the
gradient of the correction equals the gradient of sum_v q_v w_v log p_v over the
whole vocabulary (head exact, tail modelled as rho * p) for every importance
sampling mode, untruncated IS gives a zero correction, adaptive-ppo-clip picks
its bounds per position by the advantage's sign, and non-finite values at masked
positions never reach the loss or its gradients.
"""

import itertools

import pytest
import torch

from oracle.loss import clipped_pg_loss
from oracle.score_centering import score_centering_term


def _adaptive_weights(ratios, advantage):
    # lo = 0.5, hi = 2, outer = 5 written out independently of the kept-mask helper
    if advantage > 0:
        sign_bound = ratios <= 2.0
    elif advantage < 0:
        sign_bound = ratios >= 0.5
    else:
        sign_bound = torch.ones_like(ratios, dtype=torch.bool)
    return torch.where((ratios <= 5.0) & sign_bound, ratios, 0.0)


@pytest.mark.parametrize(("mode", "advantage"), [("off", 1.0), ("is", 1.0), ("tis", 1.0),
                                                 ("icepop", 1.0), ("adaptive-ppo-clip", 1.0),
                                                 ("adaptive-ppo-clip", -1.0)])
@pytest.mark.parametrize("head_probs", [(0.1, 0.6), (0.3, 0.65)])
def test_matches_full_distribution_gradient(mode, advantage, head_probs):
    logits = torch.tensor([0.6, -0.2, 0.1, -0.7], requires_grad=True)
    logp = logits.log_softmax(-1)
    q_head = torch.tensor(head_probs)
    q = torch.cat([q_head, (1 - q_head.sum()) * logp[2:].softmax(-1).detach()])
    truncated = mode in ("tis", "icepop", "adaptive-ppo-clip")
    term, _ = score_centering_term(
        logp[:2].reshape(1, 1, 2),
        sampler_topk_logprobs=q_head.log().reshape(1, 1, 2),
        importance_sampling_mode=mode,
        is_bounds=(0.5, 2.0) if truncated else None,
        token_mask=torch.ones(1, 1),
        adaptive_ppo_clip_advantages=torch.full((1, 1), advantage),
        adaptive_ppo_clip_outer_bound=5.0,
    )
    ratios = logp.detach().exp() / q
    weights = {"off": torch.ones_like(ratios), "is": ratios, "tis": ratios.clamp(0.5, 2.0),
               "icepop": torch.where((ratios >= 0.5) & (ratios <= 2.0), ratios, 0.0)}.get(mode)
    if weights is None:
        weights = _adaptive_weights(ratios, advantage)
    expected = (q * weights * logp).sum()
    got_grad = torch.autograd.grad(term.sum(), logits, retain_graph=True)[0]
    exp_grad = torch.autograd.grad(expected, logits)[0]
    torch.testing.assert_close(got_grad, exp_grad, atol=1e-6, rtol=1e-5)
    if mode == "is":
        torch.testing.assert_close(term, torch.zeros_like(term))


def test_adaptive_filters_by_each_positions_advantage():
    logits = torch.tensor([0.6, -0.2, 0.1, -0.7], requires_grad=True)
    logp = logits.log_softmax(-1)
    q_head = torch.tensor([0.1, 0.6])
    q = torch.cat([q_head, (1 - q_head.sum()) * logp[2:].softmax(-1).detach()])
    adv = torch.tensor([[1.0, -1.0, 0.0], [-1.0, 1.0, 1.0]])
    tm = torch.tensor([[1.0, 1.0, 1.0], [1.0, 0.0, 1.0]])
    term, _ = score_centering_term(
        logp[:2].expand(2, 3, 2), sampler_topk_logprobs=q_head.log().expand(2, 3, 2),
        importance_sampling_mode="adaptive-ppo-clip", is_bounds=(0.5, 2.0), token_mask=tm,
        adaptive_ppo_clip_advantages=adv, adaptive_ppo_clip_outer_bound=5.0)
    assert term[1, 1] == 0
    ratios = logp.detach().exp() / q
    for row, pos in tm.nonzero().tolist():
        w = _adaptive_weights(ratios, adv[row, pos].item())
        expected = (q * w * logp).sum()
        (a,) = torch.autograd.grad(term[row, pos], logits, retain_graph=True)
        (e,) = torch.autograd.grad(expected, logits, retain_graph=True)
        torch.testing.assert_close(a, e, atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize(("mode", "force_on_policy"),
                         [*itertools.product(("off", "is", "tis", "icepop"), (True, False)),
                          ("adaptive-ppo-clip", True)])
def test_nonfinite_masked_positions_stay_out_of_the_loss(mode, force_on_policy):
    lp = torch.tensor([0.6, -0.2, 0.1, -0.7]).log_softmax(-1)
    token_lp = torch.tensor([[lp[0], float("nan")]], requires_grad=True)
    head_lp = torch.tensor([[[lp[0], lp[1]], [float("nan"), float("inf")]]], requires_grad=True)
    data = {
        "token_mask": torch.tensor([[0.0, 1.0, 0.0]]),
        "sample_mask": torch.ones(1),
        "advantages": torch.tensor([[0.0, 1.0, float("nan")]]),
        "prev_logprobs": torch.tensor([[0.0, lp[0] - torch.log(torch.tensor(2.0)), float("nan")]]),
        "generation_logprobs": torch.tensor([[0.0, -2.3025851, float("nan")]]),
        "sampler_topk_logprobs": torch.tensor([[[0.0, 0.0], [0.1, 0.6], [float("nan")] * 2]]).log(),
    }
    truncated = mode in ("tis", "icepop", "adaptive-ppo-clip")
    cfg = dict(score_centering=True, reference_policy_kl_penalty=0,
               force_on_policy_ratio=force_on_policy,
               use_importance_sampling_correction=mode != "off",
               truncated_importance_sampling_type=mode if truncated else None,
               truncated_importance_sampling_ratio=2.0 if truncated else None,
               truncated_importance_sampling_ratio_min=0.5 if truncated else None)
    loss, _ = clipped_pg_loss(token_lp, data, torch.tensor(1.0), torch.tensor(1.0),
                              policy_logprobs_at_sampler_topk=head_lp, **cfg)
    assert torch.isfinite(loss)
    loss.backward()
    assert torch.isfinite(token_lp.grad).all() and torch.isfinite(head_lp.grad).all()
    assert token_lp.grad[0, 1] == 0 and torch.all(head_lp.grad[0, 1] == 0)
    if not force_on_policy:
        assert token_lp.grad[0, 0] == 0
    if mode in ("icepop", "adaptive-ppo-clip"):
        assert token_lp.grad[0, 0] == 0
        assert head_lp.grad[0, 0].abs().sum() > 0
