"""The CPU oracle of the ClippedPG loss against the reference's float64 goldens (CPU only)."""

import pytest
import torch

from oracle.loss import clipped_pg_loss
from tests.helpers import golden_case_inputs, load_goldens

GOLDENS = load_goldens()
CASES = GOLDENS["cases"]


def test_golden_file_is_the_reference_fixture():
    assert GOLDENS["schema_version"] == 1
    assert GOLDENS["provenance"]["dtype"] == "float64"
    assert len(CASES) == 12


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_reference_goldens(case):
    ntl, data, gvs, gvt, grad_inputs = golden_case_inputs(GOLDENS, case)
    loss, metrics = clipped_pg_loss(ntl, data, gvs, gvt, **case["config"])
    exp = case["expected"]
    torch.testing.assert_close(loss.detach(), torch.tensor(exp["loss"], dtype=torch.float64),
                               rtol=1e-12, atol=1e-12)
    grads = torch.autograd.grad(loss, [t for _, t in grad_inputs])
    for (name, _), g in zip(grad_inputs, grads):
        torch.testing.assert_close(g, torch.tensor(exp["gradients"][name], dtype=torch.float64),
                                   rtol=1e-12, atol=1e-12)
    # the goldens predate this metric; the reference test pops it and requires 0
    assert metrics.pop("policy_support_excluded_tokens") == 0
    assert set(metrics) == set(exp["metrics"]), sorted(set(metrics) ^ set(exp["metrics"]))
    for k, v in exp["metrics"].items():
        assert metrics[k] == pytest.approx(v, rel=1e-12, abs=1e-12), k


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_minimal_metrics_keep_loss_and_grads(case):
    ntl, data, gvs, gvt, grad_inputs = golden_case_inputs(GOLDENS, case)
    loss, metrics = clipped_pg_loss(ntl, data, gvs, gvt, metrics_level="minimal", **case["config"])
    exp = case["expected"]
    assert loss.item() == pytest.approx(exp["loss"], rel=1e-12, abs=1e-12)
    grads = torch.autograd.grad(loss, [t for _, t in grad_inputs])
    for (name, _), g in zip(grad_inputs, grads):
        torch.testing.assert_close(g, torch.tensor(exp["gradients"][name], dtype=torch.float64),
                                   rtol=1e-12, atol=1e-12)
    names = {"loss", "kl_penalty", "num_valid_samples", "positive_nll_loss", "token_mult_prob_error"}
    if case["config"].get("use_importance_sampling_correction", False):
        names.add("sampling_importance_ratio")
    if case["config"].get("truncated_importance_sampling_type") is not None:
        names.add("is_oob_ratio")
    assert metrics.pop("policy_support_excluded_tokens") == 0
    assert set(metrics) == names
    for k in names:
        assert metrics[k] == pytest.approx(exp["metrics"][k], rel=1e-12, abs=1e-12), k


def test_oracle_known_answer_ppo_clipping():
    """Hand-computed PPO clipping values: a mutated-input check that a dropped clamp fails.

    One token, A = 1: ratio 1.5 above 1.2 clamps the objective to -1.2; ratio
    0.5 below 0.8 keeps -0.5 (max picks the unclipped, larger term).
    """
    for ratio, expected in [(1.5, -1.2), (0.5, -0.5), (1.0, -1.0)]:
        curr = torch.tensor([[0.0, float(torch.log(torch.tensor(ratio, dtype=torch.float64)))]],
                            dtype=torch.float64)[:, 1:].clone().requires_grad_(True)
        data = {
            "token_mask": torch.tensor([[0.0, 1.0]], dtype=torch.float64),
            "sample_mask": torch.tensor([1.0], dtype=torch.float64),
            "advantages": torch.tensor([[0.0, 1.0]], dtype=torch.float64),
            "prev_logprobs": torch.zeros(1, 2, dtype=torch.float64),
            "generation_logprobs": torch.zeros(1, 2, dtype=torch.float64),
            "reference_policy_logprobs": torch.zeros(1, 2, dtype=torch.float64),
        }
        loss, _ = clipped_pg_loss(curr, data, torch.tensor(1.0, dtype=torch.float64),
                                  torch.tensor(1.0, dtype=torch.float64),
                                  reference_policy_kl_penalty=0.0)
        assert loss.item() == pytest.approx(expected / (1 + 1e-8), rel=1e-12)
