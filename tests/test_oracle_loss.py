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


# reference tests/unit/algorithms/test_loss_functions.py:1000-1039: logprobs -1, reference
# logprobs (0, -15, -30); un-clamped and clamped (input 20, output 10) KL values (rtol 1e-3)
KL_KNOWN = {
    "k1": ([-1.0, 14.0, 29.0], [-1.0, 10.0, 10.0]),
    "k2": ([0.5, 98.0, 420.5], [0.5, 10.0, 10.0]),
    "k3": ([0.7183, 13.0, 28.0], [0.7183, 10.0, 10.0]),
}


def _kl_impls():
    from oracle.loss import calculate_kl as oracle_kl
    from rl_amd.algorithms.utils import calculate_kl as api_kl

    return [oracle_kl, api_kl]


@pytest.mark.parametrize("impl", [0, 1], ids=["oracle", "api"])
@pytest.mark.parametrize("kl_type", list(KL_KNOWN))
def test_calculate_kl_known_answers(kl_type, impl):
    kl_fn = _kl_impls()[impl]
    lp = torch.tensor([[-1.0, -1.0, -1.0]])
    ref = torch.tensor([[-0.0, -15.0, -30.0]])
    raw, clamped = KL_KNOWN[kl_type]
    kl = kl_fn(lp, ref, kl_type, input_clamp_value=None, output_clamp_value=None)
    assert torch.allclose(kl, torch.tensor([raw]), rtol=1e-3)
    kl = kl_fn(lp, ref, kl_type, input_clamp_value=20.0, output_clamp_value=10.0)
    assert torch.allclose(kl, torch.tensor([clamped]), rtol=1e-3)


@pytest.mark.parametrize("impl", [0, 1], ids=["oracle", "api"])
def test_calculate_kl_importance_weight_rules(impl):
    """reference test_loss_functions.py:1042-1097: an input-clamped term detaches its IS
    weight (gradient 0 there, -1 elsewhere); the output clamp applies after the IS weight."""
    kl_fn = _kl_impls()[impl]
    lp = torch.tensor([[-3.0, -1.0]], requires_grad=True)
    kl = kl_fn(lp, torch.zeros_like(lp), "k3", input_clamp_value=2.0, output_clamp_value=None,
               importance_sampling_weights=torch.exp(lp - lp.detach()))
    torch.testing.assert_close(kl.detach(), torch.tensor([[4.389056, 0.7182818]]))
    kl.sum().backward()
    torch.testing.assert_close(lp.grad, torch.tensor([[0.0, -1.0]]), atol=1e-6, rtol=1e-6)
    lp = torch.tensor([[-1.0]], requires_grad=True)
    kl = kl_fn(lp, torch.zeros_like(lp), "k3", input_clamp_value=None, output_clamp_value=1.0,
               importance_sampling_weights=100.0 * torch.exp(lp - lp.detach()))
    torch.testing.assert_close(kl.detach(), torch.tensor([[1.0]]))
    kl.sum().backward()
    torch.testing.assert_close(lp.grad, torch.zeros_like(lp), atol=1e-6, rtol=1e-6)


def test_masked_mean_all_zeros():
    """reference test_loss_functions.py:1839-1858 (the +1e-8 keeps an empty mask at 0)."""
    from oracle.loss import masked_mean as oracle_mm
    from rl_amd.algorithms.utils import masked_mean as api_mm

    for mm in (oracle_mm, api_mm):
        values = torch.tensor([1.0, 2.0, 3.0, 4.0])
        mask = torch.zeros_like(values)
        assert mm(values, mask).item() == 0.0
        mask[0] = 1
        assert mm(values, mask).item() == pytest.approx(1.0)
        v2 = torch.tensor([[1.0, 2.0], [3.0, 4.0]])
        assert torch.equal(mm(v2, torch.zeros_like(v2), dim=1), torch.zeros(2))
