"""Pinning the GRPO advantage oracle with the reference tests' known answers (CPU only)."""

import pytest
import torch

from oracle.advantage import baseline_and_std_per_prompt, grpo_advantages
from tests.helpers import ADVANTAGE_KNOWN_ANSWERS, advantage_case_inputs, check_advantage_known_answer

P6 = torch.tensor([[1, 2, 3]] * 3 + [[4, 5, 6]] * 3)


def test_basic_loo_baseline_and_std():
    b, s, _ = baseline_and_std_per_prompt(P6, torch.tensor([1.0, 2, 3, 4, 5, 6]), torch.ones(6))
    assert torch.allclose(b, torch.tensor([2.5, 2.0, 1.5, 5.5, 5.0, 4.5]), rtol=1e-5)
    assert torch.allclose(s, torch.tensor([0.707107, 1.414214, 0.707107] * 2), rtol=1e-5)


def test_masked_sample_is_excluded():
    r = torch.tensor([1.0, 999.0, 3.0, 4.0, 5.0, 6.0])
    b, s, _ = baseline_and_std_per_prompt(P6, r, torch.tensor([1.0, 0, 1, 1, 1, 1]))
    assert torch.allclose(b, torch.tensor([3.0, 4.0, 1.0, 5.5, 5.0, 4.5]), rtol=1e-5)
    assert torch.allclose(s, torch.tensor([0.0, 0.0, 0.0, 0.707107, 1.414214, 0.707107]), rtol=1e-5)


def test_trivial_leave_one_out_set():
    r = torch.tensor([0.0] + [0.95] * 7)
    b, _, triv = baseline_and_std_per_prompt(torch.zeros(8, 1, dtype=torch.long), r, torch.ones(8))
    assert b[0].item() == pytest.approx(0.95)
    assert triv.tolist() == [True] + [False] * 7
    _, _, triv2 = baseline_and_std_per_prompt(torch.zeros(8, 1, dtype=torch.long), r, torch.ones(8), False)
    assert triv2.tolist() == [False] * 8


@pytest.mark.parametrize("loo", [False, True])
@pytest.mark.parametrize("normalize", [False, True])
def test_masked_reward_group_signal(loo, normalize):
    """reference tests/unit/algorithms/test_grpo.py:500-533 (num_valid = 3)."""
    adv = grpo_advantages(torch.zeros(3, 2, dtype=torch.long), torch.tensor([1.0, 1.0, 0.0]),
                          torch.ones(3, 2), torch.ones(3), leave_one_out=loo, normalize=normalize)
    exp = 0.5 if loo else 1.0 / 3.0
    if normalize:
        exp /= (0.5 if loo else 1.0 / 3.0) ** 0.5 + 1e-6
    assert adv[0, 0].item() == pytest.approx(exp)


def test_brute_force_random_groups():
    g = torch.Generator().manual_seed(0)
    B = 24
    prompts = torch.randint(0, 4, (B, 1), generator=g)
    r = torch.randn(B, generator=g)
    b, s, _ = baseline_and_std_per_prompt(prompts, r, torch.ones(B), False)
    for i in range(B):
        grp = r[(prompts[:, 0] == prompts[i, 0])].double()
        if len(grp) > 1:
            assert b[i].item() == pytest.approx(grp.mean().item(), abs=1e-6)
            assert s[i].item() == pytest.approx(grp.std(unbiased=True).item(), abs=1e-5)


@pytest.mark.parametrize("case", ADVANTAGE_KNOWN_ANSWERS, ids=[c[0] for c in ADVANTAGE_KNOWN_ANSWERS])
def test_reference_known_answers(case):
    """Every known answer of reference tests/unit/algorithms/test_utils.py:830-1120 (the
    id names the test and its first line)."""
    p, r, v, loo, q = advantage_case_inputs(case)
    check_advantage_known_answer(case, *baseline_and_std_per_prompt(p, r, v, loo, std_rewards=q))


def test_known_answer_checker_catches_a_dropped_leave_one_out():
    """A plausible oracle mistake (the leave-one-out count not subtracted) fails the table."""
    case = ADVANTAGE_KNOWN_ANSWERS[0]
    p, r, v, _, _ = advantage_case_inputs(case)
    b, s, t = baseline_and_std_per_prompt(p, r, v, False)  # full-group mean instead of leave-one-out
    with pytest.raises(AssertionError):
        check_advantage_known_answer(case, b, s, t)
