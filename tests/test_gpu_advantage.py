"""gfx950 GRPO advantage kernel: reference known answers and the CPU oracle (GPU)."""

import pytest
import torch

from oracle.advantage import baseline_and_std_per_prompt, grpo_advantages
from rl_amd.algorithms.advantage_estimator import AdvEstimatorConfig, GRPOAdvantageEstimator
from rl_amd.algorithms.utils import calculate_baseline_and_std_per_prompt
from tests.helpers import ADVANTAGE_KNOWN_ANSWERS, advantage_case_inputs, check_advantage_known_answer

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
P6 = torch.tensor([[1, 2, 3]] * 3 + [[4, 5, 6]] * 3)


def test_known_answers():
    b, s, _ = calculate_baseline_and_std_per_prompt(P6.to(DEV), torch.tensor([1.0, 2, 3, 4, 5, 6], device=DEV),
                                                    torch.ones(6, device=DEV))
    assert b.device.type == "cuda"
    assert torch.allclose(b.cpu(), torch.tensor([2.5, 2.0, 1.5, 5.5, 5.0, 4.5]), rtol=1e-5)
    assert torch.allclose(s.cpu(), torch.tensor([0.707107, 1.414214, 0.707107] * 2), rtol=1e-5)
    r = torch.tensor([1.0, 999.0, 3.0, 4.0, 5.0, 6.0])
    b, s, _ = calculate_baseline_and_std_per_prompt(P6, r, torch.tensor([1.0, 0, 1, 1, 1, 1]))
    assert b.device.type == "cpu"  # CPU inputs come back on the CPU
    assert torch.allclose(b, torch.tensor([3.0, 4.0, 1.0, 5.5, 5.0, 4.5]), rtol=1e-5)
    assert torch.allclose(s, torch.tensor([0.0, 0.0, 0.0, 0.707107, 1.414214, 0.707107]), rtol=1e-5)


@pytest.mark.parametrize("case", ADVANTAGE_KNOWN_ANSWERS, ids=[c[0] for c in ADVANTAGE_KNOWN_ANSWERS])
def test_reference_known_answers(case):
    """Every known answer of reference tests/unit/algorithms/test_utils.py:830-1120, on the
    device, and the oracle on the same inputs (trivial flags equal, values to fp32 rounding)."""
    p, r, v, loo, q = advantage_case_inputs(case, DEV)
    b, s, t = calculate_baseline_and_std_per_prompt(p, r, v, loo, q)
    assert b.device.type == "cuda"
    check_advantage_known_answer(case, b, s, t)
    ob, os_, ot = baseline_and_std_per_prompt(p.cpu(), r.cpu(), v.cpu(), loo, std_rewards=None if q is None else q.cpu())
    assert torch.equal(t.cpu(), ot)
    torch.testing.assert_close(b.cpu(), ob, rtol=1e-6, atol=0)
    torch.testing.assert_close(s.cpu(), os_, rtol=1e-5, atol=1e-6)


def test_trivial_flags_and_std_rewards():
    r = torch.tensor([0.0] + [0.95] * 7)
    z = torch.zeros(8, 1, dtype=torch.long)
    b, _, triv = calculate_baseline_and_std_per_prompt(z, r, torch.ones(8))
    assert b[0].item() == pytest.approx(0.95)
    assert triv.tolist() == [True] + [False] * 7
    rewards = torch.tensor([0.0, -0.2, -1.0, 1.0, 0.0, 1.0])
    std_rewards = torch.tensor([0.0, 0.0, 0.0, 1.0, 0.0, 1.0])
    prompts = torch.tensor([[0], [0], [0], [1], [1], [1]])
    _, std, triv = calculate_baseline_and_std_per_prompt(prompts, rewards, torch.ones(6), False, std_rewards)
    assert triv.tolist() == [True, True, True, False, False, False]
    assert torch.allclose(std[:3], torch.zeros(3)) and (std[3:] > 0).all()


def test_empty_batch():
    b, s, t = calculate_baseline_and_std_per_prompt(torch.empty(0, 3, dtype=torch.long), torch.tensor([]),
                                                    torch.tensor([]))
    assert b.shape == (0,) and s.shape == (0,) and t.shape == (0,)


@pytest.mark.parametrize("loo", [False, True])
@pytest.mark.parametrize("normalize", [False, True])
@pytest.mark.parametrize("num_valid", [0, 1, 2, 3])
def test_masked_reward_group_signal(loo, normalize, num_valid):
    """reference tests/unit/algorithms/test_grpo.py:500-533 ('include' policy: all valid)."""
    est = GRPOAdvantageEstimator(AdvEstimatorConfig(normalize_rewards=normalize, use_leave_one_out_baseline=loo))
    loss_mask = (torch.arange(3) < num_valid).float()
    adv = est.compute_advantage(torch.zeros(3, 2, dtype=torch.long, device=DEV),
                                torch.tensor([1.0, 1.0, 0.0], device=DEV),
                                loss_mask[:, None].expand(-1, 2).to(DEV), valid_mask=torch.ones(3, device=DEV))
    assert torch.isfinite(adv).all()
    eff = adv.cpu() * loss_mask[:, None]
    assert eff[num_valid:].count_nonzero() == 0
    if num_valid > 0:
        exp = 0.5 if loo else 1.0 / 3.0
        if normalize:
            exp /= (0.5 if loo else 1.0 / 3.0) ** 0.5 + 1e-6
        assert adv[0, 0].item() == pytest.approx(exp)


@pytest.mark.parametrize("loo", [False, True])
@pytest.mark.parametrize("B,groups", [(8, 1), (64, 8), (300, 37)])
def test_random_groups_against_oracle(loo, B, groups):
    g = torch.Generator().manual_seed(B)
    prompts = torch.randint(0, groups, (B, 1), generator=g)
    rewards = torch.bernoulli(torch.full((B,), 0.3), generator=g)
    rewards[::5] += torch.randn(len(rewards[::5]), generator=g)
    valid = (torch.rand(B, generator=g) > 0.1).float()
    mask = torch.ones(B, 16)
    exp = grpo_advantages(prompts, rewards, mask, valid, leave_one_out=loo)
    est = GRPOAdvantageEstimator(AdvEstimatorConfig(use_leave_one_out_baseline=loo))
    got = est.compute_advantage(prompts.to(DEV), rewards.to(DEV), mask.to(DEV), valid_mask=valid.to(DEV))
    assert got.shape == (B, 16)
    torch.testing.assert_close(got.cpu(), exp, rtol=1e-5, atol=1e-5)
    b0, s0, t0 = baseline_and_std_per_prompt(prompts, rewards, valid, loo)
    b1, s1, t1 = calculate_baseline_and_std_per_prompt(prompts.to(DEV), rewards.to(DEV), valid.to(DEV), loo)
    torch.testing.assert_close(b1.cpu(), b0, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(s1.cpu(), s0, rtol=1e-5, atol=1e-6)
    assert torch.equal(t1.cpu(), t0)


@pytest.mark.parametrize("loo", [False, True])
@pytest.mark.parametrize("B,groups,K", [(1024, 64, 512), (300, 37, 7), (8192, 512, 16)])
def test_prompt_token_keys_against_oracle(loo, B, groups, K):
    """Prompt-token rows as keys (the keyed path: each row hashed once, equal
    hashes confirmed by a full comparison).  Groups of rows that differ only in
    their last token must stay apart, and the result must equal the one for the
    same grouping given as single-token ids, bit for bit."""
    g = torch.Generator().manual_seed(B + K)
    base = torch.randint(0, 50000, (groups, K), generator=g)
    # pairs of groups whose keys differ in the last token only
    n_odd = base[1::2].shape[0]
    base[1::2, :-1] = base[0::2, :-1][:n_odd]
    base[1::2, -1] = (base[0::2, -1][:n_odd] + 1) % 50000
    gid = torch.randint(0, groups, (B,), generator=g)
    prompts = base[gid]
    rewards = torch.bernoulli(torch.full((B,), 0.4), generator=g)
    rewards[::7] += torch.randn(len(rewards[::7]), generator=g)
    valid = (torch.rand(B, generator=g) > 0.1).float()
    b0, s0, t0 = baseline_and_std_per_prompt(prompts, rewards, valid, loo)
    b1, s1, t1 = calculate_baseline_and_std_per_prompt(prompts.to(DEV), rewards.to(DEV), valid.to(DEV), loo)
    torch.testing.assert_close(b1.cpu(), b0, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(s1.cpu(), s0, rtol=1e-5, atol=1e-6)
    assert torch.equal(t1.cpu(), t0)
    b2, s2, t2 = calculate_baseline_and_std_per_prompt(gid[:, None].to(DEV), rewards.to(DEV), valid.to(DEV), loo)
    assert torch.equal(b1, b2) and torch.equal(s1, s2) and torch.equal(t1, t2)
