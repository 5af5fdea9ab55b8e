"""ClippedPG known answers end to end (GPU): logits built so that their log-softmax gives
chosen token logprobs, through ``prepare_loss_input`` and ``ClippedPGLossFn`` on the device.

Cases and numbers follow the reference's hand-computed tests
(tests/unit/algorithms/test_loss_functions.py): PPO clipping (:457-531, loss -0.6333),
REINFORCE (:533-586, 0.8333) and the k3 KL penalty with and without top-k filtering
(:1098-1175, 0.0362; the KL term uses the unfiltered logprobs, so top-k = 1 changes nothing).
Batch of one sequence of 4 tokens over a vocabulary of 8; masks are int64 as there.
"""

import math

import pytest
import torch

from rl_amd.algorithms.logits_sampling_utils import TrainingSamplingParams
from rl_amd.algorithms.loss import ClippedPGLossConfig, ClippedPGLossFn, prepare_loss_input

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
B, S, V = 1, 4, 8


def _data(seed):
    g = torch.Generator().manual_seed(seed)
    token_mask = torch.ones(B, S, dtype=torch.int64)
    token_mask[:, 0] = 0
    d = {
        "input_ids": torch.randint(0, V, (B, S), generator=g),
        "token_mask": token_mask,
        "sample_mask": torch.ones(B, dtype=torch.int64),
        "advantages": torch.zeros(B, S),
        "prev_logprobs": torch.zeros(B, S),
        "reference_policy_logprobs": torch.zeros(B, S),
        "generation_logprobs": torch.zeros(B, S),
    }
    return d


def _exact_logits(target_lp, input_ids):
    """[B, S, V] logits whose log-softmax at position i is target_lp[:, i] for token
    input_ids[:, i + 1]: the target logit is 0 and one other token carries
    log(exp(-lp) - 1) (a logprob of 0 puts the target at +100); the rest sit at -100."""
    x = torch.full((B, S, V), -100.0, dtype=torch.float64)
    for b in range(B):
        for i in range(target_lp.shape[1]):
            t = int(input_ids[b, i + 1])
            lp = float(target_lp[b, i])
            if lp == 0.0:
                x[b, i, t] = 100.0
            else:
                x[b, i, t] = 0.0
                x[b, i, (t + 1) % V] = math.log(math.expm1(-lp))
    return x.float()


def _run(d, curr_lp, cfg, sampling_params=None):
    logits = _exact_logits(curr_lp, d["input_ids"]).to(DEV).requires_grad_(True)
    data = {k: v.to(DEV) for k, v in d.items()}
    fn = ClippedPGLossFn(cfg)
    li, data = prepare_loss_input(logits, data, fn, sampling_params=sampling_params)
    gvs = data["sample_mask"].sum()
    gvt = (data["sample_mask"].unsqueeze(-1) * data["token_mask"]).sum()
    loss, metrics = fn(data=data, global_valid_seqs=gvs, global_valid_toks=gvt, **li)
    (grad,) = torch.autograd.grad(loss, [logits])
    assert torch.isfinite(grad).all()
    return loss.item(), data, li


def test_ppo_clipping_known_answer():
    print("[case] e2e ppo clipping", flush=True)
    d = _data(0)
    d["advantages"][0, 1:] = torch.tensor([1.0, -1.0, 2.0])
    d["prev_logprobs"][0, 1:] = -1.0
    curr = torch.tensor([[-1.69315, -1.0, -0.59453]])  # ratios 0.5, 1.0, 1.5
    loss, _, li = _run(d, curr, ClippedPGLossConfig(reference_policy_kl_penalty=0.0))
    torch.testing.assert_close(li["next_token_logprobs"].cpu(), curr, rtol=0, atol=2e-6)
    # max(-A r, -A clamp(r, 0.8, 1.2)) = -0.5, 1.0, -2.4 per token
    r = torch.exp(curr.double() + 1.0)[0]
    exact = (-r[0] + r[1] - 2.4) / 3  # tokens 0 and 1 keep -A r, token 2 is clipped
    assert loss == pytest.approx(-0.6333, rel=1e-3)
    assert loss == pytest.approx(float(exact), rel=1e-5)


def test_reinforce_known_answer():
    print("[case] e2e reinforce", flush=True)
    d = _data(1)
    d["advantages"][0, 1:] = torch.tensor([1.0, -1.0, 2.0])
    curr = torch.tensor([[-0.5, -1.0, -1.5]])
    cfg = ClippedPGLossConfig(reference_policy_kl_penalty=0.0, disable_ppo_ratio=True,
                              ratio_clip_min=0.0, ratio_clip_max=0.0)
    loss, _, _ = _run(d, curr, cfg)
    assert loss == pytest.approx(0.8333, rel=1e-3)
    assert loss == pytest.approx(2.5 / 3, rel=1e-5)  # mean of -A * logprob = (0.5, -1.0, 3.0)


@pytest.mark.parametrize("top_k", [None, 1])
def test_kl_penalty_known_answer(top_k):
    print("[case] e2e kl penalty top_k", top_k, flush=True)
    d = _data(2)
    d["reference_policy_logprobs"][0, 1:] = -1.0
    curr = torch.tensor([[0.0, -1.0, -2.0]])
    loss, data, li = _run(d, curr, ClippedPGLossConfig(reference_policy_kl_penalty=0.1),
                          TrainingSamplingParams(top_k=top_k))
    assert torch.equal(data["token_mask"].cpu(), torch.tensor([[0, 1, 1, 1]]))
    if top_k == 1:
        # the target is the argmax only where its logprob is above log(0.5)
        lp = li["next_token_logprobs"].cpu()
        assert lp[0, 0].item() == 0.0 and torch.isinf(lp[0, 1:]).all()
    # k3 per token at logr = ref - curr = (-1, 0, 1): e^-1, 0, e - 2
    exact = 0.1 * (math.exp(-1.0) + 0.0 + (math.e - 2.0)) / 3
    assert loss == pytest.approx(0.0362, rel=1e-3)
    assert loss == pytest.approx(exact, rel=1e-5)
