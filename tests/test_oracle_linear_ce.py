"""The hidden-state logprob oracle against closed forms and the already-pinned logits oracle (CPU)."""

import torch

from oracle.linear_ce import (
    hidden_state_logprob_grads,
    hidden_state_logprobs,
    logits_bf16,
    next_token_hidden_state_logprobs,
)
from oracle.logprob import selected_logprobs, selected_logprobs_grad


def _inputs(S=6, B=3, H=16, V=40, seed=0, integer=False):
    g = torch.Generator().manual_seed(seed)
    if integer:
        # small integers: every product sum is exactly representable in bf16
        hidden = torch.randint(-2, 3, (S, B, H), generator=g).to(torch.bfloat16)
        weight = torch.randint(-1, 2, (V, H), generator=g).to(torch.bfloat16)
    else:
        hidden = torch.randn(S, B, H, generator=g).to(torch.bfloat16)
        weight = (torch.randn(V, H, generator=g) * 0.3).to(torch.bfloat16)
    target = torch.randint(0, V, (B, S), generator=g)
    return hidden, weight, target


def test_logits_are_the_rounded_exact_products():
    hidden, weight, _ = _inputs()
    x = logits_bf16(hidden, weight)
    S, B, H = hidden.shape
    for s in range(S):
        for b in range(B):
            for v in (0, 7, 39):
                exact = sum(float(hidden[s, b, k]) * float(weight[v, k]) for k in range(H))
                assert x[b, s, v].item() == torch.tensor(exact, dtype=torch.float64).to(torch.bfloat16).float().item()


def test_forward_is_the_logits_path_on_the_rounded_logits():
    hidden, weight, target = _inputs(S=9, B=2, V=57)
    x = logits_bf16(hidden, weight)
    ours = hidden_state_logprobs(hidden, target, weight, 0, 57)
    ref = selected_logprobs(x, target, 0, 57)
    assert torch.equal(ours, ref)
    closed = torch.log_softmax(x.double(), -1).gather(-1, target.unsqueeze(-1)).squeeze(-1)
    assert torch.allclose(ours.double(), closed, atol=2e-6)


def test_chunking_does_not_change_the_forward():
    hidden, weight, target = _inputs(S=11, B=2, V=33)
    full = hidden_state_logprobs(hidden, target, weight, 0, 33)
    for cs in (1, 3, 11):
        assert torch.equal(hidden_state_logprobs(hidden, target, weight, 0, 33, chunk_size=cs), full)


def test_vocab_slice_masks_targets_to_zero():
    hidden, weight, target = _inputs(S=5, B=4, V=30)
    out = hidden_state_logprobs(hidden, target, weight, 10, 20)
    outside = (target < 10) | (target >= 20)
    assert torch.all(out[outside] == 0)
    shifted = (target - 10).clamp(0, 29)
    x = logits_bf16(hidden, weight)
    closed = torch.log_softmax(x.double(), -1).gather(-1, shifted.unsqueeze(-1)).squeeze(-1)
    assert torch.allclose(out[~outside].double(), closed[~outside], atol=2e-6)


def test_next_token_roll_and_drop():
    hidden, weight, target = _inputs(S=7, B=2, V=25)
    out = next_token_hidden_state_logprobs(hidden, weight, target, 0, 25)
    assert out.shape == (2, 6)
    x = logits_bf16(hidden, weight)
    for s in range(6):
        closed = torch.log_softmax(x[:, s].double(), -1).gather(-1, target[:, s + 1 : s + 2]).squeeze(-1)
        assert torch.allclose(out[:, s].double(), closed, atol=2e-6)


def test_gradients_match_autograd_when_rounding_is_exact():
    hidden, weight, target = _inputs(S=5, B=3, H=12, V=21, integer=True)
    g = torch.randn(3, 5, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    g[1, 2] = 0.0
    dh, dw, gi = hidden_state_logprob_grads(hidden, target, weight, 0, 21, g)
    h64 = hidden.double().requires_grad_(True)
    w64 = weight.double().requires_grad_(True)
    logits = torch.matmul(h64, w64.t()).transpose(0, 1)  # exact: no rounding needed
    lp = torch.log_softmax(logits, -1).gather(-1, target.unsqueeze(-1)).squeeze(-1)
    ah, aw = torch.autograd.grad((lp * g).sum(), [h64, w64])
    assert torch.allclose(dh, ah, atol=1e-12, rtol=1e-12)
    assert torch.allclose(dw, aw, atol=1e-12, rtol=1e-12)
    # rows of the logits gradient sum to zero (in-range targets)
    assert torch.allclose(gi.sum(-1), torch.zeros(3, 5, dtype=torch.float64), atol=1e-12)


def test_gradient_input_is_the_logits_path_gradient():
    hidden, weight, target = _inputs(S=6, B=2, V=19)
    g = torch.randn(2, 6, generator=torch.Generator().manual_seed(1))
    _, _, gi = hidden_state_logprob_grads(hidden, target, weight, 0, 19, g)
    x = logits_bf16(hidden, weight)
    ref = selected_logprobs_grad(x, target, 0, 19, g, out_dtype=torch.float64)
    assert torch.allclose(gi, ref.double(), atol=1e-6)


def test_masked_targets_give_minus_softmax_gradient():
    hidden, weight, target = _inputs(S=4, B=2, V=15)
    g = torch.ones(2, 4)
    _, _, gi = hidden_state_logprob_grads(hidden, target, weight, 5, 10, g)
    outside = (target < 5) | (target >= 10)
    assert torch.all(gi[outside] <= 0)
    assert torch.allclose(gi[outside].sum(-1), -torch.ones(int(outside.sum()), dtype=torch.float64), atol=1e-12)
