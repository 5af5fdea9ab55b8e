"""The oracle for logprobs at K ids and for the student/teacher divergences, pinned (CPU).

Pins: log_softmax + gather in float64 (the baseline of the reference tests,
tests/unit/distributed/test_model_utils.py:422-446, 872-940); the gradient from
autograd of that float64 closed form; closed forms of the divergences (uniform
entropy -log V, KL(p||p) = 0, CE = H(p) + KL, KL >= 0, a two-token case by hand)
and their float64 autograd gradients; chunk invariance.
"""

import math

import pytest
import torch

from oracle.vocab_reduce import (
    divergence,
    divergence_f64,
    divergence_grad,
    gather_logprobs,
    gather_logprobs_grad,
)


def _ids(g, B, S, K, V, lo=0, hi=None):
    return torch.randint(lo, V if hi is None else hi, (B, S, K), generator=g)


def test_gather_matches_float64_log_softmax():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 7, 50, generator=g) * 3
    idx = _ids(g, 2, 7, 5, 50)
    got = gather_logprobs(x, idx, 0, 50)
    ref = torch.log_softmax(x.double(), -1).gather(-1, idx)
    torch.testing.assert_close(got.double(), ref, rtol=0, atol=2e-6)


def test_gather_out_of_range_ids_are_zero_and_chunking_is_invisible():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 9, 40, generator=g)
    idx = _ids(g, 2, 9, 4, 60, lo=-10)  # some ids < 0 and >= 40
    got = gather_logprobs(x, idx, 0, 40)
    oob = (idx < 0) | (idx >= 40)
    assert oob.any() and torch.all(got[oob] == 0)
    assert torch.equal(got, gather_logprobs(x, idx, 0, 40, chunk_size=2))
    # a vocabulary slice: ids are global, the logits are columns [10, 50)
    got2 = gather_logprobs(x, idx + 10, 10, 50)
    assert torch.equal(got2, got)


def test_gather_grad_matches_float64_autograd_with_duplicate_ids():
    g = torch.Generator().manual_seed(2)
    V = 30
    x = torch.randn(2, 5, V, generator=g)
    idx = _ids(g, 2, 5, 6, V)
    idx[0, 0] = torch.tensor([3, 3, 3, 7, 7, 1])  # repeated ids accumulate
    idx[1, 2, 0] = -4  # out of range: contributes nothing
    go = torch.randn(2, 5, 6, generator=g)
    got = gather_logprobs_grad(x, idx, 0, V, go, out_dtype=torch.float64)
    xd = x.double().requires_grad_(True)
    inr = (idx >= 0) & (idx < V)
    vals = torch.log_softmax(xd, -1).gather(-1, idx.clamp(0, V - 1)) * inr
    (vals * go.double()).sum().backward()
    # The reference's softmax term uses the sum of every g_k, in range or not
    # (an id outside this vocabulary slice belongs to another rank, whose
    # logprob still depends on these logits): -p * sum_k g_k plus g_k at the
    # in-range ids.  Autograd of the masked forward leaves out the out-of-range
    # g_k, so they are added back here.
    p = torch.softmax(x.double(), -1)
    expect = xd.grad - p * (go.double() * (~inr)).sum(-1, keepdim=True)
    assert (~inr).any()
    torch.testing.assert_close(got, expect, rtol=0, atol=2e-6)
    # softmax identity: each row's gradient sums to sum_k g_k (in range) - sum_k g_k
    expect_rowsum = (go * inr).sum(-1) - go.sum(-1)
    torch.testing.assert_close(got.sum(-1).float(), expect_rowsum, rtol=0, atol=1e-5)


@pytest.mark.parametrize("kind", ["entropy", "cross_entropy", "reverse_kl"])
def test_divergence_matches_float64_closed_form(kind):
    g = torch.Generator().manual_seed(3)
    s = torch.randn(2, 6, 77, generator=g) * 2
    t = None if kind == "entropy" else torch.randn(2, 6, 77, generator=g) * 2 + 5
    got = divergence(kind, s, t)
    torch.testing.assert_close(got.double(), divergence_f64(kind, s, t), rtol=0, atol=5e-6)
    assert torch.equal(got, divergence(kind, s, t, chunk_size=4))


def test_divergence_closed_forms():
    V = 64
    uniform = torch.zeros(1, 1, V)
    assert divergence("entropy", uniform, None).item() == pytest.approx(-math.log(V), abs=1e-6)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 3, V, generator=g)
    y = torch.randn(1, 3, V, generator=g)
    # KL(p || p) = 0; KL >= 0; CE = KL - (sum p log p)
    assert divergence("reverse_kl", x, x.clone()).abs().max().item() < 1e-6
    kl = divergence("reverse_kl", x, y)
    assert (kl > 0).all()
    ce = divergence("cross_entropy", x, y)
    ent = divergence("entropy", x, None)
    torch.testing.assert_close(ce, kl - ent, rtol=0, atol=1e-5)
    # two tokens by hand: p = (a, 1-a), q = (b, 1-b)
    a, b = 0.3, 0.8
    s = torch.tensor([[[math.log(a), math.log(1 - a)]]])
    t = torch.tensor([[[math.log(b), math.log(1 - b)]]])
    assert divergence("cross_entropy", s, t).item() == pytest.approx(
        -(a * math.log(b) + (1 - a) * math.log(1 - b)), abs=1e-6)
    assert divergence("entropy", s, None).item() == pytest.approx(
        a * math.log(a) + (1 - a) * math.log(1 - a), abs=1e-6)


@pytest.mark.parametrize("kind", ["entropy", "cross_entropy", "reverse_kl"])
def test_divergence_grad_matches_float64_autograd(kind):
    g = torch.Generator().manual_seed(5)
    s = torch.randn(2, 4, 33, generator=g)
    t = None if kind == "entropy" else torch.randn(2, 4, 33, generator=g)
    go = torch.randn(2, 4, generator=g)
    got = divergence_grad(kind, s, t, go)
    sd = s.double().requires_grad_(True)
    (divergence_f64(kind, sd, t) * go.double()).sum().backward()
    torch.testing.assert_close(got.double(), sd.grad, rtol=0, atol=2e-6)
    # the gradient of a softmax expectation sums to zero over the vocabulary
    assert got.sum(-1).abs().max().item() < 1e-5


def test_divergence_grad_dtype_is_the_logits_dtype():
    g = torch.Generator().manual_seed(6)
    s = torch.randn(1, 2, 16, generator=g).bfloat16()
    t = torch.randn(1, 2, 16, generator=g).bfloat16()
    out = divergence_grad("reverse_kl", s, t, torch.ones(1, 2))
    assert out.dtype == torch.bfloat16


def test_vocab_topk_values_are_torch_topk_and_ids_point_at_them():
    """The reference test's checks (test_model_utils.py:1701-1730): values equal the fp32
    torch.topk values exactly and regathering at the ids returns them."""
    from oracle.vocab_reduce import vocab_topk

    torch.manual_seed(1337)
    x = torch.randn(2, 16, 256, dtype=torch.bfloat16)
    vals, idx = vocab_topk(x, 5)
    exp_vals, _ = torch.topk(x.float(), 5, dim=-1)
    assert torch.equal(vals, exp_vals)
    assert torch.equal(torch.gather(x.float(), -1, idx), vals)


def test_vocab_topk_brute_force_with_ties_nan_and_signed_zero():
    """Rank of element j = #{i : x_i > x_j or (x_i == x_j and i < j)}; the top k are ranks < k."""
    from oracle.vocab_reduce import vocab_topk

    x = torch.tensor([[[1.0, 3.0, 3.0, -0.0, 0.0, 2.0, 3.0, float("nan"), -1.0]]])
    vals, idx = vocab_topk(x, 6, vocab_start=100)
    xs = x[0, 0].tolist()
    import math

    def gt(a, b):  # a sorts above b
        if math.isnan(a):
            return not math.isnan(b)
        return (not math.isnan(b)) and a > b

    ranks = []
    for j, xj in enumerate(xs):
        r = sum(1 for i, xi in enumerate(xs) if gt(xi, xj) or (not gt(xj, xi) and not gt(xi, xj) and i < j))
        ranks.append(r)
    order = sorted(range(len(xs)), key=lambda j: ranks[j])[:6]
    assert idx[0, 0].tolist() == [100 + j for j in order]
    got = vals[0, 0].tolist()
    assert math.isnan(got[0]) and got[1:] == [xs[j] for j in order[1:]]
