"""Pinning the CPU logprob oracle (CPU only).

The oracle follows the reference op sequence in fp32; these tests pin it to
quantities the mathematics fixes: float64 log_softmax + gather (the baseline
the reference tests use), brute-force softmax on tiny vocabularies, the
softmax-gradient identity, chunk invariance, and masked targets.
"""

import math

import pytest
import torch

from oracle.logprob import (
    closed_form_logprobs_f64,
    next_token_logprobs,
    next_token_logprobs_grad,
    pack_input_ids,
    pack_targets,
    selected_logprobs,
    selected_logprobs_grad,
    unpack_logprobs,
)


def test_matches_float64_closed_form():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 7, 300, generator=g) * 2
    t = torch.randint(0, 300, (2, 7), generator=g)
    got = selected_logprobs(x, t, 0, 300)
    exp = closed_form_logprobs_f64(x, t)
    torch.testing.assert_close(got.double(), exp, rtol=0, atol=2e-6)


def test_brute_force_tiny_vocab():
    x = torch.tensor([[[0.5, -1.0, 2.0]]])
    for t in range(3):
        got = selected_logprobs(x, torch.tensor([[t]]), 0, 3).item()
        z = sum(math.exp(v) for v in [0.5, -1.0, 2.0])
        assert got == pytest.approx(x[0, 0, t].item() - math.log(z), abs=1e-6)


def test_out_of_range_targets_are_zero():
    x = torch.randn(1, 4, 10)
    t = torch.tensor([[3, -1, 10, 12]])
    got = selected_logprobs(x, t, 0, 10)
    assert got[0, 1] == 0 and got[0, 2] == 0 and got[0, 3] == 0
    assert got[0, 0] < 0
    # vocab shard [5, 10): target 3 is outside the shard
    got2 = selected_logprobs(x, torch.tensor([[3, 7, 5, 9]]), 5, 10)
    assert got2[0, 0] == 0


@pytest.mark.parametrize("chunk", [1, 3, 7, 37])
def test_chunk_invariance(chunk):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 11, 64, generator=g)
    t = torch.randint(0, 64, (2, 11), generator=g)
    base = selected_logprobs(x, t, 0, 64)
    torch.testing.assert_close(selected_logprobs(x, t, 0, 64, chunk), base, rtol=0, atol=0)
    gout = torch.randn(2, 11, generator=g)
    gb = selected_logprobs_grad(x, t, 0, 64, gout)
    torch.testing.assert_close(selected_logprobs_grad(x, t, 0, 64, gout, chunk), gb, rtol=0, atol=0)


def test_grad_matches_autograd_and_sums_to_zero():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 5, 50, generator=g, dtype=torch.float64)
    t = torch.randint(0, 50, (2, 5), generator=g)
    gout = torch.randn(2, 5, generator=g, dtype=torch.float64)
    xr = x.clone().requires_grad_(True)
    lp = torch.log_softmax(xr, -1).gather(-1, t.unsqueeze(-1)).squeeze(-1)
    (ref,) = torch.autograd.grad((lp * gout).sum(), xr)
    got = selected_logprobs_grad(x.float(), t, 0, 50, gout.float())
    torch.testing.assert_close(got.double(), ref, rtol=0, atol=1e-6)
    # sum_v (onehot - p) = 0 for in-range targets
    assert got.double().sum(-1).abs().max() < 1e-5


def test_next_token_shift_and_last_row():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 6, 20, generator=g)
    ids = torch.randint(0, 20, (2, 6), generator=g)
    lp = next_token_logprobs(x, ids)
    assert lp.shape == (2, 5)
    exp = closed_form_logprobs_f64(x[:, :-1], ids[:, 1:])
    torch.testing.assert_close(lp.double(), exp, rtol=0, atol=2e-6)
    gout = torch.randn(2, 5, generator=g)
    gr = next_token_logprobs_grad(x, ids, gout)
    assert gr[:, -1].abs().max() == 0


def test_packed_roll_and_unpack_match_per_sequence_reference():
    ids = torch.arange(10).unsqueeze(0)
    cu = [0, 3, 3, 7, 10]
    rolled = pack_targets(ids, cu)
    assert rolled.tolist() == [[1, 2, 0, 4, 5, 6, 3, 8, 9, 7]]
    probs = torch.arange(10, dtype=torch.float32)
    out = unpack_logprobs(probs, cu, 5)
    assert out.tolist() == [[0, 1, 0, 0], [0, 0, 0, 0], [3, 4, 5, 0], [7, 8, 0, 0]]


def test_pack_input_ids_known_answers():
    """Hand-computed packings: padded segments, per-segment roll, trailing dims."""
    ids = torch.tensor([[1, 2, 3, 0], [4, 5, 0, 0]])
    assert pack_input_ids(ids, [0, 3, 5], [0, 4, 8]).tolist() == [[1, 2, 3, 0, 4, 5, 0, 0]]
    # roll -1: each padded segment shifts left and wraps to its own first token
    assert pack_input_ids(ids, [0, 3, 5], [0, 4, 8], roll_shift=-1).tolist() == [[2, 3, 0, 1, 5, 0, 0, 4]]
    # actual length beyond the row width copies only the S real tokens
    assert pack_input_ids(ids, [0, 3, 9], [0, 4, 10]).tolist() == [[1, 2, 3, 0, 4, 5, 0, 0, 0, 0]]
    # trailing dimensions are carried along (reference test_model_utils.py:2233-2250 layout)
    ids3 = torch.arange(2 * 3 * 2).view(2, 3, 2)
    got = pack_input_ids(ids3, [0, 2, 5], [0, 2, 6], roll_shift=-1)
    assert got.tolist() == [[[2, 3], [0, 1], [8, 9], [10, 11], [0, 0], [6, 7]]]
    # the roll of an unpadded packing is pack_targets of the plain packing
    x = torch.randint(0, 50, (3, 6))
    cu = [0, 6, 8, 12]
    ids_full = torch.zeros(3, 6, dtype=torch.long)
    for i, n in enumerate([6, 2, 4]):
        ids_full[i, :n] = x[i, :n]
    plain = pack_input_ids(ids_full, cu, cu)
    assert torch.equal(pack_input_ids(ids_full, cu, cu, roll_shift=-1), pack_targets(plain, cu))
