"""Pinning the token-level post-processing oracle (CPU only).

Known answers derived by hand from the reference definitions
(nemo_rl/algorithms/utils.py:273-291, :309-326), and agreement with the
reference's own tensor expressions evaluated here on small inputs.
"""

import math

import torch

from oracle.token_metrics import mask_outside_tokens, seq_logprob_errors


def test_mask_known_answers():
    lp = torch.tensor([[-1.0, -float("inf"), -2.0], [-float("inf"), -0.5, float("nan")]])
    mask = torch.tensor([[1.0, 1.0, 0.0], [0.0, 1.0, 0.0]])
    out = mask_outside_tokens(lp, mask)
    assert out[0, 0] == -1.0 and out[0, 1] == -float("inf") and out[0, 2] == 0.0
    assert out[1, 0] == 0.0 and out[1, 1] == -0.5 and out[1, 2] == 0.0  # masked NaN -> 0
    # the reference expression on the same inputs
    assert torch.equal(out, torch.where(mask.bool(), lp, 0.0))
    # bool and broadcast masks
    assert torch.equal(mask_outside_tokens(lp, mask.bool()), out)
    row = torch.tensor([1.0, 0.0, 1.0])
    torch.testing.assert_close(mask_outside_tokens(lp, row), torch.where(row.bool(), lp, 0.0),
                               rtol=0, atol=0, equal_nan=True)  # the kept NaN stays NaN


def test_seq_errors_known_answers():
    pol = torch.tensor([[-1.0, -2.0, -3.0], [-1.0, -1.0, -1.0], [-1.0, float("nan"), -1.0],
                        [0.0, 0.0, 0.0]])
    gen = torch.tensor([[-1.5, -2.0, -1.0], [-1.0, -1.0, -1.0], [-1.0, -1.0, -1.0],
                        [0.0, 0.0, 0.0]])
    tm = torch.tensor([[1.0, 1.0, 0.0], [1.0, 1.0, 1.0], [1.0, 0.0, 1.0], [1.0, 1.0, 1.0]])
    sm = torch.tensor([1.0, 1.0, 1.0, 0.0])
    err, valid = seq_logprob_errors(pol, gen, tm, sm)
    # row 0: tokens 0, 1: (exp(0.5) + exp(0)) / 2; token 2 masked out (its error 2 ignored)
    assert math.isclose(float(err[0]), (math.exp(0.5) + 1.0) / 2, rel_tol=1e-6)
    assert float(err[1]) == 1.0  # identical logprobs: exp(0) on every token
    assert float(err[2]) == 1.0  # the NaN sits on a masked token
    assert float(err[3]) == 0.0 and not bool(valid[3])  # no valid token: 0 / max(0, 1)
    assert valid[:3].all()
    # a NaN on a valid token makes the sequence's error NaN
    pol2 = pol.clone()
    pol2[0, 0] = float("nan")
    e2, _ = seq_logprob_errors(pol2, gen, tm, sm)
    assert math.isnan(float(e2[0]))
    # the reference expression (fp32 torch ops) on the same inputs
    mask = tm * sm.unsqueeze(-1)
    counts = mask.sum(dim=-1)
    error = torch.where(mask.bool(), (gen - pol).abs(), 0.0)
    ref = (torch.exp(error * mask) * mask).sum(dim=-1) / counts.clamp(min=1)
    torch.testing.assert_close(err, ref, rtol=1e-6, atol=0)
    assert torch.equal(valid, counts > 0)


def test_seq_errors_fractional_mask():
    """A non-binary mask weights both the exponent and the term (w * exp(e * w))."""
    pol = torch.tensor([[-1.0, -1.0]])
    gen = torch.tensor([[-2.0, -1.0]])
    tm = torch.tensor([[0.5, 1.0]])
    sm = torch.tensor([1.0])
    err, _ = seq_logprob_errors(pol, gen, tm, sm)
    assert math.isclose(float(err[0]), (0.5 * math.exp(0.5) + 1.0) / 1.5, rel_tol=1e-6)
