"""Pinning the CPU top-k / top-p oracle (CPU only).

Checks against definitions evaluated independently: brute force over every
candidate set on tiny vocabularies (the top-k set is the k largest with ties;
the nucleus is the shortest descending-order prefix whose mass reaches top_p,
resolved in stable order), plus the reference tests' invariants
(tests/unit/distributed/test_model_utils.py:1402-1490).

For 16-bit tensors the reference's own op sequence decides top-p in the
tensor's dtype (logits_sampling_utils.py:189-191 on an un-upcast tensor): the
softmax output is rounded to the dtype, torch's CPU cumsum accumulates it in
fp32 and rounds every partial sum to the dtype, and the Python float 1 - top_p
is compared in the dtype.  That rule is written out below with numpy scalars
(fp32 exponentials and sums, explicit round-to-nearest-even to bf16/fp16) and
checked against the oracle on tiny rows, where the CPU softmax sums its few
terms one by one; two hand-derived rows pin the cases where the 16-bit rule and
the fp32 rule keep different sets.
"""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle.sampling import (
    apply_temperature,
    filtered_logprobs,
    filtered_logprobs_grad,
    next_token_filtered,
    temperature_recip,
    top_k_top_p,
)


def _definition_keep(x: list[float], k, p) -> set[int]:
    """Keep set from the definitions, in float64, ties broken by (value, index) ascending order."""
    order = sorted(range(len(x)), key=lambda i: (x[i], i))  # stable ascending
    kept = list(order)
    if k is not None and k > 0:
        thr = sorted(x, reverse=True)[k - 1]
        kept = [i for i in order if x[i] >= thr]
    if p is None or p == 1.0:
        return set(kept)
    m = max(x[i] for i in kept)
    e = {i: math.exp(x[i] - m) for i in kept}
    z = sum(e.values())
    cum = 0.0
    out = set()
    for pos, i in enumerate(kept):
        cum += e[i] / z
        if cum > 1 - p or pos == len(kept) - 1:
            out.update(kept[pos:])
            break
    return out


@pytest.mark.parametrize("k,p", [(1, 1.0), (2, 1.0), (3, 0.9), (None, 0.5), (None, 0.95), (4, 0.3), (5, 0.999)])
def test_matches_definition_on_tiny_rows(k, p):
    g = torch.Generator().manual_seed(0)
    for trial in range(200):
        V = 6
        x = (torch.randint(-3, 4, (V,), generator=g).float() * 0.5)  # many ties
        _, keep = top_k_top_p(x.unsqueeze(0), k, p)
        got = set(torch.nonzero(keep[0]).flatten().tolist()) if keep is not None else set(range(V))
        assert got == _definition_keep(x.tolist(), k, p), (x.tolist(), k, p)


def test_reference_invariants():
    torch.manual_seed(42)
    logits = torch.randn(2, 4, 100)
    for k, p in [(5, 1.0), (None, 0.9), (10, 0.8)]:
        filt, keep = top_k_top_p(logits, k, p)
        assert torch.equal(keep, ~torch.isinf(filt))
        probs = torch.softmax(filt, -1)
        assert torch.allclose(probs.sum(-1), torch.ones(2, 4), atol=1e-5)
        if k is not None:
            assert (keep.sum(-1) <= k).all()
            for b, s in itertools.product(range(2), range(4)):
                top = torch.topk(logits[b, s], k).indices
                assert keep[b, s][torch.tensor([i for i in range(100) if i not in top.tolist()])].sum() == 0


def test_filtered_logprob_and_grad_definitions():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 3, 40, generator=g)
    t = torch.randint(0, 40, (2, 3), generator=g)
    lp, keep = filtered_logprobs(x, t, 5, 0.8)
    kept_t = keep.gather(-1, t.unsqueeze(-1)).squeeze(-1)
    assert torch.isinf(lp[~kept_t]).all() and (lp[~kept_t] < 0).all()
    ref = torch.log_softmax(x.double().masked_fill(~keep, -float("inf")), -1).gather(-1, t.unsqueeze(-1)).squeeze(-1)
    torch.testing.assert_close(lp[kept_t].double(), ref[kept_t], rtol=0, atol=1e-6)
    gout = torch.randn(2, 3, generator=g)
    gr = filtered_logprobs_grad(x, t, 5, 0.8, gout)
    assert (gr[~keep] == 0).all()
    # inside the kept set the gradient is the renormalised softmax gradient
    p = torch.softmax(x.double().masked_fill(~keep, -float("inf")), -1)
    oh = torch.nn.functional.one_hot(t, 40).double()
    torch.testing.assert_close(gr.double(), (oh - p) * gout.unsqueeze(-1).double() * keep, rtol=0, atol=1e-6)


def _times_recip16(values, T: float, dtype) -> torch.Tensor:
    """dtype(fl32(v * fl32(1.0 / T))) element by element with numpy scalars."""
    r = np.float32(1.0 / T)
    out = [_round16(float(np.float32(np.float32(v) * r)), dtype) for v in values.reshape(-1).tolist()]
    return torch.tensor(out, dtype=torch.float32).view(values.shape)


def test_temperature_reciprocal_known_answers():
    """The in-place temperature's reciprocal is 1.0 / T formed in double and rounded once.

    At T = 1.1 that is 0x3F68BA2F, where the reciprocal of the fp32 temperature,
    1.0f / fl32(1.1), is one ulp lower: a reciprocal formed in fp32 fails here.  At
    T = 0.7 the product and the exact quotient round differently for x = 5 in fp32."""
    assert int(temperature_recip(1.1).view(torch.int32)) == 0x3F68BA2F
    wrong = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(1.1, dtype=torch.float32)
    assert int(wrong.view(torch.int32)) == 0x3F68BA2E
    x = torch.tensor([5.0], dtype=torch.float32)
    prod = apply_temperature(x, 0.7)
    assert prod.item() == float(np.float32(np.float32(5.0) * np.float32(1.0 / 0.7)))
    assert prod.item() != (x / 0.7).item()  # CPU torch's exact quotient differs by one ulp


def test_temperature_chain_bf16():
    """div_ in bf16 then the bf16 gradient chain of the reference's production path,
    against the same chain written out with numpy scalars."""
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(1, 5, 64, generator=g) * 2).to(torch.bfloat16)
    ids = torch.randint(0, 64, (1, 5), generator=g)
    gout = torch.randn(1, 4, generator=g)
    lp, keep, grad = next_token_filtered(x, ids, 8, 0.9, temperature=0.7, grad_output=gout)
    y = _times_recip16(x.float(), 0.7, torch.bfloat16)
    lp2, keep2 = filtered_logprobs(y[:, :-1], ids[:, 1:], 8, 0.9)
    assert torch.equal(keep, keep2)
    torch.testing.assert_close(lp, lp2, rtol=0, atol=0)
    assert grad.dtype == torch.bfloat16
    g32 = filtered_logprobs_grad(y[:, :-1], ids[:, 1:], 8, 0.9, gout)
    exp = _times_recip16(g32.to(torch.bfloat16).float(), 0.7, torch.bfloat16)
    torch.testing.assert_close(grad[:, :-1].float(), exp, rtol=0, atol=0)
    assert grad[:, -1].abs().max() == 0


def _round16(v: float, dtype) -> float:
    """fp32 value rounded to bf16 / fp16 (nearest even), as a Python float."""
    f = np.float32(v)
    if dtype is torch.float16:
        return float(np.float16(f))
    u = int(np.array([f], dtype=np.float32).view(np.uint32)[0])
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return float(np.array([u], dtype=np.uint32).view(np.float32)[0])


def _definition_keep16(x: list[float], k, p, dtype) -> set[int]:
    """16-bit keep set: exp and their sum in fp32 (one term at a time), probabilities
    rounded to the dtype, cumulative sum in fp32 rounded to the dtype at every step,
    compared with dtype(fp32(1 - top_p)); ties in stable ascending order."""
    order = sorted(range(len(x)), key=lambda i: (x[i], i))
    kept = list(order)
    if k is not None and k > 0:
        thr = sorted(x, reverse=True)[k - 1]
        kept = [i for i in order if x[i] >= thr]
    if p is None or p == 1.0:
        return set(kept)
    m = max(x[i] for i in kept)
    e = [np.float32(math.exp(x[i] - m)) for i in kept]
    z = np.float32(0.0)
    for v in e:
        z = np.float32(z + v)
    probs = [_round16(float(np.float32(v / z)), dtype) for v in e]
    thr16 = _round16(float(np.float32(1.0 - p)), dtype)
    cum = np.float32(0.0)
    for pos, i in enumerate(kept):
        cum = np.float32(cum + np.float32(probs[pos]))
        if _round16(float(cum), dtype) > thr16 or pos == len(kept) - 1:
            return set(kept[pos:])
    return set()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k,p", [(2, 1.0), (3, 0.9), (None, 0.5), (None, 0.95), (4, 0.3), (5, 0.999)])
def test_16bit_rule_matches_definition_on_tiny_rows(k, p, dtype):
    g = torch.Generator().manual_seed(3)
    for trial in range(200):
        V = 6
        x = (torch.randint(-3, 4, (V,), generator=g).float() * 0.5).to(dtype)
        _, keep = top_k_top_p(x.unsqueeze(0), k, p)
        got = set(torch.nonzero(keep[0]).flatten().tolist())
        assert got == _definition_keep16(x.float().tolist(), k, p, dtype), (x.tolist(), k, p)


@pytest.mark.parametrize(
    "dtype,row",
    [
        # bf16: p0 = p1 = 0.050107 (fp32) round to 0.050048828125; their bf16 cumsum
        # is 0.10009765625 = bf16(1 - 0.9), not above it, while the fp32 cumsum
        # 0.100214 exceeds fp32(1 - 0.9) = 0.099999994
        (torch.bfloat16, [-0.013, -0.013, 2.875]),
        # fp16: p0 = p1 = 0.0500014 round to 0.04998779296875; the fp16 cumsum is
        # 0.0999755859375 = fp16(1 - 0.9), not above it; the fp32 cumsum 0.1000029 is
        (torch.float16, [0.000285, 0.000285, 2.890625]),
    ],
)
def test_16bit_rule_known_answers(dtype, row):
    x = torch.tensor([row], dtype=dtype)
    _, keep16 = top_k_top_p(x, None, 0.9)
    _, keep32 = top_k_top_p(x.float(), None, 0.9)
    assert keep16.tolist() == [[False, False, True]]
    assert keep32.tolist() == [[False, True, True]]
    assert _definition_keep16(x.float()[0].tolist(), None, 0.9, dtype) == {2}
    assert _definition_keep(x.float()[0].tolist(), None, 0.9) == {1, 2}


@pytest.mark.parametrize("k,p", [(50, 0.9), (5, 0.5), (20, 0.99), (3, 0.2)])
def test_candidate_restriction_matches_full_sort(k, p):
    """The top-k-candidate evaluation equals the full-row oracle (exact normaliser) on
    random rows, tie-heavy rows and rows with a peaked head."""
    from oracle.sampling import top_k_top_p_candidates

    g = torch.Generator().manual_seed(k)
    V = 3000
    x = torch.randn(24, V, generator=g) * 2
    x[0] = (torch.randint(-4, 4, (V,), generator=g).float()) * 0.5   # heavy ties everywhere
    x[1, ::3] = 5.0                                                   # ties at the top
    x[2, 17] = 30.0                                                   # one-hot row
    x[3] = (torch.randn(V, generator=g) * 2).bfloat16().float()       # bf16 values
    x[4, :100] = 7.0                                                  # a tied block above the rest
    _, want = top_k_top_p(x, k, p, exact_normaliser=True)
    got, st = top_k_top_p_candidates(x, k, p)
    assert torch.equal(got, want)
    assert torch.equal(st["n_kept"], want.sum(-1))
    # every kept value is >= the smallest kept one, and the group counts are consistent
    assert (st["kept_in_group"] >= 1).all() and (st["kept_in_group"] <= st["group"]).all()
