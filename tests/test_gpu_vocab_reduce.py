"""gfx950 kernels for logprobs at K ids per row and for the student/teacher
divergences, against the CPU oracle (GPU).

Tolerances: values 1e-5 abs for fp32 logits and 2e-3 abs for bf16/fp16 logits
(fp32 arithmetic on the exactly widened inputs); logits gradients 1e-3 abs,
where a bf16 element may instead sit one bf16 ulp from the oracle's.  The
reference's own checks are kept where it states them: reverse KL of identical
logits within 1e-6, bf16 logits normalised in fp32 within 1e-5, gradients within
rtol 1e-4 / atol 1e-5 of autograd (tests/unit/distributed/test_model_utils.py:1930-2130).
"""

import pytest
import torch

from oracle.vocab_reduce import (
    divergence,
    divergence_f64,
    divergence_grad,
    gather_logprobs,
    gather_logprobs_grad,
)
from rl_amd.distributed.model_utils import (
    ChunkedDistributedCrossEntropyToFixedLogits,
    ChunkedDistributedEntropy,
    ChunkedDistributedGatherLogprob,
    ChunkedDistributedReverseKLToFixedLogits,
    get_policy_logprobs_at_sampler_topk,
)
from tests.helpers import assert_close_or_ulp_bf16

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
KINDS = {
    "entropy": ChunkedDistributedEntropy,
    "cross_entropy": ChunkedDistributedCrossEntropyToFixedLogits,
    "reverse_kl": ChunkedDistributedReverseKLToFixedLogits,
}


def say(*a):
    print("[case]", *a, flush=True)


def _val_tol(dtype):
    return 1e-5 if dtype == torch.float32 else 2e-3


def _check_grad(got, ref, dtype):
    if dtype == torch.bfloat16:
        assert_close_or_ulp_bf16(got, ref, 1e-3)
    else:
        torch.testing.assert_close(got.float().cpu(), ref.float(), rtol=0, atol=1e-3)


@pytest.mark.parametrize("dtype,V", [(torch.float32, 997), (torch.bfloat16, 1000),
                                     (torch.bfloat16, 1003), (torch.float16, 512),
                                     (torch.bfloat16, 151936)])
@pytest.mark.parametrize("K", [1, 5, 20, 64, 70])
def test_gather_fwd_bwd_parity(dtype, V, K):
    say("gather", dtype, "V", V, "K", K)
    g = torch.Generator().manual_seed(V + K)
    B, S = 2, 9
    x = (torch.randn(B, S, V, generator=g) * 2).to(dtype)
    idx = torch.randint(0, V, (B, S, K), generator=g)
    if K >= 5:
        idx[0, 0, :3] = idx[0, 0, 0]          # repeated ids accumulate
        idx[0, 1, K - 1] = idx[0, 1, 0]       # ... also from the first to the last k
        idx[1, 3, 1] = V + 7                  # out of range: 0 out, no scatter term
        idx[1, 4, 0] = -3
    go = torch.randn(B, S, K, generator=g)
    xd = x.to(DEV).requires_grad_(True)
    got = ChunkedDistributedGatherLogprob.apply(xd, idx.to(DEV), 0, V, 4, None, False)
    ref = gather_logprobs(x, idx, 0, V)
    assert got.shape == (B, S, K) and got.dtype == torch.float32
    torch.testing.assert_close(got.cpu(), ref, rtol=0, atol=_val_tol(dtype))
    oob = (idx < 0) | (idx >= V)
    assert torch.all(got.cpu()[oob] == 0)
    (got * go.to(DEV)).sum().backward()
    _check_grad(xd.grad, gather_logprobs_grad(x, idx, 0, V, go), dtype)


def test_gather_vocab_slice_and_strided_logits():
    """Global ids against a vocabulary slice, logits as a non-contiguous view."""
    say("gather slice/strided")
    g = torch.Generator().manual_seed(11)
    base = torch.randn(3, 6, 2, 700, generator=g).bfloat16()
    x = base[:, :, 1, 50:650]  # [3, 6, 600], row stride 1400
    idx = torch.randint(0, 1000, (3, 6, 7), generator=g)
    got = ChunkedDistributedGatherLogprob.apply(x.to(DEV), idx.to(DEV), 200, 800, 6, None, True)
    torch.testing.assert_close(got.cpu(), gather_logprobs(x, idx, 200, 800), rtol=0, atol=2e-3)


def test_reference_chunked_gather_case():
    """The reference's TP=1 case: B=2, S=16, V=256, K=3, chunk 5 (test_model_utils.py:872-940)."""
    say("reference chunked gather")
    torch.manual_seed(1337)
    full = torch.randn(2, 16, 256)
    gi = torch.randint(0, 256, (2, 16, 3))
    base = full.clone().requires_grad_(True)
    sel = torch.gather(torch.log_softmax(base, -1), -1, gi)
    sel.sum().backward()
    xd = full.to(DEV).requires_grad_(True)
    got = ChunkedDistributedGatherLogprob.apply(xd, gi.to(DEV), 0, 256, 5, None, False)
    torch.testing.assert_close(got.cpu(), sel.detach(), rtol=1e-4, atol=1e-4)
    got.sum().backward()
    torch.testing.assert_close(xd.grad.cpu(), base.grad, rtol=1e-4, atol=1e-4)


def test_policy_logprobs_at_sampler_topk_single_device():
    """Reference test_model_utils.py:422-446 on the GPU path."""
    say("sampler topk single device")
    torch.manual_seed(0)
    logits = torch.randn(2, 6, 11)
    ids = torch.randint(0, 11, (2, 6, 3), dtype=torch.int32)
    ld = logits.to(DEV).requires_grad_(True)
    got = get_policy_logprobs_at_sampler_topk(sampler_topk_token_ids=ids.to(DEV), next_token_logits=ld)
    lr = logits.clone().requires_grad_(True)
    exp = torch.log_softmax(lr, dim=-1)[:, :-1].gather(-1, ids.long()[:, 1:])
    torch.testing.assert_close(got.cpu(), exp.detach())
    got.sum().backward()
    exp.sum().backward()
    assert torch.isfinite(ld.grad).all()
    torch.testing.assert_close(ld.grad.cpu(), lr.grad, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("dtype,V", [(torch.float32, 997), (torch.bfloat16, 1000),
                                     (torch.bfloat16, 1003), (torch.float16, 640),
                                     (torch.bfloat16, 151936)])
def test_divergence_fwd_bwd_parity(kind, dtype, V):
    say("divergence", kind, dtype, "V", V)
    g = torch.Generator().manual_seed(V)
    B, S = 2, 7
    s = (torch.randn(B, S, V, generator=g) * 1.5).to(dtype)
    t = (torch.randn(B, S, V, generator=g) * 1.5 + 20).to(dtype) if kind != "entropy" else None
    go = torch.randn(B, S, generator=g)
    go[0, 2] = 0.0  # zero upstream row: written without reading
    sd = s.to(DEV).requires_grad_(True)
    fn = KINDS[kind]
    args = (sd, 4, None, False) if t is None else (sd, t.to(DEV), 4, None, False)
    got = fn.apply(*args)
    ref = divergence(kind, s, t)
    assert got.shape == (B, S) and got.dtype == torch.float32
    torch.testing.assert_close(got.cpu(), ref, rtol=0, atol=_val_tol(dtype) if V < 10000 else 5e-5)
    torch.testing.assert_close(got.cpu().double(), divergence_f64(kind, s, t), rtol=0,
                               atol=_val_tol(dtype) if V < 10000 else 5e-5)
    (got * go.to(DEV)).sum().backward()
    assert sd.grad.dtype == dtype
    _check_grad(sd.grad, divergence_grad(kind, s, t, go), dtype)
    assert torch.all(sd.grad[0, 2] == 0)


@pytest.mark.parametrize("kind", ["cross_entropy", "reverse_kl"])
def test_divergence_strided_and_misaligned_rows(kind):
    """Non-contiguous student (row kernel) and student/teacher rows at different alignments."""
    say("divergence strided", kind)
    g = torch.Generator().manual_seed(3)
    big = torch.randn(2, 5, 1031, generator=g).bfloat16()
    s = big[:, :, 1:1001]            # row start 2 bytes past alignment
    t = torch.randn(2, 5, 1000, generator=g).bfloat16()
    go = torch.randn(2, 5, generator=g)
    sd = s.to(DEV).requires_grad_(True)
    got = KINDS[kind].apply(sd, t.to(DEV), 2, None, False)
    torch.testing.assert_close(got.cpu(), divergence(kind, s, t), rtol=0, atol=2e-3)
    (got * go.to(DEV)).sum().backward()
    _check_grad(sd.grad, divergence_grad(kind, s, t, go), torch.bfloat16)


def test_reverse_kl_vanishes_for_identical_logits():
    say("rkl identical")
    torch.manual_seed(4)
    logits = torch.randn(1, 4, 13)
    got = ChunkedDistributedReverseKLToFixedLogits.apply(logits.to(DEV), logits.clone().to(DEV), 4, None, True)
    torch.testing.assert_close(got.cpu(), torch.zeros_like(got.cpu()), rtol=0, atol=1e-6)
    big = torch.randn(2, 3, 151936).bfloat16().to(DEV)
    got = ChunkedDistributedReverseKLToFixedLogits.apply(big, big.clone(), 4, None, True)
    assert got.abs().max().item() < 2e-5


def test_bf16_logits_are_normalised_in_fp32():
    """Reference test_model_utils.py:2110-2127: bf16 in, fp32 reverse KL within 1e-5."""
    say("bf16 fp32 normalisation")
    torch.manual_seed(5)
    s = torch.randn(1, 4, 8, dtype=torch.bfloat16)
    t = torch.randn(1, 4, 8, dtype=torch.bfloat16)
    got = ChunkedDistributedReverseKLToFixedLogits.apply(s.to(DEV), t.to(DEV), 2, None, True)
    exp = divergence_f64("reverse_kl", s.float(), t.float())
    torch.testing.assert_close(got.cpu().double(), exp, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("kind", ["cross_entropy", "reverse_kl"])
def test_backward_matches_float64_autograd(kind):
    """Reference test_model_utils.py:1930-1973: the shared backward drops the constant dw/dlogp."""
    say("autograd", kind)
    torch.manual_seed(2)
    teacher = torch.randn(2, 5, 9)
    go = torch.randn(2, 5)
    student = torch.randn(2, 5, 9)
    sd = student.to(DEV).requires_grad_(True)
    KINDS[kind].apply(sd, teacher.to(DEV), 3, None, False).mul(go.to(DEV)).sum().backward()
    sr = student.double().requires_grad_(True)
    (divergence_f64(kind, sr, teacher) * go.double()).sum().backward()
    torch.testing.assert_close(sd.grad.cpu().double(), sr.grad, rtol=1e-4, atol=1e-5)


def test_teacher_gets_no_gradient():
    say("teacher no grad")
    torch.manual_seed(3)
    s = torch.randn(1, 4, 6, device=DEV, requires_grad=True)
    t = torch.randn(1, 4, 6, device=DEV, requires_grad=True)
    ChunkedDistributedReverseKLToFixedLogits.apply(s, t, 2, None, False).sum().backward()
    assert s.grad is not None and t.grad is None


def test_large_vocab_rows_and_entropy_closed_form():
    """[2, 64, 151936] bf16: sampled rows against the oracle, uniform rows give -log V."""
    say("large vocab divergences")
    g = torch.Generator().manual_seed(8)
    V = 151936
    s = torch.randn(2, 64, V, generator=g).bfloat16()
    s[1, 5] = 0  # uniform row
    t = torch.randn(2, 64, V, generator=g).bfloat16()
    sd, td = s.to(DEV), t.to(DEV)
    ent = ChunkedDistributedEntropy.apply(sd, 64, None, True).cpu()
    assert ent[1, 5].item() == pytest.approx(-torch.log(torch.tensor(float(V))).item(), abs=1e-5)
    rows = [(0, 0), (0, 17), (1, 5), (1, 63)]
    for kind in KINDS:
        fn = KINDS[kind]
        got = (fn.apply(sd, 64, None, True) if kind == "entropy" else fn.apply(sd, td, 64, None, True)).cpu()
        for b, r in rows:
            ref = divergence_f64(kind, s[b:b + 1, r:r + 1], None if kind == "entropy" else t[b:b + 1, r:r + 1])
            assert abs(got[b, r].item() - ref.item()) < 5e-5, (kind, b, r)
