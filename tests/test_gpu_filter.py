"""gfx950 top-k / top-p / temperature-filtered logprobs against the CPU oracle (GPU).

Filtering decisions are made on fp32 values, as in the reference's production
chain (the logits are upcast before filtering, model_utils.py:1666 and
loss/loss_input.py:556), so 16-bit inputs are checked against the oracle run on
their fp32 upcast.  Keep sets are compared bit-exactly (boolean masks); filtered logprobs within
2e-3 abs for bf16 logits and 1e-5 for fp32 (-inf exactly where the target is
outside the kept set); gradients within 1e-3 abs or one bf16 ulp.  The oracle
resolves ties at the top-p boundary in stable (vocabulary-index) order, as the
kernels do.
"""

import pytest
import torch

from oracle.sampling import filtered_logprobs, filtered_logprobs_grad, next_token_filtered, top_k_top_p
from rl_amd.algorithms.logits_sampling_utils import apply_top_k_top_p
from rl_amd.distributed.model_utils import (
    ChunkedDistributedLogprobWithSampling,
    DistributedLogprobWithSampling,
    from_parallel_logits_to_logprobs,
)
from rl_amd.distributed.sampling import filtered_next_token_logprobs
from rl_amd.algorithms.logits_sampling_utils import TrainingSamplingParams
from tests.helpers import assert_close_or_ulp_bf16

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

CASES = [
    (50, 0.9),      # the workload's filter (fast path)
    (5, 1.0),       # top-k only
    (1, 1.0),       # argmax
    (None, 0.9),    # top-p only (general path)
    (None, 0.3),
    (700, 0.95),    # large k, fast path with 16-wave rows
    (2000, 0.99),   # k > 1024 (general path)
]


def _logits(B, S, V, dtype, seed, peaked=True, ties=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, V, generator=g)
    if ties:
        x = (x * 8).round() / 8  # many exact ties
    if peaked:
        idx = torch.randint(0, V, (B, S), generator=g)
        x.scatter_add_(-1, idx.unsqueeze(-1), torch.full((B, S, 1), 6.0))
    return x.to(dtype)


@pytest.mark.parametrize("k,p", CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_keep_mask_bit_exact(k, p, dtype):
    print("[case] keep", k, p, dtype, flush=True)
    x = _logits(3, 7, 4096, dtype, seed=1 + (k or 0))
    filt_o, keep_o = top_k_top_p(x.float(), k, p)
    filt, keep = apply_top_k_top_p(x.to(DEV), k, p)
    assert keep.dtype == torch.bool and filt.dtype == dtype
    assert torch.equal(keep.cpu(), keep_o)
    assert torch.equal(filt.cpu(), filt_o.to(dtype))


@pytest.mark.parametrize("k,p", CASES)
@pytest.mark.parametrize("dtype,T", [(torch.bfloat16, 1.0), (torch.bfloat16, 0.7), (torch.float32, 1.0),
                                     (torch.float32, 0.7), (torch.float16, 1.3)])
def test_next_token_fwd_bwd_against_oracle(k, p, dtype, T):
    print("[case] fwd/bwd", k, p, dtype, T, flush=True)
    B, S, V = 2, 9, 3001
    x = _logits(B, S, V, dtype, seed=7 + (k or 0))
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, V, (B, S), generator=g)
    # point half the targets at the row's argmax so that many are kept
    ids[:, 1::2] = x[:, :-1:2].float().argmax(-1)
    gout = torch.randn(B, S - 1, generator=g)
    lp_o, keep_o, grad_o = next_token_filtered(x, ids, k, p, temperature=T, grad_output=gout)
    xd = x.to(DEV).requires_grad_(True)
    lp = filtered_next_token_logprobs(xd, ids.to(DEV), k, p, temperature=T)
    (gr,) = torch.autograd.grad(lp, [xd], gout.to(DEV))
    lp_c = lp.detach().cpu()
    assert torch.equal(torch.isinf(lp_c), torch.isinf(lp_o))
    fin = torch.isfinite(lp_o)
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    torch.testing.assert_close(lp_c[fin], lp_o[fin], rtol=0, atol=tol)
    assert gr.dtype == dtype
    if dtype == torch.bfloat16:
        assert_close_or_ulp_bf16(gr, grad_o, 1e-3)
    else:
        torch.testing.assert_close(gr.float().cpu(), grad_o.float(), rtol=0, atol=1e-3)


def test_massive_ties_take_the_general_path():
    """All-equal rows: every element ties with the k-th value, the candidate list overflows."""
    print("[case] ties", flush=True)
    V = 5000
    x = torch.zeros(2, 3, V)
    x[1, 1, 17] = 1.0
    ids = torch.randint(0, V, (2, 3))
    for k, p in [(10, 1.0), (10, 0.5), (None, 0.5)]:
        lp_o, keep_o = filtered_logprobs(x, ids, k, p)
        lp = DistributedLogprobWithSampling.apply(x.to(DEV), ids.to(DEV), None, k, p, True)
        torch.testing.assert_close(lp.cpu(), lp_o, rtol=0, atol=1e-5)
        _, keep = apply_top_k_top_p(x.to(DEV), k, p)
        assert torch.equal(keep.cpu(), keep_o)


@pytest.mark.parametrize("chunk", [None, 3])
def test_distributed_with_sampling_api(chunk):
    print("[case] api chunk", chunk, flush=True)
    B, S, V = 2, 6, 1000
    x = _logits(B, S, V, torch.float32, seed=11)
    g = torch.Generator().manual_seed(4)
    t = torch.randint(0, V, (B, S), generator=g)
    t[:, ::2] = x[:, ::2].argmax(-1)
    gout = torch.randn(B, S, generator=g)
    lp_o, _ = filtered_logprobs(x, t, 8, 0.8)
    gr_o = filtered_logprobs_grad(x, t, 8, 0.8, gout)
    xd = x.to(DEV).requires_grad_(True)
    if chunk is None:
        lp = DistributedLogprobWithSampling.apply(xd, t.to(DEV), None, 8, 0.8)
    else:
        lp = ChunkedDistributedLogprobWithSampling.apply(xd, t.to(DEV), None, 8, 0.8, chunk)
    (gr,) = torch.autograd.grad(lp, [xd], gout.to(DEV))
    assert torch.equal(torch.isinf(lp.detach().cpu()), torch.isinf(lp_o))
    fin = torch.isfinite(lp_o)
    torch.testing.assert_close(lp.detach().cpu()[fin], lp_o[fin], rtol=0, atol=1e-5)
    torch.testing.assert_close(gr.cpu(), gr_o, rtol=0, atol=1e-5)


def test_from_parallel_logits_sampling_params():
    print("[case] from_parallel sampling", flush=True)
    B, S, V = 2, 10, 777
    x = _logits(B, S, V, torch.bfloat16, seed=5)
    ids = torch.randint(0, V, (B, S), generator=torch.Generator().manual_seed(5))
    sp = TrainingSamplingParams(top_k=20, top_p=0.7)
    got = from_parallel_logits_to_logprobs(x.to(DEV), ids.to(DEV), 0, V, None, sampling_params=sp,
                                           inference_only=True)
    exp, _, _ = next_token_filtered(x, ids, 20, 0.7)
    assert torch.equal(torch.isinf(got.cpu()), torch.isinf(exp))
    fin = torch.isfinite(exp)
    torch.testing.assert_close(got.cpu()[fin], exp[fin], rtol=0, atol=2e-3)


def test_full_size_workload_sampled_rows():
    """bf16 [4, 4096, 151936], T=0.7, k=50, p=0.9: sampled rows against the oracle (keep sets exact)."""
    print("[case] full size filtered", flush=True)
    from rl_amd import workloads

    d = workloads.topk_filter_bf16(device=DEV)
    x, ids, gout = d["logits"], d["input_ids"], d["grad"]
    B, S, V = x.shape
    x.requires_grad_(True)
    lp = filtered_next_token_logprobs(x, ids, 50, 0.9, temperature=0.7)
    (gr,) = torch.autograd.grad(lp, [x], gout)
    inside = (gout != 0)
    # targets chosen inside the kept set get finite logprobs
    assert torch.isfinite(lp[inside]).float().mean() > 0.99
    rs = torch.Generator().manual_seed(0)
    for _ in range(16):
        b = int(torch.randint(0, B, (1,), generator=rs))
        s = int(torch.randint(0, S - 1, (1,), generator=rs))
        xr = x.detach()[b : b + 1, s : s + 2].cpu()
        idr = ids[b : b + 1, s : s + 2].cpu()
        lp_o, keep_o, grad_o = next_token_filtered(xr, idr, 50, 0.9, temperature=0.7,
                                                   grad_output=gout[b : b + 1, s : s + 1].cpu())
        got = lp[b, s].item()
        if torch.isinf(lp_o).item():
            assert got == float("-inf")
        else:
            assert abs(got - lp_o.item()) <= 2e-3
        assert_close_or_ulp_bf16(gr[b : b + 1, s : s + 1], grad_o[:, :1], 1e-3)
        # keep set of this row, bit-exact
        y = (xr[:, :1].float() / 0.7).to(torch.bfloat16).float()
        _, keep_o1 = top_k_top_p(y, 50, 0.9)
        _, keep1 = apply_top_k_top_p(y.to(DEV), 50, 0.9)
        assert torch.equal(keep1.cpu(), keep_o1)
    assert gr[:, -1].abs().max().item() == 0
    del x, gr
