"""Logprobs from hidden states (fused LM-head GEMM + log-sum-exp) against the oracle (GPU).

Tolerances.  The reference's logits are a bf16 matmul output: an fp32 sum of
bf16 products rounded once to bf16.  The kernel forms the same sum on the MFMA
units in another order, so a logit can round to the neighbouring bf16 value
(one ulp, <= |x| * 2^-7).  A logprob therefore matches the oracle within
2e-3 + |x_t| * 2^-7 (the target logit enters it directly; the log-sum-exp
moves by far less), and most rows within 2e-3.  Gradients: the logits
gradient G is rounded to bf16 before the two GEMMs (the reference keeps it in
fp32), so dH and dW match the float64 oracle to 1e-2 of their largest
magnitude; fused and unfused (materialised-logits) paths agree the same way.
Out-of-range targets give exactly 0.
"""

import pytest
import torch

from oracle.linear_ce import (
    hidden_state_logprob_grads,
    hidden_state_logprobs,
    logits_bf16,
    next_token_hidden_state_logprobs,
)
from rl_amd.distributed.model_utils import (
    ChunkedDistributedHiddenStatesToLogprobs,
    from_parallel_hidden_states_to_logprobs,
    from_parallel_logits_to_logprobs,
)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def say(*a):
    print("[case]", *a, flush=True)


def _inputs(S, B, H, V, seed, scale=1.5):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(S, B, H, generator=g).to(torch.bfloat16)
    weight = (torch.randn(V, H, generator=g) * (scale / H**0.5)).to(torch.bfloat16)
    target = torch.randint(0, V, (B, S), generator=g)
    return hidden, weight, target


def _check_logprobs(got, ref, x_t):
    tol = 2e-3 + x_t.abs() * 2.0**-7
    diff = (got.cpu().double() - ref.double()).abs()
    assert torch.all(diff <= tol), f"max excess {(diff - tol).max().item():.3e}"
    # the one-ulp flips of the target logit are rare
    assert (diff > 2e-3).float().mean().item() < 0.1


def _target_logits(hidden, weight, target):
    x = logits_bf16(hidden, weight)  # [B, S, V]
    return x.gather(-1, target.clamp(0, weight.shape[0] - 1).unsqueeze(-1)).squeeze(-1)


@pytest.mark.parametrize("S,B,H,V", [(37, 3, 128, 1000), (16, 2, 256, 151936), (300, 1, 128, 4096),
                                     (5, 4, 384, 257), (29, 2, 64, 1000), (9, 3, 192, 3001)])
def test_forward_against_oracle(S, B, H, V):
    say("linear-ce fwd", S, B, H, V)
    hidden, weight, target = _inputs(S, B, H, V, seed=S + V)
    ref = hidden_state_logprobs(hidden, target, weight, 0, V)
    got = ChunkedDistributedHiddenStatesToLogprobs.apply(
        hidden.to(DEV), target.to(DEV), weight.to(DEV), 0, V, 8, None, True)
    assert got.shape == (B, S) and got.dtype == torch.float32
    _check_logprobs(got, ref, _target_logits(hidden, weight, target))


def test_vocab_slice_targets_are_exactly_zero():
    say("linear-ce vocab slice")
    S, B, H, V = 20, 3, 128, 700
    hidden, weight, target = _inputs(S, B, H, V, seed=7)
    target = torch.randint(0, 3 * V, (B, S), generator=torch.Generator().manual_seed(8))
    vs, ve = V, 2 * V
    got = ChunkedDistributedHiddenStatesToLogprobs.apply(
        hidden.to(DEV), target.to(DEV), weight.to(DEV), vs, ve, None, None, True).cpu()
    outside = (target < vs) | (target >= ve)
    assert outside.any() and (~outside).any()
    assert torch.all(got[outside] == 0)
    ref = hidden_state_logprobs(hidden, target, weight, vs, ve)
    _check_logprobs(got[~outside], ref[~outside], _target_logits(hidden, weight, target - vs)[~outside])


def test_next_token_api_and_roll():
    say("linear-ce next-token api")
    S, B, H, V = 33, 2, 128, 3000
    hidden, weight, target = _inputs(S, B, H, V, seed=11)
    got = from_parallel_hidden_states_to_logprobs(
        hidden.to(DEV), weight.to(DEV), False, target.to(DEV), 0, V, None, inference_only=True,
        chunk_size=4)
    assert got.shape == (B, S - 1)
    ref = next_token_hidden_state_logprobs(hidden, weight, target, 0, V)
    _check_logprobs(got, ref, _target_logits(hidden, weight, target.roll(-1, -1))[:, :-1])


@pytest.mark.parametrize("chunk", [None, 1, 7])
def test_gradients_against_oracle(chunk):
    say("linear-ce grads chunk", chunk)
    S, B, H, V = 24, 3, 128, 1500
    hidden, weight, target = _inputs(S, B, H, V, seed=21)
    g = torch.randn(B, S, generator=torch.Generator().manual_seed(22))
    g[:, :5] = 0.0  # zero-gradient rows
    h = hidden.to(DEV).requires_grad_(True)
    w = weight.to(DEV).requires_grad_(True)
    lp = ChunkedDistributedHiddenStatesToLogprobs.apply(h, target.to(DEV), w, 0, V, chunk, None, False)
    dh, dw = torch.autograd.grad(lp, [h, w], g.to(DEV))
    assert dh.dtype == torch.bfloat16 and dw.dtype == torch.bfloat16
    rdh, rdw, _ = hidden_state_logprob_grads(hidden, target, weight, 0, V, g)
    for got, ref in ((dh, rdh), (dw, rdw)):
        err = (got.cpu().double() - ref).abs().max().item()
        assert err <= 1e-2 * ref.abs().max().item(), (err, ref.abs().max().item())


def test_all_zero_gradient_tiles():
    say("linear-ce zero-gradient tiles")
    S, B, H, V = 300, 1, 128, 600  # 300 rows: one full 256-row tile of zeros
    hidden, weight, target = _inputs(S, B, H, V, seed=31)
    g = torch.zeros(B, S)
    g[:, 280:] = 1.0
    h = hidden.to(DEV).requires_grad_(True)
    w = weight.to(DEV).requires_grad_(True)
    lp = ChunkedDistributedHiddenStatesToLogprobs.apply(h, target.to(DEV), w, 0, V, None, None, False)
    dh, dw = torch.autograd.grad(lp, [h, w], g.to(DEV))
    assert torch.all(dh[:280].cpu() == 0)
    rdh, rdw, _ = hidden_state_logprob_grads(hidden, target, weight, 0, V, g)
    for got, ref in ((dh, rdh), (dw, rdw)):
        err = (got.cpu().double() - ref).abs().max().item()
        assert err <= 1e-2 * ref.abs().max().item(), err


def test_fused_matches_materialised_logits_path():
    """The reference's own agreement check (linear-CE fusion vs the logits path), on one GPU."""
    say("linear-ce fused vs unfused")
    S, B, H, V = 64, 2, 256, 151936
    hidden, weight, target = _inputs(S, B, H, V, seed=41)
    hd, wd, td = hidden.to(DEV), weight.to(DEV), target.to(DEV)
    fused = from_parallel_hidden_states_to_logprobs(hd, wd, False, td, 0, V, None, inference_only=True)
    logits = torch.mm(hd.view(S * B, H), wd.t().contiguous()).view(S, B, V)
    logits = logits.transpose(0, 1).contiguous()  # [B, S, V] bf16
    unfused = from_parallel_logits_to_logprobs(logits, td, 0, V, None, inference_only=True)
    x_t = logits.float().gather(-1, td.roll(-1, -1).unsqueeze(-1)).squeeze(-1)[:, :-1]
    _check_logprobs(fused, unfused.cpu(), x_t.cpu())


@pytest.mark.parametrize("H", [64, 200])
def test_unaligned_hidden_sizes_and_sliced_weight(H):
    """Hidden sizes that are not a multiple of 128 (small models' 64) and a weight that is
    a column slice of a wider matrix (row stride not a multiple of 8, unaligned start) run
    through zero-padded copies; logprobs and both gradients match the oracle."""
    say("linear-ce unaligned H", H)
    S, B, V = 19, 3, 1234
    hidden, weight, target = _inputs(S, B, H, V, seed=61 + H)
    wide = torch.zeros(V, H + 3, dtype=torch.bfloat16)
    wide[:, 1 : H + 1] = weight
    g = torch.randn(B, S, generator=torch.Generator().manual_seed(62))
    g[:, :4] = 0.0
    h = hidden.to(DEV).requires_grad_(True)
    wd = wide.to(DEV).requires_grad_(True)
    w = wd[:, 1 : H + 1]
    assert w.stride(0) % 8 != 0 and w.data_ptr() % 16 != 0
    lp = ChunkedDistributedHiddenStatesToLogprobs.apply(h, target.to(DEV), w, 0, V, 5, None, False)
    _check_logprobs(lp.detach(), hidden_state_logprobs(hidden, target, weight, 0, V),
                    _target_logits(hidden, weight, target))
    dh, dwide = torch.autograd.grad(lp, [h, wd], g.to(DEV))
    dw = dwide[:, 1 : H + 1]
    assert not dwide[:, 0].any() and not dwide[:, H + 1 :].any()
    rdh, rdw, _ = hidden_state_logprob_grads(hidden, target, weight, 0, V, g)
    for got, ref in ((dh, rdh), (dw, rdw)):
        err = (got.cpu().double() - ref).abs().max().item()
        assert err <= 1e-2 * ref.abs().max().item(), (err, ref.abs().max().item())


def test_errors():
    say("linear-ce errors")
    hidden, weight, target = _inputs(4, 2, 128, 50, seed=1)
    with pytest.raises(RuntimeError):  # mixed dtypes: torch.matmul's own error, as in the reference
        ChunkedDistributedHiddenStatesToLogprobs.apply(
            hidden.float().to(DEV), target.to(DEV), weight.to(DEV), 0, 50, None, None, True)
    with pytest.raises(ValueError):
        ChunkedDistributedHiddenStatesToLogprobs.apply(
            hidden.to(DEV), target.t().contiguous().to(DEV), weight.to(DEV), 0, 50, None, None, True)


@pytest.mark.parametrize("pattern", ["none", "all", "scattered"])
def test_gradient_row_compaction(pattern):
    """The backward runs only rows with a non-zero upstream gradient: no such row (zero
    gradients), every row (the uncompacted path) and scattered rows across chunks."""
    say("linear-ce grad rows", pattern)
    S, B, H, V = 40, 3, 128, 2000
    hidden, weight, target = _inputs(S, B, H, V, seed=51)
    gen = torch.Generator().manual_seed(52)
    g = torch.randn(B, S, generator=gen)
    if pattern == "none":
        g.zero_()
    elif pattern == "scattered":
        g *= (torch.rand(B, S, generator=gen) < 0.3).float()
    h = hidden.to(DEV).requires_grad_(True)
    w = weight.to(DEV).requires_grad_(True)
    lp = ChunkedDistributedHiddenStatesToLogprobs.apply(h, target.to(DEV), w, 0, V, 7, None, False)
    dh, dw = torch.autograd.grad(lp, [h, w], g.to(DEV))
    if pattern == "none":
        assert not dh.any() and not dw.any()
        return
    rdh, rdw, _ = hidden_state_logprob_grads(hidden, target, weight, 0, V, g)
    for got, ref in ((dh, rdh), (dw, rdw)):
        err = (got.cpu().double() - ref).abs().max().item()
        assert err <= 1e-2 * ref.abs().max().item(), (pattern, err)
    zero_rows = (g == 0).t()  # [S, B], the layout of dh
    assert not dh.cpu()[zero_rows].any()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("S,B,H,V,chunk", [(37, 3, 128, 1000, 8), (16, 2, 64, 151936, None), (9, 3, 200, 3001, 4)])
def test_fp16_fp32_forward_and_gradients(dtype, S, B, H, V, chunk):
    """fp16 inputs run the fused kernels (logits tiles on the fp16 MFMA, rounded to fp16;
    G in bf16 and W, H rounded to bf16 for dH and dW); fp32 inputs take per chunk the fp32
    tile loop (fp32 MFMA), then the logprob row kernels (the reference's chunked shape), and
    the backward's three products on the fp32 tile loop over the active rows.  The oracle
    rounds the exact products to the dtype; logprobs within 2e-3 (fp16) / 1e-5 (fp32) plus
    the target logit's last-ulp rounding, dH and dW against the float64 oracle to 1e-2
    (fp16, bf16 operands of the two products) / 1e-4 (fp32) of their largest magnitude."""
    say("linear-ce", dtype, S, B, H, V, chunk)
    g0 = torch.Generator().manual_seed(S * V + H)
    hidden = torch.randn(S, B, H, generator=g0).to(dtype)
    weight = (torch.randn(V, H, generator=g0) * (1.5 / H**0.5)).to(dtype)
    target = torch.randint(0, V + 50, (B, S), generator=g0)  # some targets outside the slice
    g = torch.randn(B, S, generator=g0)
    g[:, :2] = 0.0
    ref = hidden_state_logprobs(hidden, target, weight, 0, V)
    h = hidden.to(DEV).requires_grad_(True)
    w = weight.to(DEV).requires_grad_(True)
    lp = ChunkedDistributedHiddenStatesToLogprobs.apply(h, target.to(DEV), w, 0, V, chunk, None, False)
    assert lp.dtype == torch.float32 and lp.shape == (B, S)
    outside = target >= V
    assert torch.all(lp.detach().cpu()[outside] == 0)
    eps = 2.0**-10 if dtype == torch.float16 else 2.0**-22
    base = 2e-3 if dtype == torch.float16 else 1e-5
    x_t = _target_logits(hidden, weight, target.clamp(max=V - 1))
    diff = (lp.detach().cpu().double() - ref.double()).abs()
    assert torch.all(diff[~outside] <= base + x_t[~outside].abs() * eps), diff.max().item()
    dh, dw = torch.autograd.grad(lp, [h, w], g.to(DEV))
    assert dh.dtype == dtype and dw.dtype == dtype
    rdh, rdw, _ = hidden_state_logprob_grads(hidden, target, weight, 0, V, g)
    rel = 1e-2 if dtype == torch.float16 else 1e-4
    for got, want in ((dh, rdh), (dw, rdw)):
        err = (got.cpu().double() - want).abs().max().item()
        assert err <= rel * want.abs().max().item(), (err, want.abs().max().item())


@pytest.mark.parametrize("active", [0.0, 0.2, 0.6, 1.0])
def test_gradient_blocks_with_device_count(active):
    """Several backward blocks (600 rows, 256 per block at chunk 7): the active-row count
    lives on the device, so the blocks past it return at once and dW is rounded by the
    last block holding active rows (none, the first, the second, the third)."""
    say("linear-ce grad blocks active", active)
    S, B, H, V = 200, 3, 128, 2000
    hidden, weight, target = _inputs(S, B, H, V, seed=61)
    gen = torch.Generator().manual_seed(62)
    g = torch.randn(B, S, generator=gen) * (torch.rand(B, S, generator=gen) < active).float()
    h = hidden.to(DEV).requires_grad_(True)
    w = weight.to(DEV).requires_grad_(True)
    lp = ChunkedDistributedHiddenStatesToLogprobs.apply(h, target.to(DEV), w, 0, V, 7, None, False)
    dh, dw = torch.autograd.grad(lp, [h, w], g.to(DEV))
    if active == 0.0:
        assert not dh.any() and not dw.any()
        return
    rdh, rdw, _ = hidden_state_logprob_grads(hidden, target, weight, 0, V, g)
    for got, ref in ((dh, rdh), (dw, rdw)):
        err = (got.cpu().double() - ref).abs().max().item()
        assert err <= 1e-2 * ref.abs().max().item(), (active, err)
    assert not dh.cpu()[(g == 0).t()].any()


@pytest.mark.parametrize("R,C,lds,off,Rp,ldd,dtype", [
    (130, 77, 77, 0, 136, 136, torch.bfloat16),     # columns not a multiple of 8: element loads
    (200, 128, 136, 3, 203, 208, torch.bfloat16),   # source 6 bytes past alignment, Rp not a multiple of 8
    (64, 256, 256, 0, 64, 64, torch.float16),       # whole tiles, fp16 rounded to bf16
    (1000, 520, 520, 0, 1024, 1030, torch.bfloat16),  # destination stride not a multiple of 8
    (0, 64, 64, 0, 64, 64, torch.bfloat16),         # no rows: zeros
])
def test_transpose_shapes_and_alignments(R, C, lds, off, Rp, ldd, dtype):
    """mirl_transpose_bf16 gives dst[c, r] = bf16(src[r, c]) for r < R and 0 for
    R <= r < Rp, with the columns past Rp of each destination row left alone, for
    16-byte and element-wise pieces alike."""
    from rl_amd import _C

    say("transpose", R, C, lds, off, Rp, ldd, dtype)
    gen = torch.Generator().manual_seed(R * 7 + C)
    rows = max(R, 1)
    flat = torch.randn(rows * lds + off, generator=gen).to(dtype)
    src = flat[off:].view(rows, lds)[:, :C]
    dst_full = torch.full((C, ldd), 9.0, dtype=torch.bfloat16)
    dst = dst_full.to(DEV)
    src_d = flat.to(DEV)[off:].view(rows, lds)[:, :C]
    _C.transpose_bf16(src_d, R, dst[:, :Rp])
    ref = dst_full.clone()
    ref[:, :Rp] = 0
    ref[:, :R] = src[:R].t().to(torch.bfloat16)
    assert torch.equal(dst.cpu(), ref)


@pytest.mark.parametrize("R,C,lds,off,Rp,ldd", [
    (130, 77, 77, 0, 136, 136),     # columns not a multiple of 4: element loads
    (200, 128, 132, 1, 203, 208),   # source 4 bytes past alignment, Rp not a multiple of 4
    (64, 256, 256, 0, 64, 64),      # whole tiles
    (1000, 520, 520, 0, 1024, 1030),  # destination stride not a multiple of 4
    (0, 64, 64, 0, 64, 64),         # no rows: zeros
])
def test_transpose_f32_shapes_and_alignments(R, C, lds, off, Rp, ldd):
    """mirl_transpose_f32 gives dst[c, r] = src[r, c] for r < min(R, count - count_off) and
    0 up to Rp, with the columns past Rp of each destination row left alone."""
    from rl_amd import _C

    say("transpose f32", R, C, lds, off, Rp, ldd)
    gen = torch.Generator().manual_seed(R * 5 + C)
    rows = max(R, 1)
    flat = torch.randn(rows * lds + off, generator=gen)
    src = flat[off:].view(rows, lds)[:, :C]
    src_d = flat.to(DEV)[off:].view(rows, lds)[:, :C]
    for cnt in (None, R // 2 + 10):
        dst_full = torch.full((C, ldd), 9.0)
        dst = dst_full.to(DEV)
        count = None if cnt is None else torch.tensor([cnt], dtype=torch.int64, device=DEV)
        _C.transpose_f32(src_d, R, dst[:, :Rp], count=count, count_off=10 if cnt is not None else 0)
        n = R if cnt is None else min(R, cnt - 10)
        ref = dst_full.clone()
        ref[:, :Rp] = 0
        ref[:, :n] = src[:n].t()
        assert torch.equal(dst.cpu(), ref), cnt


def test_gemm_primitives_with_device_counts():
    """The GEMM, split sum and transpose with a device count equal the same calls on the
    host-trimmed operands, bit for bit."""
    from rl_amd import _C

    say("linear-ce primitives with device counts")
    gen = torch.Generator().manual_seed(71)
    M, N, K = 600, 300, 512
    a = torch.randn(M, K, generator=gen).to(torch.bfloat16).to(DEV)
    b = torch.randn(N, K, generator=gen).to(torch.bfloat16).to(DEV)
    for c in (0, 1, 255, 257, 600):
        cnt = torch.tensor([c + 100], dtype=torch.int64, device=DEV)  # count_off 100
        # rows: absent rows of a leave their output rows untouched
        part = torch.full((2, M, N), 7.0, device=DEV)
        _C.gemm_bf16_abt(a, b, K, part, k_splits=2, count=cnt, count_off=100, count_axis=_C.COUNT_ROWS)
        if c > 0:
            ref = torch.empty((2, c, N), device=DEV)
            _C.gemm_bf16_abt(a[:c], b, K, ref, k_splits=2)
            assert torch.equal(part[:, :c], ref)
        assert torch.all(part[:, c:] == 7.0)
        out = torch.full((M, N), 3.0, dtype=torch.bfloat16, device=DEV)
        _C.sum_splits_bf16(part, out, count=cnt, count_off=100)
        ref_out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
        _C.sum_splits_bf16(part, ref_out)
        assert torch.equal(out[:c], ref_out[:c]) and not out[c:].any()
        # a row map writes each row at its own position (here a permutation)
        rmap = torch.randperm(M, generator=gen).to(DEV)
        mapped = torch.full((M, N), 3.0, dtype=torch.bfloat16, device=DEV)
        _C.sum_splits_bf16(part, mapped, count=cnt, count_off=100, out_rows=rmap)
        assert torch.equal(mapped[rmap], out)
        # transpose with the count: zeros past it
        t = torch.full((K, 640), 5.0, dtype=torch.bfloat16, device=DEV)
        _C.transpose_bf16(a, M, t, count=torch.tensor([c], dtype=torch.int64, device=DEV))
        t_ref = torch.empty((K, 640), dtype=torch.bfloat16, device=DEV)
        _C.transpose_bf16(a, c, t_ref)
        assert torch.equal(t, t_ref)
    # reduction length: c rows of the reduction, blocks of 256 accumulated in fp32 and
    # rounded once by the last block holding rows
    at = torch.zeros((N, 768), dtype=torch.bfloat16, device=DEV)
    bt = torch.zeros((K, 768), dtype=torch.bfloat16, device=DEV)
    for c in (0, 100, 256, 300, 700):
        at.zero_()
        bt.zero_()
        at[:, :c] = torch.randn(N, c, generator=gen).to(torch.bfloat16).to(DEV)
        bt[:, :c] = torch.randn(K, c, generator=gen).to(torch.bfloat16).to(DEV)
        cnt = torch.tensor([c], dtype=torch.int64, device=DEV)
        ref32 = torch.zeros((N, K), device=DEV)
        for r0 in range(0, 768, 256):
            _C.gemm_bf16_abt(at[:, r0:r0 + 256], bt[:, r0:r0 + 256], 256, ref32, accumulate=r0 > 0)
        out16 = torch.full((N, K), 9.0, dtype=torch.bfloat16, device=DEV)
        acc32 = torch.empty((N, K), device=DEV)
        for r0 in range(0, 768, 256):
            _C.gemm_bf16_abt(at[:, r0:r0 + 256], bt[:, r0:r0 + 256], 256, acc32, accumulate=r0 > 0,
                             count=cnt, count_off=r0, count_axis=_C.COUNT_K, out_bf16=out16,
                             final_at=r0 + 256)
        assert torch.equal(out16, ref32.to(torch.bfloat16)), c


def test_gemm_f32_primitives():
    """The fp32 tile loop (four v_mfma_f32_32x32x2_f32 per fragment pair): C = A . B^T
    against float64 within fp32 summation error; k splits sum to the same product; with a
    device row count absent rows are untouched and the others equal the uncounted call bit
    for bit; a reduction-length count over blocks accumulated in fp32 equals the
    host-trimmed reduction; the fp32 transpose and split sum with counts and a row map."""
    from rl_amd import _C

    say("linear-ce fp32 primitives")
    gen = torch.Generator().manual_seed(81)
    M, N, K = 600, 300, 512
    a = torch.randn(M, K, generator=gen).to(DEV)
    b = torch.randn(N, K, generator=gen).to(DEV)
    ref = (a.double() @ b.double().t()).cpu()
    out = torch.empty((M, N), device=DEV)
    _C.gemm_f32_abt(a, b, K, out)
    bound = K * 2.0**-23 * (a.abs().double() @ b.abs().double().t()).cpu()  # fp32 summation error
    assert torch.all((out.cpu().double() - ref).abs() <= bound)
    part = torch.empty((2, M, N), device=DEV)
    _C.gemm_f32_abt(a, b, K, part, k_splits=2)
    assert torch.all((part.sum(0).cpu().double() - ref).abs() <= bound)
    # a strided B (rows of a wider buffer) and accumulation
    wide = torch.zeros((N, K + 64), device=DEV)
    wide[:, :K] = b
    acc = out.clone()
    _C.gemm_f32_abt(a, wide, K, acc, accumulate=True)
    assert torch.all((acc.cpu().double() - 2 * ref).abs() <= 2 * bound + 1e-6)
    for c in (0, 1, 255, 257, 600):
        cnt = torch.tensor([c + 100], dtype=torch.int64, device=DEV)  # count_off 100
        pc = torch.full((2, M, N), 7.0, device=DEV)
        _C.gemm_f32_abt(a, b, K, pc, k_splits=2, count=cnt, count_off=100, count_axis=_C.COUNT_ROWS)
        assert torch.equal(pc[:, :c], part[:, :c]) and torch.all(pc[:, c:] == 7.0)
        # split sum into fp32 rows, through a row map
        rmap = torch.randperm(M, generator=gen).to(DEV)
        o32 = torch.full((M, N), 3.0, device=DEV)
        _C.sum_splits_bf16(pc, o32, count=cnt, count_off=100, out_rows=rmap)
        direct = torch.empty((M, N), device=DEV)
        _C.sum_splits_bf16(part, direct)
        assert torch.equal(o32[rmap][:c], direct[:c]) and not o32[rmap][c:].any()
        assert torch.equal(direct, part[0] + part[1])
        # fp32 transpose with the count and an offset: zeros past it
        t = torch.full((K, 640), 5.0, device=DEV)
        _C.transpose_f32(a, M, t, count=torch.tensor([c + 30], dtype=torch.int64, device=DEV), count_off=30)
        t_ref = torch.zeros((K, 640), device=DEV)
        t_ref[:, :c] = a[:c].t()
        assert torch.equal(t, t_ref)
    # reduction length: c rows of the reduction over blocks of 256, accumulated in fp32
    at = torch.zeros((N, 768), device=DEV)
    bt = torch.zeros((K, 768), device=DEV)
    for c in (0, 100, 256, 300, 700):
        at.zero_()
        bt.zero_()
        at[:, :c] = torch.randn(N, c, generator=gen).to(DEV)
        bt[:, :c] = torch.randn(K, c, generator=gen).to(DEV)
        cnt = torch.tensor([c], dtype=torch.int64, device=DEV)
        ref32 = torch.zeros((N, K), device=DEV)
        for r0 in range(0, 768, 256):
            _C.gemm_f32_abt(at[:, r0:r0 + 256], bt[:, r0:r0 + 256], 256, ref32, accumulate=r0 > 0)
        acc32 = torch.full((N, K), 9.0, device=DEV)
        for r0 in range(0, 768, 256):
            _C.gemm_f32_abt(at[:, r0:r0 + 256], bt[:, r0:r0 + 256], 256, acc32, accumulate=r0 > 0,
                            count=cnt, count_off=r0, count_axis=_C.COUNT_K)
        assert torch.equal(acc32, ref32), c


def test_f32_path_runs_no_library_gemm(monkeypatch):
    """fp32 hidden states and weight: forward and backward run on this library's kernels;
    torch's GEMM entry points are made to fail during the call."""
    say("linear-ce fp32 without library GEMMs")
    S, B, H, V = 24, 2, 128, 3000
    g0 = torch.Generator().manual_seed(91)
    hidden = torch.randn(S, B, H, generator=g0)
    weight = torch.randn(V, H, generator=g0) * (1.5 / H**0.5)
    target = torch.randint(0, V, (B, S), generator=g0)
    g = torch.randn(B, S, generator=g0)
    h = hidden.to(DEV).requires_grad_(True)
    w = weight.to(DEV).requires_grad_(True)

    def refuse(*a, **k):
        raise AssertionError("a library GEMM ran on the fp32 hidden-state path")

    for name in ("matmul", "mm", "addmm", "bmm", "baddbmm", "einsum"):
        monkeypatch.setattr(torch, name, refuse)
    monkeypatch.setattr(torch.Tensor, "__matmul__", refuse)
    lp = ChunkedDistributedHiddenStatesToLogprobs.apply(h, target.to(DEV), w, 0, V, 5, None, False)
    dh, dw = torch.autograd.grad(lp, [h, w], g.to(DEV))
    monkeypatch.undo()
    ref = hidden_state_logprobs(hidden, target, weight, 0, V)
    assert (lp.detach().cpu().double() - ref.double()).abs().max().item() < 1e-4
    rdh, rdw, _ = hidden_state_logprob_grads(hidden, target, weight, 0, V, g)
    for got, want in ((dh, rdh), (dw, rdw)):
        assert (got.cpu().double() - want).abs().max().item() <= 1e-4 * want.abs().max().item()


def test_weight_written_in_place_between_backwards():
    """A weight changed without its version counter moving (``p.data.copy_``, as Megatron
    and collectives write parameters) gives the next backward the new weight: dH and dW
    equal, bit for bit, those of a fresh weight tensor holding the same values."""
    say("linear-ce weight written in place")
    S, B, H, V = 40, 2, 256, 3001
    hidden, weight, target = _inputs(S, B, H, V, seed=51)
    _, weight2, _ = _inputs(S, B, H, V, seed=52)
    g = torch.randn(B, S, generator=torch.Generator().manual_seed(53))
    h = hidden.to(DEV).requires_grad_(True)
    w = weight.to(DEV).requires_grad_(True)

    def grads(wt):
        lp = ChunkedDistributedHiddenStatesToLogprobs.apply(h, target.to(DEV), wt, 0, V, 8, None, False)
        return torch.autograd.grad(lp, [h, wt], g.to(DEV))

    dh1, dw1 = grads(w)
    version = w._version
    w.data.copy_(weight2.to(DEV))
    assert w._version == version  # the write is invisible to the version counter
    dh2, dw2 = grads(w)
    fresh = weight2.to(DEV).requires_grad_(True)
    dh_f, dw_f = grads(fresh)
    assert torch.equal(dh2, dh_f) and torch.equal(dw2, dw_f)
    assert not torch.equal(dh2, dh1)
