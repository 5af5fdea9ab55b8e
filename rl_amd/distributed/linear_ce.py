"""Token logprobs from hidden states and the output weight (fused LM head + log-softmax).

Drop-in for ``from_parallel_hidden_states_to_logprobs`` and
``ChunkedDistributedHiddenStatesToLogprobs`` (reference
nemo_rl/distributed/model_utils.py:2541-2745) with a tensor-parallel group of
size 1.  Hidden states are Megatron's sequence-first ``[S, B, H]``; the weight
is ``[V, H]``; targets are ``[B, S]``.

* forward: one gfx950 kernel forms each 256 x 256 logits tile on the MFMA units
  (bf16 or fp16 inputs, fp32 accumulation, rounded to the input dtype as the
  reference's matmul output is) and reduces it to per-row partial log-sum-exps
  and the target logit; a merge kernel finishes each row.  The ``[S*B, V]`` logits are
  never materialised (the reference materialises an fp32 copy per chunk).
* backward: the rows with a non-zero upstream gradient are moved to the front
  (the others have a zero logits gradient: zero dH rows, nothing added to dW)
  and counted on the device, where the kernels read the count (no host
  synchronisation); per block of up to ``4 * chunk_size * B`` rows a kernel recomputes the logits
  tiles and writes ``G = (onehot - softmax) * g`` in bf16 and its transpose, and
  ``dH = G . W`` and ``dW += G^T . H`` run on the same MFMA tile loop
  (``mirl_gemm_bf16_abt``) against bf16 transposed copies of W (formed in every
  backward) and of the active hidden rows, with fp32 accumulation (``dW``
  accumulated in fp32 across blocks and rounded once to the weight's dtype, by
  the kernel itself when there is one block; the reference adds each chunk into
  a buffer of the weight's dtype).  G is bf16 for fp16 inputs too: fp16's
  exponent range would flush the small ``-p * g`` terms of the vocabulary's
  tail, which together make up most of ``dH``; the transposes round fp16 W and
  H to bf16 for those two products.
* fp32 hidden states and weights keep the reference's chunked shape on this
  library's kernels: per chunk of sequence positions the fp32 logits are one
  product on the same MFMA tile loop with fp32 operands (``mirl_gemm_f32_abt``,
  four ``v_mfma_f32_32x32x2_f32`` per 16-byte fragment pair; the reference's
  ``torch.matmul`` output), and the row kernels of the logits path
  (``mirl_logprob_fwd`` / ``mirl_logprob_bwd``) form the logprobs and, in
  place, the logits gradient.  The backward moves the rows with a non-zero
  upstream gradient to the front and counts them on the device, as above; per
  block of one chunk of rows it recomputes their logits, forms G in place,
  and runs ``dH = G . W`` and ``dW += G^T . H`` in fp32 on the same tile loop
  (fp32 transposed copies of W, of the active hidden rows and of G).  An fp32
  GEMM here is bound by the fp32 MFMA rate (1/16 of bf16's) at over a
  thousand flops per byte of logits, so the per-chunk logits write and read
  that a fused epilogue would save cost under 1% of the step; skipping the
  rows with a zero upstream gradient saves most of the backward's products.
* other dtypes (fp64, or hidden states and weight of different dtypes) take
  the reference's chunked shape with the library's ``torch.matmul``.
"""

from __future__ import annotations

from typing import Any, Optional

import torch

from rl_amd import _C

__all__ = ["ChunkedDistributedHiddenStatesToLogprobs", "from_parallel_hidden_states_to_logprobs"]


def _require_single_rank(*groups: Optional[Any]) -> None:
    from rl_amd.distributed.model_utils import _require_single_rank as req

    req(*groups)


class ChunkedDistributedHiddenStatesToLogprobs(torch.autograd.Function):
    """Selected-token logprobs ``[B, S]`` (fp32) of ``hidden [S, B, H] . weight[V, H]^T``.

    Reference: model_utils.py:2572-2745 (forward 2576-2644, backward 2647-2745).
    ``target`` is already aligned with the rows (the caller rolls it); targets
    outside ``[vocab_start_index, vocab_end_index)`` give 0.
    """

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        tensor_parallel_hidden_states: torch.Tensor,
        target: torch.Tensor,
        output_weight_layer: torch.Tensor,
        vocab_start_index: int,
        vocab_end_index: int,
        chunk_size: Optional[int],
        tp_group: Optional[Any],
        inference_only: bool = False,
    ) -> torch.Tensor:
        _require_single_rank(tp_group)
        if chunk_size is not None and int(chunk_size) <= 0:
            raise ValueError("chunk_size must be positive")
        hidden = tensor_parallel_hidden_states
        if hidden.dim() != 3:
            raise ValueError(f"expected hidden states [S, B, H], got {tuple(hidden.shape)}")
        S, B, H = hidden.shape
        if tuple(target.shape) != (B, S):
            raise ValueError(f"target shape {tuple(target.shape)} does not match [B, S] = {(B, S)}")
        weight = output_weight_layer
        if weight.dim() != 2 or weight.shape[1] != H:
            raise ValueError(f"weight shape {tuple(weight.shape)} does not match hidden size {H}")
        if not hidden.is_contiguous():
            hidden = hidden.contiguous()
        if weight.stride(-1) != 1:
            weight = weight.contiguous()
        if target.dtype != torch.int64:
            target = target.long()
        if hidden.dtype == torch.float32 and weight.dtype == torch.float32:
            return _f32_forward(ctx, hidden, target, weight, vocab_start_index, vocab_end_index,
                                chunk_size, inference_only)
        if hidden.dtype not in _FUSED_DTYPES or weight.dtype != hidden.dtype:
            return _chunked_forward(ctx, hidden, target, weight, vocab_start_index, vocab_end_index,
                                    chunk_size, inference_only)
        ctx.chunked = False
        ctx.f32 = False
        h2 = hidden.view(S * B, H)
        out = torch.empty((B, S), dtype=torch.float32, device=hidden.device)
        stats = None
        if not inference_only:
            stats = torch.empty((S * B, 2), dtype=torch.float32, device=hidden.device)
        _C.linear_ce_fwd(_kernel_operand(h2), _kernel_operand(weight), B, target, vocab_start_index,
                         vocab_end_index, out, stats)
        if not inference_only:
            ctx.save_for_backward(hidden, target, weight, stats)
            ctx.vocab = (int(vocab_start_index), int(vocab_end_index))
            ctx.chunk_size = None if chunk_size is None else int(chunk_size)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):  # type: ignore[override]
        (grad_output,) = grad_outputs
        if ctx.f32:
            return _f32_backward(ctx, grad_output)
        if ctx.chunked:
            return _chunked_backward(ctx, grad_output)
        hidden, target, weight, stats = ctx.saved_tensors
        vs, ve = ctx.vocab
        S, B, H = hidden.shape
        V = weight.shape[0]
        T = S * B
        if grad_output.dtype != torch.float32:
            grad_output = grad_output.float()
        h2 = hidden.view(T, H)
        need_h = ctx.needs_input_grad[0]
        need_w = ctx.needs_input_grad[2]
        dev = hidden.device
        # Rows whose upstream gradient is exactly zero (prompt, padding) have a
        # zero logits gradient, so they add nothing to dW and their dH rows are
        # zero.  The rows are permuted so that the active ones come first (in row
        # order) and their count stays on the device: every kernel below reads it
        # and skips what lies past it, so the host never waits for the count.
        g_rows = grad_output.t().reshape(T)  # row r = (s, b) is position s of sample b
        nz = g_rows != 0
        perm = torch.argsort(torch.logical_not(nz).to(torch.uint8), stable=True)
        count = nz.sum(dtype=torch.int64).view(1)
        h_a = torch.index_select(h2, 0, perm)
        tgt_a = target.t().reshape(T).index_select(0, perm).view(1, T)
        st_a = stats.index_select(0, perm)
        g_a = g_rows.index_select(0, perm).view(1, T)
        # Blocks of up to 4 chunks of rows (whole 256-row tiles): the bf16 G
        # buffer stays below one reference chunk's fp32 logits, softmax and
        # one-hot temporaries.  Blocks past the count return at once.
        rows = T if ctx.chunk_size is None else min(T, _round_up(_BLOCK_CHUNKS * ctx.chunk_size * B, 256))
        n_blocks = -(-T // rows)
        Vp = _round_up(V, _K_ALIGN)
        # G [rows, Vp] (columns past V zero: dH's padded reduction length)
        G = torch.empty((rows, Vp), dtype=torch.bfloat16, device=dev)
        if Vp > V:
            G[:, V:].zero_()
        # G^T [V, rows rounded to 256] and H^T of the permuted rows [H, T rounded
        # to 256] for dW = (G^T) . (H^T)^T; H^T is zero past the count and G^T in
        # the tile that holds the last active row, which covers dW's reduction
        # (stopped at the count rounded up to 128)
        Gt = torch.empty((V, _padded_width(rows)), dtype=torch.bfloat16, device=dev) if need_w else None
        hT = None
        if need_w:
            hT = torch.empty((H, _padded_width(T)), dtype=torch.bfloat16, device=dev)
            _C.transpose_bf16(h_a, T, hT, count=count)
        wT, wT_ready = _weight_transposed(weight, Vp) if need_h else (None, None)
        # dH is written row by row at each permuted row's own position
        dH = torch.empty((T, H), dtype=hidden.dtype, device=dev) if need_h else None
        hk_a, wk = _kernel_operand(h_a), _kernel_operand(weight)
        if need_w:
            dW = torch.empty((V, H), dtype=weight.dtype, device=dev)
            # fp32 across blocks, rounded once by the last block with active rows
            # (allocated, never touched, when that is the first)
            dW32 = torch.empty((V, H), dtype=torch.float32, device=dev) if n_blocks > 1 else None
        for r0 in range(0, T, rows):
            n = min(rows, T - r0)
            Gc = G[:n]
            _C.linear_ce_grad(hk_a, wk, 1, tgt_a, vs, ve, st_a, g_a, r0, Gc, Gt, count=count)
            if need_h:
                # dH = G . W = G . (W^T)^T on the MFMA units, the reduction over
                # the vocabulary split so that the tiles fill the CUs; rows past
                # the count are written as zeros
                splits = _dh_splits(n, H, Vp, count_known=False)
                part = torch.empty((splits, n, H), dtype=torch.float32, device=dev)
                if wT_ready is not None:
                    torch.cuda.current_stream(dev).wait_event(wT_ready)
                    wT_ready = None
                _C.gemm_bf16_abt(Gc, wT, Vp, part, k_splits=splits, count=count, count_off=r0,
                                 count_axis=_C.COUNT_ROWS)
                _C.sum_splits_bf16(part, dH, count=count, count_off=r0, out_rows=perm[r0 : r0 + n])
                del part
            if need_w:
                nk = _round_up(n, _K_ALIGN)
                hb = hT[:, r0 : r0 + nk]
                if dW32 is None:
                    # one block: fp32 accumulation, rounded once to bf16 by the kernel
                    _C.gemm_bf16_abt(Gt, hb, nk, dW, count=count, count_off=r0, count_axis=_C.COUNT_K)
                else:
                    _C.gemm_bf16_abt(Gt, hb, nk, dW32, accumulate=r0 > 0, count=count, count_off=r0,
                                     count_axis=_C.COUNT_K, out_bf16=dW, final_at=r0 + n)
        if wT_ready is not None:  # no block ran: W^T still waits to be released after its writer
            torch.cuda.current_stream(dev).wait_event(wT_ready)
        grad_h = dH.view(S, B, H) if need_h else None
        grad_w = (dW if dW.dtype == weight.dtype else dW.to(weight.dtype)) if need_w else None
        return grad_h, None, grad_w, None, None, None, None, None


def _chunks(S: int, chunk_size: Optional[int]) -> list[tuple[int, int]]:
    cs = S if chunk_size is None else chunk_size
    return [(c0, min(S, c0 + cs)) for c0 in range(0, S, cs)] if S > 0 else []


def _chunked_forward(ctx, hidden, target, weight, vs, ve, chunk_size, inference_only):
    """fp32 (or mixed dtypes): per chunk of positions, logits = hidden[c] . weight^T in the input
    dtype (one library GEMM, [c, B, V]), then the logprob row kernel over them viewed
    as [B, c, V] (reference model_utils.py:2608-2630)."""
    S, B, H = hidden.shape
    dev = hidden.device
    out = torch.empty((B, S), dtype=torch.float32, device=dev)
    # the saved row statistics: chunk [c0, c1) is the contiguous [B, c1 - c0, 2]
    # block at offset 2 * B * c0
    stats = None if inference_only else torch.empty(2 * B * S, dtype=torch.float32, device=dev)
    for c0, c1 in _chunks(S, chunk_size):
        logits = torch.matmul(hidden[c0:c1], weight.t())  # [c, B, V]
        out_c = torch.empty((B, c1 - c0), dtype=torch.float32, device=dev)
        st_c = None if stats is None else stats[2 * B * c0 : 2 * B * c1].view(B, c1 - c0, 2)
        _C.logprob_fwd(logits.permute(1, 0, 2), target[:, c0:c1], vs, ve, out_c, st_c)
        out[:, c0:c1] = out_c
        del logits
    ctx.chunked = True
    ctx.f32 = False
    if not inference_only:
        ctx.save_for_backward(hidden, target, weight, stats)
        ctx.vocab = (int(vs), int(ve))
        ctx.chunk_size = None if chunk_size is None else int(chunk_size)
    return out


def _chunked_backward(ctx, grad_output):
    """fp32 backward (reference model_utils.py:2647-2745): per chunk the logits
    are recomputed by the library GEMM and the logprob backward kernel overwrites them
    with (onehot - softmax) * g in the input dtype; dH = G . W per chunk and
    dW = sum over chunks of G^T . H, accumulated in fp32."""
    hidden, target, weight, stats = ctx.saved_tensors
    vs, ve = ctx.vocab
    S, B, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    if grad_output.dtype != torch.float32:
        grad_output = grad_output.float()
    need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[2]
    dH = torch.empty_like(hidden) if need_h else None
    dW = torch.zeros((V, H), dtype=torch.float32, device=dev) if need_w else None
    for c0, c1 in _chunks(S, ctx.chunk_size):
        logits = torch.matmul(hidden[c0:c1], weight.t())  # [c, B, V]
        lv = logits.permute(1, 0, 2)
        st_c = stats[2 * B * c0 : 2 * B * c1].view(B, c1 - c0, 2)
        _C.logprob_bwd(lv, target[:, c0:c1], vs, ve, st_c, grad_output[:, c0:c1],
                       lv)  # the gradient overwrites the logits
        if need_h:
            torch.matmul(logits, weight, out=dH[c0:c1])
        if need_w:
            g2 = logits.reshape(-1, V)
            h2 = hidden[c0:c1].reshape(-1, H)
            if weight.dtype == torch.float32:
                torch.addmm(dW, g2.t(), h2, out=dW)
            else:
                torch.addmm(dW, g2.t(), h2, out_dtype=torch.float32, out=dW)
        del logits
    grad_w = (dW if dW.dtype == weight.dtype else dW.to(weight.dtype)) if need_w else None
    return dH, None, grad_w, None, None, None, None, None


def _f32_operand(x: torch.Tensor) -> torch.Tensor:
    """``x [N, H]`` fp32 as the fp32 tile loop reads it: ``H`` a multiple of 64, a row stride
    that is a multiple of 4 elements (16 bytes) and a 16-byte-aligned start; otherwise a
    zero-padded ``[N, round_up(H, 64)]`` copy (the padding adds exact zeros to every dot
    product)."""
    N, H = x.shape
    if (H % _F32_K_ALIGN == 0 and x.stride(-1) == 1 and x.stride(0) % 4 == 0 and x.stride(0) >= H
            and x.data_ptr() % 16 == 0):
        return x
    out = torch.zeros((N, _round_up(H, _F32_K_ALIGN)), dtype=x.dtype, device=x.device)
    out[:, :H].copy_(x)
    return out


def _f32_forward(ctx, hidden, target, weight, vs, ve, chunk_size, inference_only):
    """fp32: per chunk of positions, logits = hidden[c] . weight^T (fp32 tile loop, rows in
    (position, sample) order), then the logprob row kernel over them (reference
    model_utils.py:2608-2630).  The row statistics are saved per row r = s * B + b."""
    S, B, H = hidden.shape
    V = weight.shape[0]
    T = S * B
    dev = hidden.device
    h2 = _f32_operand(hidden.view(T, H))
    w2 = _f32_operand(weight)
    K = h2.shape[1]
    tgt_rows = target.t().reshape(1, T)  # row r = (s, b): position s of sample b
    out_rows = torch.empty((1, T), dtype=torch.float32, device=dev)
    stats = None if inference_only else torch.empty((T, 2), dtype=torch.float32, device=dev)
    chunks = _chunks(S, chunk_size)
    logits = torch.empty((max((c1 - c0) * B for c0, c1 in chunks), V), dtype=torch.float32, device=dev) \
        if chunks else None
    for c0, c1 in chunks:
        r0, r1 = c0 * B, c1 * B
        lc = logits[: r1 - r0]
        _C.gemm_f32_abt(h2[r0:r1], w2, K, lc)
        st_c = None if stats is None else stats[r0:r1].view(1, r1 - r0, 2)
        _C.logprob_fwd(lc.view(1, r1 - r0, V), tgt_rows[:, r0:r1], vs, ve, out_rows[:, r0:r1], st_c)
    del logits
    ctx.chunked = False
    ctx.f32 = True
    if not inference_only:
        ctx.save_for_backward(hidden, target, weight, stats)
        ctx.vocab = (int(vs), int(ve))
        ctx.chunk_size = None if chunk_size is None else int(chunk_size)
    return out_rows.view(S, B).t().contiguous()


def _f32_backward(ctx, grad_output):
    """fp32 backward (reference model_utils.py:2647-2745) over the rows with a non-zero
    upstream gradient, moved to the front and counted on the device (the others have a zero
    logits gradient: zero dH rows, nothing added to dW).  Per block of one chunk of rows:
    the logits recomputed on the fp32 tile loop, G = (onehot - softmax) * g written over them
    by the logprob backward kernel, dH = G . W against W^T, and dW += G^T . H, fp32
    throughout."""
    hidden, target, weight, stats = ctx.saved_tensors
    vs, ve = ctx.vocab
    S, B, H = hidden.shape
    V = weight.shape[0]
    T = S * B
    dev = hidden.device
    if grad_output.dtype != torch.float32:
        grad_output = grad_output.float()
    need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[2]
    h2 = hidden.view(T, H)
    g_rows = grad_output.t().reshape(T)
    nz = g_rows != 0
    perm = torch.argsort(torch.logical_not(nz).to(torch.uint8), stable=True)
    count = nz.sum(dtype=torch.int64).view(1)
    h_a = torch.index_select(h2, 0, perm)
    tgt_a = target.t().reshape(T).index_select(0, perm).view(1, T)
    st_a = stats.index_select(0, perm)
    g_a = g_rows.index_select(0, perm).view(1, T)
    hk_a, wk = _f32_operand(h_a), _f32_operand(weight)
    K = hk_a.shape[1]
    rows = T if ctx.chunk_size is None else min(T, _round_up(ctx.chunk_size * B, 256))
    Vp = _round_up(V, _F32_K_ALIGN)
    L = torch.empty((rows, Vp), dtype=torch.float32, device=dev)  # logits, then G
    if Vp > V:
        L[:, V:].zero_()  # dH's padded reduction length
    dH = torch.empty((T, H), dtype=torch.float32, device=dev) if need_h else None
    if need_h:
        wT = torch.empty((H, Vp), dtype=torch.float32, device=dev)
        _C.transpose_f32(weight, V, wT)
    if need_w:
        dW = torch.empty((V, H), dtype=torch.float32, device=dev)
        hT = torch.empty((H, _padded_width(T)), dtype=torch.float32, device=dev)
        _C.transpose_f32(h_a, T, hT, count=count)
        Gt = torch.empty((V, _padded_width(rows)), dtype=torch.float32, device=dev)
    for r0 in range(0, T, rows):
        n = min(rows, T - r0)
        Lc = L[:n]
        # the block's active rows (rows past the count are not computed)
        _C.gemm_f32_abt(hk_a[r0 : r0 + n], wk, K, Lc, count=count, count_off=r0,
                        count_axis=_C.COUNT_ROWS)
        lv = Lc[:, :V].view(1, n, V)
        _C.logprob_bwd(lv, tgt_a[:, r0 : r0 + n], vs, ve, st_a[r0 : r0 + n].view(1, n, 2),
                       g_a[:, r0 : r0 + n], lv)  # G over the logits; zeros past the count
        if need_h:
            splits = _dh_splits(n, H, Vp, count_known=False)
            part = torch.empty((splits, n, H), dtype=torch.float32, device=dev)
            _C.gemm_f32_abt(Lc, wT, Vp, part, k_splits=splits, count=count, count_off=r0,
                            count_axis=_C.COUNT_ROWS)
            _C.sum_splits_bf16(part, dH, count=count, count_off=r0, out_rows=perm[r0 : r0 + n])
            del part
        if need_w:
            nk = _round_up(n, _K_ALIGN)
            _C.transpose_f32(Lc[:, :V], n, Gt, count=count, count_off=r0)
            _C.gemm_f32_abt(Gt, hT[:, r0 : r0 + nk], nk, dW, accumulate=r0 > 0, count=count,
                            count_off=r0, count_axis=_C.COUNT_K)
    grad_h = dH.view(S, B, H) if need_h else None
    grad_w = dW if need_w else None
    return grad_h, None, grad_w, None, None, None, None, None


_FUSED_DTYPES = (torch.bfloat16, torch.float16)  # operand dtypes of the fused kernels
_F32_K_ALIGN = 64  # the fp32 tile loop steps through the reduction 64 elements at a time
_BLOCK_CHUNKS = 4  # chunks of active rows per backward block
_K_ALIGN = 128  # dW's reduction length is padded with zero rows to a multiple of this
_H_ALIGN = 128  # the fused kernels step through the hidden dimension 128 elements at a time


def _kernel_operand(x: torch.Tensor) -> torch.Tensor:
    """``x [N, H]`` (bf16 or fp16) as the fused kernels read it: ``H`` a multiple of 128, a row
    stride that is a multiple of 8 elements (16 bytes) and a 16-byte-aligned start.

    Other operands (small models' hidden sizes such as 64, sliced weights) are
    copied into a zero-padded ``[N, round_up(H, 128)]`` buffer: the padding adds
    exact zeros to every dot product, so the logits are the same sums.  The
    library GEMMs of the backward take the unpadded tensors.
    """
    N, H = x.shape
    if (H % _H_ALIGN == 0 and x.stride(-1) == 1 and x.stride(0) % 8 == 0 and x.stride(0) >= H
            and x.data_ptr() % 16 == 0):
        return x
    out = torch.zeros((N, _round_up(H, _H_ALIGN)), dtype=x.dtype, device=x.device)
    out[:, :H].copy_(x)
    return out


def _round_up(n: int, m: int) -> int:
    return (n + m - 1) // m * m


def _padded_width(rows: int) -> int:
    """Row length of the transposed operands of dW: whole 256-row tiles plus one
    128-byte line, so that the rows a tile reads together do not all start at the
    same offset of a power-of-two stride."""
    return _round_up(rows, 256) + 64


def _dh_splits(n: int, H: int, K: int, count_known: bool = True) -> int:
    """Splits of dH's reduction length (each adds an fp32 partial product to read
    back).  dH has few 256 x 256 tiles over a long reduction, so the count that
    fills the last round of tiles over the 256 CUs best wins, the smaller on a
    tie (measured on [5871, 151936] x [151936, 4096]: 1 split 7.62 ms, 2 6.09,
    3 6.81, 4 6.23).  The kernel cuts K into ranges of round_up(ceil(K / s), 128);
    only counts for which that gives exactly s ranges, each of at least 1024, qualify.
    With count_known False, n is an upper bound (the active rows are counted on the
    device) and at least two splits are taken where they qualify: fewer active rows
    leave the single-split tiles short of the CUs, and a second split costs one more
    fp32 partial of n x H."""
    tiles = ((n + 255) // 256) * ((H + 255) // 256)
    best, best_eff = 1, tiles / (256 * -(-tiles // 256))
    qualifying = []
    for s in range(2, 9):
        kb = _round_up(-(-K // s), 128)
        if kb < 1024 or -(-K // kb) != s:
            continue
        qualifying.append(s)
        t = tiles * s
        eff = t / (256 * -(-t // 256))
        if eff > best_eff + 1e-9:
            best, best_eff = s, eff
    if not count_known and best == 1 and qualifying:
        best = qualifying[0]
    return best


_transpose_streams: dict = {}


def _weight_transposed(weight: torch.Tensor, Vp: int):
    """W^T [H, Vp] bf16 (columns past V zero; an fp16 weight rounded), formed from the weight's current contents
    in every backward (one read and one write of W, about 0.5 ms at [151936, 4096]), and the event
    that marks it written.

    The transpose runs on a side stream (default priority) behind everything already
    enqueued on the current stream, so it overlaps the gradient kernel, which is bound by
    the MFMA units; the caller waits for the event on the current stream before the first
    product that reads W^T.  The buffer is allocated on the current stream, which frees
    it only after that product, itself ordered after the transpose.

    Nothing is kept across calls: a weight can change without its version counter
    moving (``p.data.copy_``, collectives writing into parameter storage), so a copy
    reused by key could silently give dH from an old weight."""
    V, H = weight.shape
    dev = weight.device
    wT = torch.empty((H, Vp), dtype=torch.bfloat16, device=dev)
    side = _transpose_streams.get(dev)
    if side is None:
        side = torch.cuda.Stream(dev)
        _transpose_streams[dev] = side
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        _C.transpose_bf16(weight, V, wT)
        ready = torch.cuda.Event()
        ready.record(side)
    return wT, ready


def from_parallel_hidden_states_to_logprobs(
    tensor_parallel_hidden_states: torch.Tensor,
    output_weight_layer: torch.Tensor,
    runtime_gather_output: bool,
    target: torch.Tensor,
    vocab_start_index: int,
    vocab_end_index: int,
    tp_group: Optional[Any],
    inference_only: bool = False,
    cp_group: Optional[Any] = None,
    chunk_size: Optional[int] = None,
) -> torch.Tensor:
    """Next-token logprobs ``[B, S-1]`` from ``[S, B, H]`` hidden states (reference model_utils.py:2541-2569).

    ``target`` ``[B, S]`` is rolled by -1 along the sequence, as in the
    reference; ``runtime_gather_output`` is accepted and unused, as there.
    """
    from rl_amd.distributed.model_utils import _group_size

    target = target.roll(shifts=-1, dims=-1)
    assert cp_group is None or _group_size(cp_group) == 1, (
        "Context parallelism is not supported for linear CE fusion loss"
    )
    logprobs = ChunkedDistributedHiddenStatesToLogprobs.apply(
        tensor_parallel_hidden_states,
        target,
        output_weight_layer,
        vocab_start_index,
        vocab_end_index,
        chunk_size,
        tp_group,
        inference_only,
    ).contiguous()
    return logprobs[:, :-1]
