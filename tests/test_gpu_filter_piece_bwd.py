"""The filtered backward on 8 KB pieces (rows cut into pieces in address order, ties of
rank-form cuts counted and listed per piece and settled per row) against the
row-per-workgroup walk (GPU).

Both write the gradient of the same forward records, so they must agree bit for bit on
every row: rank-form cuts of 16-bit rows (ties kept from rank rcut on, in index order)
with few ties per piece (listed) and with many (a piece's list overflows and the fix-up
reads the piece again), index-form cuts (fp32 rows), the fused temperature and an
earlier in-place one, rows with a zero upstream gradient and the rows past R, rows that
start off a 16-byte boundary (elements before the first vector and after the last).
Layouts the pieces do not take (rows at different 16-byte offsets) fall back to the
walk.  The walk itself is checked against
the oracle in test_gpu_filter.py and test_gpu_full_rows.py (which run the piece schedule
by default).
"""

import pytest
import torch

from rl_amd import _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _rows(B, S, V, dtype, seed, ties=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, V, generator=g)
    if ties:
        x = (x * 8).round() / 8
    idx = torch.randint(0, V, (B, S), generator=g)
    x.scatter_add_(-1, idx.unsqueeze(-1), torch.full((B, S, 1), 6.0))
    return x.to(dtype)


def _both(x, k, p, T, gT, g, tgt, decision=None, make_grad=None):
    """(pieces, walk) gradients of the filtered logprobs of rows 0..S-2 of x."""
    info, kidx, kp = _C.filtered_fwd(x, tgt, T, k or 0, p, None, decision)
    out = []
    for pieces in (True, False):
        gi = make_grad() if make_grad else torch.full(x.shape, 7.0, dtype=x.dtype, device=DEV)
        _C.filtered_bwd(x, tgt, T, info, kidx, kp, g, gi, grad_temperature=gT, top_k=k or 0, pieces=pieces)
        out.append(gi)
    return out, info


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("k,p", [(None, 0.9), (None, 0.3), (2000, 0.9), (1500, 1.0)])
@pytest.mark.parametrize("T,gT", [(1.0, 1.0), (0.7, 1.0), (1.0, 0.7), (0.7, 1.3)])
@pytest.mark.parametrize("ties", [True, False])
def test_pieces_equal_walk(dtype, k, p, T, gT, ties):
    print("[case] piece bwd", dtype, k, p, T, gT, ties, flush=True)
    B, S, V = 2, 17, 20000  # 5 pieces per 16-bit row, 10 per fp32 row
    x = _rows(B, S, V, dtype, seed=3 + (k or 0), ties=ties).to(DEV)
    gen = torch.Generator().manual_seed(4)
    tgt = torch.randint(0, V, (B, S - 1), generator=gen)
    tgt[:, ::2] = x[:, :-1:2].float().argmax(-1).cpu()
    g = torch.randn(B, S - 1, generator=gen)
    g[:, 3:6] = 0.0
    (pc, walk), _ = _both(x, k, p, T, gT, g.to(DEV), tgt.to(DEV), torch.float32 if dtype != torch.float32 else None)
    assert torch.equal(pc, walk)
    assert not pc[:, -1].any()  # the row past R
    assert not pc[:, 3:6].any()  # zero upstream gradient


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ties", [True, False])
def test_16bit_decisions_rank_form(dtype, ties):
    """Top-p decided in the 16-bit dtype (the histogram kernels' rank-form cuts)."""
    print("[case] piece bwd 16-bit decisions", dtype, ties, flush=True)
    B, S, V = 2, 17, 32768
    x = _rows(B, S, V, dtype, seed=11, ties=ties).to(DEV)
    gen = torch.Generator().manual_seed(12)
    tgt = torch.randint(0, V, (B, S - 1), generator=gen).to(DEV)
    g = torch.randn(B, S - 1, generator=gen).to(DEV)
    (pc, walk), info = _both(x, None, 0.9, 1.0, 1.0, g, tgt, None)
    rec = info.cpu().view(torch.int32).view(-1, 6)
    assert bool((rec[:, 3] < -1).any()), "expected rank-form cuts with rcut > 0"
    assert torch.equal(pc, walk)


def test_tie_list_overflow():
    """Rows whose cut falls inside a group of 2000 equal bf16 values (about 250 per
    piece, more than a piece lists): the fix-up reads those pieces again."""
    print("[case] piece bwd tie overflow", flush=True)
    B, S, V = 1, 9, 32768
    gen = torch.Generator().manual_seed(21)
    x = torch.randn(B, S, V, generator=gen) - 20.0
    for s in range(S):
        pos = torch.randperm(V, generator=gen)[:2001]
        x[0, s, pos[:2000]] = 1.0
        x[0, s, pos[2000]] = 1.0 + float(torch.log(torch.tensor(3000.0)))  # 1.5x the group's mass
    x = x.to(torch.bfloat16).to(DEV)
    tgt = torch.randint(0, V, (B, S - 1), generator=gen).to(DEV)
    g = torch.randn(B, S - 1, generator=gen).to(DEV)
    (pc, walk), info = _both(x, None, 0.8, 1.0, 1.0, g, tgt, torch.float32)
    rec = info.cpu().view(torch.int32).view(-1, 6)
    assert bool((rec[:, 3] < -1).all()), "expected rank-form cuts inside the tied group"
    assert torch.equal(pc, walk)
    kept = (pc[0, :-1].float() != 0).sum(-1).cpu()
    assert torch.equal(kept, rec[:, 4].long())  # every kept element has a non-zero gradient here


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("V,lo", [(12285, 1), (12287, 1), (5, 1), (12288 - 8, 3)])
def test_rows_off_a_16_byte_boundary(dtype, V, lo):
    """Logits and gradient as views starting `lo` elements into rows of 12288 (every row
    at the same 16-byte offset): elements before the first vector and after the last
    belong to the first and the last piece."""
    print("[case] piece bwd unaligned rows", dtype, V, lo, flush=True)
    B, S, W = 2, 9, 12288
    xw = torch.zeros(B, S, W, dtype=dtype)
    xw[:, :, lo:lo + V] = _rows(B, S, V, dtype, seed=41, ties=dtype != torch.float32)
    xw = xw.to(DEV)
    x = xw[:, :, lo:lo + V]
    gen = torch.Generator().manual_seed(42)
    tgt = torch.randint(0, V, (B, S - 1), generator=gen)
    tgt[:, 0] = 0
    tgt[:, 1] = V - 1
    tgt = tgt.to(DEV)
    g = torch.randn(B, S - 1, generator=gen).to(DEV)
    walls = []

    def make_grad():
        gw = torch.full((B, S, W), 7.0, dtype=dtype, device=DEV)
        walls.append(gw)
        return gw[:, :, lo:lo + V]

    p = 0.9 if V > 8 else 0.5
    (pc, walk), _ = _both(x, None, p, 0.7, 1.0, g, tgt, torch.float32 if dtype != torch.float32 else None,
                          make_grad=make_grad)
    assert torch.equal(pc, walk)
    for gw in walls:  # nothing written outside the views
        assert torch.all(gw[:, :, :lo] == 7.0) and torch.all(gw[:, :, lo + V:] == 7.0)
    # the same rows, contiguous
    xc = x.contiguous()
    (pcc, _), _ = _both(xc, None, p, 0.7, 1.0, g, tgt, torch.float32 if dtype != torch.float32 else None)
    assert torch.equal(pc, pcc)


@pytest.mark.parametrize("V", [4099, 4096])
def test_layouts_the_pieces_do_not_take(V):
    """Rows at different 16-byte offsets (V = 4099), or a gradient with its own row
    stride: the walk runs, or the pieces do, and both agree."""
    print("[case] piece bwd other layouts", V, flush=True)
    B, S = 2, 9
    x = _rows(B, S, V, torch.bfloat16, seed=31).to(DEV)
    gen = torch.Generator().manual_seed(32)
    tgt = torch.randint(0, V, (B, S - 1), generator=gen).to(DEV)
    g = torch.randn(B, S - 1, generator=gen).to(DEV)
    info, kidx, kp = _C.filtered_fwd(x, tgt, 0.7, 0, 0.9, None, torch.float32)
    wide = torch.full((B, S, V + 8), 7.0, dtype=torch.bfloat16, device=DEV)
    a, b = wide[:, :, :V], torch.full((B, S, V), 7.0, dtype=torch.bfloat16, device=DEV)
    _C.filtered_bwd(x, tgt, 0.7, info, kidx, kp, g, a, top_k=0, pieces=True)
    _C.filtered_bwd(x, tgt, 0.7, info, kidx, kp, g, b, top_k=0, pieces=False)
    assert torch.equal(a, b)
    assert torch.all(wide[:, :, V:] == 7.0)
