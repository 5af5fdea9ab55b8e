"""The early-backward recheck's redo over the listed rows (the check lists the rows whose
upstream gradient differs, the redo visits only those) against the redo over every piece,
and against a fresh backward (GPU).

After an early backward for g_used, the recheck for the real g must leave grad_in equal,
bit for bit, to the backward run for g directly: rows whose g equals g_used keep what the
early backward wrote, the others (every row of a scaled loss, a subset, rows whose real g
is zero) are rewritten, rows past R stay as they were.  Rows whose vectors do not fill
the last 4 KB piece, fp32 and fp16 logits, a target outside the vocabulary shard, and a
check that finds nothing are covered.
"""

import pytest
import torch

from rl_amd import _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _case(dtype, B, S, V, seed, vs=0):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(B, S, V, generator=g) * 2).to(dtype).to(DEV)
    R = S - 1
    tgt = torch.randint(vs, vs + V, (B, R), generator=g)
    tgt[0, 0] = vs + V + 5  # outside the shard
    tgt = tgt.to(DEV)
    out = torch.empty(B, R, device=DEV)
    stats = torch.empty(B, R, 2, device=DEV)
    _C.logprob_fwd(logits, tgt, vs, vs + V, out, stats)
    g_used = torch.randn(B, R, generator=g)
    g_used[:, : R // 4] = 0.0  # masked rows
    return logits, tgt, stats, g_used.to(DEV), g


def _early(logits, tgt, vs, V, stats, g_used):
    gin = torch.empty_like(logits)
    _C.logprob_bwd(logits, tgt, vs, vs + V, stats, g_used, gin)
    return gin


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("V", [4096, 5000])
@pytest.mark.parametrize("kind", ["scaled", "subset", "to_zero", "none"])
def test_listed_redo_equals_fresh_backward(dtype, V, kind):
    print("[case] recheck list", dtype, V, kind, flush=True)
    B, S, vs = 3, 37, 100
    logits, tgt, stats, g_used, gen = _case(dtype, B, S, V, seed=7 + V, vs=vs)
    R = S - 1
    if kind == "scaled":
        g = g_used * 0.5
    elif kind == "subset":
        g = g_used.clone()
        idx = torch.randperm(B * R, generator=gen)[: B * R // 3].to(DEV)
        g.view(-1)[idx] = torch.randn(idx.numel(), generator=gen).to(DEV)
    elif kind == "to_zero":
        g = g_used.clone()
        g[:, R // 4 : R // 2] = 0.0  # rows the early backward wrote for a non-zero g
    else:
        g = g_used.clone()
    fresh = _early(logits, tgt, vs, V, stats, g)
    outs = []
    for listed in (True, False):
        gin = _early(logits, tgt, vs, V, stats, g_used)
        flags = _C.logprob_bwd_recheck(logits, tgt, vs, vs + V, stats, g, g_used, gin, listed=listed)
        outs.append(gin)
        if kind == "none":
            assert not bool(flags.any())
    assert torch.equal(outs[0], fresh)
    assert torch.equal(outs[1], fresh)
