"""Packed-sequence glue kernels (GPU): packing, target roll and unpacking against the
oracle's per-sequence loops (reference loss/utils.py:355-408, model_utils.py:1116-1139
and :1211-1229).  These are pure copies, so every result is compared bit for bit.

* ``_pack_input_ids`` on device tensors (``mirl_pack_sequences``) over ragged
  batches: rolls 0, -1 and 2, padded boundaries, sequences longer than the
  unpacked row (the packer's overhang), empty sequences, boundary lists longer
  than the batch, a nonzero first boundary, trailing dims and 1/2/4/8-byte
  element types;
* ``mirl_packed_roll_targets`` and ``mirl_unpack_rows_fwd`` against the
  oracle's loops, ``mirl_unpack_rows_bwd`` against autograd of the oracle's
  unpacking (float64 on the CPU);
* the entry points' own guards: boundaries out of order or past the buffers
  give zeros and stay inside the buffers.
"""

import numpy as np
import pytest
import torch

from oracle.logprob import pack_input_ids, pack_targets, unpack_logprobs
from rl_amd import _C
from rl_amd.algorithms.loss.utils import _pack_input_ids

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def say(*a):
    print("[case]", *a, flush=True)


def _ragged(seed, B, S, pad_multiple, overhang=False, empty=False):
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.integers(0, S + 1, size=B)]
    if overhang:
        lens[-1] = S + 3
    if empty and B > 1:
        lens[1] = 0
    cu, cu_pad = [0], [0]
    for n in lens:
        cu.append(cu[-1] + n)
        cu_pad.append(cu_pad[-1] + ((n + pad_multiple - 1) // pad_multiple) * pad_multiple)
    return cu, cu_pad


@pytest.mark.parametrize("roll", [0, -1, 2])
@pytest.mark.parametrize("pad_multiple", [1, 4])
def test_pack_input_ids_device_matches_oracle(roll, pad_multiple):
    say("pack ids", roll, pad_multiple)
    for seed in range(8):
        B, S = 6, 17
        cu, cu_pad = _ragged(seed, B, S, pad_multiple, overhang=seed % 2 == 1, empty=seed % 3 == 0)
        g = torch.Generator().manual_seed(seed)
        ids = torch.randint(1, 1000, (B, S), generator=g)
        got = _pack_input_ids(ids.to(DEV), tuple(cu), tuple(cu_pad), roll_shift=roll)
        exp = pack_input_ids(ids, cu, cu_pad, roll_shift=roll)
        assert got.dtype == ids.dtype and got.shape == exp.shape
        assert torch.equal(got.cpu(), exp), (seed, cu, cu_pad)


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32, torch.bfloat16, torch.bool, torch.uint8])
def test_pack_input_ids_dtypes_and_trailing_dims(dtype):
    say("pack dtypes", dtype)
    B, S, K = 4, 9, 5
    cu, cu_pad = _ragged(3, B, S, 2, overhang=True)
    g = torch.Generator().manual_seed(5)
    x = torch.randint(0, 50, (B, S, K), generator=g)
    x = (x % 2 == 1) if dtype == torch.bool else x.to(dtype)
    for roll in (0, -1):
        got = _pack_input_ids(x.to(DEV), tuple(cu), tuple(cu_pad), roll_shift=roll)
        exp = pack_input_ids(x, cu, cu_pad, roll_shift=roll)
        assert got.dtype == dtype and torch.equal(got.cpu(), exp), roll


def test_pack_input_ids_boundary_lists():
    """Longer boundary lists than the batch (extra sequences stay zero, the length is
    cu_pad[-1]); a nonzero first boundary; a decreasing one raises like the reference."""
    say("pack boundary lists")
    ids = torch.arange(1, 1 + 3 * 6).reshape(3, 6)
    cu, cu_pad = [0, 4, 6, 9, 12], [0, 4, 8, 12, 16]
    got = _pack_input_ids(ids.to(DEV), tuple(cu), tuple(cu_pad), roll_shift=-1)
    assert torch.equal(got.cpu(), pack_input_ids(ids, cu, cu_pad, roll_shift=-1))
    cu, cu_pad = [2, 5, 7, 8], [3, 7, 9, 11]
    got = _pack_input_ids(ids.to(DEV), tuple(cu), tuple(cu_pad))
    assert torch.equal(got.cpu(), pack_input_ids(ids, cu, cu_pad))
    with pytest.raises(RuntimeError):
        _pack_input_ids(ids.to(DEV), (0, 2, 4, 6), (0, 4, 2, 6))
    with pytest.raises(IndexError):
        _pack_input_ids(ids.to(DEV), (0, 2), (0, 4))


def test_roll_and_unpack_kernels_against_oracle():
    say("roll and unpack kernels")
    for seed in range(30):
        rng = np.random.default_rng(seed)
        lens = rng.integers(0, 9, size=int(rng.integers(1, 6)))
        b = [int(rng.integers(0, 3))]
        for n in lens:
            b.append(b[-1] + int(n))
        T = b[-1] + int(rng.integers(0, 3))
        bdev = torch.tensor(b, dtype=torch.int64, device=DEV)
        ids = torch.arange(T, dtype=torch.int64) + 100
        got = _C.packed_roll_targets(ids.to(DEV), bdev).cpu()
        exp = torch.zeros(T, dtype=torch.int64)
        exp[b[0] : b[-1]] = pack_targets(ids.unsqueeze(0), b)[0][b[0] : b[-1]]
        assert torch.equal(got, exp), (seed, b)
        S = int(rng.integers(1, 10))
        probs = torch.randn(T, dtype=torch.float64)
        out = _C.unpack_rows_fwd(probs.float().to(DEV), bdev, S - 1).cpu()
        assert torch.equal(out, unpack_logprobs(probs.float(), b, S)), (seed, b, S)
        pr = probs.clone().requires_grad_(True)
        g = torch.randn(len(b) - 1, S - 1, dtype=torch.float64)
        u = unpack_logprobs(pr, b, S)
        # nothing copied (all sequences shorter than 2, or no columns): no graph, zero gradient
        ga = torch.autograd.grad(u, [pr], g)[0] if u.requires_grad else torch.zeros_like(probs)
        gk = _C.unpack_rows_bwd(g.float().to(DEV), bdev, T).cpu()
        assert torch.equal(gk, ga.float()), (seed, b, S)


def test_kernels_guard_boundaries():
    """Boundaries that break the ordering or point past the buffers read nothing outside them."""
    say("boundary guards")
    T = 16
    ids = torch.arange(T, dtype=torch.int64, device=DEV) + 1
    for b in ([0, 9, 4, 16], [0, 40, 50], [5, 3, 2], [0, 16, 16]):
        bdev = torch.tensor(b, dtype=torch.int64, device=DEV)
        r = _C.packed_roll_targets(ids, bdev)
        assert r.shape == (T,)
        out = _C.unpack_rows_fwd(ids.float(), bdev, 6)
        assert out.shape == (len(b) - 1, 6)
        gb = _C.unpack_rows_bwd(torch.ones(len(b) - 1, 6, device=DEV), bdev, T)
        assert gb.shape == (T,) and bool(torch.all((gb == 0) | (gb == 1)))
    torch.cuda.synchronize()
    # an unpacking past the packed rows reads zeros
    out = _C.unpack_rows_fwd(ids.float(), torch.tensor([0, 40], dtype=torch.int64, device=DEV), 50)
    assert torch.equal(out[0, 16:].cpu(), torch.zeros(34))
    assert torch.equal(out[0, :16].cpu(), ids.float().cpu())
