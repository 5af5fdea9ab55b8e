"""Packing helpers: drop-in for ``_pack_input_ids`` (reference loss/utils.py:355-408) and the
``CpuIntTuple`` helpers (reference utils/sequence_lengths.py:19-31).

The reference packs with a host loop over sequences; here the per-sequence copy
and roll are one gather on the device (context parallelism of size 1).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

CpuIntTuple = tuple[int, ...]


def to_cpu_int_tuple(values: torch.Tensor | Sequence[int]) -> CpuIntTuple:
    """Sequence metadata as a host tuple of ints (one sync for a device tensor)."""
    if torch.is_tensor(values):
        return tuple(int(v) for v in values.tolist())
    return tuple(int(v) for v in values)


def _pack_input_ids(
    input_ids: torch.Tensor,
    cu_seqlens_q: CpuIntTuple,
    cu_seqlens_q_padded: CpuIntTuple,
    cp_rank: int = 0,
    cp_size: int = 1,
    roll_shift: int = 0,
) -> torch.Tensor:
    """Pack ``[B, S, ...]`` into ``[1, T_packed, ...]`` along the padded boundaries.

    Sequence i occupies ``[cu_seqlens_q_padded[i], cu_seqlens_q_padded[i+1])``;
    its first ``min(actual_len, S)`` tokens are copied, the rest are zero, and
    the padded segment is rolled by ``roll_shift`` (``-1`` builds next-token
    targets: position p holds token p+1 of the same sequence, the last position
    wraps to the segment's first element).
    """
    if cp_size != 1:
        raise NotImplementedError("context parallelism is not supported (CP = 1)")
    dev = input_ids.device
    B, S = input_ids.shape[0], input_ids.shape[1]
    total = int(cu_seqlens_q_padded[-1])
    tail = tuple(input_ids.shape[2:])
    if B == 0 or S == 0 or total <= 0:
        return torch.zeros((1, max(total, 0), *tail), dtype=input_ids.dtype, device=dev)
    bounds = torch.tensor(cu_seqlens_q_padded, dtype=torch.int64, device=dev)
    starts, ends = bounds[:-1], bounds[1:]
    plen = ends - starts
    qb = torch.tensor(cu_seqlens_q, dtype=torch.int64, device=dev)
    copy_len = torch.clamp(qb[1:] - qb[:-1], max=S)  # real tokens copied per sequence
    pos = torch.arange(total, device=dev)
    seq = torch.bucketize(pos, ends, right=True).clamp(max=B - 1)
    inside = (pos >= starts[seq]) & (pos < ends[seq])
    off = pos - starts[seq]  # position inside the padded segment
    if roll_shift != 0:
        off = torch.remainder(off - roll_shift, plen[seq].clamp(min=1))
    valid = inside & (off >= 0) & (off < copy_len[seq])
    src = seq * S + off.clamp(min=0, max=S - 1)
    packed = input_ids.reshape(B * S, *tail)[src]
    mask = valid.view(-1, *([1] * len(tail)))
    return torch.where(mask, packed, torch.zeros_like(packed)).unsqueeze(0)
