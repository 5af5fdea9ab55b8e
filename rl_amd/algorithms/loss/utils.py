"""Packing helpers: drop-in for ``_pack_input_ids`` (reference loss/utils.py:355-408) and the
``CpuIntTuple`` helpers (reference utils/sequence_lengths.py:19-31).

The reference packs with a host loop over sequences; here the per-sequence copy
and roll are one gather on the device (context parallelism of size 1).
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np
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
    from rl_amd.distributed.model_utils import _gather_or_zero, _host_ints_to_device

    src = _pack_map(cu_seqlens_q, cu_seqlens_q_padded, S, roll_shift)
    flat = input_ids.reshape(B * S, *tail)
    return _gather_or_zero(flat, _host_ints_to_device(src, dev)).unsqueeze(0)


def _pack_map(cu_q: CpuIntTuple, cu_pad: CpuIntTuple, S: int, roll_shift: int) -> np.ndarray:
    """Row of ``input_ids.reshape(B * S)`` read by each packed position (``B * S`` reads zero)."""
    b = np.asarray(cu_pad, dtype=np.int64)
    q = np.asarray(cu_q, dtype=np.int64)
    B = b.shape[0] - 1
    total = int(b[-1])
    starts, plen = b[:-1], b[1:] - b[:-1]
    copy_len = np.minimum(q[1:] - q[:-1], S)
    src = np.full(total, B * S, dtype=np.int64)
    if B == 0 or np.any(plen < 0):
        return src
    # the padded segments tile [cu_pad[0], cu_pad[-1]) back to back
    seq = np.repeat(np.arange(B), plen)
    pos = np.arange(b[0], total, dtype=np.int64)
    off = pos - starts[seq]
    if roll_shift != 0:
        off = np.mod(off - roll_shift, plen[seq])
    ok = (off < copy_len[seq]) & (pos >= 0)
    src[pos[ok]] = seq[ok] * S + off[ok]
    return src
