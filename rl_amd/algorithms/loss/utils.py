"""Packing helpers: drop-in for ``_pack_input_ids`` (reference loss/utils.py:355-408) and the
``CpuIntTuple`` helpers (reference utils/sequence_lengths.py:19-31).

The reference packs with a host loop over sequences.  Here device tensors are
packed by one gfx950 kernel (``mirl_pack_sequences``) that reads the uploaded
boundaries; host tensors by the same position map built with numpy and applied
as one gather (context parallelism of size 1 in both).
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

    if dev.type == "cuda":
        # device path: the boundaries are uploaded once and one kernel packs
        # (and rolls) every position
        from rl_amd import _C

        # sequences 0 .. B-1 are packed (the reference loops over the batch rows)
        if len(cu_seqlens_q) < B + 1 or len(cu_seqlens_q_padded) < B + 1:
            raise IndexError(
                f"cu_seqlens have {len(cu_seqlens_q)} / {len(cu_seqlens_q_padded)} entries for {B} sequences"
            )
        pad = np.asarray(cu_seqlens_q_padded[: B + 1], dtype=np.int64)
        _check_padded_lengths(pad)
        q = np.asarray(cu_seqlens_q[: B + 1], dtype=np.int64)
        cu = _host_ints_to_device(np.concatenate([q, pad]), dev)
        x = input_ids.contiguous()
        if x.dtype == torch.bool:
            x = x.view(torch.uint8)
            return _C.pack_sequences(x, cu[: B + 1], cu[B + 1 :], roll_shift, total).view(torch.bool).unsqueeze(0)
        return _C.pack_sequences(x, cu[: B + 1], cu[B + 1 :], roll_shift, total).unsqueeze(0)
    # host tensors: the same map, built with numpy and applied as one gather
    src = _pack_map(cu_seqlens_q, cu_seqlens_q_padded, S, B, roll_shift)
    flat = input_ids.reshape(B * S, *tail)
    return _gather_or_zero(flat, _host_ints_to_device(src, dev)).unsqueeze(0)


def _check_padded_lengths(pad: np.ndarray) -> None:
    """A decreasing padded boundary is a negative sequence length (the reference's
    ``torch.zeros`` of that length raises the same error)."""
    plen = pad[1:] - pad[:-1]
    if np.any(plen < 0):
        raise RuntimeError(
            f"Trying to create tensor with negative dimension {int(plen.min())}: "
            "cu_seqlens_q_padded must be nondecreasing"
        )


def _pack_map(cu_q: CpuIntTuple, cu_pad: CpuIntTuple, S: int, B: int, roll_shift: int) -> np.ndarray:
    """Row of ``input_ids.reshape(B * S)`` read by each packed position (``B * S`` reads zero).

    Sequences ``0 .. B-1`` are packed; positions past ``cu_pad[B]`` stay zero.
    """
    if len(cu_q) < B + 1 or len(cu_pad) < B + 1:
        raise IndexError(f"cu_seqlens have {len(cu_q)} / {len(cu_pad)} entries for {B} sequences")
    total = int(cu_pad[-1])
    b = np.asarray(cu_pad[: B + 1], dtype=np.int64)
    q = np.asarray(cu_q[: B + 1], dtype=np.int64)
    _check_padded_lengths(b)
    starts, plen = b[:-1], b[1:] - b[:-1]
    copy_len = np.minimum(q[1:] - q[:-1], S)
    src = np.full(total, B * S, dtype=np.int64)
    if B == 0:
        return src
    # the padded segments tile [cu_pad[0], cu_pad[B]) back to back
    seq = np.repeat(np.arange(B), plen)
    pos = np.arange(b[0], b[B], dtype=np.int64)
    off = pos - starts[seq]
    if roll_shift != 0:
        off = np.mod(off - roll_shift, plen[seq])
    ok = (off < copy_len[seq]) & (pos >= 0) & (pos < total)
    src[pos[ok]] = seq[ok] * S + off[ok]
    return src
