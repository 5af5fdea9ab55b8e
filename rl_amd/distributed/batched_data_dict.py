"""The microbatch container handed to the loss wrappers: the part of
``nemo_rl.distributed.batched_data_dict`` the logprob/loss path touches.

``BatchedDataDict`` (reference batched_data_dict.py:152) is a ``UserDict`` of
tensors and lists that share a leading batch dimension; the packing wrappers
only use ``slice`` (reference :998-1024), ``size`` (:1152) and ``to`` (:1163).
Nested and packed tensor types of the reference are not part of this path.
"""

from __future__ import annotations

from collections import UserDict
from typing import Any, Generic, TypeVar

import torch

DictT = TypeVar("DictT")


class BatchedDataDict(UserDict, Generic[DictT]):
    """Batch of named fields sharing dimension 0."""

    def slice(self, start: int, end: int) -> "SlicedDataDict":
        """Rows ``[start, end)`` of every field (tensors must have at least ``end`` rows)."""
        out = SlicedDataDict()
        for k, v in self.data.items():
            if isinstance(v, torch.Tensor):
                assert end <= v.shape[0], (
                    f"end: {end} is greater than the shape of the tensor: {v.shape[0]} for key: {k}"
                )
            out[k] = v[start:end]
        return out

    @property
    def size(self) -> int:
        """Batch size: the leading dimension of the first field (0 when empty)."""
        if not self.data:
            return 0
        v = next(iter(self.data.values()))
        return v.shape[0] if isinstance(v, torch.Tensor) else len(v)

    def to(self, device: str | torch.device) -> "BatchedDataDict[Any]":
        """Move every tensor field to ``device`` in place; returns self."""
        for k, v in self.data.items():
            if isinstance(v, torch.Tensor):
                self.data[k] = v.to(device)
        return self


class SlicedDataDict(BatchedDataDict):
    """A ``BatchedDataDict`` obtained by slicing another one."""
