"""Host logic of the packed-sequence path (CPU only): target packing, loss-input
preparation plumbing and the sequence-packing wrappers' metric reduction.

``_pack_input_ids`` on host tensors builds its position map with numpy and
applies it as one gather (device tensors go through the gfx950 packing kernel,
tested in test_gpu_packing_kernels.py), so it runs here against the oracle's
loop restatement (reference loss/utils.py:355-408).  The logprob kernels are
replaced by stand-ins where the reference's own tests do the same
(test_sequence_packing_fusion.py:44-111).
"""

import math
from types import SimpleNamespace

import pytest
import torch

from oracle.logprob import pack_input_ids
from rl_amd.algorithms.logits_sampling_utils import TrainingSamplingParams
from rl_amd.algorithms.loss import (
    SequencePackingLossWrapper,
    prepare_loss_input,
    prepare_packed_loss_input,
    wrap_loss_fn_with_input_preparation,
)
from rl_amd.algorithms.loss.interfaces import LossInputType
from rl_amd.algorithms.loss.utils import _pack_input_ids, to_cpu_int_tuple
from rl_amd.distributed.batched_data_dict import BatchedDataDict


def _ragged(seed, B, S, pad_multiple, overhang=False, tail=()):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, S + 1, (B,), generator=g).tolist()
    if overhang:
        lens[-1] = S + 3  # the packer may absorb alignment padding into the last sequence
    ids = torch.randint(1, 1000, (B, S, *tail), generator=g)
    cu, cu_pad = [0], [0]
    for n in lens:
        cu.append(cu[-1] + n)
        cu_pad.append(cu_pad[-1] + ((n + pad_multiple - 1) // pad_multiple) * pad_multiple)
    return ids, cu, cu_pad


@pytest.mark.parametrize("roll", [0, -1, 2])
@pytest.mark.parametrize("pad_multiple", [1, 4])
@pytest.mark.parametrize("tail", [(), (3,)])
def test_pack_input_ids_matches_oracle(roll, pad_multiple, tail):
    for seed in range(6):
        ids, cu, cu_pad = _ragged(seed, B=5, S=13, pad_multiple=pad_multiple, overhang=seed % 2 == 1, tail=tail)
        got = _pack_input_ids(ids, tuple(cu), tuple(cu_pad), roll_shift=roll)
        exp = pack_input_ids(ids, cu, cu_pad, roll_shift=roll)
        assert got.dtype == ids.dtype
        assert torch.equal(got, exp), (seed, cu, cu_pad)


def test_pack_input_ids_edge_cases():
    ids = torch.ones(0, 4, dtype=torch.long)
    assert _pack_input_ids(ids, (0,), (0,)).shape == (1, 0)
    ids = torch.tensor([[7, 8]])
    assert _pack_input_ids(ids, (0, 0), (0, 0), roll_shift=-1).shape == (1, 0)
    with pytest.raises(NotImplementedError):
        _pack_input_ids(ids, (0, 2), (0, 2), cp_size=2)


def test_to_cpu_int_tuple():
    assert to_cpu_int_tuple(torch.tensor([0, 3, 5], dtype=torch.int32)) == (0, 3, 5)
    assert to_cpu_int_tuple([0, 4]) == (0, 4)


@pytest.mark.parametrize("top_k", [None, 1])
def test_prepare_packed_loss_input_preserves_prepacked_layout(monkeypatch, top_k):
    """Prepacked rows keep their layout; the targets are handed over unrolled
    (as the reference's test_prepare_packed_loss_input_preserves_prepacked_layout checks)."""
    input_ids = torch.tensor([[10, 11, 12, 0, 20, 21, 0, 0]])
    data = BatchedDataDict(
        {
            "input_ids": input_ids,
            "input_lengths": torch.tensor([8]),
            "token_mask": torch.tensor([[0, 1, 1, 0, 0, 1, 0, 0]]),
            "sample_mask": torch.ones(1),
            "cu_seqlens": [torch.tensor([0, 3, 5], dtype=torch.int32)],
            "cu_seqlens_padded": [torch.tensor([0, 4, 8], dtype=torch.int32)],
        }
    )
    cu = to_cpu_int_tuple(data["cu_seqlens"][0])
    cu_pad = to_cpu_int_tuple(data["cu_seqlens_padded"][0])
    expected = torch.arange(7, dtype=torch.float32).unsqueeze(0)
    if top_k is not None:
        expected[0, 1] = -float("inf")
    call = {}

    def fake_logprobs(logits, target, padded_boundaries, unpacked_seqlen, **kwargs):
        call.update(target=target, padded_boundaries=padded_boundaries,
                    unpacked_seqlen=unpacked_seqlen, kwargs=kwargs)
        return expected.clone()

    monkeypatch.setattr(
        "rl_amd.algorithms.loss.loss_input.from_parallel_logits_to_logprobs_packed_sequences",
        fake_logprobs,
    )
    loss_input, prepared = prepare_packed_loss_input(
        logits=torch.zeros(1, 8, 4),
        data=data,
        loss_fn=SimpleNamespace(input_type=LossInputType.LOGPROB),
        cu_seqlens_q=cu,
        cu_seqlens_q_padded=cu_pad,
        vocab_parallel_rank=0,
        vocab_parallel_group=object(),
        sampling_params=TrainingSamplingParams(top_k=top_k),
    )
    assert prepared is data
    assert torch.equal(loss_input["next_token_logprobs"], expected)
    assert torch.equal(call["target"], input_ids)
    assert call["padded_boundaries"] == cu_pad
    assert call["unpacked_seqlen"] == 8
    assert call["kwargs"]["target_is_pre_rolled"] is False
    assert call["kwargs"]["return_packed_layout"] is True
    if top_k is None:
        assert "policy_support_mask" not in loss_input
    else:
        assert torch.equal(loss_input["policy_support_mask"], ~torch.isneginf(expected))


def test_prepare_packed_loss_input_unpacked_batch_and_kl_second_pass(monkeypatch):
    """Unpacked data: targets packed with the per-sequence roll; filtering + KL adds an unfiltered pass."""
    ids = torch.tensor([[1, 2, 3, 0], [4, 5, 0, 0]])
    calls = []

    def fake_logprobs(logits, target, padded_boundaries, unpacked_seqlen, **kwargs):
        calls.append((target.clone(), kwargs["sampling_params"], kwargs["target_is_pre_rolled"]))
        return torch.zeros(2, 3)

    monkeypatch.setattr(
        "rl_amd.algorithms.loss.loss_input.from_parallel_logits_to_logprobs_packed_sequences",
        fake_logprobs,
    )
    sp = TrainingSamplingParams(top_k=4, top_p=0.9)
    loss_fn = SimpleNamespace(input_type=LossInputType.LOGPROB, reference_policy_kl_penalty=0.01)
    data = BatchedDataDict({"input_ids": ids})
    loss_input, data = prepare_packed_loss_input(
        torch.zeros(1, 8, 6), data, loss_fn, (0, 3, 5), (0, 4, 8),
        vocab_parallel_rank=0, vocab_parallel_group=object(), sampling_params=sp,
    )
    assert len(calls) == 2
    assert calls[0][0].tolist() == [[2, 3, 0, 1, 5, 0, 0, 4]] and calls[0][2] is True
    assert calls[0][1] is sp and calls[1][1] is None
    assert "curr_logprobs_unfiltered" in data and "policy_support_mask" in loss_input
    # no KL penalty -> no second pass
    calls.clear()
    loss_fn.reference_policy_kl_penalty = 0
    prepare_packed_loss_input(
        torch.zeros(1, 8, 6), BatchedDataDict({"input_ids": ids}), loss_fn, (0, 3, 5), (0, 4, 8),
        vocab_parallel_rank=0, vocab_parallel_group=object(), sampling_params=sp,
    )
    assert len(calls) == 1


def test_prepare_packed_loss_input_argument_errors():
    data = BatchedDataDict({"input_ids": torch.zeros(1, 4, dtype=torch.long)})
    with pytest.raises(ValueError, match="only supports LossInputType.LOGPROB"):
        prepare_packed_loss_input(torch.zeros(1, 4, 3), data, SimpleNamespace(input_type=LossInputType.LOGIT),
                                  (0, 4), (0, 4), vocab_parallel_rank=0, vocab_parallel_group=object())
    with pytest.raises(AssertionError, match="requires vocab_parallel_group"):
        prepare_packed_loss_input(torch.zeros(1, 4, 3), data, SimpleNamespace(input_type=LossInputType.LOGPROB),
                                  (0, 4), (0, 4))


def test_prepare_loss_input_logit_and_unsupported_types():
    x = torch.zeros(1, 3, 5)
    li, d = prepare_loss_input(x, {"input_ids": torch.zeros(1, 3)}, SimpleNamespace(input_type=LossInputType.LOGIT))
    assert li["logits"] is x
    with pytest.raises(NotImplementedError):
        prepare_loss_input(x, {}, SimpleNamespace(input_type=LossInputType.DISTILLATION))


class _FakeLoss:
    """Loss stand-in: loss = sum(logprobs), metrics from the per-sequence data."""

    input_type = LossInputType.LOGPROB

    def __init__(self):
        self.seen = []

    def __call__(self, data, global_valid_seqs, global_valid_toks, next_token_logprobs):
        self.seen.append({k: v.clone() for k, v in data.items()})
        n = int(data["token_mask"].sum())
        return next_token_logprobs.sum(), {
            "loss": next_token_logprobs.sum(),
            "probs_ratio_min": torch.tensor(math.inf) if n == 0 else torch.tensor(float(n)),
            "probs_ratio_max": torch.tensor(-math.inf) if n == 0 else torch.tensor(float(n)),
            "num_valid_samples": 1.0,
        }


def _fake_prepare(logits, data, loss_fn, **kwargs):
    # logprob of row s = its first logit, for the S-1 rows of this sequence
    L = data["input_ids"].shape[1]
    return {"next_token_logprobs": logits[:, : max(L - 1, 0), 0]}, data


def test_sequence_packing_wrapper_slices_and_reduces_metrics():
    lens = [3, 0, 5]
    cu, cu_pad = (0, 3, 3, 8), (0, 4, 4, 12)
    S = 6
    ids = torch.zeros(3, S, dtype=torch.long)
    tm = torch.zeros(3, S)
    for i, n in enumerate(lens):
        tm[i, 1:n] = 1
    data = BatchedDataDict({"input_ids": ids, "token_mask": tm, "sample_mask": torch.ones(3)})
    logits = torch.arange(12, dtype=torch.float32).view(1, 12, 1).expand(1, 12, 2).contiguous()
    fake = _FakeLoss()
    w = SequencePackingLossWrapper(fake, _fake_prepare, cu, cu_pad)
    loss, metrics = w(logits, data, torch.tensor(3.0), torch.tensor(5.0))
    # sequence 0: rows 0..1 -> 0+1; sequence 1: none; sequence 2: rows 4..7 -> 4+5+6+7
    assert float(loss) == 0 + 1 + 4 + 5 + 6 + 7
    assert metrics["probs_ratio_min"] == 2.0 and metrics["probs_ratio_max"] == 4.0  # inf sentinels skipped
    assert metrics["num_valid_samples"] == 3.0
    assert [d["token_mask"].shape[1] for d in fake.seen] == [3, 0, 5]
    assert [d["sample_mask"].shape for d in fake.seen] == [torch.Size([1])] * 3


def test_wrap_loss_fn_with_input_preparation_passes_through():
    fake = _FakeLoss()
    x = torch.arange(8, dtype=torch.float32).view(1, 4, 2)
    data = {"input_ids": torch.zeros(1, 4, dtype=torch.long), "token_mask": torch.ones(1, 4)}
    loss, m = wrap_loss_fn_with_input_preparation(x, data, torch.tensor(1.0), torch.tensor(3.0), fake, _fake_prepare)
    assert float(loss) == 0 + 2 + 4
