"""Shared test helpers: golden-case loading and tolerance checks."""

from __future__ import annotations

import copy
import json
from pathlib import Path
from typing import Any

import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "clipped_pg_loss_goldens.json"


def load_goldens() -> dict[str, Any]:
    return json.loads(GOLDEN.read_text())


def golden_case_inputs(golden: dict[str, Any], case: dict[str, Any], dtype=torch.float64, device="cpu"):
    """Build (next_token_logprobs, data, gvs, gvt, grad_inputs) the way the reference's test does
    (tests/unit/algorithms/test_clipped_pg_loss_goldens.py:129-203)."""
    inputs = copy.deepcopy(golden["base_inputs"])
    inputs.update(case.get("input_overrides", {}))

    def t(v, integer=False):
        return torch.tensor(v, dtype=torch.int64 if integer else dtype, device=device)

    ntl = t(inputs["next_token_logprobs"]).requires_grad_(True)
    data = {
        "input_ids": t(inputs["input_ids"], integer=True),
        "token_mask": t(inputs["token_mask"]),
        "sample_mask": t(inputs["sample_mask"]),
        "advantages": t(inputs["advantages"]),
        "prev_logprobs": t(inputs["prev_logprobs"]),
        "generation_logprobs": t(inputs["generation_logprobs"]),
        "reference_policy_logprobs": t(inputs["reference_policy_logprobs"]),
        "rewards": t(inputs["rewards"]),
    }
    grad_inputs = [("next_token_logprobs", ntl)]
    if "curr_logprobs_unfiltered" in inputs:
        cu = t(inputs["curr_logprobs_unfiltered"]).requires_grad_(True)
        data["curr_logprobs_unfiltered"] = cu
        grad_inputs.append(("curr_logprobs_unfiltered", cu))
    gvs = data["sample_mask"].sum()
    gvt = (data["token_mask"][:, 1:] * data["sample_mask"].unsqueeze(-1)).sum()
    return ntl, data, gvs, gvt, grad_inputs


def assert_close_or_ulp_bf16(actual: torch.Tensor, expected: torch.Tensor, atol: float):
    """bf16 gradients: |a - e| <= atol, or a and e are adjacent bf16 values.

    Rounding an fp32 gradient to bf16 can land one ulp apart when the two fp32
    values straddle a rounding boundary; one bf16 ulp at |g| ~ 4 is 0.0156.
    """
    a = actual.float().cpu()
    e = expected.float().cpu()
    diff = (a - e).abs()
    bad = diff > atol
    if bad.any():
        ai = actual.cpu().contiguous().view(torch.int16)[bad].int()
        ei = expected.cpu().to(actual.dtype).contiguous().view(torch.int16)[bad].int()
        ulps = (ai - ei).abs()
        assert int(ulps.max()) <= 1, f"{int(bad.sum())} elements off by more than 1 bf16 ulp"
    return int(bad.sum())


# Known answers of calculate_baseline_and_std_per_prompt from the reference's own tests
# (tests/unit/algorithms/test_utils.py): prompts, rewards, valid mask, leave-one-out flag,
# std_rewards, then the expected baseline, std and trivial flags (None = not pinned there).
_P23 = [[1, 2, 3], [4, 5, 6]]
ADVANTAGE_KNOWN_ANSWERS = [
    ("basic:830", [_P23[0]] * 3 + [_P23[1]] * 3, [1.0, 2, 3, 4, 5, 6], [1.0] * 6, True, None,
     [2.5, 2.0, 1.5, 5.5, 5.0, 4.5], [0.707107, 1.414214, 0.707107] * 2, None),
    ("single_generation:859", _P23, [2.5, 4.0], [1.0, 1.0], True, None, [2.5, 4.0], [0.0, 0.0], None),
    ("identical_rewards:883", [_P23[0]] * 3 + [_P23[1]] * 3, [3.0, 3, 3, 7, 7, 7], [1.0] * 6, True, None,
     [3.0, 3, 3, 7, 7, 7], [0.0] * 6, [True] * 6),
    ("trivial_leave_one_out:911", [[0]] * 8, [0.0] + [0.95] * 7, [1.0] * 8, True, None,
     None, None, [True] + [False] * 7),
    ("trivial_full_group_without_loo:974", [[0]] * 8, [0.0] + [0.95] * 7, [1.0] * 8, False, None,
     None, None, [False] * 8),
    ("trivial_from_std_rewards:954", [[0]] * 3 + [[1]] * 3, [0.0, -0.2, -1.0, 1.0, 0.0, 1.0], [1.0] * 6, False,
     [0.0, 0.0, 0.0, 1.0, 0.0, 1.0], None, [0.0, 0.0, 0.0, None, None, None], [True] * 3 + [False] * 3),
    ("mixed_prompt_sizes:991", [_P23[0]] * 2 + [_P23[1]] * 3, [1.0, 2, 4, 5, 6], [1.0] * 5, True, None,
     [2.0, 1.0, 5.5, 5.0, 4.5], [0.0, 0.0, 0.707107, 1.414214, 0.707107], None),
    ("masked_sample:1034", [_P23[0]] * 3 + [_P23[1]] * 3, [1.0, 999, 3, 4, 5, 6], [1.0, 0, 1, 1, 1, 1], True,
     None, [3.0, 4.0, 1.0, 5.5, 5.0, 4.5], [0.0, 0.0, 0.0, 0.707107, 1.414214, 0.707107], None),
    ("two_per_prompt:1063", [_P23[0]] * 2 + [_P23[1]] * 2, [1.0, 2, 3, 4], [1.0] * 4, True, None,
     [2.0, 1.0, 4.0, 3.0], [0.0] * 4, None),
    ("numerical_precision:1095", [_P23[0]] * 3 + [_P23[1]] * 3, [1e-8, 2e-8, 3e-8, 1e8, 2e8, 3e8], [1.0] * 6,
     True, None, [2.5e-8, 2e-8, 1.5e-8, 2.5e8, 2e8, 1.5e8], None, None),
]


def check_advantage_known_answer(case, baseline, std, trivial) -> None:
    """Compares one result of calculate_baseline_and_std_per_prompt with a known answer
    (rtol 1e-5, as the reference's tests; std must be finite everywhere)."""
    name, _, _, _, _, _, eb, es, et = case
    baseline, std, trivial = baseline.cpu().double(), std.cpu().double(), trivial.cpu()
    assert torch.isfinite(std).all(), name
    if eb is not None:
        assert torch.allclose(baseline, torch.tensor(eb, dtype=torch.float64), rtol=1e-5), (name, baseline)
    if es is not None:
        for i, e in enumerate(es):
            if e is None:
                assert std[i] > 0, (name, i, std)
            else:
                assert abs(std[i].item() - e) <= 1e-5 * abs(e) + 1e-8, (name, i, std)
    if et is not None:
        assert trivial.tolist() == et, (name, trivial)


def advantage_case_inputs(case, device="cpu"):
    _, prompts, rewards, valid, loo, std_rewards, _, _, _ = case
    p = torch.tensor(prompts, dtype=torch.long, device=device)
    r = torch.tensor(rewards, dtype=torch.float32, device=device)
    v = torch.tensor(valid, dtype=torch.float32, device=device)
    q = None if std_rewards is None else torch.tensor(std_rewards, dtype=torch.float32, device=device)
    return p, r, v, loo, q


def keep_from_row_info(y: torch.Tensor, info: torch.Tensor) -> torch.Tensor:
    """Keep sets [N, V] of the rows a filtered forward recorded, decoded from its row
    records (``mirl_filter_row_info``: m, logsum, v_cut, i_cut, n_kept, flags).

    ``y`` [N, V] holds the values the kernel filtered (after the temperature) as fp32
    on the CPU; ``info`` is the forward's raw record buffer for those N rows.  Kept:
    y > v_cut, or y == v_cut and, with i_cut >= 0, index >= i_cut; with i_cut < 0 (rank
    form), rank among the row's values equal to v_cut in index order >= -1 - i_cut.
    The decoded set's size is checked against n_kept."""
    rec = info.cpu().view(torch.int32).view(-1, 6)
    n = y.shape[0]
    assert rec.shape[0] == n
    v_cut = rec[:, 2].clone().view(torch.float32)
    i_cut = rec[:, 3].long()
    n_kept = rec[:, 4].long()
    V = y.shape[1]
    j = torch.arange(V)
    gt = y > v_cut[:, None]
    tie = y == v_cut[:, None]
    by_index = gt | (tie & (j[None, :] >= i_cut[:, None]))
    rank = tie.long().cumsum(-1) - 1
    by_rank = gt | (tie & (rank >= (-1 - i_cut)[:, None]))
    keep = torch.where((i_cut >= 0)[:, None], by_index, by_rank)
    assert torch.equal(keep.sum(-1), n_kept), "decoded keep set size differs from n_kept"
    return keep


def kept_lists_match(keep: torch.Tensor, info: torch.Tensor, kidx: torch.Tensor) -> int:
    """Rows whose saved kept list (ids of kept entries, for rows with at most 1024 kept
    and flags bit 2 clear) differs from the keep set; returns the number of rows checked."""
    rec = info.cpu().view(torch.int32).view(-1, 6)
    kidx = kidx.cpu()
    checked = 0
    for r in range(keep.shape[0]):
        nk, flags = int(rec[r, 4]), int(rec[r, 5])
        if nk > kidx.shape[1] or (flags & 4):
            continue
        got = torch.sort(kidx[r, :nk].long()).values
        exp = torch.nonzero(keep[r]).view(-1)
        assert torch.equal(got, exp), f"row {r}: kept list differs from the keep set"
        checked += 1
    return checked
