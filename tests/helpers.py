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
