"""fp32 rows (the two-pass kernel), and fp16 rows decided in fp32 (the compact kernel
over the full 65536-key table, entries holding key and count only), filtered with top-p
alone or k > 1024, against the oracle (GPU).

The oracle is the fp32 rule of ``top_k_top_p(..., exact_normaliser=True)``
(reference nemo_rl/algorithms/logits_sampling_utils.py:111-212 on the fp32
tensor that get_next_token_logprobs_from_logits filters, model_utils.py:1660-1666).
Keep sets are compared bit-exactly, decoded from the forward's row records;
logprobs within 1e-5 abs (-inf exactly where the target is dropped); gradients
within 1e-3 abs.  Row records tell which kernel finished a row: the two-pass
and compact kernels write no kept list (flags bit 2), the kernels they hand rows
over to do (flags 0), so the tests also check that ordinary rows stay on the
first kernel and that fp32 rows outside its table reach the radix kernel.
"""

import pytest
import torch

from oracle.sampling import apply_temperature, temperature_recip, top_k_top_p
from rl_amd import _C, workloads
from rl_amd.distributed.sampling import filtered_next_token_logprobs
from tests.helpers import keep_from_row_info

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

# (top_k, top_p): top-p alone at several masses, k > 1024 with and without top-p
CASES = [(None, 0.9), (None, 0.5), (None, 0.99), (None, 0.05), (2000, 0.9), (5000, 0.3), (1100, 1.0)]


def _rows(S: int, seed: int, dtype=torch.float32) -> torch.Tensor:
    """Rows shaped like the filtered workload: N(0, 1) plus a Zipf-ranked +8 boost."""
    d = workloads.general_filter_bf16(B=1, S=S, top_k=None, top_p=0.9, seed=seed, dtype=dtype)
    return d["logits"]


def _expected(y: torch.Tensor, keep: torch.Tensor, tgt: torch.Tensor, gout=None, T: float = 1.0):
    """Logprobs [N] (and the raw-logits gradient [N, V] for upstream `gout`) of the
    reference's chain on the kept sets `keep` (model_utils.py:382-479 after the
    filter): fp32 log_softmax over the kept values, gathered; gradient
    (onehot - softmax) * g on the kept set, times fl32(1 / T) (the in-place
    division's backward)."""
    filt = torch.where(keep, y, torch.full_like(y, -float("inf")))
    lsm = torch.log_softmax(filt, -1)
    lp = lsm.gather(-1, tgt[:, None])[:, 0]
    if gout is None:
        return lp, None
    oh = torch.nn.functional.one_hot(tgt, y.shape[-1]).float()
    gy = (oh - lsm.exp()) * gout[:, None] * keep
    return lp, gy * temperature_recip(T) if T != 1.0 else gy


def _check_rows(x: torch.Tensor, k, p, T: float, expect_two_pass: bool):
    """x [1, S, V] (fp32 or fp16) on the CPU: forward records, keep sets and logprobs
    against the oracle on y = dtype(x * fl32(1 / T)) upcast to fp32."""
    S, V = x.shape[1], x.shape[2]
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, V, (1, S), generator=g)
    y = apply_temperature(x, T)[0, :-1].float()
    # half the targets on the row maximum (kept), the rest uniform
    ids[0, 1::2] = y[::2].argmax(-1)
    xd = x.to(DEV)
    lp = torch.empty(1, S - 1, device=DEV)
    info, _, _ = _C.filtered_fwd(xd, ids.to(DEV)[:, 1:], T, k or 0, p, lp, torch.float32)
    _, keep_exp = top_k_top_p(y, k, p, exact_normaliser=True)
    if keep_exp is None:
        keep_exp = torch.ones_like(y, dtype=torch.bool)
    keep = keep_from_row_info(y, info)
    bad = (keep != keep_exp).any(-1).nonzero().view(-1).tolist()
    assert not bad, f"keep sets differ on rows {bad[:8]}"
    lp_o, _ = _expected(y, keep_exp, ids[0, 1:])
    lp_c = lp.cpu()[0]
    assert torch.equal(torch.isinf(lp_c), torch.isinf(lp_o))
    fin = torch.isfinite(lp_o)
    torch.testing.assert_close(lp_c[fin], lp_o[fin], rtol=0, atol=1e-5)
    flags = info.cpu().view(torch.int32).view(-1, 6)[:, 5]
    if expect_two_pass:
        assert bool((flags == 4).all()), "rows left the two-pass kernel"
    return flags


@pytest.mark.parametrize("k,p", CASES)
@pytest.mark.parametrize("T", [1.0, 0.7])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_workload_rows_keep_sets_exact(k, p, T, dtype):
    print("[case] two-pass", dtype, k, p, T, flush=True)
    x = _rows(65, seed=31 + (k or 0), dtype=dtype)
    _check_rows(x, k, p, T, expect_two_pass=True)


@pytest.mark.parametrize("k,p", [(None, 0.9), (2000, 0.9), (None, 0.5)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_exact_third_pass(k, p, dtype, monkeypatch):
    """Every row's mass below the bracket summed exactly (the pass an undecided
    bound falls back to): same keep sets."""
    print("[case] third pass", dtype, k, p, flush=True)
    monkeypatch.setenv("MIRL_F32_FILTER_EXACT_BELOW", "1")
    x = _rows(33, seed=77, dtype=dtype)
    _check_rows(x, k, p, 0.7, expect_two_pass=True)


def test_bf16_valued_rows_ties():
    """fp32 rows holding bf16 values (an upcast): every bin is one value with many
    ties, so the cut falls inside a tie group and is resolved by index."""
    print("[case] f32 ties", flush=True)
    x = _rows(33, seed=12).to(torch.bfloat16).float()
    for k, p in [(None, 0.9), (2000, 0.9), (None, 0.3)]:
        _check_rows(x, k, p, 1.0, expect_two_pass=True)


def test_rows_outside_the_table_take_the_radix_kernel():
    """Rows with -inf, a value of magnitude >= 512, or 70000 equal values are
    handed to the radix kernel; the other rows stay on the two-pass kernel."""
    print("[case] f32 handover", flush=True)
    x = _rows(9, seed=3)
    x[0, 1, 17] = -float("inf")
    x[0, 3, 5] = 600.0
    x[0, 5, :70000] = 0.25
    for k, p in [(None, 0.9), (2000, 0.9)]:
        flags = _check_rows(x, k, p, 1.0, expect_two_pass=False)
        handed = {1, 3, 5}
        for r in range(flags.numel()):
            assert (flags[r] != 4) == (r in handed), (r, int(flags[r]))


@pytest.mark.parametrize("k,p", [(None, 0.9), (3000, 0.8)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_backward_against_oracle(k, p, dtype):
    """The row backward with the two-pass kernel's index cut: gradient within 1e-3 for
    fp32 rows, 2e-3 for fp16 rows (the fp16 gradient and the division's backward round
    twice, half an fp16 ulp each)."""
    print("[case] backward", dtype, k, p, flush=True)
    x = _rows(17, seed=41, dtype=dtype)
    S, V = x.shape[1], x.shape[2]
    T = 0.7
    g = torch.Generator().manual_seed(8)
    ids = torch.randint(0, V, (1, S), generator=g)
    y = apply_temperature(x, T)[0, :-1].float()
    ids[0, 1::2] = y[::2].argmax(-1)
    gout = torch.randn(1, S - 1, generator=g)
    _, keep_exp = top_k_top_p(y, k, p, exact_normaliser=True)
    lp_o, gy = _expected(y, keep_exp, ids[0, 1:], gout[0], T)
    xd = x.to(DEV).requires_grad_(True)
    lp = filtered_next_token_logprobs(xd, ids.to(DEV), k, p, temperature=T, decision_dtype=torch.float32)
    (gr,) = torch.autograd.grad(lp, [xd], gout.to(DEV))
    fin = torch.isfinite(lp_o)
    torch.testing.assert_close(lp.detach().cpu()[0][fin], lp_o[fin], rtol=0, atol=1e-5)
    grc = gr.cpu()[0].float()
    torch.testing.assert_close(grc[:-1], gy, rtol=0, atol=1e-3 if dtype == torch.float32 else 2e-3)
    assert grc[-1].abs().max().item() == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_mask_entry_point(dtype):
    """mirl_top_k_top_p_mask on fp32 rows, and on fp16 rows decided in fp32 (top-p
    alone): the oracle's keep mask."""
    print("[case] mask", dtype, flush=True)
    x = _rows(17, seed=50, dtype=dtype)[0]
    keep_exp = top_k_top_p(x.float(), None, 0.9, exact_normaliser=True)[1]
    _, keep = _C.top_k_top_p_mask(x.to(DEV), 0, 0.9, decision_dtype=torch.float32)
    assert torch.equal(keep.cpu(), keep_exp)
