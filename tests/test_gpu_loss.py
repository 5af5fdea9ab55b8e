"""gfx950 ClippedPG kernel against the reference's goldens and the CPU oracle (GPU).

fp64 runs reproduce the float64 goldens at 1e-10 (the goldens themselves hold
at 1e-12 on the CPU; GPU exp/log differ in the last ulp).  fp32 runs are
checked against the float64 goldens at 1e-5 relative, inside the 1e-4
relative loss tolerance of the contract.
"""

import zlib

import pytest
import torch

from oracle.loss import clipped_pg_loss
from rl_amd.algorithms.loss import ClippedPGLossConfig, ClippedPGLossFn
from tests.helpers import golden_case_inputs, load_goldens

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
GOLDENS = load_goldens()
CASES = GOLDENS["cases"]


def _run(case, dtype, metrics_level="full"):
    ntl, data, gvs, gvt, grad_inputs = golden_case_inputs(GOLDENS, case, dtype=dtype, device=DEV)
    fn = ClippedPGLossFn(ClippedPGLossConfig(metrics_level=metrics_level, **case["config"]))
    loss, metrics = fn(next_token_logprobs=ntl, data=data, global_valid_seqs=gvs, global_valid_toks=gvt)
    grads = torch.autograd.grad(loss, [t for _, t in grad_inputs])
    return loss, {n: g for (n, _), g in zip(grad_inputs, grads)}, metrics


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 1e-5)])
@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_goldens_full(case, dtype, tol):
    print("[case]", case["name"], dtype, flush=True)
    loss, grads, metrics = _run(case, dtype)
    exp = case["expected"]
    assert loss.item() == pytest.approx(exp["loss"], rel=tol, abs=tol)
    assert set(grads) == set(exp["gradients"])
    for n, g in grads.items():
        torch.testing.assert_close(g.double().cpu(), torch.tensor(exp["gradients"][n], dtype=torch.float64),
                                   rtol=tol, atol=tol)
    assert metrics.pop("policy_support_excluded_tokens") == 0
    assert set(metrics) == set(exp["metrics"])
    for k, v in exp["metrics"].items():
        assert metrics[k] == pytest.approx(v, rel=tol, abs=tol), k


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_goldens_minimal(case):
    loss, grads, metrics = _run(case, torch.float64, "minimal")
    exp = case["expected"]
    assert loss.item() == pytest.approx(exp["loss"], rel=1e-10, abs=1e-10)
    for n, g in grads.items():
        torch.testing.assert_close(g.cpu(), torch.tensor(exp["gradients"][n], dtype=torch.float64),
                                   rtol=1e-10, atol=1e-10)
    assert metrics.pop("policy_support_excluded_tokens") == 0
    names = {"loss", "kl_penalty", "num_valid_samples", "positive_nll_loss", "token_mult_prob_error"}
    if case["config"].get("use_importance_sampling_correction", False):
        names.add("sampling_importance_ratio")
    if case["config"].get("truncated_importance_sampling_type") is not None:
        names.add("is_oob_ratio")
    assert set(metrics) == names


RANDOM_CONFIGS = {
    "grpo_default_kl": dict(),
    "ppo_no_kl": dict(reference_policy_kl_penalty=0.0),
    "k1_seq_level": dict(reference_policy_kl_type="k1", token_level_loss=False),
    "k2_onpolicy": dict(reference_policy_kl_type="k2", use_on_policy_kl_approximation=True),
    "dual_clip_is": dict(ratio_clip_c=3.0, use_importance_sampling_correction=True),
    "gspo_tis": dict(use_importance_sampling_correction=True, sequence_level_importance_ratios=True,
                     token_level_loss=False, truncated_importance_sampling_type="tis",
                     truncated_importance_sampling_ratio=1.1),
    "icepop": dict(use_importance_sampling_correction=True, truncated_importance_sampling_type="icepop",
                   truncated_importance_sampling_ratio=1.05, truncated_importance_sampling_ratio_min=0.95),
    "seq_mask_tis": dict(use_importance_sampling_correction=True,
                         truncated_importance_sampling_type="seq-mask-tis",
                         truncated_importance_sampling_ratio=1.01,
                         truncated_importance_sampling_ratio_min=0.99),
    "adaptive": dict(use_importance_sampling_correction=True, force_on_policy_ratio=True,
                     truncated_importance_sampling_type="adaptive-ppo-clip",
                     truncated_importance_sampling_ratio=1.05,
                     truncated_importance_sampling_ratio_min=0.95),
    "cispo": dict(use_cispo=True, use_importance_sampling_correction=True),
    "reinforce": dict(disable_ppo_ratio=True),
    "vapo": dict(positive_example_nll_weight=0.3),
    "minimal_metrics": dict(metrics_level="minimal"),
}


def _random_batch(B, S, seed, support=False, unfiltered=False):
    g = torch.Generator().manual_seed(seed)
    curr = -torch.rand(B, S - 1, generator=g) * 3
    tm = (torch.rand(B, S, generator=g) > 0.3).float()
    tm[:, 0] = 0
    tm[0] = 0  # a row without tokens
    data = {
        "token_mask": tm,
        "sample_mask": (torch.rand(B, generator=g) > 0.1).float(),
        "advantages": torch.randn(B, 1, generator=g).expand(B, S).contiguous(),
        "prev_logprobs": torch.cat([torch.zeros(B, 1), curr + torch.randn(B, S - 1, generator=g) * 0.1], 1),
        "generation_logprobs": torch.cat([torch.zeros(B, 1), curr + torch.randn(B, S - 1, generator=g) * 0.1], 1),
        "reference_policy_logprobs": torch.cat([torch.zeros(B, 1), curr + torch.randn(B, S - 1, generator=g) * 0.2], 1),
        "rewards": (torch.rand(B, generator=g) > 0.5).float(),
    }
    psm = None
    if support:
        psm = torch.rand(B, S - 1, generator=g) > 0.1
        curr = torch.where(psm, curr, torch.full_like(curr, float("-inf")))
    if unfiltered:
        data["curr_logprobs_unfiltered"] = (curr.clamp(min=-5) + torch.randn(B, S - 1, generator=g) * 0.05)
    return curr, data, psm


@pytest.mark.parametrize("support,unfiltered", [(False, False), (True, True)])
@pytest.mark.parametrize("name", list(RANDOM_CONFIGS))
def test_random_batches_against_oracle(name, support, unfiltered):
    print("[case]", name, "support", support, "unfiltered", unfiltered, flush=True)
    cfg = RANDOM_CONFIGS[name]
    # a fixed seed per case (Python's str hash is salted per process)
    curr, data, psm = _random_batch(6, 97, seed=zlib.crc32(name.encode()) % 1000, support=support,
                                    unfiltered=unfiltered)
    gvs = data["sample_mask"].sum()
    gvt = (data["token_mask"][:, 1:] * data["sample_mask"][:, None]).sum()
    # oracle
    c_o = curr.double().clone().requires_grad_(True)
    d_o = {k: v.double() for k, v in data.items()}
    inputs_o = [c_o]
    if unfiltered:
        d_o["curr_logprobs_unfiltered"] = d_o["curr_logprobs_unfiltered"].requires_grad_(True)
        inputs_o.append(d_o["curr_logprobs_unfiltered"])
    loss_o, m_o = clipped_pg_loss(c_o, d_o, gvs.double(), gvt.double(), policy_support_mask=psm, **cfg)
    g_o = torch.autograd.grad(loss_o, inputs_o, allow_unused=True)
    # kernel (fp32)
    c = curr.to(DEV).requires_grad_(True)
    d = {k: v.to(DEV) for k, v in data.items()}
    inputs = [c]
    if unfiltered:
        d["curr_logprobs_unfiltered"] = d["curr_logprobs_unfiltered"].requires_grad_(True)
        inputs.append(d["curr_logprobs_unfiltered"])
    fn = ClippedPGLossFn(ClippedPGLossConfig(**cfg))
    loss, m = fn(c, d, gvs.to(DEV), gvt.to(DEV),
                 policy_support_mask=None if psm is None else psm.to(DEV))
    g = torch.autograd.grad(loss, inputs, allow_unused=True)
    assert loss.item() == pytest.approx(loss_o.item(), rel=1e-4, abs=1e-6)
    for a, b in zip(g, g_o):
        if b is None:
            assert a is None or a.abs().max() == 0
            continue
        torch.testing.assert_close(a.double().cpu(), b, rtol=1e-4, atol=1e-6)
    assert set(m) == set(m_o)
    for k, v in m_o.items():
        assert m[k] == pytest.approx(v, rel=1e-4, abs=1e-6), k


def test_grpo_workload_shape_loss():
    """The loss at the benchmark shape [8, 2048] against the oracle."""
    from rl_amd import workloads

    d = workloads.grpo_step_bf16(B=8, S=2048, V=64, seed=2)
    cur = -torch.rand(8, 2047, generator=torch.Generator().manual_seed(1)) * 8
    d = workloads.finish_grpo_step(d, cur)
    adv = torch.randn(8, 1).expand(8, 2048).contiguous()
    data = {k: d[k] for k in ("token_mask", "sample_mask", "prev_logprobs", "generation_logprobs",
                              "reference_policy_logprobs")}
    data["advantages"] = adv
    gvs = data["sample_mask"].sum()
    gvt = (data["token_mask"][:, 1:] * data["sample_mask"][:, None]).sum()
    c_o = cur.clone().requires_grad_(True)
    loss_o, m_o = clipped_pg_loss(c_o, data, gvs, gvt, reference_policy_kl_penalty=0.0)
    (g_o,) = torch.autograd.grad(loss_o, [c_o])
    c = cur.to(DEV).requires_grad_(True)
    fn = ClippedPGLossFn(ClippedPGLossConfig(reference_policy_kl_penalty=0.0))
    loss, m = fn(c, {k: v.to(DEV) for k, v in data.items()}, gvs.to(DEV), gvt.to(DEV))
    (g,) = torch.autograd.grad(loss, [c])
    assert loss.item() == pytest.approx(loss_o.item(), rel=1e-4)
    torch.testing.assert_close(g.cpu(), g_o, rtol=1e-4, atol=1e-9)
    for k, v in m_o.items():
        assert m[k] == pytest.approx(v, rel=1e-4, abs=1e-7), k


@pytest.mark.parametrize("clamped", [False, True])
@pytest.mark.parametrize("kl_type", ["k1", "k2", "k3"])
def test_fused_kl_known_answers(kl_type, clamped):
    """The kernel's KL term on the reference's calculate_kl known answers
    (tests/unit/algorithms/test_loss_functions.py:1000-1039): logprobs -1 against reference
    logprobs (0, -15, -30), no actor term (zero advantages, ratio 1); the kl_penalty metric
    is the token mean of the per-token values."""
    print("[case] fused kl", kl_type, clamped, flush=True)
    vals = {"k1": ([-1.0, 14.0, 29.0], [-1.0, 10.0, 10.0]), "k2": ([0.5, 98.0, 420.5], [0.5, 10.0, 10.0]),
            "k3": ([0.7182818, 13.0, 28.0], [0.7182818, 10.0, 10.0])}[kl_type][int(clamped)]
    curr = torch.full((1, 3), -1.0, device=DEV, requires_grad=True)
    pad = torch.zeros(1, 1, device=DEV)
    data = {
        "token_mask": torch.ones(1, 4, device=DEV),
        "sample_mask": torch.ones(1, device=DEV),
        "advantages": torch.zeros(1, 4, device=DEV),
        "prev_logprobs": torch.cat([pad, curr.detach()], 1),
        "generation_logprobs": torch.cat([pad, curr.detach()], 1),
        "reference_policy_logprobs": torch.tensor([[0.0, -0.0, -15.0, -30.0]], device=DEV),
    }
    clamps = {} if clamped else {"kl_input_clamp_value": None, "kl_output_clamp_value": None}
    fn = ClippedPGLossFn(ClippedPGLossConfig(reference_policy_kl_penalty=0.5, reference_policy_kl_type=kl_type,
                                             **clamps))
    loss, m = fn(curr, data, torch.tensor(1.0, device=DEV), torch.tensor(3.0, device=DEV))
    mean = sum(vals) / 3
    assert m["kl_penalty"] == pytest.approx(mean, rel=1e-3)
    assert loss.item() == pytest.approx(0.5 * mean, rel=1e-3)
