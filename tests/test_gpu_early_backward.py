"""The ClippedPG loss starts the logits backward early (launch_early_backward); the
backward autograd later runs checks it against the real upstream gradient on the device
(GPU).

Every case compares the logits gradient with the one obtained when the early launch is
impossible (the logprobs passed through a clone, so the loss does not see the row
kernel's output): bit-identical for the plain loss, and still exact when the guess is
wrong (a scaled loss, a second consumer of the logprobs) because the device-side check
recomputes.  Without a backward, the early buffers are released with the graph.
"""

import pytest
import torch

from rl_amd import workloads
from rl_amd.algorithms.loss import ClippedPGLossConfig, ClippedPGLossFn
from rl_amd.distributed.model_utils import from_parallel_logits_to_logprobs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def say(*a):
    print("[case]", *a, flush=True)


def _setup(seed=3):
    d = workloads.grpo_step_bf16(B=4, S=256, V=4096, prompt_len=64, resp_min=64, resp_max=150,
                                 seed=seed, device=DEV)
    logits = d["logits"]
    V = logits.shape[-1]
    with torch.no_grad():
        cur = from_parallel_logits_to_logprobs(logits, d["input_ids"], 0, V, None, inference_only=True)
    d = workloads.finish_grpo_step(d, cur)
    d["advantages"] = torch.randn(d["token_mask"].shape, device=DEV)
    gvs = d["sample_mask"].sum()
    gvt = (d["token_mask"][:, 1:] * d["sample_mask"][:, None]).sum()
    return d, gvs, gvt


def _grad(d, gvs, gvt, early: bool, extra=None, scale=1.0):
    logits = d["logits"].detach().clone().requires_grad_(True)
    V = logits.shape[-1]
    lp = from_parallel_logits_to_logprobs(logits, d["input_ids"], 0, V, None)
    feed = lp if early else lp.clone()
    fn = ClippedPGLossFn(ClippedPGLossConfig(reference_policy_kl_penalty=0.0))
    loss, _ = fn(feed, d, gvs, gvt)
    total = loss * scale
    if extra is not None:
        total = total + (lp * extra).sum()
    started = getattr(lp.grad_fn, "early", None) is not None
    (g,) = torch.autograd.grad(total, [logits])
    return g, started


def test_plain_loss_bit_identical():
    say("early backward: plain")
    d, gvs, gvt = _setup()
    g1, started = _grad(d, gvs, gvt, early=True)
    g0, started0 = _grad(d, gvs, gvt, early=False)
    assert started and not started0
    assert torch.equal(g1, g0)


@pytest.mark.parametrize("scale", [2.0, 0.5])
def test_scaled_loss_recomputes(scale):
    say("early backward: scaled", scale)
    d, gvs, gvt = _setup(4)
    g1, started = _grad(d, gvs, gvt, early=True, scale=scale)
    g0, _ = _grad(d, gvs, gvt, early=False, scale=scale)
    assert started
    assert torch.equal(g1, g0)


def test_second_consumer_recomputes():
    say("early backward: second consumer")
    d, gvs, gvt = _setup(5)
    w = torch.randn(d["input_ids"].shape[0], d["input_ids"].shape[1] - 1, device=DEV) * 1e-3
    g1, started = _grad(d, gvs, gvt, early=True, extra=w)
    g0, _ = _grad(d, gvs, gvt, early=False, extra=w)
    assert started
    assert torch.equal(g1, g0)


def test_no_backward_releases_memory():
    say("early backward: no backward")
    d, gvs, gvt = _setup(6)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(DEV)
    logits = d["logits"].detach().clone().requires_grad_(True)
    lp = from_parallel_logits_to_logprobs(logits, d["input_ids"], 0, logits.shape[-1], None)
    loss, _ = ClippedPGLossFn(ClippedPGLossConfig(reference_policy_kl_penalty=0.0))(lp, d, gvs, gvt)
    assert getattr(lp.grad_fn, "early", None) is not None
    del loss, lp, logits
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(DEV) == base
