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
from rl_amd.distributed.early_backward import POLICY, set_early_backward
from rl_amd.distributed.model_utils import from_parallel_logits_to_logprobs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _speculate_always():
    """These cases test the device-side check, so every eligible call speculates."""
    set_early_backward("always")
    yield
    set_early_backward("adaptive")


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


@pytest.mark.parametrize("scale", [2.0, 0.5, 0.0])
def test_scaled_loss_recomputes(scale):
    """The redo rewrites the rows whose upstream gradient changed (all active rows; at
    scale 0 they become zeros) and leaves the zero-gradient rows as the early launch
    wrote them."""
    say("early backward: scaled", scale)
    d, gvs, gvt = _setup(4)
    g1, started = _grad(d, gvs, gvt, early=True, scale=scale)
    g0, _ = _grad(d, gvs, gvt, early=False, scale=scale)
    assert started
    assert torch.equal(g1, g0)


@pytest.mark.parametrize("where", ["all", "first", "last"])
def test_second_consumer_recomputes(where):
    """A second consumer of every logprob, or of only the first or the last one (a
    difference that only one checking workgroup sees)."""
    say("early backward: second consumer", where)
    d, gvs, gvt = _setup(5)
    w = torch.randn(d["input_ids"].shape[0], d["input_ids"].shape[1] - 1, device=DEV) * 1e-3
    if where != "all":
        keep = torch.zeros_like(w)
        keep.view(-1)[0 if where == "first" else -1] = 1.0
        w = w * keep
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


def _packed_setup(seed):
    """A small packed batch: 4 sequences in one padded row, bf16 logits."""
    from rl_amd.algorithms.loss.utils import _pack_input_ids

    g = torch.Generator().manual_seed(seed)
    lens, S, V = [37, 80, 5, 64], 96, 2048
    B = len(lens)
    cu, cu_pad = [0], [0]
    for n in lens:
        cu.append(cu[-1] + n)
        cu_pad.append(cu_pad[-1] + -(-n // 8) * 8)
    ids = torch.randint(0, V, (B, S), generator=g)
    mask = (torch.arange(S)[None, :] < torch.tensor(lens)[:, None]).float()
    d = {
        "input_ids": ids.to(DEV),
        "token_mask": mask.to(DEV),
        "sample_mask": torch.ones(B, device=DEV),
        "advantages": torch.randn(B, S, generator=g).to(DEV),
        "prev_logprobs": (-3.0 + 0.1 * torch.randn(B, S, generator=g)).to(DEV),
        "generation_logprobs": (-3.0 + 0.1 * torch.randn(B, S, generator=g)).to(DEV),
        "logits": (1.5 * torch.randn(1, cu_pad[-1], V, generator=g)).to(torch.bfloat16).to(DEV),
    }
    d["packed_ids"] = _pack_input_ids(d["input_ids"], tuple(cu), tuple(cu_pad))
    gvs = d["sample_mask"].sum()
    gvt = (d["token_mask"][:, 1:]).sum()
    return d, tuple(cu_pad), S, gvs, gvt


def _packed_grad(d, cu_pad, S, gvs, gvt, early: bool, scale=1.0):
    from rl_amd.distributed.model_utils import from_parallel_logits_to_logprobs_packed_sequences

    logits = d["logits"].detach().clone().requires_grad_(True)
    V = logits.shape[-1]
    lp = from_parallel_logits_to_logprobs_packed_sequences(logits, d["packed_ids"], cu_pad, S, 0, V, None)
    feed = lp if early else lp.clone()
    fn = ClippedPGLossFn(ClippedPGLossConfig(reference_policy_kl_penalty=0.0))
    loss, _ = fn(feed, d, gvs, gvt)
    started = getattr(lp.grad_fn.src, "early", None) is not None
    (g,) = torch.autograd.grad(loss * scale, [logits])
    return g, started


@pytest.mark.parametrize("scale", [1.0, 3.0])
def test_packed_sequences_early_backward(scale):
    """Packed logprobs: the early launch goes through the unpacking's backward; exact either way."""
    say("early backward: packed", scale)
    d, cu_pad, S, gvs, gvt = _packed_setup(7)
    g1, started = _packed_grad(d, cu_pad, S, gvs, gvt, early=True, scale=scale)
    g0, started0 = _packed_grad(d, cu_pad, S, gvs, gvt, early=False, scale=scale)
    assert started and not started0
    assert g0.abs().sum() > 0
    assert torch.equal(g1, g0)


def _sc_setup(seed):
    """Score-centering inputs: next-token and 5 sampler-id logprobs from one K+1-id gather."""
    from types import SimpleNamespace

    from rl_amd.algorithms.loss import LossInputType, prepare_loss_input

    d = workloads.score_centering_bf16(K=5, seed=seed, device=DEV, B=4, S=256, V=4096,
                                       prompt_len=64, resp_min=64, resp_max=150)
    probe = SimpleNamespace(input_type=LossInputType.LOGPROB, score_centering=True)
    with torch.no_grad():
        cur, _ = prepare_loss_input(d["logits"], {"input_ids": d["input_ids"],
                                                  "sampler_topk_token_ids": d["sampler_topk_token_ids"],
                                                  "sampler_topk_logprobs": d["sampler_noise"]}, probe)
    d = workloads.finish_score_centering_step(d, cur["next_token_logprobs"], cur["policy_logprobs_at_sampler_topk"])
    d["advantages"] = torch.randn(d["token_mask"].shape, device=DEV)
    gvs = d["sample_mask"].sum()
    gvt = (d["token_mask"][:, 1:] * d["sample_mask"][:, None]).sum()
    return d, gvs, gvt


def _sc_grad(d, gvs, gvt, early: bool, scale=1.0, extra=None):
    from rl_amd.algorithms.loss import prepare_loss_input

    logits = d["logits"].detach().clone().requires_grad_(True)
    fn = ClippedPGLossFn(ClippedPGLossConfig(reference_policy_kl_penalty=0.0, score_centering=True))
    batch = {k: d[k] for k in ("input_ids", "token_mask", "sample_mask", "prev_logprobs", "advantages",
                               "generation_logprobs", "sampler_topk_token_ids", "sampler_topk_logprobs")}
    li, _ = prepare_loss_input(logits, batch, fn)
    node = li["next_token_logprobs"]._mirl_gather_node
    if not early:
        li = {k: v.clone() for k, v in li.items()}  # the clones are not the gather's views
    loss, _ = fn(data=batch, global_valid_seqs=gvs, global_valid_toks=gvt, **li)
    started = getattr(node, "early", None) is not None
    total = loss * scale
    if extra is not None:
        total = total + (li["policy_logprobs_at_sampler_topk"] * extra).sum()
    (g,) = torch.autograd.grad(total, [logits])
    return g, started


@pytest.mark.parametrize("case", ["plain", "scaled", "second-consumer", "one-id"])
def test_score_centering_gather_early_backward(case):
    """The K+1-id gather's backward starts early from both gradients of the loss; the
    gather's own backward checks it on the device and recomputes when the guess is wrong."""
    say("early backward: score-centering gather", case)
    d, gvs, gvt = _sc_setup(9)
    kw = {}
    if case == "scaled":
        kw["scale"] = 0.25
    elif case == "second-consumer":
        B, S = d["input_ids"].shape
        kw["extra"] = torch.randn(B, S - 1, 5, device=DEV) * 1e-3
    elif case == "one-id":
        # one sampler id of the last token: only the last checking workgroup sees it
        B, S = d["input_ids"].shape
        extra = torch.zeros(B, S - 1, 5, device=DEV)
        extra[-1, -1, -1] = 1e-3
        kw["extra"] = extra
    g1, started = _sc_grad(d, gvs, gvt, early=True, **kw)
    g0, started0 = _sc_grad(d, gvs, gvt, early=False, **kw)
    assert started and not started0
    assert g0.abs().sum() > 0
    assert torch.equal(g1, g0)


def test_adaptive_policy_skips_after_miss():
    """Adaptive mode: a scaled loss makes the check miss; once the flags have reached the host
    the next retry_after eligible calls run the plain backward, then speculation resumes.
    Gradients are exact throughout."""
    say("early backward: adaptive policy")
    set_early_backward("adaptive", retry_after=2)
    d, gvs, gvt = _setup(8)
    g_ref, _ = _grad(d, gvs, gvt, early=False, scale=0.5)
    seen = []
    for _ in range(4):
        g, started = _grad(d, gvs, gvt, early=True, scale=0.5)
        torch.cuda.synchronize()  # the check's flags reach the host before the next decision
        seen.append(started)
        assert torch.equal(g, g_ref)
    assert seen == [True, False, False, True]
    POLICY._drain()  # read the last check too
    assert POLICY.misses == 2 and POLICY.skipped == 2
    # an unscaled loss: every check agrees, every call speculates
    set_early_backward("adaptive", retry_after=2)
    g_ref, _ = _grad(d, gvs, gvt, early=False)
    for _ in range(3):
        g, started = _grad(d, gvs, gvt, early=True)
        torch.cuda.synchronize()
        assert started and torch.equal(g, g_ref)
    assert POLICY.misses == 0


def test_never_mode_runs_plain_backward():
    say("early backward: never")
    set_early_backward("never")
    d, gvs, gvt = _setup(8)
    g_ref, _ = _grad(d, gvs, gvt, early=False)
    g, started = _grad(d, gvs, gvt, early=True)
    assert not started and torch.equal(g, g_ref)


def _misses_after(run, n=3):
    """Run `run()` n times in adaptive mode, each check's flags reaching the host before the
    next decision; the number of checks that found a different gradient."""
    for _ in range(n):
        run()
        torch.cuda.synchronize()
    POLICY._drain()
    return POLICY.misses


@pytest.mark.parametrize("path", ["rows", "packed", "score-centering"])
@pytest.mark.parametrize("scale,hint", [(8.0, 8.0), (8.0, 4.0), (0.5, 0.5), (1.0, 2.0)])
def test_loss_scale_hint(path, scale, hint):
    """A stated loss scale (set_early_backward(loss_scale=...)): with the scale the caller
    really applies, the early backward uses the scaled gradient and no check misses; with a
    wrong one every check recomputes.  The gradients are bit-identical to the plain
    backward's either way."""
    say("early backward: loss-scale hint", path, scale, hint)
    if path == "rows":
        d, gvs, gvt = _setup(10)
        run = lambda early: _grad(d, gvs, gvt, early=early, scale=scale)  # noqa: E731
    elif path == "packed":
        d, cu_pad, S, gvs, gvt = _packed_setup(11)
        run = lambda early: _packed_grad(d, cu_pad, S, gvs, gvt, early=early, scale=scale)  # noqa: E731
    else:
        d, gvs, gvt = _sc_setup(12)
        run = lambda early: _sc_grad(d, gvs, gvt, early=early, scale=scale)  # noqa: E731
    g_ref, _ = run(False)
    set_early_backward("adaptive", retry_after=0, loss_scale=hint)
    got = []

    def one():
        g, started = run(True)
        assert started
        got.append(g)

    misses = _misses_after(one)
    for g in got:
        assert torch.equal(g, g_ref)
    assert misses == (0 if hint == scale else len(got))
