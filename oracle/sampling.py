"""Top-k / top-p filtering and filtered logprobs, restated on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Follows
nemo_rl/algorithms/logits_sampling_utils.py:69-212 (the filter),
nemo_rl/distributed/model_utils.py:352-479 (DistributedLogprobWithSampling at
TP=1) and nemo_rl/models/automodel/train.py:248-262 (in-place temperature).

Two points follow the reference as it runs on the GPU rather than CPU torch:
- the ascending sort is stable (ties ordered by vocabulary index), which is
  what the reference's GPU sort does; CPU torch.sort is unstable, so the CPU
  reference's choice among tokens tied at the top-p boundary is arbitrary.
  The top-k set (all ties at the k-th value kept) does not depend on tie order;
- the in-place temperature ``logits.div_(T)`` is the product with
  ``fl32(1.0 / T)`` that torch's GPU division by a Python scalar computes
  (forward and autograd backward), not CPU torch's exact quotient
  (``temperature_recip``).
"""

from __future__ import annotations

from typing import Optional

import torch


def temperature_recip(temperature: float) -> torch.Tensor:
    """fl32(1.0 / T) as a 0-d fp32 tensor (the quotient formed in double, rounded once).

    The reference divides its logits by a Python float on the GPU, where torch
    evaluates ``x.div_(T)`` as ``x * fl32(1.0 / T)`` in fp32 and its autograd
    backward as ``g * fl32(1.0 / T)``; CPU torch divides exactly instead, so the
    oracle writes the product out."""
    return torch.tensor(1.0 / temperature, dtype=torch.float32)


def apply_temperature(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """logits.div_(T) in the logits dtype as the reference runs it on the GPU
    (automodel/train.py:248-262): dtype(fl32(float(x) * fl32(1.0 / T)))."""
    if temperature == 1.0:
        return logits.clone()
    return (logits.float() * temperature_recip(temperature)).to(logits.dtype)


def top_k_only(logits: torch.Tensor, top_k: int):
    """reference logits_sampling_utils.py:69-108: keep = x >= k-th largest (ties kept)."""
    vals, _ = torch.topk(logits, top_k, dim=-1)
    thr = vals[..., -1:].expand_as(logits)
    keep = logits >= thr
    return torch.where(keep, logits, torch.tensor(-float("inf"), dtype=logits.dtype)), keep


def _softmax_exact_normaliser(srt: torch.Tensor) -> torch.Tensor:
    """softmax of sorted rows with the normaliser summed in float64 and rounded
    once to fp32 (CPU torch sums it in fp32, in vector-lane order); the
    probabilities are fp32 exp * (1 / Z) for fp32 rows and exp / Z rounded to
    the dtype for 16-bit rows."""
    x = srt.float()
    e = torch.exp(x - x.amax(-1, keepdim=True))
    z = e.double().sum(-1, keepdim=True).float()
    if srt.dtype == torch.float32:
        return e * (1.0 / z)
    return (e / z).to(srt.dtype)


def top_k_top_p(logits: torch.Tensor, top_k: Optional[int], top_p: float, chunk_size: int = 256,
                exact_normaliser: bool = False):
    """reference logits_sampling_utils.py:111-212 with a stable ascending sort.

    ``exact_normaliser`` replaces the softmax's fp32 normaliser by the exactly
    rounded one (see _softmax_exact_normaliser); it isolates CPU torch's
    summation rounding from the filter's rule."""
    need_k = top_k is not None and top_k > 0
    need_p = top_p is not None and top_p != 1.0
    if not need_p:
        if not need_k:
            return logits, None
        return top_k_only(logits, top_k)
    shape = logits.shape
    V = shape[-1]
    x = logits.reshape(-1, V)
    out = torch.empty_like(x)
    keep = torch.empty(x.shape, dtype=torch.bool)
    for a in range(0, x.shape[0], chunk_size):
        b = min(a + chunk_size, x.shape[0])
        srt, idx = x[a:b].sort(dim=-1, descending=False, stable=True)
        kmask = None
        if need_k:
            thr = srt.gather(-1, torch.full(srt.shape[:-1], V - top_k, dtype=torch.long).unsqueeze(-1))
            kmask = srt >= thr
            srt = srt.masked_fill(~kmask, -float("inf"))
        probs = _softmax_exact_normaliser(srt) if exact_normaliser else srt.softmax(dim=-1)
        cum = torch.cumsum(probs, dim=-1)
        pmask = cum > 1 - top_p
        pmask[..., -1] = True
        srt = srt.masked_fill(~pmask, -float("inf"))
        out[a:b] = srt.scatter(-1, idx, srt)
        m = pmask if kmask is None else (kmask & pmask)
        keep[a:b] = m.scatter(-1, idx, m)
    return out.view(shape), keep.view(shape)


def filtered_logprobs(logits: torch.Tensor, target: torch.Tensor, top_k, top_p):
    """[B, S, V] -> [B, S] fp32: DistributedLogprobWithSampling.forward at TP=1
    (reference model_utils.py:382-432): filter, fp32 log_softmax, gather (no target
    masking: targets outside the kept set give -inf)."""
    filt, keep = top_k_top_p(logits, top_k, top_p)
    lsm = torch.log_softmax(filt.to(torch.float32), dim=-1)
    return torch.gather(lsm, -1, target.unsqueeze(-1)).squeeze(-1), keep


def filtered_logprobs_grad(logits: torch.Tensor, target: torch.Tensor, top_k, top_p, grad_output):
    """DistributedLogprobWithSampling.backward at TP=1 (reference model_utils.py:434-479):
    (onehot - softmax(filtered)) * g * keep, fp32."""
    filt, keep = top_k_top_p(logits, top_k, top_p)
    p = torch.softmax(filt.to(torch.float32), dim=-1)
    onehot = torch.nn.functional.one_hot(target, num_classes=logits.shape[-1]).float()
    g = (onehot - p) * grad_output.unsqueeze(-1).float()
    if keep is not None:
        g = g * keep
    return g


def next_token_filtered(logits_raw, input_ids, top_k, top_p, temperature=1.0, grad_output=None):
    """The full production chain for one microbatch (reference get_next_token_logprobs_from_logits,
    model_utils.py:1660-1718, no-group path): in-place temperature in the logits dtype (as
    torch runs it on the GPU, see temperature_recip), fp32
    upcast, drop the last position, filter, log_softmax, gather input_ids[:, 1:].

    Returns (logprobs [B, S-1] fp32, keep [B, S-1, V] or None, grad w.r.t. the raw logits in the
    logits dtype or None).  The gradient chain is autograd's: masked filter, fp32 -> dtype cast,
    then the division by T in the logits dtype.
    """
    x = logits_raw.clone().requires_grad_(grad_output is not None)
    # the logits-dtype division as a product with fl32(1.0 / T), rounded to the
    # dtype, and through autograd its backward, dtype(fl32(float(g) * fl32(1.0 / T)))
    if temperature != 1.0:
        y = (x.float() * temperature_recip(temperature)).to(x.dtype)
    else:
        y = x * 1
    yf = y.to(torch.float32)[:, :-1]
    with torch.no_grad():
        _, keep = top_k_top_p(yf.detach(), top_k, top_p)
    filt = yf if keep is None else torch.where(keep, yf, torch.full_like(yf, -float("inf")))
    lsm = torch.log_softmax(filt, dim=-1)
    lp = lsm.gather(-1, input_ids[:, 1:].unsqueeze(-1)).squeeze(-1)
    grad = None
    if grad_output is not None:
        (grad,) = torch.autograd.grad(lp, [x], grad_output)
    return lp.detach(), keep, grad


def top_k_top_p_candidates(logits: torch.Tensor, top_k: int, top_p: float, z_ulps: int = 0):
    """Keep masks of ``top_k_top_p(logits, top_k, top_p, exact_normaliser=True)`` for fp32
    rows, evaluated on the top-k candidates only, plus per-row statistics of the cut.

    After the top-k mask every other entry of the sorted row is -inf: it adds an exact zero
    to the normaliser and to the ascending cumulative sum, so the row reduces to its
    candidates (every value >= the k-th largest, ties included) in (value, index) order.
    ``z_ulps`` moves the normaliser by that many fp32 ulps (the sensitivity of the cut to
    the normaliser's rounding).  Returns (keep [R, V] bool, stats dict of [R] tensors:
    n_kept, group (elements equal to the smallest kept value), kept_in_group)."""
    x = logits.reshape(-1, logits.shape[-1]).float()
    R, V = x.shape
    kth = torch.topk(x, top_k, dim=-1).values[:, -1:]
    cand = x >= kth
    L = int(cand.sum(-1).max())
    vals, idx = torch.topk(x, L, dim=-1)
    # (value, index) ascending: sort by index, then stably by value
    o = idx.argsort(dim=-1)
    vals, idx = vals.gather(-1, o), idx.gather(-1, o)
    o = vals.argsort(dim=-1, stable=True)
    vals, idx = vals.gather(-1, o), idx.gather(-1, o)
    real = vals >= kth
    v = vals.masked_fill(~real, -float("inf"))
    e = torch.exp(v - v.amax(-1, keepdim=True))
    z = e.double().sum(-1, keepdim=True).float()
    for _ in range(abs(z_ulps)):
        z = torch.nextafter(z, torch.full_like(z, float("inf") if z_ulps > 0 else 0.0))
    p = e * (1.0 / z)
    cum = torch.cumsum(p, dim=-1)
    pm = cum > 1 - top_p
    pm[:, -1] = True
    pm &= real
    keep = torch.zeros((R, V), dtype=torch.bool)
    keep.scatter_(-1, idx, pm)
    vmin = torch.where(pm, vals, torch.full_like(vals, float("inf"))).amin(-1, keepdim=True)
    group = (real & (vals == vmin)).sum(-1)
    kept_in_group = (pm & (vals == vmin)).sum(-1)
    return keep.view(logits.shape), {"n_kept": pm.sum(-1), "group": group, "kept_in_group": kept_in_group}
