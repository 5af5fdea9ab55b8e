"""Seeded synthetic inputs of the benchmark workloads (shapes of the GRPO hot path).

Each builder returns a dict of tensors generated on the CPU with a fixed
torch.Generator (so a CPU checker sees identical bits) and optionally moved to
a device.  Sizes default to the full workloads; tests pass smaller sizes.

* logprob_fwd_f32   logits fp32 [2, 256, 32000] ~ N(0, 2^2), uniform targets
* grpo_step_bf16    logits bf16 [8, 2048, 151936] ~ N(0, 1.5^2); one prompt x 8
                    generations, 512-token prompt (mask 0), responses of
                    U{256..1536} tokens (mask 1), right padding (mask 0);
                    rewards ~ Bernoulli(0.5); prev = current logprobs + N(0, 0.05^2)
* long_context_bf16 logits bf16 [1, 32768, 131072] ~ N(0, 1), g ~ N(0, 1)
* topk_filter_bf16  logits bf16 [4, 4096, 151936] = N(0, 1) + a +8 boost per row
                    at a Zipf(1.1)-ranked vocabulary id; temperature 0.7,
                    top_k 50, top_p 0.9; 90% of targets from the row's kept set,
                    10% outside it (those rows get a zero upstream gradient)
* packed_grpo_kl_bf16 64 sequences of U{64..1024} tokens packed into logits bf16
                    [1, ~34.8k, 256000] ~ N(0, 1.5^2); 8 prompts x 8 generations,
                    rewards ~ Bernoulli(0.3); reference = current + N(0, 0.1^2)
* distill_rkl_bf16  student and teacher logits bf16 [8, 2048, 151936], both
                    ~ N(0, 1.5^2); the GRPO batch's response mask (512-token
                    prompt, U{256..1536} response tokens, padding)
* score_centering_bf16 the GRPO step plus 20 sampler top-k ids per position
                    (the sampled token first, then uniform ids); the sampler's
                    log-probs are the current ones + N(0, 0.05^2) (see
                    finish_score_centering_step)
* linear_ce_bf16    hidden states bf16 [2048, 8, 4096] ~ N(0, 1) and an LM-head
                    weight bf16 [151936, 4096] ~ N(0, (1.5 / 64)^2) (logits
                    ~ N(0, 1.5^2)); uniform token ids; upstream gradient zero on
                    the 512 prompt positions and the padding, N(0, 1) on
                    U{256..1536} response positions
"""

from __future__ import annotations

from typing import Optional

import torch


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def _randn_bf16(shape, std: float, g: torch.Generator, device: Optional[torch.device],
                dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """N(0, std^2) rounded to `dtype` (bf16 by default), generated in row blocks to
    bound memory.

    On a GPU device the values come from a device generator seeded from `g`
    (fast); checkers copy the rows they need back to the host.
    """
    B, S, V = shape
    out = torch.empty(shape, dtype=dtype, device=device)
    step = max(1, (1 << 26) // V)  # ~64M elements per block
    dev = torch.device(device) if device is not None else torch.device("cpu")
    if dev.type == "cuda":
        gd = torch.Generator(device=dev).manual_seed(int(torch.randint(0, 2**62, (1,), generator=g)))
    else:
        gd = g
    for b in range(B):
        for s0 in range(0, S, step):
            s1 = min(S, s0 + step)
            blk = torch.randn((s1 - s0, V), generator=gd, device=dev) * std
            out[b, s0:s1].copy_(blk.to(dtype))
    return out


def logprob_fwd_f32(B: int = 2, S: int = 256, V: int = 32000, seed: int = 0, device=None):
    g = _gen(seed)
    logits = (torch.randn((B, S, V), generator=g) * 2.0).to(device)
    ids = torch.randint(0, V, (B, S), generator=g).to(device)
    return {"logits": logits, "input_ids": ids}


def grpo_step_bf16(
    B: int = 8,
    S: int = 2048,
    V: int = 151936,
    prompt_len: int = 512,
    resp_min: int = 256,
    resp_max: int = 1536,
    seed: int = 2,
    device=None,
):
    """Inputs of one GRPO ClippedPG step except prev/generation logprobs (see finish_grpo_step)."""
    g = _gen(seed)
    logits = _randn_bf16((B, S, V), 1.5, g, device)
    ids = torch.randint(0, V, (B, S), generator=g)
    lens = torch.randint(resp_min, resp_max + 1, (B,), generator=g)
    pos = torch.arange(S).unsqueeze(0)
    token_mask = ((pos >= prompt_len) & (pos < prompt_len + lens.unsqueeze(1))).float()
    rewards = torch.bernoulli(torch.full((B,), 0.5), generator=g)
    noise = torch.randn((B, S), generator=g) * 0.05
    out = {
        "logits": logits,
        "input_ids": ids,
        "token_mask": token_mask,
        "sample_mask": torch.ones(B),
        "rewards": rewards,
        "prompt_ids": torch.zeros((B, 1), dtype=torch.int64),
        "prev_noise": noise,
        "response_lengths": lens,
    }
    return {k: (v.to(device) if k != "logits" else v) for k, v in out.items()}


def finish_grpo_step(data: dict, current_logprobs: torch.Tensor) -> dict:
    """prev = generation = current + noise; reference = prev (the KL term is off for this workload)."""
    B, S = data["input_ids"].shape
    prev = torch.zeros((B, S), dtype=torch.float32, device=current_logprobs.device)
    prev[:, 1:] = current_logprobs.detach().float() + data["prev_noise"][:, 1:].to(current_logprobs.device)
    data = dict(data)
    data["prev_logprobs"] = prev
    data["generation_logprobs"] = prev.clone()
    data["reference_policy_logprobs"] = prev.clone()
    return data


def long_context_bf16(B: int = 1, S: int = 32768, V: int = 131072, seed: int = 3, device=None):
    g = _gen(seed)
    logits = _randn_bf16((B, S, V), 1.0, g, device)
    ids = torch.randint(0, V, (B, S), generator=g).to(device)
    grad = torch.randn((B, S - 1), generator=g).to(device)
    return {"logits": logits, "input_ids": ids, "grad": grad}


def _recip(temperature: float, dev) -> torch.Tensor:
    """fl32(1.0 / T): the in-place temperature on the GPU multiplies by it."""
    return torch.tensor(1.0 / temperature, dtype=torch.float32, device=dev)


def topk_filter_bf16(
    B: int = 4,
    S: int = 4096,
    V: int = 151936,
    temperature: float = 0.7,
    top_k: int = 50,
    top_p: float = 0.9,
    seed: int = 4,
    device=None,
):
    g = _gen(seed)
    dev = torch.device(device) if device is not None else torch.device("cpu")
    logits = _randn_bf16((B, S, V), 1.0, g, device)
    perm = torch.randperm(V, generator=g)
    ranks = torch.arange(1, V + 1, dtype=torch.float64)
    w = ranks.pow(-1.1)
    pick = torch.multinomial(w, B * S, replacement=True, generator=g)  # rank - 1
    boost_idx = perm[pick].view(B, S).to(dev)
    flat = logits.view(B * S, V)
    rows = torch.arange(B * S, device=dev)
    flat[rows, boost_idx.view(-1)] = (flat[rows, boost_idx.view(-1)].float() + 8.0).to(torch.bfloat16)
    # the kept set of each row (top-k, then the top-p nucleus over it), used only
    # to choose targets: 90% inside it, 10% outside
    y = (flat.float() * _recip(temperature, dev)).to(torch.bfloat16).float()
    vals, idx = torch.topk(y, top_k, dim=-1)  # descending
    p = torch.softmax(vals.double(), -1)
    asc_cum = torch.cumsum(p.flip(-1), -1).flip(-1)  # mass of each element and everything below it
    nucleus = (asc_cum > 1 - top_p)
    nucleus[:, 0] = True
    n_in = nucleus.sum(-1)
    u = torch.rand(B * S, generator=g).to(dev)
    choose = (u * n_in).long().clamp(max=top_k - 1)
    inside = idx.gather(1, choose.unsqueeze(1)).squeeze(1)
    outside = torch.randint(0, V, (B * S,), generator=g).to(dev)
    use_inside = torch.rand(B * S, generator=g).to(dev) < 0.9
    tgt = torch.where(use_inside, inside, outside).view(B, S)
    ids = torch.roll(tgt, shifts=1, dims=1)  # ids[:, 1:] are the targets of rows 0..S-2
    grad = torch.randn((B, S - 1), generator=g).to(dev) * use_inside.view(B, S)[:, :-1].float()
    return {"logits": logits, "input_ids": ids, "grad": grad, "temperature": temperature,
            "top_k": top_k, "top_p": top_p}


def general_filter_bf16(
    B: int = 4,
    S: int = 4096,
    V: int = 151936,
    temperature: float = 0.7,
    top_k: Optional[int] = None,
    top_p: float = 0.9,
    seed: int = 9,
    device=None,
    dtype: torch.dtype = torch.bfloat16,
):
    """Logits shaped like the filtered workload (N(0, 1) plus one Zipf-ranked +8
    boost per row) for filters that keep large sets (top-p alone, k = 2000);
    targets 90% uniform over each row's kept set (found with a descending sort
    in chunks of 512 rows), 10% uniform over the vocabulary.  `dtype` is the
    logits dtype (bf16, fp16 or fp32)."""
    g = _gen(seed)
    dev = torch.device(device) if device is not None else torch.device("cpu")
    logits = _randn_bf16((B, S, V), 1.0, g, device, dtype)
    perm = torch.randperm(V, generator=g)
    ranks = torch.arange(1, V + 1, dtype=torch.float64)
    pick = torch.multinomial(ranks.pow(-1.1), B * S, replacement=True, generator=g)
    boost_idx = perm[pick].view(B, S).to(dev)
    flat = logits.view(B * S, V)
    rows = torch.arange(B * S, device=dev)
    flat[rows, boost_idx.view(-1)] = (flat[rows, boost_idx.view(-1)].float() + 8.0).to(dtype)
    u = torch.rand(B * S, generator=g).to(dev)
    outside = torch.randint(0, V, (B * S,), generator=g).to(dev)
    use_inside = torch.rand(B * S, generator=g).to(dev) < 0.9
    inside = torch.empty(B * S, dtype=torch.long, device=dev)
    for a in range(0, B * S, 512):
        y = (flat[a : a + 512].float() * _recip(temperature, dev)).to(dtype).float()
        vals, idx = torch.sort(y, dim=-1, descending=True)
        n_in = torch.full((vals.shape[0],), V, device=dev)
        if top_k is not None and top_k > 0:
            n_in = torch.clamp(n_in, max=top_k)
            vals = torch.where(torch.arange(V, device=dev) < top_k, vals, torch.full_like(vals, -float("inf")))
        p = torch.softmax(vals.double(), -1)
        below = 1.0 - torch.cumsum(p, -1) + p  # mass of each element and everything after it
        n_in = torch.minimum(n_in, (below > 1 - top_p).sum(-1).clamp(min=1))
        choose = (u[a : a + 512] * n_in).long().clamp(max=V - 1)
        inside[a : a + 512] = idx.gather(1, choose.unsqueeze(1)).squeeze(1)
        del y, vals, idx, p, below
    tgt = torch.where(use_inside, inside, outside).view(B, S)
    ids = torch.roll(tgt, shifts=1, dims=1)
    grad = torch.randn((B, S - 1), generator=g).to(dev) * use_inside.view(B, S)[:, :-1].float()
    return {"logits": logits, "input_ids": ids, "grad": grad, "temperature": temperature,
            "top_k": top_k, "top_p": top_p}


def packed_grpo_kl_bf16(
    n_seq: int = 64,
    len_min: int = 64,
    len_max: int = 1024,
    V: int = 256000,
    group_size: int = 8,
    seed: int = 5,
    device=None,
):
    """Packed GRPO step with a k3 KL penalty: one row [1, T, V] of n_seq sequences.

    Sequence lengths ~ U{len_min..len_max}, packed back to back (cu_seqlens is
    the cumulative sum, no padding); logits bf16 ~ N(0, 1.5^2); token ids
    uniform; token_mask is 1 on every position but the first of a sequence;
    n_seq / group_size prompts x group_size generations, rewards ~
    Bernoulli(0.3).  The reference-policy noise ~ N(0, 0.1^2) is applied by
    finish_packed_grpo_step once the current logprobs are known.
    """
    g = _gen(seed)
    lens = torch.randint(len_min, len_max + 1, (n_seq,), generator=g)
    cu = [0]
    for n in lens.tolist():
        cu.append(cu[-1] + n)
    T, S = cu[-1], int(lens.max())
    logits = _randn_bf16((1, T, V), 1.5, g, device)
    pos = torch.arange(S).unsqueeze(0)
    live = pos < lens.unsqueeze(1)
    ids = torch.randint(0, V, (n_seq, S), generator=g) * live
    token_mask = (live & (pos > 0)).float()
    rewards = torch.bernoulli(torch.full((n_seq,), 0.3), generator=g)
    prompt_ids = (torch.arange(n_seq) // group_size).unsqueeze(1)
    ref_noise = torch.randn((n_seq, S), generator=g) * 0.1
    out = {
        "input_ids": ids,
        "input_lengths": lens,
        "token_mask": token_mask,
        "sample_mask": torch.ones(n_seq),
        "rewards": rewards,
        "prompt_ids": prompt_ids,
        "ref_noise": ref_noise,
    }
    out = {k: v.to(device) for k, v in out.items()}
    out["logits"] = logits
    out["cu_seqlens"] = tuple(cu)
    return out


def finish_packed_grpo_step(data: dict, current_logprobs: torch.Tensor) -> dict:
    """generation = prev = current (on policy); reference = current + noise; [B, S-1] -> [B, S]."""
    B, S = data["input_ids"].shape
    cur = torch.zeros((B, S), dtype=torch.float32, device=current_logprobs.device)
    cur[:, 1:] = current_logprobs.detach().float()
    data = dict(data)
    data["prev_logprobs"] = cur
    data["generation_logprobs"] = cur.clone()
    data["reference_policy_logprobs"] = cur + data["ref_noise"].to(cur.device)
    return data


def linear_ce_bf16(
    S: int = 2048,
    B: int = 8,
    H: int = 4096,
    V: int = 151936,
    prompt_len: int = 512,
    resp_min: int = 256,
    resp_max: int = 1536,
    seed: int = 6,
    device=None,
):
    """Inputs of the hidden-state logprob path (Megatron's sequence-first [S, B, H] layout)."""
    g = _gen(seed)
    hidden = _randn_bf16((S, B, H), 1.0, g, device)
    weight = _randn_bf16((1, V, H), 1.5 / H**0.5, g, device)[0]
    ids = torch.randint(0, V, (B, S), generator=g)
    lens = torch.randint(resp_min, resp_max + 1, (B,), generator=g)
    pos = torch.arange(S).unsqueeze(0)
    live = (pos >= prompt_len) & (pos < prompt_len + lens.unsqueeze(1))
    grad = torch.randn((B, S - 1), generator=g) * live[:, 1:].float()
    return {"hidden": hidden, "weight": weight, "input_ids": ids.to(device), "grad": grad.to(device)}


def _response_mask(B, S, prompt_len, resp_min, resp_max, g):
    lens = torch.randint(resp_min, resp_max + 1, (B,), generator=g)
    pos = torch.arange(S).unsqueeze(0)
    return ((pos >= prompt_len) & (pos < prompt_len + lens.unsqueeze(1))).float()


def distill_rkl_bf16(
    B: int = 8,
    S: int = 2048,
    V: int = 151936,
    prompt_len: int = 512,
    resp_min: int = 256,
    resp_max: int = 1536,
    seed: int = 7,
    device=None,
):
    """Student/teacher logits of a full-vocabulary reverse-KL distillation step."""
    g = _gen(seed)
    student = _randn_bf16((B, S, V), 1.5, g, device)
    teacher = _randn_bf16((B, S, V), 1.5, g, device)
    token_mask = _response_mask(B, S, prompt_len, resp_min, resp_max, g)
    return {"student": student, "teacher": teacher, "token_mask": token_mask.to(device)}


def score_centering_bf16(K: int = 20, seed: int = 8, device=None, **grpo_kw):
    """The GRPO step's inputs plus sampler top-k ids [B, S, K] (id 0 = the sampled token)."""
    data = grpo_step_bf16(device=device, **grpo_kw)
    g = _gen(seed)
    B, S = data["input_ids"].shape
    V = data["logits"].shape[-1]
    ids = torch.randint(0, V, (B, S, K), generator=g).to(data["input_ids"].device)
    ids[..., 0] = data["input_ids"]
    data["sampler_topk_token_ids"] = ids
    data["sampler_noise"] = (torch.randn((B, S, K), generator=g) * 0.05).to(ids.device)
    return data


def finish_score_centering_step(data: dict, current_logprobs: torch.Tensor,
                                current_topk_logprobs: torch.Tensor) -> dict:
    """finish_grpo_step plus sampler log-probs = current top-k log-probs + noise, [B, S, K]."""
    data = finish_grpo_step(data, current_logprobs)
    B, S, K = data["sampler_topk_token_ids"].shape
    q = torch.zeros((B, S, K), dtype=torch.float32, device=current_topk_logprobs.device)
    q[:, 1:] = current_topk_logprobs.detach().float() + data["sampler_noise"][:, 1:]
    data["sampler_topk_logprobs"] = q
    return data
