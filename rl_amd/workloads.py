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
"""

from __future__ import annotations

from typing import Optional

import torch


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def _randn_bf16(shape, std: float, g: torch.Generator, device: Optional[torch.device]) -> torch.Tensor:
    """N(0, std^2) rounded to bf16, generated in row blocks to bound memory.

    On a GPU device the values come from a device generator seeded from `g`
    (fast); checkers copy the rows they need back to the host.
    """
    B, S, V = shape
    out = torch.empty(shape, dtype=torch.bfloat16, device=device)
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
            out[b, s0:s1].copy_(blk.to(torch.bfloat16))
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
