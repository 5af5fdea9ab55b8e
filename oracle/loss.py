"""ClippedPG loss restated with PyTorch autograd on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Follows the reference op
sequence of ClippedPGLossFn.__call__ (reference
nemo_rl/algorithms/loss/loss_functions.py:698-1183), clipped_pg_actor_objective
and clipped_pg_diagnostic_metrics (nemo_rl/algorithms/loss/clipped_pg.py:53-194),
calculate_kl and masked_mean (nemo_rl/algorithms/utils.py:56-115, :294-306).
Gradients come from autograd over the same ops, so they follow PyTorch's
backward rules exactly.  Pinned by the reference's float64 goldens.
"""

from __future__ import annotations

from typing import Any, Optional

import torch

DEFAULTS: dict[str, Any] = dict(
    disable_ppo_ratio=False,
    token_level_loss=True,
    sequence_level_importance_ratios=False,
    ratio_clip_min=0.2,
    ratio_clip_max=0.2,
    ratio_clip_c=None,
    reference_policy_kl_penalty=0.01,
    reference_policy_kl_type="k3",
    kl_input_clamp_value=20.0,
    kl_output_clamp_value=10.0,
    use_kl_in_reward=False,
    use_importance_sampling_correction=False,
    truncated_importance_sampling_type=None,
    truncated_importance_sampling_ratio=None,
    truncated_importance_sampling_ratio_min=None,
    truncated_importance_sampling_adaptive_outer_bound=50.0,
    adaptive_ppo_clip_k=0.0,
    use_on_policy_kl_approximation=False,
    force_on_policy_ratio=False,
    use_cispo=False,
    positive_example_nll_weight=0.0,
    metrics_level="full",
    score_centering=False,
)


def masked_mean(values, mask, dim=None, global_normalization_factor=None):
    """reference utils.py:294-306"""
    n = torch.sum(mask, dim=dim) if global_normalization_factor is None else global_normalization_factor
    return torch.sum(values * mask, dim=dim) / (n + 1e-8)


def calculate_kl(logprobs, logprobs_reference, kl_type="k3", input_clamp_value=20.0,
                 output_clamp_value=10.0, importance_sampling_weights=None):
    """reference utils.py:56-115"""
    logr = logprobs_reference - logprobs
    if input_clamp_value is not None:
        lc = logr.clamp(min=-input_clamp_value, max=input_clamp_value)
        if importance_sampling_weights is not None:
            importance_sampling_weights = torch.where(
                logr == lc, importance_sampling_weights, importance_sampling_weights.detach()
            )
        logr = lc
    if kl_type == "k1":
        kl = -logr
    elif kl_type == "k2":
        kl = torch.square(logr) / 2
    elif kl_type == "k3":
        kl = torch.exp(logr) - 1 - logr
    else:
        raise ValueError(f"Invalid KL type: {kl_type}")
    if importance_sampling_weights is not None:
        kl = importance_sampling_weights * kl
    if output_clamp_value is not None:
        kl = kl.clamp(min=-output_clamp_value, max=output_clamp_value)
    return kl


def _actor_objective(curr, prev, adv, token_mask, mask, sample_mask, iw, gvt, gvs, c):
    """reference clipped_pg.py:131-194"""
    if c["force_on_policy_ratio"]:
        ratios = (curr - curr.detach()).exp()
        ratios_clamped = ratios
    elif not c["disable_ppo_ratio"]:
        log_ratios = curr - prev
        if c["sequence_level_importance_ratios"]:
            seq = masked_mean(log_ratios, token_mask, dim=-1).unsqueeze(-1).exp()
            ratios = seq.expand(-1, adv.shape[1])
        else:
            ratios = log_ratios.exp()
        ratios_clamped = ratios.clamp(1.0 - c["ratio_clip_min"], 1.0 + c["ratio_clip_max"])
    else:
        ratios = curr
        ratios_clamped = curr
    if c["use_cispo"]:
        clip_loss = -adv * ratios_clamped.detach() * curr
    else:
        clip_loss = torch.maximum(-adv * ratios, -adv * ratios_clamped)
    rc = c["ratio_clip_c"] if c["ratio_clip_c"] is not None else -1.0
    if rc > 0:
        clip_loss = torch.where(adv < 0, torch.minimum(clip_loss, -adv * rc), clip_loss)
    vals = clip_loss if iw is None else iw * clip_loss
    if c["token_level_loss"]:
        actor = masked_mean(vals, mask, global_normalization_factor=gvt)
    else:
        actor = masked_mean(masked_mean(vals, token_mask, dim=-1), sample_mask, global_normalization_factor=gvs)
    return actor, ratios, ratios_clamped


def clipped_pg_loss(
    next_token_logprobs: torch.Tensor,
    data: dict,
    global_valid_seqs: torch.Tensor,
    global_valid_toks: torch.Tensor,
    policy_support_mask: Optional[torch.Tensor] = None,
    policy_logprobs_at_sampler_topk: Optional[torch.Tensor] = None,
    **cfg: Any,
) -> tuple[torch.Tensor, dict[str, float]]:
    """Loss and metric dict of ClippedPGLossFn.__call__ (reference loss_functions.py:698-1183)."""
    c = dict(DEFAULTS)
    c.update(cfg)
    beta = 0 if c["use_kl_in_reward"] else c["reference_policy_kl_penalty"]
    full = c["metrics_level"] == "full"
    need_iw = full or c["use_importance_sampling_correction"]
    gvt, gvs = global_valid_toks, global_valid_seqs

    curr = next_token_logprobs
    token_mask = data["token_mask"][:, 1:]
    sample_mask = data["sample_mask"]
    adv = data["advantages"][:, 1:]
    prev = None if c["force_on_policy_ratio"] else data["prev_logprobs"][:, 1:]
    gen = data["generation_logprobs"][:, 1:]
    if beta != 0:
        ref = data["reference_policy_logprobs"][:, 1:]
        cu = data.get("curr_logprobs_unfiltered", curr)

    sample_mask = sample_mask * token_mask.bool().any(dim=-1)
    mask = token_mask * sample_mask.unsqueeze(-1)
    if c["force_on_policy_ratio"]:
        prev = curr.detach()
    if policy_support_mask is not None:
        policy_support_mask = policy_support_mask & ~torch.isneginf(prev) & ~torch.isneginf(gen)

    kl_token_mask, kl_sample_mask, kl_mask = token_mask, sample_mask, mask
    kl_gen = torch.where(kl_mask.bool(), gen, 0.0)
    if beta != 0:
        cu = torch.where(kl_mask.bool(), cu, 0.0)
        ref = torch.where(kl_mask.bool(), ref, 0.0)
    if policy_support_mask is not None:
        token_mask = token_mask * policy_support_mask.to(token_mask.dtype)
        sample_mask = sample_mask * token_mask.bool().any(dim=-1).to(sample_mask.dtype)
    mask = token_mask * sample_mask.unsqueeze(-1)
    curr = torch.where(mask.bool(), curr, 0.0)
    prev = torch.where(mask.bool(), prev, 0.0)
    gen = torch.where(mask.bool(), gen, 0.0)
    if c["score_centering"]:
        adv = torch.where(mask.bool(), adv.detach(), 0.0)

    if beta != 0:
        if c["use_on_policy_kl_approximation"]:
            kiw = torch.exp(cu - kl_gen)
        else:
            kiw = torch.exp(cu - cu.detach())
        kiw = torch.nan_to_num(kiw, nan=0.0, posinf=0.0, neginf=0.0)
        kl = beta * calculate_kl(cu, ref, c["reference_policy_kl_type"], c["kl_input_clamp_value"],
                                 c["kl_output_clamp_value"], kiw)
        if c["token_level_loss"]:
            kl = masked_mean(kl, kl_mask, global_normalization_factor=gvt)
        else:
            kl = masked_mean(masked_mean(kl, kl_token_mask, dim=-1), kl_sample_mask,
                             global_normalization_factor=gvs)
    else:
        kl = curr.new_zeros(())

    filt: dict = {}
    if not need_iw:
        iw = None
    elif c["sequence_level_importance_ratios"]:
        d = ((prev - gen) * mask).sum(dim=-1)
        iw = torch.nan_to_num(torch.exp(d).detach(), nan=0.0, posinf=0.0, neginf=0.0).unsqueeze(-1)
    else:
        iw = torch.nan_to_num(torch.exp(prev - gen), nan=0.0, posinf=0.0, neginf=0.0)
    tis_ratio = c["truncated_importance_sampling_ratio"]
    tis_type = c["truncated_importance_sampling_type"]
    tis_min = c["truncated_importance_sampling_ratio_min"]
    if tis_ratio is not None:
        if tis_type == "tis":
            lo = 0.0 if tis_min is None else tis_min
            oob = (iw > tis_ratio) | (iw < lo)
            filt["is_oob_ratio"] = masked_mean(oob.float(), mask, global_normalization_factor=gvt)
            iw = torch.clamp(iw, min=lo, max=tis_ratio)
        elif tis_type == "icepop":
            kept = (iw >= tis_min) & (iw <= tis_ratio)
            filt["is_oob_ratio"] = masked_mean((~kept).float(), mask, global_normalization_factor=gvt)
            iw = torch.where(kept, iw, torch.zeros_like(iw))
        elif tis_type == "adaptive-ppo-clip":
            hi = tis_ratio + c["adaptive_ppo_clip_k"]
            outer = c["truncated_importance_sampling_adaptive_outer_bound"]
            kept = (iw <= outer) & ((adv >= 0) | (iw >= tis_min)) & ((adv <= 0) | (iw <= hi))
            filt["is_oob_ratio"] = masked_mean((~kept).float(), mask, global_normalization_factor=gvt)
            iw = torch.where(kept, iw, torch.zeros_like(iw))
        elif tis_type == "seq-mask-tis":
            lir = torch.nan_to_num(prev - gen, nan=0.0, posinf=0.0, neginf=0.0)
            g = torch.exp(masked_mean(lir, token_mask, dim=-1)).detach()
            kept = ((g >= tis_min) & (g <= tis_ratio)).float()
            filt["is_oob_ratio"] = masked_mean(1.0 - kept, sample_mask, global_normalization_factor=gvs)
            iw = iw * kept.unsqueeze(-1)
        else:
            raise ValueError(f"Invalid truncated importance sampling type: {tis_type}")

    use_iw = iw if c["use_importance_sampling_correction"] else None
    actor, ratios, ratios_c = _actor_objective(curr, prev, adv, token_mask, mask, sample_mask,
                                               use_iw, gvt, gvs, c)
    sc_metrics: dict = {}
    if c["score_centering"]:
        # reference loss_functions.py:1070-1097 with _get_score_centering_is_bounds (:659-671)
        from oracle.score_centering import score_centering_term

        mode = (tis_type or "is") if c["use_importance_sampling_correction"] else "off"
        if mode in ("tis", "icepop"):
            bounds = (tis_min or 0.0, tis_ratio)
        elif mode == "adaptive-ppo-clip":
            bounds = (tis_min, tis_ratio + c["adaptive_ppo_clip_k"])
        else:
            bounds = None
        centering, head_mass = score_centering_term(
            policy_logprobs_at_sampler_topk,
            sampler_topk_logprobs=data["sampler_topk_logprobs"][:, 1:],
            importance_sampling_mode=mode,
            is_bounds=bounds,
            token_mask=mask,
            adaptive_ppo_clip_advantages=adv,
            adaptive_ppo_clip_outer_bound=c["truncated_importance_sampling_adaptive_outer_bound"],
        )
        correction = adv * centering
        if c["token_level_loss"]:
            actor = actor + masked_mean(correction, mask, global_normalization_factor=gvt)
        else:
            actor = actor + masked_mean(masked_mean(correction, token_mask, dim=-1), sample_mask,
                                        global_normalization_factor=gvs)
        sc_metrics["score_centering_head_mass"] = masked_mean(head_mass, mask,
                                                              global_normalization_factor=gvt)
    if need_iw:
        if c["sequence_level_importance_ratios"]:
            sir = masked_mean(iw.squeeze(-1), sample_mask, global_normalization_factor=gvs)
        else:
            sir = masked_mean(iw, mask, global_normalization_factor=gvt)

    nll = curr.new_zeros(())
    mu = c["positive_example_nll_weight"]
    if mu > 0 and "rewards" in data:
        cm = mask * (data["rewards"] > 0).float().unsqueeze(-1)
        cvt = cm.sum()
        nll = torch.where(cvt > 0, masked_mean(-curr, cm, global_normalization_factor=cvt), curr.new_zeros(()))

    loss = actor + kl + mu * nll
    m: dict[str, torch.Tensor] = {"loss": loss.detach()}
    with torch.no_grad():
        m["token_mult_prob_error"] = masked_mean(torch.exp(torch.abs(gen - prev) * mask), mask,
                                                 global_normalization_factor=gvt)
        if full:
            kt = c["reference_policy_kl_type"]
            lm = torch.log(0.5 * torch.exp(prev) + 0.5 * torch.exp(gen))
            a, b = prev - lm, gen - lm
            js = 0.5 * (torch.exp(a) - a - 1) + 0.5 * (torch.exp(b) - b - 1)
            valid = mask.bool()
            m.update({
                "probs_ratio": masked_mean(ratios, mask, global_normalization_factor=gvt),
                "probs_ratio_clamped": masked_mean(ratios_c, mask, global_normalization_factor=gvt),
                "probs_ratio_min": torch.where(valid, ratios, float("inf")).min(),
                "probs_ratio_max": torch.where(valid, ratios, float("-inf")).max(),
                "probs_ratio_clamped_min": torch.where(valid, ratios_c, float("inf")).min(),
                "probs_ratio_clamped_max": torch.where(valid, ratios_c, float("-inf")).max(),
                "gen_kl_error": masked_mean(calculate_kl(gen, prev, kt, None, None), mask,
                                            global_normalization_factor=gvt),
                "policy_kl_error": masked_mean(calculate_kl(prev, gen, kt, None, None), mask,
                                               global_normalization_factor=gvt),
                "js_divergence_error": masked_mean(js, mask, global_normalization_factor=gvt),
                "approx_entropy": -masked_mean(torch.exp(curr - gen) * curr, mask,
                                               global_normalization_factor=gvt),
            })
        if need_iw:
            m["sampling_importance_ratio"] = sir
        m["kl_penalty"] = kl / beta if beta != 0 else curr.new_zeros(())
        m["num_valid_samples"] = sample_mask.sum()
        m["positive_nll_loss"] = nll
        m.update(filt)
        m.update({k: v.detach() for k, v in sc_metrics.items()})
        m["policy_support_excluded_tokens"] = (kl_mask - mask).sum()
    vals = torch.stack([v.detach().to(loss.dtype).reshape(()) for v in m.values()]).tolist()
    return loss, dict(zip(m, vals))
