"""Clipped policy-gradient loss: drop-in for ``ClippedPGLossFn`` (reference loss_functions.py:173-1183).

Construction, validation and the metric-normaliser table follow the reference
line by line (same assertions and messages).  ``__call__`` runs one fused
kernel pair over the ``[B, S-1]`` tokens that produces the loss, every metric
and the closed-form gradient with respect to ``next_token_logprobs`` (and
``curr_logprobs_unfiltered`` when it is a separate tensor).  The metrics come
back to the host in one device-to-host copy, as the reference's
``materialize_scalar_metrics`` does.

With ``score_centering`` the same kernels add the score-centering correction
(reference score_centering.py:22-129, loss_functions.py:1070-1097) and its
gradient with respect to ``policy_logprobs_at_sampler_topk``.

Unsupported options raise ``NotImplementedError``: ``opd_full`` and
``seq_logprob_error_in_loss``.
"""

from __future__ import annotations

from typing import Any, Literal, Mapping, Optional, TypedDict

import torch
from pydantic import BaseModel, Field

from rl_amd import _C
from rl_amd.algorithms.loss.interfaces import (
    LossFunction,
    LossInputType,
    LossType,
    MetricNormalizer,
)

KL_PENALTY_KEY = "kl_penalty"
APPROX_ENTROPY_KEY = "approx_entropy"


class ClippedPGLossConfig(BaseModel, extra="allow"):
    """Field-for-field copy of the reference config (reference loss_functions.py:173-260)."""

    disable_ppo_ratio: bool = False
    token_level_loss: bool = True
    sequence_level_importance_ratios: bool = False
    ratio_clip_min: float = 0.2
    ratio_clip_max: float = 0.2
    ratio_clip_c: Optional[float] = None
    reference_policy_kl_penalty: float = Field(default=0.01, ge=0, allow_inf_nan=False)
    reference_policy_kl_type: str = "k3"
    kl_input_clamp_value: Optional[float] = 20.0
    kl_output_clamp_value: Optional[float] = 10.0
    use_kl_in_reward: bool = False
    use_importance_sampling_correction: bool = False
    truncated_importance_sampling_type: Optional[str] = None
    truncated_importance_sampling_ratio: Optional[float] = None
    truncated_importance_sampling_ratio_min: Optional[float] = None
    truncated_importance_sampling_adaptive_target_entropy: float = Field(default=0.3, ge=0.0)
    truncated_importance_sampling_adaptive_k_step: float = Field(default=0.25, gt=0.0)
    truncated_importance_sampling_adaptive_k_max: float = Field(default=1.0, ge=0.0)
    truncated_importance_sampling_adaptive_outer_bound: float = Field(default=50.0, gt=0.0)
    use_on_policy_kl_approximation: bool = False
    force_on_policy_ratio: bool = False
    seq_logprob_error_in_loss: bool = False
    use_cispo: bool = False
    positive_example_nll_weight: float = 0.0
    metrics_level: Literal["full", "minimal"] = "full"
    enable_torch_compile: bool = False
    score_centering: bool = False


class ClippedPGLossDataDict(TypedDict, total=False):
    """Keys read by the loss (reference :263-275)."""

    input_ids: torch.Tensor
    advantages: torch.Tensor
    prev_logprobs: torch.Tensor
    generation_logprobs: torch.Tensor
    reference_policy_logprobs: torch.Tensor
    token_mask: torch.Tensor
    sample_mask: torch.Tensor


class ClippedPGLossFn(LossFunction):
    """PPO / GRPO / GSPO / CISPO / REINFORCE clipped policy-gradient loss with KL.

    ``L = E_t[max(-A r_t, -A clip(r_t, 1-eps_min, 1+eps_max))] + beta * KL``
    plus dual clipping, truncated importance sampling, VAPO NLL and the
    on-policy / force-on-policy variants of the reference.
    """

    input_type = LossInputType.LOGPROB

    def __init__(
        self,
        cfg: ClippedPGLossConfig,
        use_fused_linear_logprobs: bool = False,
        opd_full: Optional[Any] = None,
        *,
        seq_logprob_error_threshold: float | None = None,
    ):
        if isinstance(cfg, Mapping):
            cfg = ClippedPGLossConfig(**cfg)
        self.seq_logprob_error_in_loss = cfg.seq_logprob_error_in_loss
        self.seq_logprob_error_threshold = seq_logprob_error_threshold
        if self.seq_logprob_error_in_loss:
            if seq_logprob_error_threshold is None:
                raise ValueError(
                    "loss_fn.seq_logprob_error_in_loss requires seq_logprob_error_threshold"
                )
            if not cfg.force_on_policy_ratio or not cfg.token_level_loss:
                raise ValueError(
                    "In-loss sequence filtering requires force_on_policy_ratio and token_level_loss"
                )
            if cfg.positive_example_nll_weight != 0:
                raise ValueError("In-loss sequence filtering does not support NLL")
        self.use_fused_linear_logprobs = use_fused_linear_logprobs
        self.opd_full = opd_full if opd_full is not None and getattr(opd_full, "enabled", False) else None
        self.input_type = LossInputType.OPD_FULL if self.opd_full is not None else LossInputType.LOGPROB
        self.disable_ppo_ratio = cfg.disable_ppo_ratio
        self.ratio_clip_min = cfg.ratio_clip_min
        self.ratio_clip_max = cfg.ratio_clip_max
        self.ratio_clip_c = cfg.ratio_clip_c
        if self.ratio_clip_c is not None:
            assert self.ratio_clip_c > 1, (
                f"ratio_clip_c must exceed 1 representing a lower bound of the ratios, got {self.ratio_clip_c}."
            )
        self.reference_policy_kl_penalty = (
            cfg.reference_policy_kl_penalty if not cfg.use_kl_in_reward else 0
        )
        self.reference_policy_kl_type = cfg.reference_policy_kl_type
        self.kl_input_clamp_value = cfg.kl_input_clamp_value
        self.kl_output_clamp_value = cfg.kl_output_clamp_value
        self.use_importance_sampling_correction = cfg.use_importance_sampling_correction
        self.truncated_importance_sampling_type = cfg.truncated_importance_sampling_type
        self.truncated_importance_sampling_ratio = cfg.truncated_importance_sampling_ratio
        self.truncated_importance_sampling_ratio_min = cfg.truncated_importance_sampling_ratio_min
        self.truncated_importance_sampling_adaptive_target_entropy = (
            cfg.truncated_importance_sampling_adaptive_target_entropy
        )
        self.truncated_importance_sampling_adaptive_k_step = (
            cfg.truncated_importance_sampling_adaptive_k_step
        )
        self.truncated_importance_sampling_adaptive_k_max = (
            cfg.truncated_importance_sampling_adaptive_k_max
        )
        self.truncated_importance_sampling_adaptive_outer_bound = (
            cfg.truncated_importance_sampling_adaptive_outer_bound
        )
        self.use_on_policy_kl_approximation = cfg.use_on_policy_kl_approximation
        self.force_on_policy_ratio = cfg.force_on_policy_ratio
        self.sequence_level_importance_ratios = cfg.sequence_level_importance_ratios
        self.positive_example_nll_weight = cfg.positive_example_nll_weight
        self.metrics_level = cfg.metrics_level
        self.enable_torch_compile = cfg.enable_torch_compile
        self.loss_type = LossType.TOKEN_LEVEL if cfg.token_level_loss else LossType.SEQUENCE_LEVEL
        if self.sequence_level_importance_ratios:
            assert self.loss_type == LossType.SEQUENCE_LEVEL, (
                "sequence-level importance sampling (e.g. GSPO) is mutually exclusive with token-level loss"
            )
        self.use_cispo = cfg.use_cispo
        if self.use_cispo:
            assert not self.disable_ppo_ratio, (
                "use_cispo is incompatible with disable_ppo_ratio; "
                "CISPO needs the pi_theta/pi_theta_old ratio but disable_ppo_ratio removes it"
            )
            if self.force_on_policy_ratio:
                assert (
                    self.use_importance_sampling_correction
                    and self.truncated_importance_sampling_type == "tis"
                ), "CISPO with force_on_policy_ratio requires IS correction with TIS"
            assert not self.sequence_level_importance_ratios, (
                "use_cispo is incompatible with sequence_level_importance_ratios; "
                "CISPO uses token-level importance weights"
            )
            assert self.ratio_clip_c is None, (
                "use_cispo is incompatible with dual clipping (ratio_clip_c); "
                "the dual-clip block runs after the CISPO loss assembly and would "
                "silently overwrite it. Set ratio_clip_c=null when use_cispo=True."
            )
            assert self.loss_type == LossType.TOKEN_LEVEL, (
                "use_cispo requires token_level_loss=True (LossType.TOKEN_LEVEL)."
            )
        if self.truncated_importance_sampling_type is not None:
            assert self.use_importance_sampling_correction, (
                "truncated importance sampling is only supported when use_importance_sampling_correction is True"
            )
            assert self.truncated_importance_sampling_type in (
                "tis",
                "icepop",
                "adaptive-ppo-clip",
                "seq-mask-tis",
            ), (
                "truncated_importance_sampling_type must be 'tis', 'icepop', "
                "'adaptive-ppo-clip', or 'seq-mask-tis', "
                f"got {self.truncated_importance_sampling_type}"
            )
            assert (
                self.truncated_importance_sampling_ratio is not None
                and self.truncated_importance_sampling_ratio > 0
            ), "truncated_importance_sampling_ratio should be positive"
            if self.truncated_importance_sampling_ratio_min is not None:
                assert (
                    self.truncated_importance_sampling_ratio_min
                    <= self.truncated_importance_sampling_ratio
                ), (
                    "truncated_importance_sampling_ratio_min must be <= "
                    "truncated_importance_sampling_ratio"
                )
            if self.truncated_importance_sampling_type in ("icepop", "adaptive-ppo-clip", "seq-mask-tis"):
                assert self.truncated_importance_sampling_ratio_min is not None, (
                    "truncated_importance_sampling_ratio_min should be set when "
                    "truncated_importance_sampling_type is 'icepop', "
                    "'adaptive-ppo-clip', or 'seq-mask-tis'"
                )
            if self.truncated_importance_sampling_type == "seq-mask-tis":
                assert not self.sequence_level_importance_ratios, (
                    "seq-mask-tis uses token-level IS correction with sequence-level masking, "
                    "and is incompatible with sequence_level_importance_ratios=True"
                )
            if self.truncated_importance_sampling_type == "adaptive-ppo-clip":
                assert self.force_on_policy_ratio, (
                    "adaptive-ppo-clip is intended for async RL; set "
                    "force_on_policy_ratio=True to use it"
                )
                assert self.metrics_level == "full", (
                    "adaptive-ppo-clip adapts its upper bound from approx_entropy, "
                    "which only metrics_level='full' computes"
                )
                assert not self.sequence_level_importance_ratios, (
                    "adaptive-ppo-clip uses token-level advantage-aware filtering "
                    "and is incompatible with sequence_level_importance_ratios=True"
                )
        self.cur_adaptive_ppo_clip_k: float | None = 0.0 if self.has_adaptive_loss_state() else None
        self.score_centering = cfg.score_centering
        if self.score_centering:
            assert self.opd_full is None and not use_fused_linear_logprobs, (
                "score_centering needs the policy-gradient loss on full logits"
            )
            assert not self.sequence_level_importance_ratios and (
                not self.use_importance_sampling_correction
                or self.truncated_importance_sampling_type in (None, "tis", "icepop", "adaptive-ppo-clip")
            ), (
                "score_centering composes only with importance sampling off or "
                "token-level untruncated IS, 'tis', 'icepop', or 'adaptive-ppo-clip'"
            )
        self._score_centering_is_mode = (
            (self.truncated_importance_sampling_type or "is")
            if self.use_importance_sampling_correction
            else "off"
        )
        if self.reference_policy_kl_type not in _C.KL_TYPES and self.reference_policy_kl_penalty != 0:
            # the reference raises at call time (calculate_kl); keep that timing
            pass

        grad_normalizer = (
            MetricNormalizer.TOKENS if self.loss_type == LossType.TOKEN_LEVEL else MetricNormalizer.SEQUENCES
        )
        self.metric_normalizations: dict[str, MetricNormalizer] = {
            "loss": grad_normalizer,
            KL_PENALTY_KEY: grad_normalizer,
            "probs_ratio": MetricNormalizer.TOKENS,
            "probs_ratio_clamped": MetricNormalizer.TOKENS,
            "token_mult_prob_error": MetricNormalizer.TOKENS,
            "gen_kl_error": MetricNormalizer.TOKENS,
            "policy_kl_error": MetricNormalizer.TOKENS,
            "js_divergence_error": MetricNormalizer.TOKENS,
            APPROX_ENTROPY_KEY: MetricNormalizer.TOKENS,
            "sampling_importance_ratio": (
                MetricNormalizer.SEQUENCES if self.sequence_level_importance_ratios else MetricNormalizer.TOKENS
            ),
            "policy_support_excluded_tokens": MetricNormalizer.NONE,
            "num_valid_samples": MetricNormalizer.NONE,
            "seq_logprob_error_valid_tokens": MetricNormalizer.NONE,
            "seq_logprob_error_valid_seqs": MetricNormalizer.NONE,
            "num_masked_seqs_by_logprob_error": MetricNormalizer.NONE,
            "positive_nll_loss": MetricNormalizer.NONE,
            "probs_ratio_min": MetricNormalizer.NONE,
            "probs_ratio_max": MetricNormalizer.NONE,
            "probs_ratio_clamped_min": MetricNormalizer.NONE,
            "probs_ratio_clamped_max": MetricNormalizer.NONE,
        }
        if self.metrics_level == "minimal":
            minimal = {
                "loss",
                "kl_penalty",
                "num_valid_samples",
                "policy_support_excluded_tokens",
                "positive_nll_loss",
                "token_mult_prob_error",
            }
            if self.use_importance_sampling_correction:
                minimal.add("sampling_importance_ratio")
            if self.seq_logprob_error_in_loss:
                minimal.update(
                    {
                        "seq_logprob_error_valid_tokens",
                        "seq_logprob_error_valid_seqs",
                        "num_masked_seqs_by_logprob_error",
                    }
                )
            self.metric_normalizations = {
                k: v for k, v in self.metric_normalizations.items() if k in minimal
            }
        if self.truncated_importance_sampling_type is not None:
            self.metric_normalizations["is_oob_ratio"] = (
                MetricNormalizer.SEQUENCES
                if self.truncated_importance_sampling_type == "seq-mask-tis"
                else MetricNormalizer.TOKENS
            )
        if self.score_centering:
            self.metric_normalizations["score_centering_head_mass"] = MetricNormalizer.TOKENS

    # ---- adaptive-ppo-clip controller state (reference :637-696) --------------
    def has_adaptive_loss_state(self) -> bool:
        return self.truncated_importance_sampling_type == "adaptive-ppo-clip"

    def set_adaptive_ppo_clip_k(self, k: float) -> None:
        if not self.has_adaptive_loss_state():
            return
        self.cur_adaptive_ppo_clip_k = min(
            self.truncated_importance_sampling_adaptive_k_max, max(0.0, float(k))
        )

    def _get_adaptive_ppo_clip_bounds(self) -> tuple[float, float]:
        tis_min = self.truncated_importance_sampling_ratio_min
        tis_max = self.truncated_importance_sampling_ratio
        cur_k = self.cur_adaptive_ppo_clip_k
        assert tis_min is not None and tis_max is not None and cur_k is not None
        return tis_min, tis_max + cur_k

    def update_adaptive_loss_state(self, entropy: float) -> None:
        if not self.has_adaptive_loss_state():
            return
        cur_k = self.cur_adaptive_ppo_clip_k
        assert cur_k is not None
        target = self.truncated_importance_sampling_adaptive_target_entropy
        if entropy > target:
            cur_k -= self.truncated_importance_sampling_adaptive_k_step
        elif entropy < target:
            cur_k += self.truncated_importance_sampling_adaptive_k_step
        self.set_adaptive_ppo_clip_k(cur_k)

    def _get_score_centering_is_bounds(self) -> tuple[float, float] | None:
        """Bounds that set the score-centering head and tail masses this step (reference :659-671)."""
        if self._score_centering_is_mode in ("tis", "icepop"):
            assert self.truncated_importance_sampling_ratio is not None
            return (
                self.truncated_importance_sampling_ratio_min or 0.0,
                self.truncated_importance_sampling_ratio,
            )
        elif self._score_centering_is_mode == "adaptive-ppo-clip":
            return self._get_adaptive_ppo_clip_bounds()
        return None

    @property
    def requires_survivor_normalization(self) -> bool:
        return self.seq_logprob_error_in_loss

    # ---- kernel configuration ---------------------------------------------------
    def _kernel_config(self, has_rewards: bool, has_support: bool, has_unfiltered: bool) -> _C.PgConfig:
        if self.reference_policy_kl_penalty != 0 and self.reference_policy_kl_type not in _C.KL_TYPES:
            raise ValueError(f"Invalid KL type: {self.reference_policy_kl_type}")
        full = self.metrics_level == "full"
        c = _C.PgConfig()
        c.ratio_clip_min = float(self.ratio_clip_min)
        c.ratio_clip_max = float(self.ratio_clip_max)
        c.ratio_clip_c = float(self.ratio_clip_c) if self.ratio_clip_c is not None else -1.0
        c.kl_penalty = float(self.reference_policy_kl_penalty)
        c.has_kl_input_clamp = int(self.kl_input_clamp_value is not None)
        c.kl_input_clamp = float(self.kl_input_clamp_value or 0.0)
        c.has_kl_output_clamp = int(self.kl_output_clamp_value is not None)
        c.kl_output_clamp = float(self.kl_output_clamp_value or 0.0)
        c.kl_type = _C.KL_TYPES.get(self.reference_policy_kl_type, 3)
        tis = self.truncated_importance_sampling_type
        if self.truncated_importance_sampling_ratio is not None and tis not in _C.TIS_TYPES:
            raise ValueError(f"Invalid truncated importance sampling type: {tis}")
        if self.truncated_importance_sampling_ratio is not None and tis is None:
            raise ValueError(f"Invalid truncated importance sampling type: {tis}")
        c.tis_type = _C.TIS_TYPES[tis] if self.truncated_importance_sampling_ratio is not None else 0
        c.tis_ratio = float(self.truncated_importance_sampling_ratio or 0.0)
        c.tis_ratio_min = float(self.truncated_importance_sampling_ratio_min or 0.0)
        if tis == "adaptive-ppo-clip":
            lo, hi = self._get_adaptive_ppo_clip_bounds()
            c.tis_ratio_min = float(lo)
            c.adaptive_hi = float(hi)
        c.adaptive_outer = float(self.truncated_importance_sampling_adaptive_outer_bound)
        c.nll_weight = float(self.positive_example_nll_weight)
        c.disable_ppo_ratio = int(self.disable_ppo_ratio)
        c.token_level_loss = int(self.loss_type == LossType.TOKEN_LEVEL)
        c.sequence_level_is = int(self.sequence_level_importance_ratios)
        c.use_is_correction = int(self.use_importance_sampling_correction)
        c.use_on_policy_kl = int(self.use_on_policy_kl_approximation)
        c.force_on_policy = int(self.force_on_policy_ratio)
        c.use_cispo = int(self.use_cispo)
        c.full_metrics = int(full)
        c.need_is = int(full or self.use_importance_sampling_correction)
        c.has_rewards = int(has_rewards)
        c.has_support_mask = int(has_support)
        c.has_unfiltered = int(has_unfiltered)
        return c

    def _metric_keys(self) -> list[str]:
        full = self.metrics_level == "full"
        keys = ["loss", "token_mult_prob_error"]
        if full:
            keys += [
                "probs_ratio",
                "probs_ratio_clamped",
                "probs_ratio_min",
                "probs_ratio_max",
                "probs_ratio_clamped_min",
                "probs_ratio_clamped_max",
                "gen_kl_error",
                "policy_kl_error",
                "js_divergence_error",
                "approx_entropy",
            ]
        if full or self.use_importance_sampling_correction:
            keys.append("sampling_importance_ratio")
        keys += ["kl_penalty", "num_valid_samples", "positive_nll_loss"]
        if self.truncated_importance_sampling_ratio is not None:
            keys.append("is_oob_ratio")
        if self.score_centering:
            keys.append("score_centering_head_mass")
        keys.append("policy_support_excluded_tokens")
        return keys

    # ---- the loss -----------------------------------------------------------------
    def __call__(
        self,
        next_token_logprobs: Optional[torch.Tensor] = None,
        data: Optional[Mapping[str, Any]] = None,
        global_valid_seqs: Optional[torch.Tensor] = None,
        global_valid_toks: Optional[torch.Tensor] = None,
        opd_full_divergence: Optional[torch.Tensor] = None,
        opd_full_entropy: Optional[torch.Tensor] = None,
        opd_full_cross_entropy: Optional[torch.Tensor] = None,
        policy_support_mask: Optional[torch.Tensor] = None,
        policy_logprobs_at_sampler_topk: Optional[torch.Tensor] = None,
    ) -> tuple[torch.Tensor, dict]:
        """Scalar loss (differentiable w.r.t. ``next_token_logprobs``) and its metric dict."""
        loss, metrics, early = self._loss_on_device(
            next_token_logprobs, data, global_valid_seqs, global_valid_toks, opd_full_divergence,
            opd_full_entropy, opd_full_cross_entropy, policy_support_mask,
            policy_logprobs_at_sampler_topk,
        )
        fetch = _C.start_fetch(metrics)
        if early is not None:
            # d(loss)/d(curr) is known now (grad_loss = 1): start the logits
            # backward behind the metrics copy, before the host waits for it
            from rl_amd.distributed.model_utils import launch_early_backward, launch_early_backward_pair

            (launch_early_backward if len(early) == 2 else launch_early_backward_pair)(*early)
        return loss, self.metrics_from_values(_C.finish_fetch(fetch))

    def metrics_from_values(self, values: list) -> dict:
        """The metric dict from the kernel's metric slots (a host list)."""
        return {k: float(values[_C.PG_METRIC_SLOTS[k]]) for k in self._metric_keys()}

    def _loss_on_device(
        self,
        next_token_logprobs: Optional[torch.Tensor],
        data: Optional[Mapping[str, Any]],
        global_valid_seqs: Optional[torch.Tensor],
        global_valid_toks: Optional[torch.Tensor],
        opd_full_divergence: Optional[torch.Tensor] = None,
        opd_full_entropy: Optional[torch.Tensor] = None,
        opd_full_cross_entropy: Optional[torch.Tensor] = None,
        policy_support_mask: Optional[torch.Tensor] = None,
        policy_logprobs_at_sampler_topk: Optional[torch.Tensor] = None,
    ) -> tuple[torch.Tensor, torch.Tensor, Optional[tuple]]:
        """The loss, the device metric slots ``[MIRL_NUM_METRICS]`` and, when the early
        logits backward applies, its ``(logprobs, gradient)`` pair; nothing is synchronised."""
        assert data is not None, "ClippedPGLossFn requires data"
        assert global_valid_seqs is not None, "ClippedPGLossFn requires global_valid_seqs"
        assert global_valid_toks is not None, "ClippedPGLossFn requires global_valid_toks"
        if self.opd_full is not None:
            raise NotImplementedError("opd_full is not supported by the rl_amd loss")
        if self.seq_logprob_error_in_loss:
            raise NotImplementedError("seq_logprob_error_in_loss is not supported by the rl_amd loss")
        assert next_token_logprobs is not None, "ClippedPGLossFn requires next_token_logprobs"

        curr = next_token_logprobs
        dtype = curr.dtype if curr.dtype in (torch.float32, torch.float64) else torch.float32
        dev = curr.device

        def prep(x: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
            if x is None:
                return None
            x = torch.as_tensor(x)
            if x.dtype != dtype or x.device != dev:
                x = x.to(device=dev, dtype=dtype)
            return x

        def sl(x: torch.Tensor) -> torch.Tensor:
            return prep(x)[:, 1:]

        token_mask = sl(data["token_mask"])
        advantages = sl(data["advantages"])
        prev = None if self.force_on_policy_ratio else sl(data["prev_logprobs"])
        generation = sl(data["generation_logprobs"])
        has_kl = self.reference_policy_kl_penalty != 0
        reference = sl(data["reference_policy_logprobs"]) if has_kl else None
        unfiltered = None
        if has_kl and "curr_logprobs_unfiltered" in data:
            u = data["curr_logprobs_unfiltered"]
            if u is not curr:
                unfiltered = u if u.dtype == dtype else u.to(dtype)
        sample_mask = prep(data["sample_mask"]).contiguous()
        rewards = None
        if self.positive_example_nll_weight > 0 and "rewards" in data:
            rewards = prep(data["rewards"]).contiguous()
        support = None
        if policy_support_mask is not None:
            support = policy_support_mask.to(device=dev, dtype=torch.bool)
        gvs = prep(global_valid_seqs).reshape(())
        gvt = prep(global_valid_toks).reshape(())
        curr_k = curr if curr.dtype == dtype else curr.to(dtype)
        cfg = self._kernel_config(rewards is not None, support is not None, unfiltered is not None)
        plog = None
        sc = None
        if self.score_centering:
            assert policy_logprobs_at_sampler_topk is not None, (
                "score_centering requires policy_logprobs_at_sampler_topk from prepare_loss_input"
            )
            plog = policy_logprobs_at_sampler_topk
            if plog.dtype != dtype:
                plog = plog.to(dtype)
            qlog = data["sampler_topk_logprobs"][:, 1:]
            qlog = torch.as_tensor(qlog).to(device=dev, dtype=dtype).detach()
            if plog.dim() != 3 or tuple(plog.shape[:2]) != tuple(curr.shape):
                raise ValueError(
                    f"policy_logprobs_at_sampler_topk shape {tuple(plog.shape)} does not match "
                    f"next_token_logprobs {tuple(curr.shape)} + [k]"
                )
            if tuple(qlog.shape) != tuple(plog.shape):
                raise ValueError(
                    f"sampler_topk_logprobs[:, 1:] shape {tuple(qlog.shape)} does not match "
                    f"policy_logprobs_at_sampler_topk {tuple(plog.shape)}"
                )
            bounds = self._get_score_centering_is_bounds()
            sc = (self._score_centering_is_mode, bounds,
                  self.truncated_importance_sampling_adaptive_outer_bound, qlog)

        loss, metrics = _ClippedPGFunction.apply(
            curr_k, unfiltered, cfg, token_mask, advantages, prev, generation, reference,
            support, sample_mask, rewards, gvs, gvt, plog, sc,
        )
        early = None
        if curr_k is curr and loss.grad_fn is not None and curr.requires_grad:
            early = (curr, loss.grad_fn.grad_curr)
            if plog is not None:
                # score centering: the gradient of the sampler-id logprobs too
                early = (curr, loss.grad_fn.grad_curr, plog, loss.grad_fn.grad_plog) if (
                    plog is policy_logprobs_at_sampler_topk and plog.requires_grad) else None
        return loss, metrics.detach(), early


class _ClippedPGFunction(torch.autograd.Function):
    """Loss value + metrics from the fused kernel; backward scales the saved closed-form gradient."""

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        curr: torch.Tensor,
        unfiltered: Optional[torch.Tensor],
        cfg: _C.PgConfig,
        token_mask: torch.Tensor,
        advantages: torch.Tensor,
        prev: Optional[torch.Tensor],
        generation: torch.Tensor,
        reference: Optional[torch.Tensor],
        support: Optional[torch.Tensor],
        sample_mask: torch.Tensor,
        rewards: Optional[torch.Tensor],
        gvs: torch.Tensor,
        gvt: torch.Tensor,
        plog: Optional[torch.Tensor],
        sc: Optional[tuple],
    ):
        sc_args = None
        grad_plog = None
        if plog is not None:
            mode, bounds, outer, qlog = sc
            grad_plog = torch.empty(plog.shape, dtype=plog.dtype, device=plog.device)
            sc_args = _C.score_centering_args(mode, bounds, outer, plog, qlog, grad_plog)
        # the kernel writes the loss into its own 0-d tensor too: a copy out of
        # the metrics would sit on the stream between the loss and the early backward
        loss = torch.empty((), dtype=curr.dtype, device=curr.device)
        metrics, grad_curr, grad_unf = _C.clipped_pg(
            cfg, curr, unfiltered, token_mask, advantages, prev, generation, reference, support,
            sample_mask, rewards, gvs, gvt, sc_args, loss_out=loss,
        )
        ctx.save_for_backward(grad_curr, grad_unf, grad_plog)
        ctx.grad_curr = grad_curr  # d(loss)/d(curr) at grad_loss = 1, for launch_early_backward
        ctx.grad_plog = grad_plog
        ctx.mark_non_differentiable(metrics)
        # no zero-filled gradient for the metrics output on the way back
        ctx.set_materialize_grads(False)
        return loss, metrics

    @staticmethod
    def backward(ctx: Any, grad_loss: torch.Tensor, grad_metrics: torch.Tensor):  # type: ignore[override]
        grad_curr, grad_unf, grad_plog = ctx.saved_tensors
        if grad_loss is None:
            return (None,) * 15
        gc = grad_curr * grad_loss if ctx.needs_input_grad[0] else None
        gu = grad_unf * grad_loss if (grad_unf is not None and ctx.needs_input_grad[1]) else None
        gp = grad_plog * grad_loss if (grad_plog is not None and ctx.needs_input_grad[13]) else None
        return (gc, gu) + (None,) * 11 + (gp, None)
