"""Benchmark of the GRPO logprob + ClippedPG-loss forward/backward step on one MI355X.

Workload (one "step" = one pass of the hot path over one batch):
  bf16 logits [B=8, S=2048, V=151936] ~ N(0, 1.5^2), one prompt x 8 generations,
  512-token prompt (mask 0), responses U{256..1536} (mask 1), right padding;
  GRPO advantages (rewards ~ Bernoulli(0.5), group mean/std, no leave-one-out);
  prev = generation = current logprobs + N(0, 0.05^2); ClippedPG with clip
  0.2/0.2, token-level masked mean, no KL term.
  step = advantages -> next-token logprobs (fwd) -> loss fwd+bwd -> logprob bwd
  through the drop-in API (torch autograd), inputs resident in HBM.

Prints one JSON line.  `value` is next-token rows (tokens) per second for the
whole step; `roofline` is the dominant kernel (the logprob backward) measured
with HIP events around each of its launches inside the timed region;
`cpu_baseline` times the CPU oracle (a restatement of the reference's PyTorch
op sequence) on a bounded sample of the same workload.

`--workload` selects another workload of the same path for its kernel
roofline (the default line above is the headline measurement):
  fwd_f32      logprob forward only, fp32 [2, 256, 32000] (8 rotating input copies)
  long_context chunked logprob fwd+bwd, bf16 [1, 32768, 131072], chunk 4096
  topk_filter  filtered logprob fwd+bwd, bf16 [4, 4096, 151936], T=0.7, k=50, p=0.9,
               through the reference's call shape: the model's logits divided in place
               (apply_temperature_scaling), get_next_token_logprobs_from_logits with the
               sampling params, backward to the raw logits
  topk_filter_fused  the same rows with the temperature fused into the filter
               (filtered_next_token_logprobs(..., temperature=T))
  topp_only    as topk_filter with top-p 0.9 alone (no top-k): the histogram path
  topk2000     as topk_filter with k = 2000, p = 0.9: the histogram path
  topp_only_f32 as topp_only with fp32 logits: the fp32 two-pass path
  topp_only_f16 as topp_only with fp16 logits: the histogram path over the full 65536-key table
  filtered16_fwd  forward-only filtered logprobs decided in bf16 (the Megatron logprob
               post-processor's call on the scaled bf16 logits), T=0.7, p=0.9
  packed_kl    packed GRPO step with k3 KL, 64 sequences in bf16 [1, ~34.8k, 256000],
               through SequencePackingFusionLossWrapper
  linear_ce    logprobs from hidden states, fwd+bwd: bf16 hidden [2048, 8, 4096] and
               LM-head weight [151936, 4096], chunk 256 positions (MFMA-bound: TFLOP/s)
  distill_rkl, score_centering, topk_export: the other rows of the path (see below)

Every line carries a `cpu_baseline`: the oracle timed on this host's cores on a
bounded sample of the same workload (stated in `sample`), with the CPU model
and torch version.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path
from typing import Optional

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "logprob+PG-loss fwd/bwd tokens/s and HBM GB/s (% peak) at V=151936 bf16"
PEAK_HBM_GBPS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # dense bf16 MFMA (fp16 the same)
PEAK_FP32_TFLOPS = 157.3  # dense fp32 MFMA


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", default="grpo",
                    choices=["grpo", "fwd_f32", "long_context", "topk_filter", "topk_filter_fused",
                             "topp_only", "topk2000", "topp_only_f32", "topp_only_f16", "filtered16_fwd", "packed_kl",
                             "linear_ce",
                             "distill_rkl", "score_centering", "topk_export"])
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "fp16", "fp32"],
                    help="linear_ce: dtype of the hidden states and weight")
    ap.add_argument("--loss-scale", type=float, default=1.0,
                    help="grpo: multiply the loss by this before the backward (as callers that "
                         "scale the loss by the data-parallel size or microbatch count do)")
    ap.add_argument("--hint-loss-scale", action="store_true",
                    help="grpo: state --loss-scale to the early backward "
                         "(set_early_backward(loss_scale=...)), as a data-parallel caller would")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="minimum CPU time of the cpu_baseline sample")
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-chunk", type=int, default=128,
                    help="sequence positions per chunk of the CPU oracle (bounds its memory)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy-gib", type=float, default=0.0,
                    help="also run a plain device copy of this many GiB (HBM counter calibration)")
    return ap.parse_args()


def _cpu_threads() -> int:
    import torch

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    threads = min(threads, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    return threads


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _cpu_fields(value: float, unit: str, threads: int, sample: str) -> dict:
    import torch

    return {"value": value, "unit": unit, "cores": threads, "kind": "port", "sample": sample,
            "cpu_model": _cpu_model(), "torch": torch.__version__,
            "cpu_capability": torch.backends.cpu.get_cpu_capability()}


def _cpu_timed(run_pass, rows_per_pass: int, sample: str, min_seconds: float,
               max_passes: int = 200, unit: str = "tokens/s") -> dict:
    """Repeat the oracle pass `run_pass` until `min_seconds` have run; rows per second."""
    threads = _cpu_threads()
    passes = 0
    t0 = time.perf_counter()
    while True:
        run_pass()
        passes += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds or passes >= max_passes:
            break
    return _cpu_fields(passes * rows_per_pass / dt, unit, threads,
                       f"{sample}; {passes} pass(es) in {dt:.1f} s")


def cpu_baseline(x, tgt, d: dict, chunk: int, min_seconds: float = 10.0, max_passes: int = 3) -> dict:
    """The CPU oracle (reference op sequence in PyTorch) on the whole step's rows.

    x: [B, S-1, V] bf16 logits rows, tgt: [B, S-1] targets, d: the loss's [B, S]
    data.  Whole passes (chunked forward, ClippedPG loss, chunked backward) are
    repeated until at least ``min_seconds`` have run (at most ``max_passes``).
    """
    import torch

    from oracle.logprob import selected_logprobs, selected_logprobs_grad
    from oracle.loss import clipped_pg_loss

    threads = _cpu_threads()
    B, R, V = x.shape
    passes = 0
    t0 = time.perf_counter()
    while True:
        lp = selected_logprobs(x, tgt, 0, V, chunk_size=chunk)
        lpr = lp.clone().requires_grad_(True)
        loss, _ = clipped_pg_loss(lpr, d, d["sample_mask"].sum(), d["gvt"], reference_policy_kl_penalty=0.0)
        (g,) = torch.autograd.grad(loss, [lpr])
        grad = selected_logprobs_grad(x, tgt, 0, V, g, chunk_size=chunk)
        del grad, lp, lpr, loss, g
        passes += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds or passes >= max_passes:
            break
    return _cpu_fields(passes * B * R / dt, "tokens/s", threads,
                       f"the whole step's {B}x{R} next-token rows (V={V}, bf16) x {passes} pass(es): "
                       f"fwd in chunks of {chunk} positions + ClippedPG loss + bwd, {dt:.1f} s")


def main() -> None:
    args = parse()
    if args.gpus != 1:
        sys.exit(f"bench.py runs on one GPU only (got --gpus {args.gpus}): there is no multi-GPU "
                 "path; the rows of the workload are independent, so it would shard by rows "
                 "with no exchange of logits")
    if args.workload != "grpo":
        bench_workload(args)
        return
    import torch

    from rl_amd import _C, workloads
    from rl_amd.algorithms.advantage_estimator import AdvEstimatorConfig, GRPOAdvantageEstimator
    from rl_amd.algorithms.loss import ClippedPGLossConfig, ClippedPGLossFn
    from rl_amd.distributed.model_utils import from_parallel_logits_to_logprobs

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    print(f"[bench] device {torch.cuda.get_device_name(dev)}; building inputs", file=sys.stderr, flush=True)
    if args.hint_loss_scale:
        from rl_amd.distributed.model_utils import set_early_backward

        set_early_backward("adaptive", loss_scale=args.loss_scale)
    data = workloads.grpo_step_bf16(device=dev)
    logits = data["logits"].requires_grad_(True)
    ids = data["input_ids"]
    B, S, V = logits.shape
    with torch.no_grad():
        cur = from_parallel_logits_to_logprobs(logits, ids, 0, V, None, inference_only=True)
    data = workloads.finish_grpo_step(data, cur)
    loss_cfg = ClippedPGLossConfig(reference_policy_kl_penalty=0.0)
    loss_fn = ClippedPGLossFn(loss_cfg)
    est = GRPOAdvantageEstimator(AdvEstimatorConfig(use_leave_one_out_baseline=False), loss_cfg)
    gvs = data["sample_mask"].sum()
    gvt = (data["token_mask"][:, 1:] * data["sample_mask"][:, None]).sum()
    batch = {k: data[k] for k in ("token_mask", "sample_mask", "prev_logprobs",
                                   "generation_logprobs", "reference_policy_logprobs")}

    def step():
        adv = est.compute_advantage(data["prompt_ids"], data["rewards"], data["token_mask"])
        batch["advantages"] = adv
        lp = from_parallel_logits_to_logprobs(logits, ids, 0, V, None)
        loss, metrics = loss_fn(lp, batch, gvs, gvt)
        if args.loss_scale != 1.0:
            loss = loss * args.loss_scale
        (grad,) = torch.autograd.grad(loss, [logits])
        return grad, lp, metrics

    # active rows: rows whose upstream gradient is non-zero (the bwd reads only those)
    grad, lp, metrics = step()
    lp2 = lp.detach().requires_grad_(True)
    l2, _ = loss_fn(lp2, batch, gvs, gvt)
    (glp,) = torch.autograd.grad(l2, [lp2])
    active_rows = int((glp != 0).sum().item())
    del grad, lp, lp2, l2, glp

    main_kernels = ["mirl_logprob_fwd", "mirl_logprob_bwd", "mirl_logprob_bwd_recheck"]
    ms_step, ms = _timed(step, args.steps, args.warmup, main_kernels)
    always = None
    if args.loss_scale != 1.0 and not args.hint_loss_scale:
        # the default (adaptive) policy stops speculating after the first checked
        # miss; time the redo itself with speculation forced on every step
        from rl_amd.distributed.model_utils import set_early_backward

        set_early_backward("always")
        always = _timed(step, args.steps, args.warmup, main_kernels)
        set_early_backward("adaptive")

    def avg_ms(name):
        return ms.get(name, 0.0)

    rows = B * (S - 1)
    esz = logits.element_size()
    fwd_bytes = rows * V * esz
    bwd_bytes = active_rows * V * esz + B * S * V * esz
    redo_bytes = 2 * active_rows * V * esz
    fwd_ms, bwd_ms = avg_ms("mirl_logprob_fwd"), avg_ms("mirl_logprob_bwd")
    # with a scaled loss the early backward (launched for the unit loss gradient)
    # is checked and redone by the recheck launch; both are the step's backward
    recheck_ms = avg_ms("mirl_logprob_bwd_recheck")
    if always is not None:
        recheck_ms = always[1].get("mirl_logprob_bwd_recheck", 0.0)
    loss_ms, adv_ms = avg_ms("mirl_clipped_pg"), avg_ms("mirl_grpo_advantage")
    bwd_gbps = bwd_bytes / (bwd_ms * 1e-3) / 1e9
    fwd_gbps = fwd_bytes / (fwd_ms * 1e-3) / 1e9
    step_gbps = (fwd_bytes + bwd_bytes) / (ms_step * 1e-3) / 1e9

    traffic = _traffic("grpo", "mirl_logprob_bwd")

    _calibration_copy(args, dev)

    cpu = None
    if not args.no_cpu_baseline:
        x_rows = logits.detach()[:, :-1].cpu()
        tgt_rows = ids[:, 1:].cpu()
        d = {
            "token_mask": data["token_mask"].cpu(),
            "sample_mask": data["sample_mask"].cpu(),
            "advantages": batch["advantages"].cpu().contiguous(),
            "prev_logprobs": data["prev_logprobs"].cpu(),
            "generation_logprobs": data["generation_logprobs"].cpu(),
            "reference_policy_logprobs": data["reference_policy_logprobs"].cpu(),
            "gvt": gvt.cpu(),
        }
        print(f"[bench] timing the CPU oracle on the step's {x_rows.shape[0] * x_rows.shape[1]} rows",
              file=sys.stderr, flush=True)
        cpu = cpu_baseline(x_rows, tgt_rows, d, chunk=args.cpu_chunk, min_seconds=args.cpu_seconds)
        del x_rows

    out = {
        "metric": METRIC,
        "value": rows / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "grpo_clipped_pg_logprob_fwd_bwd",
            "logits": [B, S, V],
            "next_token_rows": rows,
            "active_rows": active_rows,
            "loss": "ClippedPG clip 0.2/0.2 token-level, no KL; GRPO adv (no LOO)",
            "loss_scale": args.loss_scale,
            "loss_scale_hinted": bool(args.hint_loss_scale),
            "parallelism": "single-gpu",
        },
        "hbm_gbps_step": step_gbps,
        "hbm_frac_step": step_gbps / PEAK_HBM_GBPS,
        "kernels_ms": {"logprob_fwd": fwd_ms, "logprob_bwd": bwd_ms, "clipped_pg": loss_ms,
                       "grpo_advantage": adv_ms, "logprob_bwd_recheck": recheck_ms},
        "logprob_fwd_gbps": fwd_gbps,
        # loss_scale != 1 only: the step with the early backward forced on every
        # step (wasted early backward + check + redo), and the redo's rate
        "always_speculate_ms_per_step": None if always is None else always[0],
        # the redo reads and rewrites the rows whose upstream gradient the scale
        # changed (the active rows) and leaves the zero-gradient rows as they are
        "logprob_bwd_recheck_gbps": (redo_bytes / (recheck_ms * 1e-3) / 1e9) if always is not None and recheck_ms > 0 else None,
        "roofline": {
            "kernel": "mirl_logprob_bwd",
            "bound": "hbm",
            "achieved": bwd_gbps,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": bwd_gbps / PEAK_HBM_GBPS,
            "traffic": traffic,
            "algorithmic_bytes": bwd_bytes,
        },
        "cpu_baseline": cpu,
    }
    from rl_amd.distributed.early_backward import POLICY

    POLICY._drain()
    out["early_backward"] = {"mode": POLICY.mode, "loss_scale_hint": POLICY.loss_scale,
                             "checks_missed": POLICY.misses, "opportunities_skipped": POLICY.skipped}
    print(json.dumps(out), flush=True)


def _calibration_copy(args, dev) -> None:
    """A plain device copy of --calibrate-copy-gib GiB (three times), whose HBM
    counter readings scale FETCH_SIZE / WRITE_SIZE to bytes."""
    if args.calibrate_copy_gib <= 0:
        return
    import torch

    n = int(args.calibrate_copy_gib * (1 << 30)) // 4
    a = torch.empty(n, dtype=torch.float32, device=dev).fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def _timed(step, steps: int, warmup: int, main_kernels: list, region_events: Optional[dict] = None):
    """Run `warmup` untimed steps, then `steps` timed ones; (ms per step, ms per entry point).

    Inside the timed region HIP events bracket only the `main_kernels` entry
    points (each event pair adds a few microseconds of GPU time between
    neighbouring launches); the other entry points are timed afterwards over a
    few more steps.  With `region_events` (a dict), one event pair on the
    current stream also brackets the whole timed region and its GPU time per
    step is stored under "gpu_ms_per_step".
    """
    import torch

    from rl_amd import _C

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    timer = _C.enable_launch_timing(main_kernels) if main_kernels else None
    torch.cuda.synchronize()
    if region_events is not None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    if region_events is not None:
        e0.record()
    for _ in range(steps):
        step()
    if region_events is not None:
        e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    if region_events is not None:
        region_events["gpu_ms_per_step"] = e0.elapsed_time(e1) / steps
    _C.disable_launch_timing()
    if timer is None:
        timer = {}
    ms = {k: sum(a.elapsed_time(b) for a, b in v) / max(1, len(v)) for k, v in timer.items()}
    rest = _C.enable_launch_timing()
    for _ in range(min(steps, 5)):
        step()
    torch.cuda.synchronize()
    _C.disable_launch_timing()
    for k, v in rest.items():
        if k not in ms:
            ms[k] = sum(a.elapsed_time(b) for a, b in v) / max(1, len(v))
    return (t1 - t0) * 1e3 / steps, ms


def _traffic(workload: str, entry_point: str):
    """HBM bytes per call of `entry_point` in `workload`, from the committed rocprof counter runs.

    profiles/traffic.json holds FETCH_SIZE + WRITE_SIZE per dispatch of the
    entry point's kernels, scaled by what the same counters read for a 1 GiB
    device copy; None when that entry point was not measured in that workload.
    """
    tf = ROOT / "profiles" / "traffic.json"
    try:
        return json.loads(tf.read_text())["workloads"][workload][entry_point]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError, TypeError):
        return None


def _roofline(kernel: str, nbytes: float, ms: float, workload: str) -> dict:
    gbps = nbytes / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
    return {"kernel": kernel, "bound": "hbm", "achieved": gbps, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "frac": gbps / PEAK_HBM_GBPS, "traffic": _traffic(workload, kernel), "algorithmic_bytes": nbytes}


def _timed_split(prepare, path, steps: int, warmup: int, main_kernels: list):
    """Like _timed, for steps whose inputs must be rebuilt first (in-place work):
    `prepare()` runs outside the timed window of each step; the step time is
    the mean of HIP-event intervals around `path(prepare())` on the current stream."""
    import torch

    from rl_amd import _C

    for _ in range(warmup):
        path(prepare())
    torch.cuda.synchronize()
    timer = _C.enable_launch_timing(main_kernels)
    evs = []
    for _ in range(steps):
        x = prepare()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        path(x)
        e1.record()
        evs.append((e0, e1))
    torch.cuda.synchronize()
    _C.disable_launch_timing()
    ms = {k: sum(a.elapsed_time(b) for a, b in v) / max(1, len(v)) for k, v in timer.items()}
    step_ms = sum(a.elapsed_time(b) for a, b in evs) / max(1, len(evs))
    rest = _C.enable_launch_timing()
    for _ in range(min(steps, 5)):
        path(prepare())
    torch.cuda.synchronize()
    _C.disable_launch_timing()
    for k, v in rest.items():
        if k not in ms:
            ms[k] = sum(a.elapsed_time(b) for a, b in v) / max(1, len(v))
    return step_ms, ms


def _dominant(candidates: list, ms: dict, workload: str) -> dict:
    """Roofline of the entry point with the largest average time among
    (name, algorithmic bytes) candidates."""
    name, nbytes = max(candidates, key=lambda c: ms.get(c[0], 0.0))
    return _roofline(name, nbytes, ms.get(name, 0.0), workload)


def _filtered_cpu(x, ids, g, k, p, T, rows: int, min_seconds: float, forward_only: bool = False,
                  decide_16bit: bool = False):
    """The oracle's filtered chain on the first `rows` next-token rows of sequence 0."""
    import torch

    from oracle.sampling import apply_temperature, filtered_logprobs, next_token_filtered

    xs = x[0:1, : rows + 1].detach().cpu()
    ids_s = ids[0:1, : rows + 1].cpu()
    gs = None if g is None else g[0:1, :rows].cpu()
    dt = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[x.dtype]
    if decide_16bit:
        def run():
            y = apply_temperature(xs, T)
            filtered_logprobs(y[:, :-1], ids_s[:, 1:], k, p)
        what = "T-division in bf16, top-p decided in bf16, forward"
    else:
        def run():
            next_token_filtered(xs, ids_s, k, p, temperature=T, grad_output=None if forward_only else gs)
        what = f"T-division in {dt}, fp32 upcast, filter, log_softmax, gather" + (
            "" if forward_only else ", backward to the raw logits")
    return lambda: _cpu_timed(run, rows, f"{rows} next-token rows of [1, {rows + 1}, {x.shape[-1]}] {dt} "
                              f"(k={k}, p={p}, T={T}): {what}", min_seconds)


def bench_workload(args) -> None:
    """The non-default workloads: one JSON line each, same fields as the headline line.

    Algorithmic bytes per next-token row of V entries of s bytes: forward V*s
    (read); unfiltered backward V*s read for rows with a non-zero upstream
    gradient plus V*s written for every row; filtered backward V*s written
    (the kept set saved by the forward replaces the re-read) plus, for rows
    without a kept list (top-p alone, k > 1024), V*s read for rows with a
    non-zero upstream gradient; the in-place temperature division V*s read +
    V*s written for every row.
    """
    import torch

    from rl_amd import _C, workloads
    from rl_amd.distributed.model_utils import from_parallel_logits_to_logprobs

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w = args.workload
    print(f"[bench] device {torch.cuda.get_device_name(dev)}; workload {w}", file=sys.stderr, flush=True)
    extra: dict = {}
    cpu_fn = None
    secs = args.cpu_seconds
    if w == "fwd_f32":
        copies = [workloads.logprob_fwd_f32(device=dev) for _ in range(8)]  # 8 x 65.5 MB > on-die cache
        B, S, V = copies[0]["logits"].shape
        it = [0]

        def step():
            c = copies[it[0] % len(copies)]
            it[0] += 1
            return from_parallel_logits_to_logprobs(c["logits"], c["input_ids"], 0, V, None, inference_only=True)

        # No events inside the timed steps: an event pair around a 13-us launch
        # costs host and GPU time of its own (with them the step read 23 us
        # against 10 us of host work per call and a 13-us kernel).
        region = {}
        ms_step, ms = _timed(step, args.steps, args.warmup, [], region)
        rows = B * (S - 1)
        esz = 4
        # The kernel's launch duration comes from one pair of events around a
        # burst of back-to-back launches of the entry point (the same inputs and
        # outputs, the rotating copies in turn).
        outs = [torch.empty((B, S - 1), dtype=torch.float32, device=dev) for _ in copies]
        tgts = [c["input_ids"][:, 1:] for c in copies]
        burst = 200
        for k in range(len(copies)):
            _C.logprob_fwd(copies[k]["logits"], tgts[k], 0, V, outs[k], None)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for k in range(burst):
            j = k % len(copies)
            _C.logprob_fwd(copies[j]["logits"], tgts[j], 0, V, outs[j], None)
        e1.record()
        torch.cuda.synchronize()
        extra["logprob_fwd_event_pair_ms"] = ms.get("mirl_logprob_fwd", 0.0)
        extra["logprob_fwd_burst_ms"] = e0.elapsed_time(e1) / burst
        # the launch duration: GPU time of the timed region (one event pair on
        # the launch stream around all timed steps, one launch per step) per step
        ms["mirl_logprob_fwd"] = region["gpu_ms_per_step"]
        extra["launch_duration_from"] = ("one event pair around the timed steps (one launch per step); "
                                         f"burst of {burst} back-to-back launches alongside")
        roof = _roofline("mirl_logprob_fwd", rows * V * esz, ms.get("mirl_logprob_fwd", 0.0), w)
        step_bytes = rows * V * esz
        cfg = {"workload": "logprob_fwd_f32", "logits": [B, S, V], "next_token_rows": rows,
               "rotating_copies": len(copies)}
        dtype = "f32"
        xc, tc = copies[0]["logits"].cpu(), copies[0]["input_ids"].cpu()

        def cpu_fn():
            from oracle.logprob import selected_logprobs

            return _cpu_timed(lambda: selected_logprobs(xc[:, :-1], tc[:, 1:], 0, V), rows,
                              f"the whole fp32 [{B}, {S}, {V}] batch ({rows} next-token rows), forward", secs,
                              max_passes=100000)
    elif w == "long_context":
        d = workloads.long_context_bf16(device=dev)
        logits = d["logits"].requires_grad_(True)
        ids, g = d["input_ids"], d["grad"]
        B, S, V = logits.shape

        def step():
            lp = from_parallel_logits_to_logprobs(logits, ids, 0, V, None, chunk_size=4096)
            return torch.autograd.grad(lp, [logits], g)

        ms_step, ms = _timed(step, args.steps, args.warmup, ["mirl_logprob_fwd", "mirl_logprob_bwd"])
        rows = B * (S - 1)
        active = int((g != 0).sum().item())
        esz = 2
        bwd_bytes = (active + B * S) * V * esz
        roof = _roofline("mirl_logprob_bwd", bwd_bytes, ms.get("mirl_logprob_bwd", 0.0), w)
        step_bytes = rows * V * esz + bwd_bytes
        extra["logprob_fwd_gbps"] = rows * V * esz / (ms.get("mirl_logprob_fwd", 1e9) * 1e-3) / 1e9
        cfg = {"workload": "long_context_chunked_logprob_fwd_bwd", "logits": [B, S, V], "chunk_size": 4096,
               "next_token_rows": rows, "active_rows": active}
        dtype = "bf16"
        n_s = 2048
        xs, ts, gs = logits.detach()[:, :n_s].cpu(), ids[:, 1 : n_s + 1].cpu(), g[:, :n_s].cpu()

        def cpu_fn():
            from oracle.logprob import selected_logprobs, selected_logprobs_grad

            def run():
                selected_logprobs(xs, ts, 0, V, chunk_size=4096)
                selected_logprobs_grad(xs, ts, 0, V, gs, chunk_size=4096, out_dtype=torch.bfloat16)

            return _cpu_timed(run, n_s, f"the first {n_s} of the {rows} next-token rows (V={V}, bf16, "
                              "chunk 4096): forward + backward", secs)
    elif w in ("topk_filter", "topp_only", "topk2000", "topp_only_f32", "topp_only_f16", "filtered16_fwd"):
        from rl_amd.algorithms.logits_sampling_utils import TrainingSamplingParams, apply_temperature_scaling
        from rl_amd.distributed.model_utils import get_next_token_logprobs_from_logits

        if w == "topk_filter":
            d = workloads.topk_filter_bf16(device=dev)
        elif w == "topk2000":
            d = workloads.general_filter_bf16(top_k=2000, top_p=0.9, device=dev)
        elif w == "topp_only_f32":
            d = workloads.general_filter_bf16(top_k=None, top_p=0.9, device=dev, dtype=torch.float32)
        elif w == "topp_only_f16":
            d = workloads.general_filter_bf16(top_k=None, top_p=0.9, device=dev, dtype=torch.float16)
        else:
            d = workloads.general_filter_bf16(top_k=None, top_p=0.9, device=dev)
        raw = d["logits"]
        ids, g = d["input_ids"], d["grad"]
        B, S, V = raw.shape
        k, p, T = d["top_k"], d["top_p"], d["temperature"]
        sp = TrainingSamplingParams(top_k=k, top_p=p, temperature=T)
        rows = B * (S - 1)
        esz = raw.element_size()
        scale_bytes = 2 * B * S * V * esz
        fwd_bytes, bwd_bytes = rows * V * esz, B * S * V * esz
        kept_list = k is not None and 1 <= k <= 1024
        if not kept_list:
            # No kept list is saved for these rows (top-p alone keeps most of the
            # vocabulary: a list of kept ids and probabilities would outweigh the
            # row), so the backward re-reads the logits of every row with a
            # non-zero upstream gradient: those bytes are compulsory here.
            bwd_bytes += int((g[:, : S - 1] != 0).sum().item()) * V * esz
        if w == "filtered16_fwd":
            work = torch.empty_like(raw)

            def prepare():
                work.copy_(raw)  # the model's output of this step, outside the timed window
                return work

            def path(logits):
                apply_temperature_scaling(logits, sp)
                return from_parallel_logits_to_logprobs(logits, ids, 0, V, None, inference_only=True,
                                                        sampling_params=sp)

            ms_step, ms = _timed_split(prepare, path, args.steps, args.warmup,
                                       ["mirl_temperature_scale", "mirl_filtered_logprob_fwd"])
            roof = _dominant([("mirl_temperature_scale", scale_bytes),
                              ("mirl_filtered_logprob_fwd", fwd_bytes)], ms, w)
            step_bytes = scale_bytes + fwd_bytes
            cfg = {"workload": "bf16_decided_filtered_logprob_fwd", "logits": [B, S, V], "temperature": T,
                   "top_k": k, "top_p": p, "next_token_rows": rows,
                   "call": "apply_temperature_scaling in place, then from_parallel_logits_to_logprobs("
                           "sampling_params, inference_only=True): top-p decided in bf16"}
            cpu_fn = _filtered_cpu(raw, ids, None, k, p, T, 1024, secs, forward_only=True, decide_16bit=True)
        else:
            raw.requires_grad_(True)

            class _ModelOutput(torch.autograd.Function):
                """Stands in for the LM head: a fresh logits tensor each step (copied from
                the resident logits outside the timed window); its backward hands the
                raw-logits gradient on unchanged."""

                @staticmethod
                def forward(ctx, x):  # type: ignore[override]
                    return x.detach().clone()

                @staticmethod
                def backward(ctx, grad):  # type: ignore[override]
                    return grad

            def prepare():
                return _ModelOutput.apply(raw)

            def path(logits):
                logits = apply_temperature_scaling(logits, sp)
                lp = get_next_token_logprobs_from_logits(ids, logits, sampling_params=sp)
                return torch.autograd.grad(lp, [raw], g)

            kern = ["mirl_temperature_scale", "mirl_filtered_logprob_fwd", "mirl_filtered_logprob_bwd"]
            ms_step, ms = _timed_split(prepare, path, args.steps, args.warmup, kern)
            roof = _dominant([("mirl_temperature_scale", scale_bytes), ("mirl_filtered_logprob_fwd", fwd_bytes),
                              ("mirl_filtered_logprob_bwd", bwd_bytes)], ms, w)
            step_bytes = scale_bytes + fwd_bytes + bwd_bytes
            cfg = {"workload": {"topk_filter": "topk_topp_temperature_filtered_logprob_fwd_bwd",
                                "topp_only": "topp_temperature_filtered_logprob_fwd_bwd",
                                "topk2000": "topk2000_topp_temperature_filtered_logprob_fwd_bwd",
                                "topp_only_f32": "fp32_topp_temperature_filtered_logprob_fwd_bwd",
                                "topp_only_f16": "fp16_topp_temperature_filtered_logprob_fwd_bwd"}[w],
                   "logits": [B, S, V], "temperature": T, "top_k": k, "top_p": p, "next_token_rows": rows,
                   "call": "apply_temperature_scaling in place, get_next_token_logprobs_from_logits("
                           "sampling_params), backward to the raw logits (the division's backward "
                           "folded into the filtered backward)"}
            cpu_fn = _filtered_cpu(raw, ids, g, k, p, T, 1024, secs)
        fwd_ms = ms.get("mirl_filtered_logprob_fwd", 0.0)
        bwd_ms = ms.get("mirl_filtered_logprob_bwd", 0.0)
        sc_ms = ms.get("mirl_temperature_scale", 0.0)
        extra["filtered_fwd_gbps"] = fwd_bytes / (fwd_ms * 1e-3) / 1e9 if fwd_ms > 0 else None
        extra["filtered_bwd_gbps"] = bwd_bytes / (bwd_ms * 1e-3) / 1e9 if bwd_ms > 0 else None
        extra["temperature_scale_gbps"] = scale_bytes / (sc_ms * 1e-3) / 1e9 if sc_ms > 0 else None
        dtype = "fp32" if esz == 4 else ("fp16" if raw.dtype == torch.float16 else "bf16")
    elif w == "topk_filter_fused":
        from rl_amd.distributed.sampling import filtered_next_token_logprobs

        d = workloads.topk_filter_bf16(device=dev)
        logits = d["logits"].requires_grad_(True)
        ids, g = d["input_ids"], d["grad"]
        B, S, V = logits.shape
        k, p, T = d["top_k"], d["top_p"], d["temperature"]

        def step():
            lp = filtered_next_token_logprobs(logits, ids, k, p, temperature=T, decision_dtype=torch.float32)
            return torch.autograd.grad(lp, [logits], g)

        ms_step, ms = _timed(step, args.steps, args.warmup,
                             ["mirl_filtered_logprob_fwd", "mirl_filtered_logprob_bwd"])
        rows = B * (S - 1)
        esz = 2
        fwd_bytes, bwd_bytes = rows * V * esz, B * S * V * esz
        fwd_ms, bwd_ms = ms.get("mirl_filtered_logprob_fwd", 0.0), ms.get("mirl_filtered_logprob_bwd", 0.0)
        roof = _roofline("mirl_filtered_logprob_fwd", fwd_bytes, fwd_ms, w)
        extra["filtered_bwd_gbps"] = bwd_bytes / (bwd_ms * 1e-3) / 1e9 if bwd_ms > 0 else None
        step_bytes = fwd_bytes + bwd_bytes
        cfg = {"workload": "topk_topp_temperature_filtered_logprob_fwd_bwd_fused", "logits": [B, S, V],
               "temperature": T, "top_k": k, "top_p": p, "next_token_rows": rows,
               "call": "filtered_next_token_logprobs(..., temperature=T, decision_dtype=float32): the "
                       "division fused into the filter (an extension of the reference's API)"}
        dtype = "bf16"
        cpu_fn = _filtered_cpu(logits, ids, g, k, p, T, 1024, secs)
    elif w == "linear_ce":
        from rl_amd.distributed.model_utils import from_parallel_hidden_states_to_logprobs

        d = workloads.linear_ce_bf16(device=dev)
        tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[args.dtype]
        hidden = d["hidden"].to(tdt).requires_grad_(True)
        weight = d["weight"].to(tdt).requires_grad_(True)
        del d["hidden"], d["weight"]
        ids, g = d["input_ids"], d["grad"]
        S, B, H = hidden.shape
        V = weight.shape[0]

        def step():
            lp = from_parallel_hidden_states_to_logprobs(hidden, weight, False, ids, 0, V, None,
                                                         chunk_size=256)
            return torch.autograd.grad(lp, [hidden, weight], g)

        lce_kernels = (["mirl_linear_ce_fwd", "mirl_linear_ce_grad", "mirl_gemm_bf16_abt",
                        "mirl_transpose_bf16", "mirl_sum_splits_bf16"] if args.dtype != "fp32" else
                       ["mirl_gemm_f32_abt", "mirl_logprob_fwd", "mirl_logprob_bwd", "mirl_transpose_f32",
                        "mirl_sum_splits_bf16"])
        region = {}
        ms_step, ms = _timed(step, args.steps, args.warmup, lce_kernels, region_events=region)
        rows = B * (S - 1)
        gemm = 2.0 * S * B * H * V  # one [S*B, H] x [H, V] product
        # the backward moves the rows with a non-zero upstream gradient to the front
        # and runs all rows in blocks of _BLOCK_CHUNKS * chunk_size * B rows (counted
        # on the device; launches of blocks past the active rows return at once):
        # per-step kernel times are the average launch times the launches per step
        from rl_amd.distributed.linear_ce import _BLOCK_CHUNKS

        active = int((g != 0).sum().item())
        fwd_ms = ms.get("mirl_linear_ce_fwd", 0.0)
        T = S * B
        n_blocks = -(-T // min(T, -(-(_BLOCK_CHUNKS * 256 * B) // 256) * 256))
        grad_ms = ms.get("mirl_linear_ce_grad", 0.0) * n_blocks
        gemm_act = 2.0 * active * H * V
        tflops = gemm / (fwd_ms * 1e-3) / 1e12 if fwd_ms > 0 else 0.0
        peak = PEAK_FP32_TFLOPS if args.dtype == "fp32" else PEAK_BF16_TFLOPS
        if args.dtype == "fp32":
            # the fp32 tile loop per chunk (forward logits; per backward block the active
            # rows' logits, dH and dW) plus the logprob row kernels and the transposes: the
            # whole step's algorithmic flops over its GPU time (one event pair around the
            # timed steps)
            gpu_ms = region.get("gpu_ms_per_step", ms_step)
            tflops = (gemm + 3 * gemm_act) / (gpu_ms * 1e-3) / 1e12
            roof = {"kernel": "step (mirl_gemm_f32_abt + mirl_logprob_fwd/bwd)", "bound": "mfma",
                    "achieved": tflops, "peak": peak, "unit": "TFLOP/s", "frac": tflops / peak,
                    "traffic": None, "algorithmic_flops": gemm + 3 * gemm_act}
        else:
            roof = {"kernel": "mirl_linear_ce_fwd", "bound": "mfma", "achieved": tflops, "peak": peak,
                    "unit": "TFLOP/s", "frac": tflops / peak,
                    "traffic": _traffic(w if args.dtype == "bf16" else f"{w}_{args.dtype}", "mirl_linear_ce_fwd"),
                    "algorithmic_flops": gemm}
        extra["tflops_step"] = (gemm + 3 * gemm_act) / (ms_step * 1e-3) / 1e12
        extra["grad_kernel_ms_per_step"] = grad_ms
        extra["grad_kernel_tflops"] = gemm_act / (grad_ms * 1e-3) / 1e12 if grad_ms > 0 else None
        # dH and dW: two products of 2 * active * H * V each on mirl_gemm_bf16_abt
        # (average launch x launches per step: one dH and one dW per block)
        gemm_ms = ms.get("mirl_gemm_bf16_abt", 0.0) * 2 * n_blocks
        extra["dh_dw_gemm_ms_per_step"] = gemm_ms
        extra["dh_dw_gemm_tflops"] = 2 * gemm_act / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else None
        step_bytes = None
        cfg = {"workload": "hidden_state_logprobs_fwd_bwd", "hidden": [S, B, H], "weight": [V, H],
               "chunk_size": 256, "next_token_rows": rows, "active_rows": active,
               "flops_per_step": "2*S*B*H*V (fused fwd) + 3 x 2*active*H*V (fused grad recompute, dH, dW)"}
        dtype = args.dtype
        n_pos = 32
        hs, ws_, ts = hidden.detach()[:n_pos].cpu(), weight.detach().cpu(), torch.roll(ids, -1, 1)[:, :n_pos].cpu()

        def cpu_fn():
            from oracle.linear_ce import hidden_state_logprobs

            return _cpu_timed(lambda: hidden_state_logprobs(hs, ts, ws_, 0, V), n_pos * B,
                              f"{n_pos * B} rows ({n_pos} positions x {B}) of the hidden states against "
                              f"the whole [{V}, {H}] weight: forward (logits, log-sum-exp, gather)", secs)
    elif w == "distill_rkl":
        from rl_amd.distributed.model_utils import ChunkedDistributedReverseKLToFixedLogits

        d = workloads.distill_rkl_bf16(device=dev)
        student = d["student"].requires_grad_(True)
        teacher = d["teacher"]
        B, S, V = student.shape
        m = d["token_mask"][:, 1:]
        n_tok = m.sum()

        def step():
            rkl = ChunkedDistributedReverseKLToFixedLogits.apply(student, teacher, 4096, None, False)
            loss = (rkl[:, :-1] * m).sum() / n_tok
            return torch.autograd.grad(loss, [student])

        ms_step, ms = _timed(step, args.steps, args.warmup, ["mirl_divergence_fwd", "mirl_divergence_bwd"])
        rows = B * (S - 1)
        active = int((m != 0).sum().item())
        esz = 2
        fwd_bytes = 2 * B * S * V * esz
        bwd_bytes = (2 * active + B * S) * V * esz
        fwd_ms, bwd_ms = ms.get("mirl_divergence_fwd", 0.0), ms.get("mirl_divergence_bwd", 0.0)
        roof = _roofline("mirl_divergence_bwd", bwd_bytes, bwd_ms, w)
        extra["divergence_fwd_gbps"] = fwd_bytes / (fwd_ms * 1e-3) / 1e9 if fwd_ms > 0 else None
        step_bytes = fwd_bytes + bwd_bytes
        cfg = {"workload": "reverse_kl_to_fixed_teacher_fwd_bwd", "student": [B, S, V], "teacher": [B, S, V],
               "next_token_rows": rows, "active_rows": active,
               "loss": "masked mean of per-token reverse KL over response tokens"}
        dtype = "bf16"
        n_s = 1024
        ss, tt = student.detach()[0:1, :n_s].cpu(), teacher[0:1, :n_s].cpu()
        gg = torch.ones(1, n_s)

        def cpu_fn():
            from oracle.vocab_reduce import divergence, divergence_grad

            def run():
                divergence("reverse_kl", ss, tt, chunk_size=4096)
                divergence_grad("reverse_kl", ss, tt, gg, chunk_size=4096)

            return _cpu_timed(run, n_s, f"{n_s} rows of the student/teacher [1, {n_s}, {V}] bf16 pair: "
                              "reverse KL forward + backward", secs)
    elif w == "score_centering":
        from types import SimpleNamespace

        from rl_amd.algorithms.advantage_estimator import AdvEstimatorConfig, GRPOAdvantageEstimator
        from rl_amd.algorithms.loss import (
            ClippedPGLossConfig,
            ClippedPGLossFn,
            LossInputType,
            prepare_loss_input,
        )

        d = workloads.score_centering_bf16(device=dev)
        logits = d["logits"].requires_grad_(True)
        B, S, V = logits.shape
        K = d["sampler_topk_token_ids"].shape[-1]
        probe = SimpleNamespace(input_type=LossInputType.LOGPROB, score_centering=True)
        with torch.no_grad():
            cur, _ = prepare_loss_input(logits, {"input_ids": d["input_ids"],
                                                 "sampler_topk_token_ids": d["sampler_topk_token_ids"],
                                                 "sampler_topk_logprobs": d["sampler_noise"]}, probe)
        d = workloads.finish_score_centering_step(d, cur["next_token_logprobs"],
                                                  cur["policy_logprobs_at_sampler_topk"])
        loss_cfg = ClippedPGLossConfig(reference_policy_kl_penalty=0.0, score_centering=True)
        loss_fn = ClippedPGLossFn(loss_cfg)
        est = GRPOAdvantageEstimator(AdvEstimatorConfig(use_leave_one_out_baseline=False), loss_cfg)
        gvs = d["sample_mask"].sum()
        gvt = (d["token_mask"][:, 1:] * d["sample_mask"][:, None]).sum()
        batch = {k: d[k] for k in ("input_ids", "token_mask", "sample_mask", "prev_logprobs",
                                   "generation_logprobs", "reference_policy_logprobs",
                                   "sampler_topk_token_ids", "sampler_topk_logprobs")}

        def step():
            batch["advantages"] = est.compute_advantage(d["prompt_ids"], d["rewards"], d["token_mask"])
            li, _ = prepare_loss_input(logits, batch, loss_fn)
            loss, _ = loss_fn(data=batch, global_valid_seqs=gvs, global_valid_toks=gvt, **li)
            return torch.autograd.grad(loss, [logits])

        # rows whose upstream gradient is non-zero, for each of the two logprob outputs
        batch["advantages"] = est.compute_advantage(d["prompt_ids"], d["rewards"], d["token_mask"])
        lp_leaf = cur["next_token_logprobs"].detach().requires_grad_(True)
        pk_leaf = cur["policy_logprobs_at_sampler_topk"].detach().requires_grad_(True)
        l2, _ = loss_fn(next_token_logprobs=lp_leaf, policy_logprobs_at_sampler_topk=pk_leaf, data=batch,
                        global_valid_seqs=gvs, global_valid_toks=gvt)
        g_lp, g_pk = torch.autograd.grad(l2, [lp_leaf, pk_leaf])
        # the one K+1-id backward reads a row when g_target + sum_k g_k != 0
        active = int(((g_lp + g_pk.sum(-1)) != 0).sum().item())
        del lp_leaf, pk_leaf, l2, g_lp, g_pk

        ms_step, ms = _timed(step, args.steps, args.warmup,
                             ["mirl_gather_logprob_fwd", "mirl_gather_logprob_bwd"])
        rows = B * (S - 1)
        esz = 2
        # next-token and top-k logprobs share one K+1-id pass over all B*S rows;
        # one backward reads the active rows and writes every row
        fwd_bytes = B * S * V * esz
        bwd_bytes = (active + B * S) * V * esz
        gfwd_ms, gbwd_ms = ms.get("mirl_gather_logprob_fwd", 0.0), ms.get("mirl_gather_logprob_bwd", 0.0)
        roof = _roofline("mirl_gather_logprob_bwd", bwd_bytes, gbwd_ms, w)
        extra["gather_fwd_gbps"] = fwd_bytes / (gfwd_ms * 1e-3) / 1e9 if gfwd_ms > 0 else None
        step_bytes = fwd_bytes + bwd_bytes
        cfg = {"workload": "grpo_score_centering_fwd_bwd", "logits": [B, S, V], "sampler_topk": K,
               "next_token_rows": rows, "active_rows": active, "ids_per_row": K + 1,
               "loss": "ClippedPG clip 0.2/0.2 token-level + score centering (IS off); GRPO adv"}
        dtype = "bf16"
        n_s = 1024
        xs = logits.detach()[0:1, :n_s].cpu()
        idx = torch.cat([d["input_ids"][0:1, 1 : n_s + 1].unsqueeze(-1),
                         d["sampler_topk_token_ids"][0:1, :n_s]], -1).cpu()
        gg = torch.randn(idx.shape, generator=torch.Generator().manual_seed(0))

        def cpu_fn():
            from oracle.vocab_reduce import gather_logprobs, gather_logprobs_grad

            def run():
                gather_logprobs(xs, idx, 0, V)
                gather_logprobs_grad(xs, idx, 0, V, gg)

            return _cpu_timed(run, n_s, f"{n_s} rows of [1, {n_s}, {V}] bf16 at {K + 1} ids per row: "
                              "log-softmax gather forward + backward (the loss kernels excluded)", secs)
    elif w == "topk_export":
        from rl_amd.distributed.model_utils import distributed_vocab_topk

        d = workloads.distill_rkl_bf16(device=dev)
        teacher = d["teacher"]
        del d
        B, S, V = teacher.shape
        k = 64

        def step():
            return distributed_vocab_topk(teacher, k, None, vocab_start_index=0, vocab_end_index=V)

        ms_step, ms = _timed(step, args.steps, args.warmup, ["mirl_vocab_topk"])
        rows = B * S
        esz = 2
        fwd_bytes = rows * V * esz + rows * k * 12
        roof = _roofline("mirl_vocab_topk", fwd_bytes, ms.get("mirl_vocab_topk", 0.0), w)
        step_bytes = fwd_bytes
        cfg = {"workload": "teacher_topk_export", "logits": [B, S, V], "k": k, "rows": rows,
               "outputs": "fp32 values + int64 ids [B, S, k]"}
        dtype = "bf16"
        n_s = 1024
        xs = teacher[0:1, :n_s].cpu()

        def cpu_fn():
            from oracle.vocab_reduce import vocab_topk

            return _cpu_timed(lambda: vocab_topk(xs, k), n_s,
                              f"{n_s} rows of [1, {n_s}, {V}] bf16: top-{k} values and ids", secs,
                              unit="rows/s")
    else:  # packed_kl
        import torch.distributed as dist

        from rl_amd.algorithms.advantage_estimator import AdvEstimatorConfig, GRPOAdvantageEstimator
        from rl_amd.algorithms.loss import (
            ClippedPGLossConfig,
            ClippedPGLossFn,
            SequencePackingFusionLossWrapper,
            prepare_packed_loss_input,
        )
        from rl_amd.distributed.batched_data_dict import BatchedDataDict

        if not dist.is_initialized():
            # gloo reports its (empty) peer set on stdout; keep stdout for the JSON line
            sys.stdout.flush()
            saved = os.dup(1)
            os.dup2(2, 1)
            try:
                dist.init_process_group("gloo", store=dist.HashStore(), rank=0, world_size=1)
            finally:
                sys.stdout.flush()
                os.dup2(saved, 1)
                os.close(saved)
        group = dist.group.WORLD
        d = workloads.packed_grpo_kl_bf16(device=dev)
        logits, cu = d["logits"], d["cu_seqlens"]
        _, T, V = logits.shape
        n_seq = len(cu) - 1
        cfg_kw = dict(reference_policy_kl_penalty=0.01, reference_policy_kl_type="k3",
                      ratio_clip_min=0.2, ratio_clip_max=0.2, token_level_loss=False)
        loss_fn = ClippedPGLossFn(ClippedPGLossConfig(**cfg_kw))
        with torch.no_grad():
            cur, _ = prepare_packed_loss_input(
                logits, BatchedDataDict({"input_ids": d["input_ids"]}), loss_fn, cu, cu,
                vocab_parallel_rank=0, vocab_parallel_group=group)
        d = workloads.finish_packed_grpo_step(d, cur["next_token_logprobs"])
        est = GRPOAdvantageEstimator(AdvEstimatorConfig(use_leave_one_out_baseline=False))
        batch = BatchedDataDict({k: d[k] for k in ("input_ids", "token_mask", "sample_mask", "prev_logprobs",
                                                   "generation_logprobs", "reference_policy_logprobs")})
        gvs = d["sample_mask"].sum()
        gvt = d["token_mask"][:, 1:].sum()
        wrapper = SequencePackingFusionLossWrapper(loss_fn, prepare_packed_loss_input, cu, cu,
                                                   vocab_parallel_rank=0, vocab_parallel_group=group)
        logits.requires_grad_(True)

        def step():
            batch["advantages"] = est.compute_advantage(d["prompt_ids"], d["rewards"], d["token_mask"])
            loss, _ = wrapper(logits, batch, gvs, gvt)
            return torch.autograd.grad(loss, [logits])

        # active rows: next-token rows whose upstream gradient is non-zero
        batch["advantages"] = est.compute_advantage(d["prompt_ids"], d["rewards"], d["token_mask"])
        lp_leaf = cur["next_token_logprobs"].detach().requires_grad_(True)
        l2, _ = loss_fn(next_token_logprobs=lp_leaf, data=batch, global_valid_seqs=gvs, global_valid_toks=gvt)
        (glp,) = torch.autograd.grad(l2, [lp_leaf])
        active = int((glp != 0).sum().item())
        del lp_leaf, l2, glp
        ms_step, ms = _timed(step, args.steps, args.warmup, ["mirl_logprob_fwd", "mirl_logprob_bwd"])
        rows = T - n_seq
        esz = 2
        fwd_bytes = rows * V * esz
        bwd_bytes = (active + T) * V * esz
        roof = _roofline("mirl_logprob_bwd", bwd_bytes, ms.get("mirl_logprob_bwd", 0.0), w)
        extra["logprob_fwd_gbps"] = fwd_bytes / (ms.get("mirl_logprob_fwd", 1e9) * 1e-3) / 1e9
        step_bytes = fwd_bytes + bwd_bytes
        cfg = {"workload": "packed_grpo_kl_fused_wrapper", "logits": [1, T, V], "sequences": n_seq,
               "next_token_rows": rows, "active_rows": active,
               "loss": "ClippedPG clip 0.2/0.2, k3 KL beta 0.01, sequence-level mean; GRPO adv (no LOO)"}
        dtype = "bf16"
        n_s = 2048
        xs = logits.detach()[:, :n_s].cpu()
        ts = _packed_targets(d["input_ids"], cu)[:, :n_s].cpu()
        gg = torch.randn(1, n_s, generator=torch.Generator().manual_seed(0))

        def cpu_fn():
            from oracle.logprob import selected_logprobs, selected_logprobs_grad

            def run():
                selected_logprobs(xs, ts, 0, V, chunk_size=1024)
                selected_logprobs_grad(xs, ts, 0, V, gg, chunk_size=1024, out_dtype=torch.bfloat16)

            return _cpu_timed(run, n_s, f"the first {n_s} of the {T} packed rows (V={V}, bf16): logprob "
                              "forward + backward in chunks of 1024 rows (the loss, ~0.3% of the "
                              "step, excluded)", secs)

    _calibration_copy(args, dev)
    cfg["parallelism"] = "single-gpu"
    step_gbps = step_bytes / (ms_step * 1e-3) / 1e9 if step_bytes is not None else None
    cpu = None
    if not args.no_cpu_baseline and cpu_fn is not None:
        print("[bench] timing the CPU oracle", file=sys.stderr, flush=True)
        cpu = cpu_fn()
    out = {
        "metric": f"{w}: next-token rows/s and HBM GB/s (% peak)",
        "value": rows / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": cfg,
        "hbm_gbps_step": step_gbps,
        "hbm_frac_step": step_gbps / PEAK_HBM_GBPS if step_gbps is not None else None,
        "kernels_ms": {k.replace("mirl_", ""): v for k, v in ms.items()},
        **extra,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def _packed_targets(input_ids, cu):
    """Packed next-token targets [1, T] of the [n, S] ids (the oracle's packing with the
    per-sequence roll), for the CPU baseline's sample."""
    from oracle.logprob import pack_input_ids

    return pack_input_ids(input_ids.cpu(), list(cu), list(cu), roll_shift=-1)


if __name__ == "__main__":
    main()
