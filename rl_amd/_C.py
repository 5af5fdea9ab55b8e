"""ctypes binding of libmirl.so (the gfx950 kernels behind include/mirl.h).

Every wrapper takes torch tensors that already live on a ROCm device, passes
raw pointers, element strides and the current HIP stream, and raises
:class:`MirlError` when the library reports a failure.  The library is loaded
lazily; a missing or unloadable library raises immediately — there is no
fallback implementation.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().with_name("libmirl.so")

DTYPE_CODES = {
    torch.float32: 0,
    torch.bfloat16: 1,
    torch.float16: 2,
    torch.float64: 3,
}

KL_TYPES = {"k1": 1, "k2": 2, "k3": 3}
TIS_TYPES = {None: 0, "tis": 1, "icepop": 2, "adaptive-ppo-clip": 3, "seq-mask-tis": 4}

# metric slots of the ClippedPG kernel (MIRL_M_* in include/mirl.h)
PG_METRIC_SLOTS = {
    "loss": 0,
    "token_mult_prob_error": 1,
    "probs_ratio": 2,
    "probs_ratio_clamped": 3,
    "probs_ratio_min": 4,
    "probs_ratio_max": 5,
    "probs_ratio_clamped_min": 6,
    "probs_ratio_clamped_max": 7,
    "gen_kl_error": 8,
    "policy_kl_error": 9,
    "js_divergence_error": 10,
    "approx_entropy": 11,
    "sampling_importance_ratio": 12,
    "kl_penalty": 13,
    "num_valid_samples": 14,
    "positive_nll_loss": 15,
    "is_oob_ratio": 16,
    "policy_support_excluded_tokens": 17,
    "score_centering_head_mass": 18,
}
PG_NUM_METRICS = 19

# score-centering importance-sampling modes (MIRL_SC_* in include/mirl.h)
SC_MODES = {"off": 0, "is": 1, "tis": 2, "icepop": 3, "adaptive-ppo-clip": 4}

# divergence kinds (MIRL_DIV_* in include/mirl.h)
DIV_KINDS = {"entropy": 0, "cross_entropy": 1, "reverse_kl": 2}


class MirlError(RuntimeError):
    """A libmirl entry point returned a non-zero status."""


class PgConfig(ctypes.Structure):
    _fields_ = [
        ("ratio_clip_min", ctypes.c_double),
        ("ratio_clip_max", ctypes.c_double),
        ("ratio_clip_c", ctypes.c_double),
        ("kl_penalty", ctypes.c_double),
        ("kl_input_clamp", ctypes.c_double),
        ("kl_output_clamp", ctypes.c_double),
        ("tis_ratio", ctypes.c_double),
        ("tis_ratio_min", ctypes.c_double),
        ("adaptive_hi", ctypes.c_double),
        ("adaptive_outer", ctypes.c_double),
        ("nll_weight", ctypes.c_double),
        ("kl_type", ctypes.c_int32),
        ("tis_type", ctypes.c_int32),
        ("has_kl_input_clamp", ctypes.c_int32),
        ("has_kl_output_clamp", ctypes.c_int32),
        ("disable_ppo_ratio", ctypes.c_int32),
        ("token_level_loss", ctypes.c_int32),
        ("sequence_level_is", ctypes.c_int32),
        ("use_is_correction", ctypes.c_int32),
        ("use_on_policy_kl", ctypes.c_int32),
        ("force_on_policy", ctypes.c_int32),
        ("use_cispo", ctypes.c_int32),
        ("full_metrics", ctypes.c_int32),
        ("need_is", ctypes.c_int32),
        ("has_rewards", ctypes.c_int32),
        ("has_support_mask", ctypes.c_int32),
        ("has_unfiltered", ctypes.c_int32),
    ]


class View2D(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("sb", ctypes.c_int64), ("sl", ctypes.c_int64)]


class ScArgs(ctypes.Structure):
    """mirl_score_centering_args."""

    _fields_ = [
        ("mode", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("K", ctypes.c_int64),
        ("lo", ctypes.c_double),
        ("hi", ctypes.c_double),
        ("outer", ctypes.c_double),
        ("plog", ctypes.c_void_p),
        ("p_sb", ctypes.c_int64),
        ("p_sl", ctypes.c_int64),
        ("p_sk", ctypes.c_int64),
        ("qlog", ctypes.c_void_p),
        ("q_sb", ctypes.c_int64),
        ("q_sl", ctypes.c_int64),
        ("q_sk", ctypes.c_int64),
        ("grad", ctypes.c_void_p),
    ]


# exported symbol -> (restype, argtypes)
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
SIGNATURES = {
    "mirl_last_error": (ctypes.c_char_p, []),
    "mirl_version": (ctypes.c_char_p, []),
    "mirl_logprob_fwd": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _P],
    ),
    "mirl_logprob_bwd": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _I64,
         _I64, _P, _I64, _I64, _P],
    ),
    "mirl_logprob_bwd_recheck": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _I64,
         _I64, _P, _P, _I64, _I64, _P, _P, _P],
    ),
    "mirl_clipped_pg_workspace_elems": (_I64, [_I64, _I64, _I]),
    "mirl_clipped_pg": (
        _I,
        [ctypes.POINTER(PgConfig), _I, _I64, _I64] + [View2D] * 8 + [_P] * 8
        + [ctypes.POINTER(ScArgs), _P, _P],
    ),
    "mirl_clipped_pg_noalloc_max_scratch_bytes": (_I64, []),
    "mirl_clipped_pg_noalloc": (
        _I,
        [ctypes.POINTER(PgConfig), _I, _I64, _I64] + [View2D] * 8 + [_P] * 8
        + [ctypes.POINTER(ScArgs), _P],
    ),
    "mirl_score_centering_term": (
        _I,
        [_I, _I64, _I64, ctypes.POINTER(ScArgs), View2D, View2D, _P, _P, _P],
    ),
    "mirl_gather_logprob_fwd": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P,
         _P],
    ),
    "mirl_gather_logprob_workspace_elems": (_I64, [_I64, _I64]),
    "mirl_gather_logprob_bwd": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P,
         _I64, _I64, _I64, _P, _P, _I64, _I64, _P],
    ),
    "mirl_gather_logprob_bwd_recheck": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P,
         _I64, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _P],
    ),
    "mirl_vocab_topk_workspace_bytes": (_I64, [_I64]),
    "mirl_vocab_topk": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _I, _I64, _P, _P, _P, _P],
    ),
    "mirl_divergence_fwd": (
        _I,
        [_I, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P],
    ),
    "mirl_divergence_bwd": (
        _I,
        [_I, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _P,
         _I64, _I64, _P],
    ),
    "mirl_grpo_advantage": (
        _I,
        [_P, _I64, _I64, _I64, _P, _P, _P, _I, _I, _P, _P, _P, _P, _P],
    ),
    "mirl_filtered_logprob_fwd": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, ctypes.c_double, _I,
         ctypes.c_double, _I, _P, _P, _P, _P, _P],
    ),
    "mirl_filtered_logprob_bwd": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, ctypes.c_double,
         ctypes.c_double, _I, _P, _P, _P, _P, _I64, _I64, _P, _I64, _I64, _P, _P],
    ),
    "mirl_filtered_logprob_bwd_workspace_bytes": (_I64, [_I, _I64, _I64, _I64]),
    "mirl_temperature_scale": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, ctypes.c_double, _P]),
    "mirl_temperature_scale_grad": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, ctypes.c_double, _P, _I64, _I64,
         _P],
    ),
    "mirl_linear_ce_workspace_elems": (_I64, [_I64, _I64]),
    "mirl_linear_ce_fwd": (
        _I,
        [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64,
         _I64, _P, _P, _P],
    ),
    "mirl_linear_ce_grad": (
        _I,
        [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _P,
         _I64, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P],
    ),
    "mirl_gemm_bf16_abt": (
        _I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I, _P, _I64, _I, _P, _I64, _I,
             _I64, _P]
    ),
    "mirl_sum_splits_bf16": (_I, [_P, _I64, _I64, _I64, _I64, _P, _I64, _I, _P, _I64, _P, _I64,
                                  _P]),
    "mirl_transpose_bf16": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _P, _P]),
    "mirl_gemm_f32_abt": (
        _I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I, _P, _I64, _I, _P]
    ),
    "mirl_transpose_f32": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "mirl_top_k_top_p_mask": (
        _I,
        [_P, _I, _I64, _I64, _I64, _I, ctypes.c_double, _I, _P, _P, _P, _P, _I64, _P, _I64, _P],
    ),
    "mirl_pack_sequences": (
        _I,
        [_P, _I64, _I64, _I64, ctypes.c_int32, _P, _P, _I64, _P, _I64, _P],
    ),
    "mirl_packed_roll_targets": (_I, [_P, _I64, _P, _I64, _P, _P]),
    "mirl_mask_outside_tokens": (_I, [_P, _I, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P]),
    "mirl_seq_logprob_errors": (
        _I, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _P]
    ),
    "mirl_unpack_rows_fwd": (_I, [_P, _I64, _P, _I64, _I64, _P, _P]),
    "mirl_unpack_rows_bwd": (_I, [_P, _I64, _I64, _P, _I64, _P, _P]),
}

FILTER_KEEP_CAP = 1024  # MIRL_FILTER_KEEP_CAP
FILTER_ROW_INFO_BYTES = 24  # sizeof(mirl_filter_row_info)

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()

# Optional per-launch timing: when set, wrapped entry points record a pair of
# events on the launch stream around each call, keyed by entry-point name.
_timer: Optional[dict] = None
_timer_names: Optional[frozenset] = None


def enable_launch_timing(names: Optional[list] = None) -> dict:
    """Start recording (start, end) torch.cuda.Event pairs per entry point; returns the dict.

    `names` restricts the recording to those entry points (each event pair
    costs a few microseconds of GPU time between neighbouring launches).
    """
    global _timer, _timer_names
    _timer = {}
    _timer_names = None if names is None else frozenset(names)
    return _timer


def disable_launch_timing() -> None:
    global _timer
    _timer = None


class _Timed:
    def __init__(self, name: str, dev: torch.device):
        self.name, self.dev = name, dev
        self.ev = None

    def __enter__(self):
        if _timer is not None and (_timer_names is None or self.name in _timer_names):
            self.ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            self.ev[0].record(torch.cuda.current_stream(self.dev))
        return self

    def __exit__(self, *exc):
        if self.ev is not None and _timer is not None and exc[0] is None:
            self.ev[1].record(torch.cuda.current_stream(self.dev))
            _timer.setdefault(self.name, []).append(self.ev)
        return False


def load() -> ctypes.CDLL:
    """Load libmirl.so (once) and declare the C signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise MirlError(
                    f"{LIB_PATH} is not built; run `python -m rl_amd.csrc.build` "
                    "(or __graft_entry__.build()) first"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def version() -> str:
    return load().mirl_version().decode()


def _check(status: int, what: str) -> None:
    if status != 0:
        msg = load().mirl_last_error().decode()
        raise MirlError(f"{what} failed (status {status}): {msg}")


def _require(cond: bool, what: str) -> None:
    """Argument check that survives ``python -O``: a wrong layout or dtype would
    otherwise reach the kernels as raw pointers."""
    if not cond:
        raise MirlError(f"invalid argument: {what}")


def _require_gpu(*tensors: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        d = t.device
        if dev is None:
            if d.type != "cuda":
                raise MirlError(
                    "rl_amd kernels run on a ROCm GPU; got a tensor on "
                    f"{d} (move inputs to a cuda device)"
                )
            dev = d
        elif d != dev:
            raise MirlError(f"tensors on different devices: {dev} and {d}")
    if dev is None:
        raise MirlError("no device tensor given")
    return dev


def start_fetch(t: torch.Tensor):
    """Enqueue a copy of a small device tensor into a pinned host buffer and
    record an event after it; finish_fetch waits for that event, poll_fetch
    only tests it.

    The copy runs on a side stream (default priority) behind everything already
    enqueued on the current stream, so work the caller enqueues next on the
    current stream (the early logits backward) starts without waiting for the
    copy, and the wait does not include that work either.  Pinned buffers come
    from a pool keyed on (device, dtype, power-of-two size class) and go back to
    it when the values have been read, so overlapping fetches never share a
    buffer and varying sizes reuse a few buffers."""
    n = t.numel()
    dev = t.device
    key = (dev, t.dtype, max(16, 1 << max(n - 1, 0).bit_length()))
    pool = _pinned.setdefault(key, [])
    buf = pool.pop() if pool else torch.empty(key[2], dtype=t.dtype, pin_memory=True)
    side = _fetch_streams.get(dev)
    if side is None:
        side = torch.cuda.Stream(dev)
        _fetch_streams[dev] = side
    side.wait_stream(torch.cuda.current_stream(dev))
    src = t.reshape(-1)
    with torch.cuda.stream(side):
        buf[:n].copy_(src, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(side)
    src.record_stream(side)  # the allocator keeps src until the side stream has read it
    return [buf, ev, n, key]


def _read_fetch(handle) -> list:
    buf, _, n, key = handle
    values = buf[:n].tolist()
    handle[0] = None
    _pinned[key].append(buf)  # reusable: the copy into it has completed
    return values


def finish_fetch(handle) -> list:
    """Wait for start_fetch's copy by polling its event (wakes up sooner than a
    blocking device-to-host copy) and return the values as a list."""
    _require(handle[0] is not None, "this fetch was already read")
    ev = handle[1]
    while not ev.query():
        pass
    return _read_fetch(handle)


def poll_fetch(handle) -> Optional[list]:
    """start_fetch's values if its copy has completed, else None (never waits)."""
    _require(handle[0] is not None, "this fetch was already read")
    if not handle[1].query():
        return None
    return _read_fetch(handle)


def wait_and_fetch(t: torch.Tensor) -> list:
    """Copy a small device tensor to the host and return it as a list."""
    return finish_fetch(start_fetch(t))


_pinned: dict = {}
_fetch_streams: dict = {}


try:  # raw handle of the current stream without building a Stream object
    _raw_stream = torch._C._cuda_getCurrentRawStream  # type: ignore[attr-defined]
except AttributeError:  # pragma: no cover - older torch
    _raw_stream = None


def _stream(dev: torch.device) -> ctypes.c_void_p:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(idx))
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


class _OnDevice:
    """Make `dev` current for the duration of a launch (no-op when it already is)."""

    __slots__ = ("dev", "prev")

    def __init__(self, dev: torch.device):
        self.dev = dev
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if self.dev.index is not None and cur != self.dev.index:
            self.prev = cur
            torch.cuda.set_device(self.dev)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def _launch(name: str, dev: torch.device, *args):
    """Call entry point `name` with `dev` current (and timed when launch timing is on)."""
    fn = getattr(_lib if _lib is not None else load(), name)
    if _timer is None and (dev.index is None or dev.index == torch.cuda.current_device()):
        return fn(*args)
    with _OnDevice(dev), _Timed(name, dev):
        return fn(*args)


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise MirlError(f"unsupported dtype {t.dtype}") from None


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# logprob forward / backward
# ---------------------------------------------------------------------------
def logprob_fwd(
    logits: torch.Tensor,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    out: torch.Tensor,
    stats: Optional[torch.Tensor],
) -> None:
    """out[b, r] = log_softmax(logits[b, r])[target[b, r] - vocab_start] (0 when out of range).

    logits: [B, >=R, V] (unit stride on V); target: [B, R] int64; out: [B, R]
    fp32 contiguous; stats: [B, R, 2] fp32 contiguous or None.
    """
    dev = _require_gpu(logits, target, out, stats)
    B, R = target.shape
    V = logits.shape[-1]
    _require(logits.stride(-1) == 1 and out.is_contiguous(), "logits.stride(-1) == 1 and out.is_contiguous()")
    _require(stats is None or stats.is_contiguous(), "stats is None or stats.is_contiguous()")
    st = _launch(
        "mirl_logprob_fwd", dev,
        logits.data_ptr(), _dtype_code(logits), B, R, V, logits.stride(0), logits.stride(1),
        target.data_ptr(), target.stride(0), target.stride(1), int(vocab_start),
        int(vocab_end), out.data_ptr(), _ptr(stats), _stream(dev),
    )
    _check(st, "mirl_logprob_fwd")


def logprob_bwd(
    logits: torch.Tensor,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    stats: torch.Tensor,
    grad_out: torch.Tensor,
    grad_in: torch.Tensor,
) -> None:
    """grad_in[b, r, :] = (onehot(target) - softmax(logits[b, r])) * grad_out[b, r].

    Rows r >= R (= target.shape[1]) of grad_in are zeroed.  grad_in may be logits itself.
    """
    dev = _require_gpu(logits, target, stats, grad_out, grad_in)
    B, R = target.shape
    Rt = grad_in.shape[1]
    V = logits.shape[-1]
    _require(grad_in.stride(-1) == 1 and logits.stride(-1) == 1, "grad_in.stride(-1) == 1 and logits.stride(-1) == 1")
    _require(grad_in.dtype == logits.dtype and grad_out.dtype == torch.float32, "grad_in.dtype == logits.dtype and grad_out.dtype == torch.float32")
    st = _launch(
        "mirl_logprob_bwd", dev,
        logits.data_ptr(), _dtype_code(logits), B, R, Rt, V, logits.stride(0),
        logits.stride(1), target.data_ptr(), target.stride(0), target.stride(1),
        int(vocab_start), int(vocab_end), stats.data_ptr(), grad_out.data_ptr(),
        grad_out.stride(0), grad_out.stride(1), grad_in.data_ptr(), grad_in.stride(0),
        grad_in.stride(1), _stream(dev),
    )
    _check(st, "mirl_logprob_bwd")


def logprob_bwd_recheck(
    logits: torch.Tensor,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    stats: torch.Tensor,
    grad_out: torch.Tensor,
    grad_used: torch.Tensor,
    grad_in: torch.Tensor,
    listed: bool = True,
) -> torch.Tensor:
    """grad_in was written by logprob_bwd for grad_used; make it right for grad_out (device-side check).

    Returns the check's flags ([64] int32 on the device, all zero when grad_out
    equals grad_used bit for bit): one flag per check workgroup (with ``listed``,
    the number of its rows that differ; the redo then visits only those rows)."""
    dev = _require_gpu(logits, target, stats, grad_out, grad_used, grad_in)
    B, R = target.shape
    Rt = grad_in.shape[1]
    V = logits.shape[-1]
    _require(grad_used.is_contiguous() and tuple(grad_used.shape) == (B, R), "grad_used.is_contiguous() and tuple(grad_used.shape) == (B, R)")
    _require(grad_out.dtype == torch.float32 and grad_used.dtype == torch.float32, "grad_out.dtype == torch.float32 and grad_used.dtype == torch.float32")
    flag = torch.empty(64, dtype=torch.int32, device=dev)  # MIRL_RECHECK_FLAGS
    rows_ws = torch.empty(max(1, B * R), dtype=torch.int32, device=dev) if listed else None
    st = _launch(
        "mirl_logprob_bwd_recheck", dev,
        logits.data_ptr(), _dtype_code(logits), B, R, Rt, V, logits.stride(0), logits.stride(1),
        target.data_ptr(), target.stride(0), target.stride(1), int(vocab_start), int(vocab_end),
        stats.data_ptr(), grad_out.data_ptr(), grad_out.stride(0), grad_out.stride(1),
        grad_used.data_ptr(), grad_in.data_ptr(), grad_in.stride(0), grad_in.stride(1),
        flag.data_ptr(), _ptr(rows_ws), _stream(dev),
    )
    _check(st, "mirl_logprob_bwd_recheck")
    return flag[: min(B * R, 64)]  # one flag per check workgroup


# ---------------------------------------------------------------------------
# ClippedPG loss
# ---------------------------------------------------------------------------
def _view(t: Optional[torch.Tensor]) -> View2D:
    if t is None:
        return View2D(None, 0, 0)
    return View2D(t.data_ptr(), t.stride(0), t.stride(1))


def clipped_pg(
    cfg: PgConfig,
    curr: torch.Tensor,
    unfiltered: Optional[torch.Tensor],
    token_mask: torch.Tensor,
    advantages: torch.Tensor,
    prev: Optional[torch.Tensor],
    generation: torch.Tensor,
    reference: Optional[torch.Tensor],
    support_mask: Optional[torch.Tensor],
    sample_mask: torch.Tensor,
    rewards: Optional[torch.Tensor],
    global_valid_seqs: torch.Tensor,
    global_valid_toks: torch.Tensor,
    score_centering: Optional[ScArgs] = None,
    loss_out: Optional[torch.Tensor] = None,
    noalloc: bool = False,
) -> tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Run the fused ClippedPG kernel; returns (metrics[19], grad_curr, grad_unfiltered).

    ``loss_out`` (optional, one element of the loss dtype) receives the loss as
    well, written by the kernel itself (no copy out of the metrics).

    ``noalloc=True`` calls ``mirl_clipped_pg_noalloc``, whose scratch is the
    library's fixed per-GPU array instead of a workspace tensor (the outputs
    are still allocated here).

    With ``score_centering`` (a filled ScArgs whose ``grad`` points at a
    [B, L, K] buffer of the loss dtype) the correction is added to the loss and
    dloss/dplog is written into that buffer.
    """
    B, L = curr.shape
    dtype = curr.dtype
    if loss_out is not None and (
        loss_out.numel() != 1 or loss_out.dtype != dtype or not loss_out.is_contiguous()
        or loss_out.device != curr.device
    ):
        raise MirlError(
            f"loss_out must be one contiguous {dtype} element on {curr.device}; got "
            f"{tuple(loss_out.shape)} {loss_out.dtype} on {loss_out.device}"
        )
    dev = _require_gpu(curr, token_mask, advantages, generation, sample_mask)
    metrics = torch.empty(PG_NUM_METRICS, dtype=dtype, device=dev)
    grad_curr = torch.empty((B, L), dtype=dtype, device=dev)
    grad_unf = torch.empty((B, L), dtype=dtype, device=dev) if unfiltered is not None else None
    lib = load()
    args = [
        ctypes.byref(cfg), _dtype_code(curr), B, L, _view(curr), _view(unfiltered),
        _view(token_mask), _view(advantages), _view(prev), _view(generation),
        _view(reference), _view(support_mask), sample_mask.data_ptr(), _ptr(rewards),
        global_valid_seqs.data_ptr(), global_valid_toks.data_ptr(), metrics.data_ptr(),
        _ptr(loss_out), grad_curr.data_ptr(), _ptr(grad_unf),
        None if score_centering is None else ctypes.byref(score_centering),
    ]
    if noalloc:
        name = "mirl_clipped_pg_noalloc"
        st = _launch(name, dev, *args, _stream(dev))
    else:
        name = "mirl_clipped_pg"
        ws = torch.empty(
            int(lib.mirl_clipped_pg_workspace_elems(B, L, int(score_centering is not None))),
            dtype=dtype, device=dev,
        )
        st = _launch(name, dev, *args, ws.data_ptr(), _stream(dev))
    _check(st, name)
    return metrics, grad_curr, grad_unf


def score_centering_args(
    mode: str,
    bounds: Optional[tuple],
    outer: Optional[float],
    plog: torch.Tensor,
    qlog: torch.Tensor,
    grad: torch.Tensor,
) -> ScArgs:
    """Fill mirl_score_centering_args for [B, L, K] views plog / qlog and a contiguous grad buffer."""
    try:
        code = SC_MODES[mode]
    except KeyError:
        raise ValueError(f"Unsupported score-centering IS mode {mode!r}") from None
    _require(plog.dim() == 3 and qlog.shape == plog.shape and grad.shape == plog.shape, "plog.dim() == 3 and qlog.shape == plog.shape and grad.shape == plog.shape")
    _require(plog.dtype == qlog.dtype == grad.dtype and grad.is_contiguous(), "plog.dtype == qlog.dtype == grad.dtype and grad.is_contiguous()")
    lo, hi = bounds if bounds is not None else (0.0, 0.0)
    return ScArgs(
        code, 0, plog.shape[2], float(lo), float(hi), float(outer if outer is not None else 0.0),
        plog.data_ptr(), plog.stride(0), plog.stride(1), plog.stride(2),
        qlog.data_ptr(), qlog.stride(0), qlog.stride(1), qlog.stride(2),
        grad.data_ptr(),
    )


def score_centering_term(
    args: ScArgs,
    dtype: torch.dtype,
    token_mask: torch.Tensor,
    advantages: Optional[torch.Tensor],
    term: torch.Tensor,
    head_mass: torch.Tensor,
) -> None:
    """term / head_mass [B, L] (contiguous) and coef (into args.grad) of compute_score_centering_term."""
    dev = _require_gpu(token_mask, advantages, term, head_mass)
    B, L = token_mask.shape
    _require(term.is_contiguous() and head_mass.is_contiguous(), "term.is_contiguous() and head_mass.is_contiguous()")
    st = _launch(
        "mirl_score_centering_term", dev,
        DTYPE_CODES[dtype], B, L, ctypes.byref(args), _view(token_mask), _view(advantages),
        term.data_ptr(), head_mass.data_ptr(), _stream(dev),
    )
    _check(st, "mirl_score_centering_term")


# ---------------------------------------------------------------------------
# logprobs at K ids per row
# ---------------------------------------------------------------------------
def gather_logprob_fwd(
    logits: torch.Tensor,
    indices: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    out: torch.Tensor,
    stats: Optional[torch.Tensor],
) -> None:
    """out[b, r, k] = log_softmax(logits[b, r])[indices[b, r, k] - vocab_start] (0 out of range).

    logits: [B, R, V] (unit stride on V); indices: [B, R, K] int64; out: [B, R, K]
    fp32 contiguous; stats: [B, R, 2] fp32 contiguous or None.
    """
    dev = _require_gpu(logits, indices, out, stats)
    B, R, K = indices.shape
    V = logits.shape[-1]
    _require(logits.stride(-1) == 1 and out.is_contiguous() and indices.dtype == torch.int64, "logits.stride(-1) == 1 and out.is_contiguous() and indices.dtype == torch.int64")
    _require(stats is None or stats.is_contiguous(), "stats is None or stats.is_contiguous()")
    st = _launch(
        "mirl_gather_logprob_fwd", dev,
        logits.data_ptr(), _dtype_code(logits), B, R, V, logits.stride(0), logits.stride(1),
        indices.data_ptr(), K, indices.stride(0), indices.stride(1), indices.stride(2),
        int(vocab_start), int(vocab_end), out.data_ptr(), _ptr(stats), _stream(dev),
    )
    _check(st, "mirl_gather_logprob_fwd")


def gather_logprob_bwd(
    logits: torch.Tensor,
    indices: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    stats: torch.Tensor,
    grad_out: torch.Tensor,
    grad_in: torch.Tensor,
) -> None:
    """grad_in = -softmax * sum_k g_k + scatter of g_k at the in-range ids (rounded once)."""
    dev = _require_gpu(logits, indices, stats, grad_out, grad_in)
    B, R, K = indices.shape
    V = logits.shape[-1]
    _require(grad_in.stride(-1) == 1 and logits.stride(-1) == 1, "grad_in.stride(-1) == 1 and logits.stride(-1) == 1")
    _require(grad_in.dtype == logits.dtype and grad_out.dtype == torch.float32, "grad_in.dtype == logits.dtype and grad_out.dtype == torch.float32")
    lib = load()
    ws = torch.empty(int(lib.mirl_gather_logprob_workspace_elems(B, R)), dtype=torch.float32,
                     device=dev)
    st = _launch(
        "mirl_gather_logprob_bwd", dev,
        logits.data_ptr(), _dtype_code(logits), B, R, V, logits.stride(0), logits.stride(1),
        indices.data_ptr(), K, indices.stride(0), indices.stride(1), indices.stride(2),
        int(vocab_start), int(vocab_end), stats.data_ptr(), grad_out.data_ptr(),
        grad_out.stride(0), grad_out.stride(1), grad_out.stride(2), ws.data_ptr(),
        grad_in.data_ptr(), grad_in.stride(0), grad_in.stride(1), _stream(dev),
    )
    _check(st, "mirl_gather_logprob_bwd")


def gather_logprob_bwd_recheck(
    logits: torch.Tensor,
    indices: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    stats: torch.Tensor,
    grad_out: torch.Tensor,
    grad_used: torch.Tensor,
    grad_in: torch.Tensor,
) -> torch.Tensor:
    """Recompute grad_in from grad_out on the device only if it differs from grad_used.

    Returns the check's flags (int32 on the device, all zero when nothing differed)."""
    dev = _require_gpu(logits, indices, stats, grad_out, grad_used, grad_in)
    B, R, K = indices.shape
    V = logits.shape[-1]
    _require(grad_in.stride(-1) == 1 and logits.stride(-1) == 1, "grad_in.stride(-1) == 1 and logits.stride(-1) == 1")
    _require(grad_out.dtype == torch.float32 and grad_used.dtype == torch.float32, "grad_out.dtype == torch.float32 and grad_used.dtype == torch.float32")
    _require(grad_used.is_contiguous() and tuple(grad_used.shape) == (B, R, K), "grad_used.is_contiguous() and tuple(grad_used.shape) == (B, R, K)")
    lib = load()
    ws = torch.empty(int(lib.mirl_gather_logprob_workspace_elems(B, R)), dtype=torch.float32,
                     device=dev)
    flags = torch.empty(64, dtype=torch.int32, device=dev)  # MIRL_RECHECK_FLAGS
    st = _launch(
        "mirl_gather_logprob_bwd_recheck", dev,
        logits.data_ptr(), _dtype_code(logits), B, R, V, logits.stride(0), logits.stride(1),
        indices.data_ptr(), K, indices.stride(0), indices.stride(1), indices.stride(2),
        int(vocab_start), int(vocab_end), stats.data_ptr(), grad_out.data_ptr(),
        grad_out.stride(0), grad_out.stride(1), grad_out.stride(2), grad_used.data_ptr(),
        flags.data_ptr(), ws.data_ptr(), grad_in.data_ptr(), grad_in.stride(0), grad_in.stride(1),
        _stream(dev),
    )
    _check(st, "mirl_gather_logprob_bwd_recheck")
    return flags[: min(B * R * K, 64)]  # one flag per check workgroup


def vocab_topk(logits: torch.Tensor, k: int, vocab_start: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(values fp32 [B, R, k], global ids int64 [B, R, k]) of the k largest logits per row."""
    dev = _require_gpu(logits)
    B, R, V = logits.shape
    _require(logits.stride(-1) == 1, "logits.stride(-1) == 1")
    vals = torch.empty((B, R, k), dtype=torch.float32, device=dev)
    idx = torch.empty((B, R, k), dtype=torch.int64, device=dev)
    lib = load()
    ws = torch.empty(max(1, int(lib.mirl_vocab_topk_workspace_bytes(B * R))), dtype=torch.uint8,
                     device=dev)
    st = _launch(
        "mirl_vocab_topk", dev,
        logits.data_ptr(), _dtype_code(logits), B, R, V, logits.stride(0), logits.stride(1),
        int(k), int(vocab_start), vals.data_ptr(), idx.data_ptr(), ws.data_ptr(), _stream(dev),
    )
    _check(st, "mirl_vocab_topk")
    return vals, idx


# ---------------------------------------------------------------------------
# student / teacher divergences
# ---------------------------------------------------------------------------
def divergence_fwd(
    kind: str,
    student: torch.Tensor,
    teacher: Optional[torch.Tensor],
    out: torch.Tensor,
    stats: Optional[torch.Tensor],
) -> None:
    """out[b, r] = entropy / cross entropy / reverse KL of the row; stats [B, R, 4] or None."""
    dev = _require_gpu(student, teacher, out, stats)
    B, R, V = student.shape
    _require(student.stride(-1) == 1 and out.is_contiguous(), "student.stride(-1) == 1 and out.is_contiguous()")
    _require(teacher is None or (teacher.stride(-1) == 1 and teacher.dtype == student.dtype), "teacher is None or (teacher.stride(-1) == 1 and teacher.dtype == student.dtype)")
    _require(stats is None or stats.is_contiguous(), "stats is None or stats.is_contiguous()")
    t = teacher if teacher is not None else student
    st = _launch(
        "mirl_divergence_fwd", dev,
        DIV_KINDS[kind], student.data_ptr(), _ptr(teacher), _dtype_code(student), B, R, V,
        student.stride(0), student.stride(1), t.stride(0), t.stride(1), out.data_ptr(),
        _ptr(stats), _stream(dev),
    )
    _check(st, "mirl_divergence_fwd")


def divergence_bwd(
    kind: str,
    student: torch.Tensor,
    teacher: Optional[torch.Tensor],
    out: torch.Tensor,
    stats: torch.Tensor,
    grad_out: torch.Tensor,
    grad_in: torch.Tensor,
) -> None:
    """grad_in[b, r, v] = (p_v (w_v - out[b, r])) * grad_out[b, r] in the logits dtype."""
    dev = _require_gpu(student, teacher, out, stats, grad_out, grad_in)
    B, R, V = student.shape
    _require(grad_in.stride(-1) == 1 and grad_in.dtype == student.dtype, "grad_in.stride(-1) == 1 and grad_in.dtype == student.dtype")
    _require(grad_out.dtype == torch.float32, "grad_out.dtype == torch.float32")
    t = teacher if teacher is not None else student
    st = _launch(
        "mirl_divergence_bwd", dev,
        DIV_KINDS[kind], student.data_ptr(), _ptr(teacher), _dtype_code(student), B, R, V,
        student.stride(0), student.stride(1), t.stride(0), t.stride(1), out.data_ptr(),
        stats.data_ptr(), grad_out.data_ptr(), grad_out.stride(0), grad_out.stride(1),
        grad_in.data_ptr(), grad_in.stride(0), grad_in.stride(1), _stream(dev),
    )
    _check(st, "mirl_divergence_bwd")


# ---------------------------------------------------------------------------
# GRPO advantages
# ---------------------------------------------------------------------------
def grpo_advantage(
    prompts: torch.Tensor,
    rewards: torch.Tensor,
    valid_mask: Optional[torch.Tensor],
    leave_one_out: bool,
    normalize: bool,
    want_stats: bool = False,
    std_rewards: Optional[torch.Tensor] = None,
) -> tuple[
    torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor], Optional[torch.Tensor]
]:
    """GRPO advantages [B]; with want_stats also (baseline, std, trivial) per sample."""
    dev = _require_gpu(prompts, rewards, valid_mask)
    B = rewards.shape[0]
    K = prompts.shape[1]
    _require(prompts.dtype == torch.int64 and prompts.stride(1) == 1, "prompts.dtype == torch.int64 and prompts.stride(1) == 1")
    _require(rewards.dtype == torch.float32 and rewards.is_contiguous(), "rewards.dtype == torch.float32 and rewards.is_contiguous()")
    adv = torch.empty(B, dtype=torch.float32, device=dev)
    base = torch.empty_like(adv) if want_stats else None
    std = torch.empty_like(adv) if want_stats else None
    trivial = torch.empty(B, dtype=torch.bool, device=dev) if want_stats else None
    st = _launch(
        "mirl_grpo_advantage", dev,
        prompts.data_ptr(), B, K, prompts.stride(0), rewards.data_ptr(), _ptr(std_rewards),
        _ptr(valid_mask),
        int(bool(leave_one_out)), int(bool(normalize)), adv.data_ptr(), _ptr(base), _ptr(std),
        _ptr(trivial), _stream(dev),
    )
    _check(st, "mirl_grpo_advantage")
    return adv, base, std, trivial


# ---------------------------------------------------------------------------
# packed-sequence glue
# ---------------------------------------------------------------------------
def pack_sequences(
    x: torch.Tensor, cu_seqlens: torch.Tensor, cu_seqlens_padded: torch.Tensor, roll_shift: int,
    total: int,
) -> torch.Tensor:
    """``[B, S, ...]`` rows packed to ``[total, ...]`` along the padded boundaries (device int64)."""
    dev = _require_gpu(x, cu_seqlens, cu_seqlens_padded)
    _require(x.is_contiguous() and x.dim() >= 2, "x.is_contiguous() and x.dim() >= 2")
    _require(cu_seqlens.dtype == torch.int64 and cu_seqlens_padded.dtype == torch.int64, "cu_seqlens.dtype == torch.int64 and cu_seqlens_padded.dtype == torch.int64")
    B, S = x.shape[0], x.shape[1]
    tail = tuple(x.shape[2:])
    row = 1
    for d in tail:
        row *= d
    out = torch.empty((total, *tail), dtype=x.dtype, device=dev)
    if total == 0 or row == 0:
        return out.zero_()
    st = _launch(
        "mirl_pack_sequences", dev,
        x.data_ptr(), B, S, row, x.element_size(), cu_seqlens.data_ptr(),
        cu_seqlens_padded.data_ptr(), int(roll_shift), out.data_ptr(), total, _stream(dev),
    )
    _check(st, "mirl_pack_sequences")
    return out


def packed_roll_targets(target: torch.Tensor, bounds: torch.Tensor) -> torch.Tensor:
    """Per-segment roll by -1 of packed int64 targets ``[n]`` (0 outside the segments)."""
    dev = _require_gpu(target, bounds)
    _require(target.dtype == torch.int64 and target.is_contiguous() and bounds.dtype == torch.int64, "target.dtype == torch.int64 and target.is_contiguous() and bounds.dtype == torch.int64")
    out = torch.empty_like(target)
    st = _launch(
        "mirl_packed_roll_targets", dev,
        target.data_ptr(), target.numel(), bounds.data_ptr(), bounds.numel() - 1, out.data_ptr(),
        _stream(dev),
    )
    _check(st, "mirl_packed_roll_targets")
    return out


def unpack_rows_fwd(packed: torch.Tensor, bounds: torch.Tensor, cols: int) -> torch.Tensor:
    """Packed fp32 rows ``[n_rows]`` -> ``[n_seq, cols]`` (zeros after each sequence)."""
    dev = _require_gpu(packed, bounds)
    _require(packed.dtype == torch.float32 and packed.is_contiguous() and bounds.dtype == torch.int64, "packed.dtype == torch.float32 and packed.is_contiguous() and bounds.dtype == torch.int64")
    n_seq = bounds.numel() - 1
    out = torch.empty((n_seq, cols), dtype=torch.float32, device=dev)
    st = _launch(
        "mirl_unpack_rows_fwd", dev,
        packed.data_ptr(), packed.numel(), bounds.data_ptr(), n_seq, cols, out.data_ptr(),
        _stream(dev),
    )
    _check(st, "mirl_unpack_rows_fwd")
    return out


def unpack_rows_bwd(grad_out: torch.Tensor, bounds: torch.Tensor, n_rows: int) -> torch.Tensor:
    """Backward of unpack_rows_fwd: ``[n_seq, cols]`` -> ``[n_rows]`` (zeros for rows not copied)."""
    dev = _require_gpu(grad_out, bounds)
    g = grad_out.float().contiguous()
    n_seq, cols = g.shape
    out = torch.empty(n_rows, dtype=torch.float32, device=dev)
    st = _launch(
        "mirl_unpack_rows_bwd", dev,
        g.data_ptr(), n_seq, cols, bounds.data_ptr(), n_rows, out.data_ptr(), _stream(dev),
    )
    _check(st, "mirl_unpack_rows_bwd")
    return out


# ---------------------------------------------------------------------------
# top-k / top-p filtered logprobs
# ---------------------------------------------------------------------------
def _filter_scratch(rows: int, dev: torch.device):
    info = torch.empty(rows * FILTER_ROW_INFO_BYTES, dtype=torch.uint8, device=dev)
    kidx = torch.empty((rows, FILTER_KEEP_CAP), dtype=torch.int32, device=dev)
    kp = torch.empty((rows, FILTER_KEEP_CAP), dtype=torch.float32, device=dev)
    return info, kidx, kp


def _decision_code(logits: torch.Tensor, decision_dtype: Optional[torch.dtype]) -> int:
    """MIRL dtype code of the top-p decision: the logits dtype (None) or fp32."""
    d = logits.dtype if decision_dtype is None else decision_dtype
    if d not in (torch.float32, logits.dtype):
        raise MirlError(f"top-p decision dtype must be float32 or the logits dtype {logits.dtype}, got {d}")
    return DTYPE_CODES[d]


def filtered_fwd(
    logits: torch.Tensor,
    target: torch.Tensor,
    temperature: float,
    top_k: int,
    top_p: float,
    out: Optional[torch.Tensor],
    decision_dtype: Optional[torch.dtype] = None,
):
    """Filtered logprobs of rows 0..R-1 (R = target.shape[1]); returns (info, kept_idx, kept_p).

    ``decision_dtype`` is the dtype the top-p probabilities and their cumulative
    sum are formed in: None = the logits dtype (the reference on that tensor),
    torch.float32 = after an fp32 upcast."""
    dev = _require_gpu(logits, target, out)
    B, R = target.shape
    V = logits.shape[-1]
    _require(logits.stride(-1) == 1 and (out is None or out.is_contiguous()), "logits.stride(-1) == 1 and (out is None or out.is_contiguous())")
    info, kidx, kp = _filter_scratch(B * R, dev)
    st = _launch(
        "mirl_filtered_logprob_fwd", dev,
        logits.data_ptr(), _dtype_code(logits), B, R, V, logits.stride(0), logits.stride(1),
        target.data_ptr(), target.stride(0), target.stride(1), float(temperature),
        int(top_k), float(top_p), _decision_code(logits, decision_dtype), _ptr(out),
        info.data_ptr(), kidx.data_ptr(), kp.data_ptr(), _stream(dev),
    )
    _check(st, "mirl_filtered_logprob_fwd")
    return info, kidx, kp


def filtered_bwd(
    logits: torch.Tensor,
    target: torch.Tensor,
    temperature: float,
    info: torch.Tensor,
    kidx: torch.Tensor,
    kp: torch.Tensor,
    grad_out: torch.Tensor,
    grad_in: torch.Tensor,
    grad_temperature: float = 1.0,
    top_k: int = 0,
    pieces: bool = True,
) -> None:
    """``grad_temperature`` != 1 applies the backward of an in-place division of the
    logits by it, made before the forward, to the written gradient last (the product
    with ``fl32(1.0 / grad_temperature)`` in the dtype), folded into this write.  ``top_k`` is the forward's; it picks the
    kernel schedule only (rows with kept lists for 1 <= top_k <= 1024).  Rows without
    kept lists are written in 4 KB pieces with a workspace allocated here (``pieces``;
    False walks each row with a workgroup of its own: the same gradient)."""
    dev = _require_gpu(logits, target, grad_out, grad_in)
    B, R = target.shape
    Rt = grad_in.shape[1]
    V = logits.shape[-1]
    _require(grad_in.dtype == logits.dtype and grad_out.dtype == torch.float32, "grad_in.dtype == logits.dtype and grad_out.dtype == torch.float32")
    ws = None
    if pieces and not (1 <= top_k <= FILTER_KEEP_CAP) and B * R > 0:
        lib = _lib if _lib is not None else load()
        nbytes = int(lib.mirl_filtered_logprob_bwd_workspace_bytes(_dtype_code(logits), B, R, V))
        _require(nbytes >= 0, "workspace size")
        ws = torch.empty(max(1, (nbytes + 3) // 4), dtype=torch.int32, device=dev)
    st = _launch(
        "mirl_filtered_logprob_bwd", dev,
        logits.data_ptr(), _dtype_code(logits), B, R, Rt, V, logits.stride(0),
        logits.stride(1), target.data_ptr(), target.stride(0), target.stride(1),
        float(temperature), float(grad_temperature), int(top_k), info.data_ptr(), kidx.data_ptr(),
        kp.data_ptr(),
        grad_out.data_ptr(), grad_out.stride(0), grad_out.stride(1), grad_in.data_ptr(),
        grad_in.stride(0), grad_in.stride(1), _ptr(ws), _stream(dev),
    )
    _check(st, "mirl_filtered_logprob_bwd")


def _rows3(t: torch.Tensor):
    """(B, R, V, stride_b, stride_r) of a tensor viewed as [B, R, V] rows of its last dim."""
    _require(t.dim() >= 1 and (t.dim() == 1 or t.stride(-1) == 1 or t.shape[-1] == 1),
             "the last dimension must have unit stride")
    if t.dim() == 1:
        return 1, 1, t.shape[0], t.shape[0], t.shape[0]
    if t.dim() == 2:
        return 1, t.shape[0], t.shape[1], t.shape[0] * t.stride(0), t.stride(0)
    lead = t.shape[:-2]
    B = 1
    for d in lead:
        B *= d
    # leading dims must collapse to one stride
    sb = t.stride(-3) if t.dim() >= 3 else t.shape[-2] * t.stride(-2)
    expect = sb
    for i in range(t.dim() - 3, -1, -1):
        _require(t.shape[i] == 1 or t.stride(i) == expect, "leading dimensions do not collapse")
        expect *= t.shape[i]
    return B, t.shape[-2], t.shape[-1], sb, t.stride(-2)


def temperature_scale_(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """In place: logits = dtype(fl32(float(logits) * fl32(1.0 / T))), torch's GPU
    ``div_`` by a Python scalar (mirl_temperature_scale)."""
    dev = _require_gpu(logits)
    B, R, V, sb, sr = _rows3(logits)
    st = _launch("mirl_temperature_scale", dev, logits.data_ptr(), _dtype_code(logits), B, R, V,
                 sb, sr, float(temperature), _stream(dev))
    _check(st, "mirl_temperature_scale")
    return logits


def temperature_scale_grad(grad: torch.Tensor, grad2: Optional[torch.Tensor],
                           temperature: float) -> torch.Tensor:
    """dtype(fl32(float(grad [+ grad2, accumulated in the dtype]) * fl32(1.0 / T))) as a new
    tensor: the autograd backward of the in-place division."""
    dev = _require_gpu(grad, grad2)
    if grad2 is not None:
        _require(grad2.shape == grad.shape and grad2.dtype == grad.dtype, "grad2 matches grad")
    out = torch.empty(grad.shape, dtype=grad.dtype, device=dev)
    if grad.stride(-1) != 1:
        grad = grad.contiguous()
    if grad2 is not None and grad2.stride(-1) != 1:
        grad2 = grad2.contiguous()
    B, R, V, sb, sr = _rows3(grad)
    if grad2 is not None:
        _, _, _, sb2, sr2 = _rows3(grad2)
    else:
        sb2 = sr2 = 0
    _, _, _, osb, osr = _rows3(out)
    st = _launch("mirl_temperature_scale_grad", dev, grad.data_ptr(), _dtype_code(grad), B, R, V,
                 sb, sr, _ptr(grad2), sb2, sr2, float(temperature), out.data_ptr(), osb, osr,
                 _stream(dev))
    _check(st, "mirl_temperature_scale_grad")
    return out


def top_k_top_p_mask(x2d: torch.Tensor, top_k: int, top_p: float,
                     decision_dtype: Optional[torch.dtype] = None):
    """[N, V] rows -> (filtered [N, V] in x's dtype, keep [N, V] bool); ``decision_dtype``
    as for filtered_fwd."""
    dev = _require_gpu(x2d)
    N, V = x2d.shape
    _require(x2d.stride(1) == 1, "x2d.stride(1) == 1")
    info, kidx, kp = _filter_scratch(N, dev)
    filt = torch.empty((N, V), dtype=x2d.dtype, device=dev)
    keep = torch.empty((N, V), dtype=torch.bool, device=dev)
    st = _launch(
        "mirl_top_k_top_p_mask", dev,
        x2d.data_ptr(), _dtype_code(x2d), N, V, x2d.stride(0), int(top_k), float(top_p),
        _decision_code(x2d, decision_dtype), info.data_ptr(), kidx.data_ptr(), kp.data_ptr(), filt.data_ptr(), filt.stride(0),
        keep.data_ptr(), keep.stride(0), _stream(dev),
    )
    _check(st, "mirl_top_k_top_p_mask")
    return filt, keep


# ---------------------------------------------------------------------------
# logprobs from hidden states (fused LM-head GEMM + log-sum-exp)
# ---------------------------------------------------------------------------
_LCE_DTYPES = (torch.bfloat16, torch.float16)


def _check_linear_ce(hidden2d: torch.Tensor, weight: torch.Tensor) -> None:
    if hidden2d.dtype not in _LCE_DTYPES or weight.dtype != hidden2d.dtype:
        raise NotImplementedError(
            "the fused hidden-state kernels take bf16 or fp16 hidden states and weight of one "
            f"dtype (got {hidden2d.dtype} and {weight.dtype})"
        )
    if hidden2d.stride(-1) != 1 or weight.stride(-1) != 1:
        raise MirlError("hidden states and weight need a unit stride on the hidden dimension")


def linear_ce_fwd(
    hidden2d: torch.Tensor,
    weight: torch.Tensor,
    bsz: int,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    out: torch.Tensor,
    stats: Optional[torch.Tensor],
) -> None:
    """out[b, s] = log_softmax(dtype(hidden2d[s*bsz+b] . weight^T))[target[b, s] - vocab_start].

    hidden2d: [T, H] bf16 or fp16 rows (row r is position (r // bsz, r % bsz)); weight:
    [V, H] of the same dtype; target: [B, S] int64; out: [B, S] fp32; stats: [T, 2] fp32
    or None.
    """
    dev = _require_gpu(hidden2d, weight, target, out, stats)
    _check_linear_ce(hidden2d, weight)
    T, H = hidden2d.shape
    V = weight.shape[0]
    _require(target.dtype == torch.int64 and out.dtype == torch.float32, "target.dtype == torch.int64 and out.dtype == torch.float32")
    _require(stats is None or (stats.is_contiguous() and stats.dtype == torch.float32), "stats is None or (stats.is_contiguous() and stats.dtype == torch.float32)")
    lib = _lib if _lib is not None else load()
    ws = torch.empty(max(1, int(lib.mirl_linear_ce_workspace_elems(T, V))), dtype=torch.float32, device=dev)
    st = _launch(
        "mirl_linear_ce_fwd", dev,
        hidden2d.data_ptr(), _dtype_code(hidden2d), T, H, hidden2d.stride(0), weight.data_ptr(), V, weight.stride(0),
        int(bsz), target.data_ptr(), target.stride(0), target.stride(1), int(vocab_start),
        int(vocab_end), out.data_ptr(), out.stride(0), out.stride(1), _ptr(stats), ws.data_ptr(),
        _stream(dev),
    )
    _check(st, "mirl_linear_ce_fwd")


def linear_ce_grad(
    hidden2d: torch.Tensor,
    weight: torch.Tensor,
    bsz: int,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    stats: torch.Tensor,
    grad_out: torch.Tensor,
    row0: int,
    grad_logits: torch.Tensor,
    grad_logits_t: Optional[torch.Tensor] = None,
    count: Optional[torch.Tensor] = None,
) -> None:
    """grad_logits[i, :] = bf16((onehot(t) - softmax(logits)) * g) for rows row0 .. row0 + n - 1
    (bf16 for either operand dtype);
    grad_logits_t (or None) receives the transpose [V, >= round_up(n, 256)].  `count` (a
    device int64 tensor of one element, or None): rows at or past it are absent."""
    dev = _require_gpu(hidden2d, weight, target, stats, grad_out, grad_logits)
    _check_count(count, dev)
    _check_linear_ce(hidden2d, weight)
    T, H = hidden2d.shape
    V = weight.shape[0]
    n = grad_logits.shape[0]
    _require(grad_out.dtype == torch.float32 and grad_logits.dtype == torch.bfloat16, "grad_out.dtype == torch.float32 and grad_logits.dtype == torch.bfloat16")
    _require(grad_logits.stride(-1) == 1, "grad_logits.stride(-1) == 1")
    st = _launch(
        "mirl_linear_ce_grad", dev,
        hidden2d.data_ptr(), _dtype_code(hidden2d), T, H, hidden2d.stride(0), weight.data_ptr(), V, weight.stride(0),
        int(bsz), target.data_ptr(), target.stride(0), target.stride(1), int(vocab_start),
        int(vocab_end), stats.data_ptr(), grad_out.data_ptr(), grad_out.stride(0),
        grad_out.stride(1), int(row0), int(n), grad_logits.data_ptr(), grad_logits.stride(0),
        _ptr(grad_logits_t), 0 if grad_logits_t is None else grad_logits_t.stride(0), _ptr(count),
        _stream(dev),
    )
    _check(st, "mirl_linear_ce_grad")


COUNT_ROWS = 0  # MIRL_COUNT_ROWS
COUNT_K = 1  # MIRL_COUNT_K


def _check_count(count: Optional[torch.Tensor], dev: torch.device) -> None:
    if count is None:
        return
    _require(count.dtype == torch.int64 and count.numel() == 1 and count.device == dev,
             "count is a one-element int64 tensor on the operands' device")


def gemm_bf16_abt(a: torch.Tensor, b: torch.Tensor, k: int, out: torch.Tensor, k_splits: int = 1,
                  accumulate: bool = False, count: Optional[torch.Tensor] = None,
                  count_off: int = 0, count_axis: int = COUNT_ROWS,
                  out_bf16: Optional[torch.Tensor] = None, final_at: int = 0) -> None:
    """out = a[:, :k] . b[:, :k]^T with fp32 accumulation on the MFMA units.

    a [M, >=k], b [N, >=k] bf16 (unit stride, rows multiples of 8 elements, k a
    multiple of 128); out bf16 or fp16 [M, N] (k_splits 1, no accumulation), fp32 [M, N]
    (out = or +=), or fp32 [k_splits, M, N] (one partial product per k range).
    `count` (device int64, one element) with c = count - count_off: COUNT_ROWS
    leaves rows of a at or past c absent; COUNT_K stops the reduction at
    round_up(c, 128), and with `out_bf16` (a bf16 or fp16 [M, N] tensor, out fp32 [M, N])
    the result goes to out_bf16 = its dtype(product (+ out when accumulate)) when
    count <= final_at, to out otherwise."""
    dev = _require_gpu(a, b, out)
    _check_count(count, dev)
    _require(a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16, "bf16 operands")
    _require(a.stride(-1) == 1 and b.stride(-1) == 1 and out.stride(-1) == 1, "unit stride on the last dim")
    M, N = a.shape[0], b.shape[0]
    cb_dtype = 1
    if out.dtype in _LCE_DTYPES:
        _require(out_bf16 is None, "out_bf16 goes with an fp32 out")
        cb, ldcb, c, ldc = out.data_ptr(), out.stride(0), None, 0
        cb_dtype = _dtype_code(out)
    else:
        _require(out.dtype == torch.float32, "out is bf16, fp16 or fp32")
        cb, ldcb, c, ldc = None, 0, out.data_ptr(), out.stride(-2)
        if out_bf16 is not None:
            _require(out_bf16.dtype in _LCE_DTYPES and out_bf16.device == dev
                     and out_bf16.stride(-1) == 1 and tuple(out_bf16.shape) == (M, N),
                     "out_bf16 is a bf16 [M, N] tensor with unit stride on the last dim")
            _require(out.dim() == 2 and tuple(out.shape) == (M, N), "out is fp32 [M, N]")
            cb, ldcb = out_bf16.data_ptr(), out_bf16.stride(0)
            cb_dtype = _dtype_code(out_bf16)
    st = _launch(
        "mirl_gemm_bf16_abt", dev, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), M, N,
        int(k), int(k_splits), c, ldc, int(bool(accumulate)), cb, ldcb, cb_dtype, _ptr(count),
        int(count_off), int(count_axis), int(final_at), _stream(dev),
    )
    _check(st, "mirl_gemm_bf16_abt")


def gemm_f32_abt(a: torch.Tensor, b: torch.Tensor, k: int, out: torch.Tensor, k_splits: int = 1,
                 accumulate: bool = False, count: Optional[torch.Tensor] = None,
                 count_off: int = 0, count_axis: int = COUNT_ROWS) -> None:
    """out = a[:, :k] . b[:, :k]^T in fp32 on the MFMA units (fp32 MFMA).

    a [M, >=k], b [N, >=k] fp32 (unit stride, row strides multiples of 4 elements,
    16-byte aligned, k a multiple of 64); out fp32 [M, N] (out = or +=), or
    [k_splits, M, N] (one partial product per k range).  `count` (device int64, one
    element) with c = count - count_off: COUNT_ROWS leaves rows of a at or past c
    absent (not read, not written); COUNT_K stops the reduction at round_up(c, 64)."""
    dev = _require_gpu(a, b, out)
    _check_count(count, dev)
    _require(a.dtype == torch.float32 and b.dtype == torch.float32 and out.dtype == torch.float32,
             "fp32 operands and output")
    _require(a.stride(-1) == 1 and b.stride(-1) == 1 and out.stride(-1) == 1, "unit stride on the last dim")
    M, N = a.shape[0], b.shape[0]
    st = _launch(
        "mirl_gemm_f32_abt", dev, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), M, N, int(k),
        int(k_splits), out.data_ptr(), out.stride(-2), int(bool(accumulate)), _ptr(count), int(count_off),
        int(count_axis), _stream(dev),
    )
    _check(st, "mirl_gemm_f32_abt")


def transpose_f32(src: torch.Tensor, rows: int, dst: torch.Tensor, count: Optional[torch.Tensor] = None,
                  count_off: int = 0) -> None:
    """dst[c, r] = src[r, c] (fp32) for r < rows, zero for rows <= r < dst.shape[1]; rows is
    lowered to count - count_off (`count` a device int64, one element) when that is given."""
    dev = _require_gpu(src, dst)
    _check_count(count, dev)
    _require(src.dtype == torch.float32 and dst.dtype == torch.float32, "fp32 source and destination")
    _require(src.stride(-1) == 1 and dst.stride(-1) == 1, "unit stride on the last dim")
    C = src.shape[1]
    _require(dst.shape[0] >= C, "dst has a row per source column")
    _require(src.shape[0] >= rows, "src has the rows to transpose")
    st = _launch("mirl_transpose_f32", dev, src.data_ptr(), int(rows), C, src.stride(0), dst.data_ptr(),
                 dst.stride(0), dst.shape[1], _ptr(count), int(count_off), _stream(dev))
    _check(st, "mirl_transpose_f32")


def sum_splits_bf16(part: torch.Tensor, out: torch.Tensor, count: Optional[torch.Tensor] = None,
                    count_off: int = 0, out_rows: Optional[torch.Tensor] = None) -> None:
    """out [M, N] bf16, fp16 or fp32 = sum over dim 0 of part [S, M, N] fp32, in order; with `count`,
    rows at or past count - count_off are zeros (part not read there).  With `out_rows`
    (int64 [M] on the device) row m goes to out[out_rows[m]] instead (out [R, N], rows
    mapped outside [0, R) skipped)."""
    dev = _require_gpu(part, out)
    _check_count(count, dev)
    S, M, N = part.shape
    _require(part.is_contiguous() and part.dtype == torch.float32
             and (out.dtype in _LCE_DTYPES or out.dtype == torch.float32)
             and out.stride(-1) == 1 and out.dim() == 2 and out.shape[1] == N,
             "contiguous fp32 partials and a bf16, fp16 or fp32 [R, N] output")
    if out_rows is None:
        _require(out.shape[0] == M, "out has the partials' rows")
    else:
        _require(out_rows.dtype == torch.int64 and out_rows.device == dev and out_rows.dim() == 1
                 and out_rows.shape[0] == M and out_rows.is_contiguous(),
                 "out_rows is a contiguous int64 [M] tensor on the device")
    st = _launch("mirl_sum_splits_bf16", dev, part.data_ptr(), S, M, N, N, out.data_ptr(),
                 out.stride(0), _dtype_code(out), _ptr(out_rows), out.shape[0], _ptr(count), int(count_off),
                 _stream(dev))
    _check(st, "mirl_sum_splits_bf16")


def transpose_bf16(src: torch.Tensor, rows: int, dst: torch.Tensor,
                   count: Optional[torch.Tensor] = None) -> None:
    """dst[c, r] = bf16(src[r, c]) for r < rows, zero for rows <= r < dst.shape[1] (src
    bf16 or fp16, dst bf16); rows is lowered to `count` (device int64, one element) when
    that is given."""
    dev = _require_gpu(src, dst)
    _check_count(count, dev)
    _require(src.dtype in _LCE_DTYPES and dst.dtype == torch.bfloat16, "bf16 or fp16 source, bf16 destination")
    _require(src.stride(-1) == 1 and dst.stride(-1) == 1, "unit stride on the last dim")
    C = src.shape[1]
    _require(dst.shape[0] >= C, "dst has a row per source column")
    _require(src.shape[0] >= rows, "src has the rows to transpose")
    st = _launch("mirl_transpose_bf16", dev, src.data_ptr(), _dtype_code(src), int(rows), C, src.stride(0),
                 dst.data_ptr(), dst.stride(0), dst.shape[1], _ptr(count), _stream(dev))
    _check(st, "mirl_transpose_bf16")


# ---------------------------------------------------------------------------
# token-level post-processing of logprobs
# ---------------------------------------------------------------------------
def _as_f32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.float32 else t.to(torch.float32)


def mask_outside_tokens(logprobs: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """where(mask != 0, logprobs, 0) for [B, S] (or [S]) logprobs of any float dtype and a
    mask that broadcasts to them; returns a new tensor of the logprobs' dtype."""
    dev = _require_gpu(logprobs, mask)
    _require(logprobs.dim() in (1, 2), "logprobs of shape [B, S] or [S]")
    lp = logprobs if logprobs.dim() == 2 else logprobs.unsqueeze(0)
    m = _as_f32(mask)
    m = m if m.dim() == 2 else m.reshape((1,) * (2 - m.dim()) + tuple(m.shape))
    m = m.expand(lp.shape)
    out = torch.empty(lp.shape, dtype=lp.dtype, device=dev)
    B, S = lp.shape
    st = _launch(
        "mirl_mask_outside_tokens", dev, lp.data_ptr(), _dtype_code(lp), B, S, lp.stride(0),
        lp.stride(1), m.data_ptr(), m.stride(0), m.stride(1), out.data_ptr(), out.stride(0),
        out.stride(1), _stream(dev),
    )
    _check(st, "mirl_mask_outside_tokens")
    return out if logprobs.dim() == 2 else out[0]


def seq_logprob_errors(policy: torch.Tensor, generation: torch.Tensor, token_mask: torch.Tensor,
                       sample_mask: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(errors fp32 [B], valid bool [B]) of the mean multiplicative logprob error per sequence."""
    dev = _require_gpu(policy, generation, token_mask, sample_mask)
    _require(policy.dim() == 2 and tuple(generation.shape) == tuple(policy.shape),
             "policy and generation logprobs of one [B, S] shape")
    B, S = policy.shape
    _require(policy.dtype == torch.float32 and generation.dtype == torch.float32,
             "policy.dtype == generation.dtype == torch.float32")
    tm = _as_f32(token_mask).expand(B, S)
    sm = _as_f32(sample_mask)
    _require(sm.dim() == 1 and sm.shape[0] == B, "sample_mask of shape [B]")
    errors = torch.empty(B, dtype=torch.float32, device=dev)
    valid = torch.empty(B, dtype=torch.bool, device=dev)
    st = _launch(
        "mirl_seq_logprob_errors", dev, policy.data_ptr(), policy.stride(0), policy.stride(1),
        generation.data_ptr(), generation.stride(0), generation.stride(1), tm.data_ptr(),
        tm.stride(0), tm.stride(1), sm.data_ptr(), sm.stride(0), B, S, errors.data_ptr(),
        valid.data_ptr(), _stream(dev),
    )
    _check(st, "mirl_seq_logprob_errors")
    return errors, valid
