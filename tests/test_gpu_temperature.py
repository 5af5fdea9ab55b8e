"""In-place temperature scaling and the reference's call sequence around it (GPU).

The reference divides the model's logits in place (apply_temperature_scaling,
nemo_rl/models/automodel/train.py:248-262) and then calls
prepare_loss_input(sampling_params=...), whose get_next_token path upcasts and
filters (model_utils.py:1660-1718); autograd runs the division's backward on
the summed gradient of every consumer.  The reference runs this on the GPU,
where torch's own division by a Python scalar is a product with fl32(1.0 / T)
(forward and backward), rounded to the dtype: the kernel is compared bit for
bit with the oracle's restatement of it, and the oracle with torch's GPU div_
and its autograd backward (for fp16 at logits-like sizes, where torch takes
its vectorised kernel; its element-wise fp16 path rounds differently).  The
chains after the division are compared with the CPU oracle: values and
gradients bit-exactly where the arithmetic is the same rounding sequence,
filtered logprobs within 2e-3, bf16 gradients within 1e-3 or one bf16 ulp.
"""

import numpy as np
import pytest
import torch

from oracle.sampling import apply_temperature, next_token_filtered, temperature_recip, top_k_top_p
from rl_amd.algorithms.logits_sampling_utils import TrainingSamplingParams, apply_temperature_scaling
from rl_amd.distributed.model_utils import get_next_token_logprobs_from_logits
from tests.helpers import assert_close_or_ulp_bf16

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

# temperatures where fl32(1.0 / T) and the fp32 reciprocal of fl32(T) differ (1.1,
# 2.2020148549027954) and ordinary ones
TEMPS = [0.7, 1.3, 0.3, 1.1, 2.2020148549027954]


def _torch_gpu_rounds_like_the_oracle(dtype, n_elems):
    """Whether torch's own GPU division of a tensor of n_elems is the oracle's rounding.

    bf16 and fp32: always.  fp16: torch's vectorised kernel (what logits-sized tensors
    take) rounds the fp32 product to fp16, but its element-wise path (small tensors,
    remainders) rounds the exact product to fp16 once (measured: a [2, 3, 50] fp16 tensor
    at T = 0.3 rounds 24 of 300 elements differently, a [2^18] one none), so torch is
    compared at logits-like sizes only."""
    return dtype != torch.float16 or n_elems >= (1 << 16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T", TEMPS)
@pytest.mark.parametrize("shape,offset", [((3, 7, 1001), 0), ((2, 5, 4096), 3), ((1, 1, 9), 1),
                                          ((4, 8, 8192), 0)])
def test_in_place_division_bits(dtype, T, shape, offset):
    """x.div_(T) in the dtype, for aligned and unaligned (offset) rows: bit-equal to the
    oracle's product, which is torch's own GPU division bit for bit."""
    print("[case] scale", dtype, T, shape, offset, flush=True)
    n = 1
    for d in shape:
        n *= d
    g = torch.Generator().manual_seed(1)
    flat = (torch.randn(n + offset, generator=g) * 3).to(dtype)
    x_cpu = flat[offset:].view(shape)
    want = apply_temperature(x_cpu, T)
    if _torch_gpu_rounds_like_the_oracle(dtype, n):
        assert torch.equal(flat.to(DEV)[offset:].view(shape).clone().div_(T).cpu(), want)
    xd = flat.to(DEV)[offset:].view(shape)
    out = apply_temperature_scaling(xd, TrainingSamplingParams(temperature=T))
    assert out is xd
    assert torch.equal(xd.cpu(), want)
    # a strided view (every other row) is divided in place as well
    y = (torch.randn(4, 6, 33, generator=g) * 3).to(dtype)
    want = y.clone()
    want[:, ::2] = apply_temperature(y[:, ::2], T)
    yd = y.to(DEV)
    apply_temperature_scaling(yd[:, ::2], TrainingSamplingParams(temperature=T))
    assert torch.equal(yd.cpu(), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("T", TEMPS)
@pytest.mark.parametrize("shape", [(2, 3, 50), (4, 16, 4096)])
def test_division_backward_alone(dtype, T, shape):
    """A plain consumer: the gradient through the in-place division is the oracle's
    autograd of the product, dtype(fl32(g * fl32(1.0 / T))), which is torch's GPU
    autograd of div_ bit for bit."""
    print("[case] scale backward", dtype, T, shape, flush=True)
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(*shape, generator=g) * 2).to(dtype)
    w = torch.randn(*shape, generator=g).to(dtype)
    r = np.float32(1.0 / T)
    assert temperature_recip(T).item() == float(r)
    xl = x.clone().requires_grad_(True)
    (gx_o,) = torch.autograd.grad((apply_temperature_oracle_autograd(xl, T) * w).sum(), [xl])
    if _torch_gpu_rounds_like_the_oracle(dtype, x.numel()):
        xt = x.to(DEV).requires_grad_(True)
        yt = xt * 1
        yt.div_(T)
        (gx_t,) = torch.autograd.grad((yt * w.to(DEV)).sum(), [xt])  # torch on the GPU
        assert torch.equal(gx_t.cpu(), gx_o)
    xd = x.to(DEV).requires_grad_(True)
    yd = xd * 1
    apply_temperature_scaling(yd, TrainingSamplingParams(temperature=T))
    (gx,) = torch.autograd.grad((yd * w.to(DEV)).sum(), [xd])
    assert torch.equal(gx.cpu(), gx_o)


def apply_temperature_oracle_autograd(x, T):
    """The oracle's division with autograd: dtype(fl32(float(x) * fl32(1.0 / T)))."""
    return (x.float() * temperature_recip(T)).to(x.dtype)


def _reference_chain(x, ids, sp, gout, gout2=None):
    """CPU torch, the reference's op sequence: model output -> div_ in place (as torch
    runs it on the GPU: the product with fl32(1.0 / T)) -> the get_next_token path (fp32
    upcast, filter, log_softmax, gather), and with gout2 the unfiltered second pass of
    prepare_loss_input (its own upcast); backward of the sum."""
    xl = x.clone().requires_grad_(True)
    y = apply_temperature_oracle_autograd(xl * 1, sp.temperature)
    yf = y.to(torch.float32)
    wo_last = yf[:, :-1]
    with torch.no_grad():
        _, keep = top_k_top_p(wo_last.detach(), sp.top_k, sp.top_p)
    filt = torch.where(keep, wo_last, torch.full_like(wo_last, -float("inf")))
    lp = torch.log_softmax(filt, -1).gather(-1, ids[:, 1:].unsqueeze(-1)).squeeze(-1)
    loss = (lp * gout).sum()
    lp2 = None
    if gout2 is not None:
        yf2 = y.to(torch.float32)
        lp2 = torch.log_softmax(yf2[:, :-1], -1).gather(-1, ids[:, 1:].unsqueeze(-1)).squeeze(-1)
        loss = loss + (lp2 * gout2).sum()
    (gx,) = torch.autograd.grad(loss, [xl])
    return lp.detach(), None if lp2 is None else lp2.detach(), gx


@pytest.mark.parametrize("k,p", [(50, 0.9), (None, 0.9), (5, 1.0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_drop_in_sequence_single_consumer(k, p, dtype):
    """apply_temperature_scaling then get_next_token_logprobs_from_logits(sampling_params):
    the filtered backward writes the raw-logits gradient with the division folded in."""
    print("[case] drop-in sequence", k, p, dtype, flush=True)
    B, S, V = 2, 9, 3001
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(B, S, V, generator=g) * 2).to(dtype)
    ids = torch.randint(0, V, (B, S), generator=g)
    ids[:, 1::2] = x[:, :-1:2].float().argmax(-1)
    gout = torch.randn(B, S - 1, generator=g)
    sp = TrainingSamplingParams(top_k=k, top_p=p, temperature=0.7)
    lp_o, _, gx_o = _reference_chain(x, ids, sp, gout)
    lp_o2, _, gx_o2 = next_token_filtered(x, ids, k, p, temperature=0.7, grad_output=gout)
    assert torch.equal(gx_o, gx_o2)  # the two restatements agree

    xd = x.to(DEV).requires_grad_(True)
    logits = xd * 1  # a non-leaf model output
    logits = apply_temperature_scaling(logits, sp)
    lp = get_next_token_logprobs_from_logits(ids.to(DEV), logits, sampling_params=sp)
    (gx,) = torch.autograd.grad(lp, [xd], gout.to(DEV))
    lp_c = lp.detach().cpu()
    assert torch.equal(torch.isinf(lp_c), torch.isinf(lp_o))
    fin = torch.isfinite(lp_o)
    torch.testing.assert_close(lp_c[fin], lp_o[fin], rtol=0, atol=2e-3)
    assert gx.dtype == dtype
    if dtype == torch.bfloat16:
        assert_close_or_ulp_bf16(gx, gx_o, 1e-3)
    else:
        torch.testing.assert_close(gx.float().cpu(), gx_o.float(), rtol=0, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_drop_in_sequence_two_consumers(dtype):
    """Filtered + unfiltered logprobs of the same scaled logits (prepare_loss_input's KL pass):
    the two gradients are accumulated in the dtype before the division, as autograd does."""
    print("[case] two consumers", dtype, flush=True)
    B, S, V = 2, 7, 2003
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(B, S, V, generator=g) * 2).to(dtype)
    ids = torch.randint(0, V, (B, S), generator=g)
    ids[:, 1::2] = x[:, :-1:2].float().argmax(-1)
    gout, gout2 = torch.randn(B, S - 1, generator=g), torch.randn(B, S - 1, generator=g)
    sp = TrainingSamplingParams(top_k=40, top_p=0.9, temperature=0.8)
    lp_o, lp2_o, gx_o = _reference_chain(x, ids, sp, gout, gout2)

    xd = x.to(DEV).requires_grad_(True)
    logits = apply_temperature_scaling(xd * 1, sp)
    lp = get_next_token_logprobs_from_logits(ids.to(DEV), logits, sampling_params=sp)
    lp2 = get_next_token_logprobs_from_logits(ids.to(DEV), logits, sampling_params=None)
    loss = (lp * gout.to(DEV)).sum() + (lp2 * gout2.to(DEV)).sum()
    (gx,) = torch.autograd.grad(loss, [xd])
    fin = torch.isfinite(lp_o)
    torch.testing.assert_close(lp.detach().cpu()[fin], lp_o[fin], rtol=0, atol=2e-3)
    torch.testing.assert_close(lp2.detach().cpu(), lp2_o, rtol=0, atol=2e-3)
    if dtype == torch.bfloat16:
        assert_close_or_ulp_bf16(gx, gx_o, 1e-3)
    else:
        torch.testing.assert_close(gx.float().cpu(), gx_o.float(), rtol=0, atol=1e-3)


@pytest.mark.parametrize("mode", ["retain_grad", "fold_off"])
def test_gradient_of_the_scaled_logits_themselves(mode):
    """The gradient of the scaled tensor holds the filtered logprobs' part, as in the
    reference: with retain_grad on it (detected, the fold is skipped) and with the fold
    switched off for autograd.grad with the scaled tensor as an input."""
    from rl_amd.distributed.sampling import set_temperature_fold

    print("[case] scaled-logits gradient", mode, flush=True)
    dtype = torch.bfloat16
    B, S, V = 2, 9, 3001
    g = torch.Generator().manual_seed(6)
    x = (torch.randn(B, S, V, generator=g) * 2).to(dtype)
    ids = torch.randint(0, V, (B, S), generator=g)
    ids[:, 1::2] = x[:, :-1:2].float().argmax(-1)
    gout = torch.randn(B, S - 1, generator=g)
    sp = TrainingSamplingParams(top_k=50, top_p=0.9, temperature=0.7)
    # oracle: the gradients of the raw and of the scaled logits
    xl = x.clone().requires_grad_(True)
    y = apply_temperature_oracle_autograd(xl * 1, sp.temperature)
    y.retain_grad()
    wo_last = y.to(torch.float32)[:, :-1]
    with torch.no_grad():
        _, keep = top_k_top_p(wo_last.detach(), sp.top_k, sp.top_p)
    filt = torch.where(keep, wo_last, torch.full_like(wo_last, -float("inf")))
    lp_o = torch.log_softmax(filt, -1).gather(-1, ids[:, 1:].unsqueeze(-1)).squeeze(-1)
    (lp_o * gout).sum().backward()
    gy_o, gx_o = y.grad, xl.grad

    xd = x.to(DEV).requires_grad_(True)
    logits = apply_temperature_scaling(xd * 1, sp)
    if mode == "retain_grad":
        logits.retain_grad()
        lp = get_next_token_logprobs_from_logits(ids.to(DEV), logits, sampling_params=sp)
        (lp * gout.to(DEV)).sum().backward()
        gy, gx = logits.grad, xd.grad
    else:
        set_temperature_fold(False)
        try:
            lp = get_next_token_logprobs_from_logits(ids.to(DEV), logits, sampling_params=sp)
            gy, gx = torch.autograd.grad((lp * gout.to(DEV)).sum(), [logits, xd])
        finally:
            set_temperature_fold(True)
    assert gy is not None and gy.dtype == dtype
    assert_close_or_ulp_bf16(gy, gy_o, 1e-3)
    assert_close_or_ulp_bf16(gx, gx_o, 1e-3)
    assert torch.equal(gy.cpu() == 0, gy_o == 0)  # zero exactly outside the kept set
