"""GPU tests of the device AdamW (optimizer_runtime.py:68-116) and its fused
persistent low-bit refresh (layers.py:353-407).

The update is checked per step against a float64 evaluation of the same
formula, started from the device's fp32 state, and against the reference's
sequence of torch ops run on the device.  The refreshed codes and scales are
bit-exact against the oracle quantizers applied to the updated parameter."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import assert_bits_equal, seeded, to_np32
from oracle import oracle as O

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def _state(n, seed, device):
    g = torch.Generator().manual_seed(seed)
    p = (torch.randn(n, generator=g) * 0.02).to(device)
    m = (torch.randn(n, generator=g) * 1e-3).to(device)
    v = (torch.rand(n, generator=g) * 1e-6).to(device)
    return p, m, v


def _adamw64(p, m, v, g, step):
    """The reference update (optimizer_runtime.py:93-109) evaluated in float64
    with the float32 scalars torch uses.  Returns the three results and, for
    each, the largest operand magnitude of its last operation (the scale of a
    few-ulp error bound when terms cancel)."""
    from lowbit.optim import adamw_scalars

    sc = {k: np.float64(v_) for k, v_ in adamw_scalars(step=step, **HP).items()}
    p, m, v, g = (np.asarray(t, dtype=np.float64) for t in (p, m, v, g))
    m1, m2 = sc["beta1"] * m, sc["one_minus_beta1"] * g
    v1, v2 = sc["beta2"] * v, sc["one_minus_beta2"] * g * g
    m, v = m1 + m2, v1 + v2
    return (m, v), (np.maximum(np.abs(m1), np.abs(m2)), np.maximum(np.abs(v1), np.abs(v2)))


def _param64(p, m, v, step):
    """The parameter update in float64 from given (fp32) m and v, so its check
    covers only the denominator, the division and the two updates of p."""
    from lowbit.optim import adamw_scalars

    sc = {k: np.float64(v_) for k, v_ in adamw_scalars(step=step, **HP).items()}
    p, m, v = (np.asarray(t, dtype=np.float64) for t in (p, m, v))
    d = np.sqrt(v) * sc["inv_bc2_sqrt"] + sc["eps"]
    p1, p2 = p * sc["decay"], sc["neg_step_size"] * m / d
    return p1 + p2, np.maximum(np.abs(p1), np.abs(p2))


def _within_ulps(got, want, mag, k):
    return np.all(np.abs(got.astype(np.float64) - want) <= k * np.spacing(mag.astype(np.float32)).astype(np.float64))


def _ulps(a, b):
    a = np.asarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


@pytest.mark.parametrize("grad_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("param_dtype", [torch.bfloat16, torch.float32])
def test_adamw_matches_float64_per_step(gpu_device, grad_dtype, param_dtype):
    from lowbit.optim import adamw_step_refresh

    n = 5003
    mp, m, v = _state(n, 20260701, gpu_device)
    param = torch.empty(n, dtype=param_dtype, device=gpu_device)
    for step in range(1, 4):
        g = seeded((n,), seed=20260710 + step, std=1e-2, dtype=grad_dtype).to(gpu_device)
        before = [to_np32(t) for t in (mp, m, v)]
        adamw_step_refresh(mp, g, m, v, param=param, step=step, **HP)
        torch.cuda.synchronize()
        (m64, v64), (mmag, vmag) = _adamw64(*before, to_np32(g), step)
        # two roundings each for m and v; p: sqrt, divide, add, divide, multiply, FMA
        assert _within_ulps(to_np32(m), m64, mmag, 2)
        assert _within_ulps(to_np32(v), v64, vmag, 2)
        p64, pmag = _param64(before[0], to_np32(m), to_np32(v), step)
        assert _within_ulps(to_np32(mp), p64, pmag, 4)
        assert torch.equal(param, mp.to(param_dtype))


def test_adamw_matches_reference_torch_ops(gpu_device):
    """The reference's torch op sequence (optimizer_runtime.py:98-109), run on
    the device on the same fp32 state: bit-identical results."""
    from lowbit.optim import adamw_step_refresh

    n = 1 << 16
    mp, m, v = _state(n, 20260702, gpu_device)
    rp, rm, rv = mp.clone(), m.clone(), v.clone()
    b1, b2 = HP["betas"]
    for step in range(1, 4):
        g = seeded((n,), seed=20260720 + step, std=1e-2).float().to(gpu_device)
        adamw_step_refresh(mp, g, m, v, step=step, **HP)
        rm.mul_(b1).add_(g, alpha=1.0 - b1)
        rv.mul_(b2).addcmul_(g, g, value=1.0 - b2)
        bc1, bc2 = 1.0 - b1 ** step, 1.0 - b2 ** step
        denom = rv.sqrt().div_(bc2 ** 0.5).add_(HP["eps"])
        rp.mul_(1.0 - HP["lr"] * HP["weight_decay"])
        rp.addcdiv_(rm, denom, value=-(HP["lr"] / bc1))
        torch.cuda.synchronize()
        for got, ref in ((m, rm), (v, rv), (mp, rp)):
            assert _ulps(to_np32(got), to_np32(ref)).max() == 0
        # continue both from the same state
        rp.copy_(mp), rm.copy_(m), rv.copy_(v)


@pytest.mark.parametrize("refresh,block", [("nf4", 64), ("nf4", 2048), ("nf4", 8), ("fp8", 256), ("fp8", 1024)])
def test_fused_refresh_matches_oracle(gpu_device, refresh, block):
    from lowbit.optim import adamw_step_refresh

    n = 4 * 2048 + 40  # a ragged last block
    mp, m, v = _state(n, 20260703, gpu_device)
    mp[17] = float("nan") if refresh == "nf4" else mp[17]
    param = torch.empty(n, dtype=torch.bfloat16, device=gpu_device)
    nb = -(-n // block)
    codes = torch.empty((n + 1) // 2 if refresh == "nf4" else n, dtype=torch.uint8, device=gpu_device)
    scales = torch.empty(nb, dtype=torch.float32, device=gpu_device)
    g = seeded((n,), seed=20260730, std=1e-2).to(gpu_device)
    adamw_step_refresh(mp, g, m, v, param=param, refresh=refresh, block=block, codes=codes, scales=scales, step=1,
                       **HP)
    torch.cuda.synchronize()
    w = to_np32(param)
    if refresh == "nf4":
        c_ref, s_ref = O.nf4_quant(w, block)
    else:
        c_ref, s_ref = O.fp8_persistent_quant(w, block)
    assert_bits_equal(codes.cpu().numpy(), c_ref, "codes")
    assert_bits_equal(scales.cpu().numpy(), s_ref, "scales")


@pytest.mark.parametrize("mode", ["fp4", "fp8"])
def test_optimizer_refreshes_layers(gpu_device, mode):
    """PrecisionAdamW with attach_lowbit_refresh: after step() the module
    buffers equal a fresh refresh_persistent_lowbit_params() of the stepped
    weight, for a weight the fused pass takes (rows of 256) and one it does
    not (rows of 384)."""
    from test_gpu_layers import _linear, _resolver

    from lowbit.optim import PrecisionAdamW

    flags = {"fp4": dict(fp4_param=True), "fp8": dict(fp8_param=True)}[mode]
    _, res = _resolver(bf16=True, persistent_scale_granularity="per_channel", persistent_lowbit_include=["fc"],
                       compute_lowbit_mode=None, **flags)
    model = torch.nn.Sequential(_linear(res, 256, 64, path="fc.a", bias=False),
                                _linear(res, 384, 128, path="fc.b", bias=False))
    opt = PrecisionAdamW(model.parameters(), **HP)
    assert opt.attach_lowbit_refresh(model) == 2
    for layer in model:
        layer.refresh_persistent_lowbit_params()
    x = seeded((16, 256), seed=20260740).to(gpu_device)
    x2 = seeded((16, 384), seed=20260741).to(gpu_device)
    ((model[0](x).float() ** 2).mean() + (model[1](x2).float() ** 2).mean()).backward()
    opt.step()
    torch.cuda.synchronize()
    for layer in model:
        st = opt.state[layer.weight]
        assert torch.equal(layer.weight.detach(), st["main_param"].to(torch.bfloat16))
        if mode == "fp4":
            got = (layer._persistent_fp4_codes.clone(), layer._persistent_scale.clone())
        else:
            got = (layer._persistent_fp8_weight.view(torch.uint8).clone(), layer._persistent_scale.clone())
        layer.refresh_persistent_lowbit_params()
        want = (layer._persistent_fp4_codes, layer._persistent_scale) if mode == "fp4" else \
            (layer._persistent_fp8_weight.view(torch.uint8), layer._persistent_scale)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
        assert got[1].shape == want[1].shape
