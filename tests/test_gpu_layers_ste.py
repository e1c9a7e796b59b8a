"""GPU tests of the straight-through operands and gradients of HipLowBitBackend:

- ``ops.ste_value`` against torch's own evaluation of ``t + (t_dq - t)`` (the
  expression of te_backend.py:250-251) for bf16, fp16 and fp32, bit for bit;
- under stochastic rounding, the reference-mode forward and the
  straight-through gradients multiply that expression's values (they differ
  from bf16(q * s) on some elements, which the test shows), against the
  oracle's seeded codes;
- float16 layers: both forward modes and the straight-through backward
  against the oracle with operands rounded to fp16 (te_backend.py:173-202
  casts the dequantized operand to the input dtype);
- a retained graph: backward twice gives the same gradients.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import rel_fro_bf16, seeded, to_np32
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _backend(act="tile_1x128", wgt="block_128x128", rounding="nearest", fmt="e4m3", forward="blockscaled",
             seed=None, i=384, o=200):
    from lowbit.backend import HipLowBitBackend
    from lowbit.contracts import LowBitKernelSpec

    spec = LowBitKernelSpec("linear", i, o, True, act, wgt, rounding)
    return HipLowBitBackend(mode="fp8", kernel_spec=spec, code_format=fmt, forward=forward, seed=seed)


def _same_values(a: torch.Tensor, b: torch.Tensor) -> bool:
    """equal bit for bit, every NaN counted equal to every NaN"""
    a, b = a.detach().cpu(), b.detach().cpu()
    nan = torch.isnan(a.float())
    if not torch.equal(nan, torch.isnan(b.float())):
        return False
    it = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}[a.dtype]
    return torch.equal(a.view(it)[~nan], b.view(it)[~nan])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n,offset", [(4096 * 37 + 5, 0), (1000, 3), (7, 1)])
def test_ste_value_matches_torch_expression(gpu_device, dtype, n, offset):
    from lowbit import ops

    g = torch.Generator().manual_seed(20262301 + n)
    t = torch.randn(n + offset, generator=g) * torch.exp(torch.randn(n + offset, generator=g) * 4)
    dq = t + torch.randn(n + offset, generator=g) * t.abs() * torch.rand(n + offset, generator=g)
    specials = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), 1e-30, -3e38, 65504.0])
    k = min(len(specials), n)
    t[offset:offset + k] = specials[:k]
    dq[offset:offset + k] = specials.flip(0)[:k]
    t, dq = t.to(dtype), dq.to(dtype)
    ref = t[offset:] + (dq[offset:] - t[offset:])  # torch CPU, the reference's op sequence
    out = ops.ste_value(t.to(gpu_device)[offset:], dq.to(gpu_device)[offset:])
    assert out.dtype == dtype and out.shape == ref.shape
    assert _same_values(out, ref)


def _with_outliers(shape, seed: int, std: float) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * std
    return torch.where(torch.rand(*shape, generator=g) < 0.01, x * 1000, x).to(torch.bfloat16)


def _oracle_dq(t: np.ndarray, gran: str, *, grid, rounding, seed, offset) -> np.ndarray:
    if gran == "tile_1x128":
        return O.quant_tile_1x128(t, grid=grid, rounding=rounding, seed=seed, offset=offset)[3]
    return O.quant_block_128x128(t, grid=grid, rounding=rounding, seed=seed, offset=offset)[3]


def _reference_operand(t: torch.Tensor, dq32: np.ndarray) -> torch.Tensor:
    """t + (t_dq - t) in t's dtype on the CPU, t_dq = dq cast to that dtype (te_backend.py:173-202, :250-251)"""
    tc = t.detach().cpu()
    dq = torch.from_numpy(dq32).to(tc.dtype)
    return tc + (dq - tc)


@pytest.mark.parametrize("fmt", ["int_grid", "e4m3"])
@pytest.mark.parametrize("forward", ["reference", "blockscaled"])
def test_stochastic_rounding_multiplies_the_reference_operands(gpu_device, fmt, forward):
    grid = O.GRID_E4M3 if fmt == "e4m3" else O.GRID_INT
    be = _backend(rounding="stochastic", fmt=fmt, forward=forward, seed=4242)
    # outliers x1000 give large scales, so many x / s lie where a stochastic
    # code can be several times x / s (e4m3's subnormals, the int grid's 0/1)
    x = _with_outliers((2, 70, 384), 20262311, 1.0).to(gpu_device).requires_grad_(True)
    w = _with_outliers((200, 384), 20262312, 0.02).to(gpu_device).requires_grad_(True)
    b = seeded((200,), seed=20262313).to(gpu_device).requires_grad_(True)
    dy = seeded((2, 70, 200), seed=20262314, std=1e-3).to(gpu_device)
    y = be.linear(x, w, b)
    y.backward(dy)
    # the first call of a backend keys x at offset 0 and w at offset 1
    xdq = _oracle_dq(to_np32(x).reshape(-1, 384), "tile_1x128", grid=grid, rounding=O.ROUND_STOCHASTIC, seed=4242,
                     offset=0)
    wdq = _oracle_dq(to_np32(w), "block_128x128", grid=grid, rounding=O.ROUND_STOCHASTIC, seed=4242, offset=1)
    xq = _reference_operand(x.reshape(-1, 384), xdq)
    wq = _reference_operand(w, wdq)
    # the expression differs from bf16(q * s) on some elements: the test tells the two apart
    differ = (xq.float() != torch.from_numpy(O.round_bf16(xdq))).sum() + \
        (wq.float() != torch.from_numpy(O.round_bf16(wdq))).sum()
    assert int(differ) > 0
    xq64, wq64 = xq.double().numpy(), wq.double().numpy()
    if forward == "reference":
        err = rel_fro_bf16(y.reshape(-1, 200), O.gemm_ref(xq64, wq64, to_np32(b)))
        assert err <= 2.5e-4, err
    else:
        err = rel_fro_bf16(y.reshape(-1, 200), O.gemm_ref(xdq, wdq, to_np32(b)))
        assert err <= 1e-3, err
    dyn = to_np32(dy).reshape(-1, 200).astype(np.float64)
    assert rel_fro_bf16(x.grad.reshape(-1, 384), dyn @ wq64) <= 1e-3
    assert rel_fro_bf16(w.grad, dyn.T @ xq64) <= 1e-3


def _rel_fro_f16(y: torch.Tensor, ref64: np.ndarray) -> float:
    a = to_np32(y)
    b = ref64.astype(np.float16).astype(np.float32)
    return O.rel_frobenius(a, b)


@pytest.mark.parametrize("forward", ["blockscaled", "reference"])
@pytest.mark.parametrize("act,wgt", [("tile_1x128", "block_128x128"), ("channel", "block_128x128"),
                                     ("tensor", "channel")])
def test_float16_layer_forward_and_ste_backward(gpu_device, forward, act, wgt):
    """A float16 layer: the blockscaled forward multiplies fp32 q * s, the
    reference forward fp16(q * s), and the straight-through gradients
    dY @ fp16(W_dq), dY^T @ fp16(X_dq) (the reference's casts, te_backend.py:173-202)."""
    from test_gpu_layers import _oracle_operand

    be = _backend(act=act, wgt=wgt, forward=forward)
    x = seeded((2, 70, 384), seed=20262321, outliers=0.01, dtype=torch.float16).to(gpu_device).requires_grad_(True)
    w = seeded((200, 384), seed=20262322, std=0.02, dtype=torch.float16).to(gpu_device).requires_grad_(True)
    b = seeded((200,), seed=20262323, dtype=torch.float16).to(gpu_device).requires_grad_(True)
    dy = seeded((2, 70, 200), seed=20262324, std=1e-3, dtype=torch.float16).to(gpu_device)
    y = be.linear(x, w, b)
    assert y.dtype == torch.float16
    y.backward(dy)
    xd = _oracle_operand(to_np32(x).reshape(-1, 384), act, is_weight=False, grid=O.GRID_E4M3, bits=8, dim=3)
    wd = _oracle_operand(to_np32(w), wgt, is_weight=True, grid=O.GRID_E4M3, bits=8, dim=2)
    xd16 = xd.astype(np.float16).astype(np.float64)
    wd16 = wd.astype(np.float16).astype(np.float64)
    if forward == "reference":
        ref = O.gemm_ref(xd16, wd16, to_np32(b))
        bound = 1e-4
    else:
        ref = O.gemm_ref(xd, wd, to_np32(b))
        bound = 1e-3
    assert _rel_fro_f16(y.reshape(-1, 200), ref) <= bound
    dyn = to_np32(dy).reshape(-1, 200).astype(np.float64)
    assert _rel_fro_f16(x.grad.reshape(-1, 384), dyn @ wd16) <= 1e-4
    assert _rel_fro_f16(w.grad, dyn.T @ xd16) <= 1e-4
    db = dyn.sum(0)
    assert np.allclose(to_np32(b.grad), db.astype(np.float16).astype(np.float32), rtol=2 ** -10, atol=1e-7)


@pytest.mark.parametrize("dtype,rounding", [(torch.bfloat16, "nearest"), (torch.float32, "nearest"),
                                            (torch.bfloat16, "stochastic")])
def test_retained_graph_runs_backward_twice(gpu_device, dtype, rounding):
    """The codes (or the reference's operands) are saved for backward, not
    dropped after the first pass: backward(retain_graph=True) then backward
    again gives the same gradients."""
    be = _backend(rounding=rounding, seed=7)
    x = seeded((130, 384), seed=20262331, dtype=dtype).to(gpu_device).requires_grad_(True)
    w = seeded((200, 384), seed=20262332, std=0.02, dtype=dtype).to(gpu_device).requires_grad_(True)
    b = torch.zeros(200, device=gpu_device, dtype=dtype, requires_grad=True)
    dy = seeded((130, 200), seed=20262333, std=1e-3, dtype=dtype).to(gpu_device)
    y = be.linear(x, w, b)
    y.backward(dy, retain_graph=True)
    g1 = [t.grad.clone() for t in (x, w, b)]
    for t in (x, w, b):
        t.grad = None
    y.backward(dy)
    for a, c in zip(g1, (x.grad, w.grad, b.grad)):
        assert _same_values(a, c)
