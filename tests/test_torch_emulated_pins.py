"""Pins for oracle/torch_emulated.py, the torch-op restatement of the
reference's emulated path that bench.py times as its CPU baseline.  It must
give the C oracle's dequantized values bit for bit (the C oracle is pinned in
test_oracle_pins.py) for every granularity, special values and ragged shapes
included, and its forward and autograd gradients must equal float64 products
of those values."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_emulated as T


def _x(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * std
    x = torch.where(torch.rand(*shape, generator=g) < 0.01, x * 50, x)
    return x


def _bits_equal(a: torch.Tensor, b: np.ndarray) -> bool:
    a = a.float().numpy().astype(np.float32)
    b = b.astype(np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | nan))


GRAN_GROUPS = {  # granularity, channel axis -> oracle (gr, gc) on a 2-D operand [R, K]
    ("tile_1x128", -1): lambda R, K: (1, 128),
    ("block_128x128", 0): lambda R, K: (128, 128),
    ("tensor", -1): lambda R, K: (R, K),
    ("channel", -1): lambda R, K: (R, 1),
    ("channel", 0): lambda R, K: (1, K),
}


@pytest.mark.parametrize("gran,axis", list(GRAN_GROUPS))
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("shape", [(256, 384), (129, 257), (3, 70)])
def test_quantize_dequantize_matches_c_oracle(gran, axis, bits, shape):
    x = _x(shape, 20263001 + shape[0])
    x[1, 2] = float("nan")
    x[2, 5] = float("inf")
    x[0, :] = 0.0
    R, K = shape
    gr, gc = GRAN_GROUPS[(gran, axis)](R, K)
    got = T.quantize_dequantize(x, bits=bits, granularity=gran, rounding="nearest", channel_axis=axis)
    want = O.quant_grouped(x.numpy(), gr, gc, bits=bits)[3]
    assert _bits_equal(got, want)


def test_unknown_granularity_is_the_scale_first_tensor_rule():
    """_ste_fake_quantize (te_backend.py:40-58): amax checked before the
    division, so a subnormal amax gives scale amax/qmax, and zero gives 1."""
    x = torch.full((4, 130), 1e-39)
    got = T.quantize_dequantize(x, bits=8, granularity="other", rounding="nearest", channel_axis=-1)
    want = O.quant_grouped(x.numpy(), 4, 130, scale_rule=O.SCALE_BEFORE_DIVIDE)[3]
    assert _bits_equal(got, want)


def test_bf16_operand_is_the_rounded_fp32_dq():
    x = _x((64, 256), 20263011).to(torch.bfloat16)
    got = T.quantize_dequantize(x, bits=8, granularity="tile_1x128", rounding="nearest", channel_axis=-1)
    want = O.round_bf16(O.quant_tile_1x128(x.float().numpy())[3])
    assert got.dtype == torch.bfloat16 and _bits_equal(got, want)


def test_stochastic_rounding_brackets():
    x = _x((64, 256), 20263021)
    dq = T.quantize_dequantize(x, bits=8, granularity="tile_1x128", rounding="stochastic", channel_axis=-1)
    lo = O.quant_tile_1x128(x.numpy())[3]  # nearest: within one scale step of the stochastic value
    s = O.quant_tile_1x128(x.numpy())[1].repeat(128, axis=1)[:, :256]
    assert np.all(np.abs(dq.numpy() - lo) <= s * 1.001)  # at most one scale step (fp32 products aside)


def test_linear_forward_and_straight_through_gradients():
    x = _x((96, 384), 20263031).requires_grad_(True)
    w = (_x((160, 384), 20263032) * 0.02).requires_grad_(True)
    b = _x((160,), 20263033).requires_grad_(True)
    dy = _x((96, 160), 20263034) * 1e-3
    y = T.emulated_linear(x, w, b)
    y.backward(dy)
    xd = O.quant_tile_1x128(x.detach().numpy())[3].astype(np.float64)
    wd = O.quant_block_128x128(w.detach().numpy())[3].astype(np.float64)
    ref = xd @ wd.T + b.detach().numpy().astype(np.float64)
    assert O.rel_frobenius(y.detach().numpy(), ref) <= 1e-6
    d = dy.numpy().astype(np.float64)
    assert O.rel_frobenius(x.grad.numpy(), d @ wd) <= 1e-6
    assert O.rel_frobenius(w.grad.numpy(), d.T @ xd) <= 1e-6
    assert np.allclose(b.grad.numpy(), d.sum(0), rtol=1e-5, atol=1e-7)


def test_nf4_dequantize_matches_c_oracle():
    w = _x((64, 256), 20263041) * 0.02
    packed, scales = O.nf4_quant(w.numpy(), 64)
    got = T.nf4_dequantize(torch.from_numpy(packed), torch.from_numpy(scales), numel=w.numel(), block=64,
                           dtype=torch.float32)
    assert _bits_equal(got, O.nf4_dequant(packed, scales, w.numel(), 64))


@pytest.mark.parametrize("grid", [O.GRID_INT, O.GRID_E4M3])
@pytest.mark.parametrize("gr,gc", [(1, 128), (128, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_reference_operand_is_the_dequant_only_under_nearest(grid, gr, gc, dtype):
    """The reference multiplies x + (x_dq - x) in x's dtype (te_backend.py:250-251),
    x_dq = dtype(q * s).  Under round to nearest that is x_dq itself (q * s and
    x lie within a factor of two, so the difference is exact), which is why
    the kernels may decode dtype(q * s) from codes.  Under stochastic rounding
    a code can land far from x / s; the difference then rounds and the
    expression differs from x_dq, exactly where dtype(x_dq - x) is inexact."""
    # outliers x1000 make large scales, so many x / s sit in e4m3's
    # subnormal range, where a stochastic code can be several times x / s
    g = torch.Generator().manual_seed(20262341)
    x = torch.randn(256, 512, generator=g)
    x = torch.where(torch.rand(256, 512, generator=g) < 0.01, x * 1000, x).to(dtype)
    x32 = x.float().numpy()
    for rounding in (O.ROUND_NEAREST, O.ROUND_STOCHASTIC):
        dq = O.quant_grouped(x32, gr, gc, grid=grid, rounding=rounding, seed=5, offset=2)[3]
        dq_t = torch.from_numpy(dq).to(dtype)
        xq = x + (dq_t - x)
        same = (xq.float() == dq_t.float()) | (torch.isnan(xq.float()) & torch.isnan(dq_t.float()))
        if rounding == O.ROUND_NEAREST:
            assert bool(same.all())
        else:
            assert 0 < int((~same).sum()) < 0.05 * x.numel()
            diff64 = dq_t.double() - x.double()
            inexact = (dq_t - x).double() != diff64
            assert bool(inexact[~same].all())


def test_autograd_accumulates_gathered_token_gradients_in_descending_expert_order():
    """The reference's loop gathers tokens[token_indices] once per expert
    (moe.py:1086, :488); autograd runs the later experts' backward first, so a
    token's gradient is its experts' contributions added in descending expert
    id, each add rounded to bf16 (ntlb_moe_token_grad mirrors this order).  An
    ascending order or one fp32 sum gives other bits."""
    torch.manual_seed(0)
    T, H, E, k = 64, 32, 5, 3
    tok = torch.randn(T, H).bfloat16().requires_grad_(True)
    idx = torch.stack([torch.randperm(E)[:k] for _ in range(T)])
    contrib = {}
    out = torch.zeros_like(tok)
    for e in range(E):
        ti = (idx == e).nonzero()[:, 0]
        c = (torch.randn(ti.numel(), H) * 1.37).bfloat16()
        contrib[e] = (ti, c)
        out[ti] += tok[ti] * c
    d = torch.randn(T, H).bfloat16()
    out.backward(d)

    def accum(order):
        acc = None
        for e in order:
            ti, c = contrib[e]
            full = torch.zeros(T, H, dtype=torch.bfloat16)
            full[ti] = d[ti] * c
            acc = full if acc is None else acc + full
        return acc

    assert torch.equal(accum(range(E - 1, -1, -1)), tok.grad)
    assert not torch.equal(accum(range(E)), tok.grad)


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


@pytest.mark.parametrize("forward", ["reference", "fp32_dq"])
@pytest.mark.parametrize("capacity", [0, 5])
def test_local_moe_loop_matches_a_dense_restatement(forward, capacity):
    """local_moe_loop (the reference's gather / ExpertMLP / index-add loop
    under autograd) against a dense float64 restatement with no gathers:
    out[t] = sum over kept slots s of w[t, s] * down_e(silu(gate_e(x_t)) *
    up_e(x_t)), e = idx[t, s], where gate row j of w_gate_up is row
    256 * (j // 128) + j % 128 and up row j is 128 rows after it, and a slot is
    kept when fewer than `capacity` assignments of its expert have a larger
    weight.  The quantizer is the identity here, so the straight-through
    gradients are the function's exact gradients; the bar is bf16's rounding
    of the loop's intermediates.  A swapped gate/up block, a dropped routing
    weight or a wrong capacity choice is off by O(1)."""
    Tn, H, I, E, k = 24, 128, 256, 4, 2
    g = torch.Generator().manual_seed(20262531)
    tokens = torch.randn(Tn, H, generator=g).bfloat16()
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(Tn)])
    w = torch.softmax(torch.randn(Tn, k, generator=g) * 2, dim=-1)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * H ** -0.5).bfloat16()
    wd = (torch.randn(E, H, I, generator=g) * I ** -0.5).bfloat16()
    leaves = [t.clone().requires_grad_(True) for t in (tokens, w, wgu, wd)]
    out = T.local_moe_loop(leaves[0], idx, leaves[1], leaves[2], leaves[3], capacity=capacity, forward=forward,
                           qdq=lambda t, gr, gc: t)
    d_out = torch.randn(Tn, H, generator=g).bfloat16()
    out.backward(d_out)
    # the dense restatement
    ref = [t.detach().double().requires_grad_(True) for t in (tokens, w, wgu, wd)]
    x64, w64, gu64, d64 = ref
    j = torch.arange(I)
    gate_rows = 256 * (j // 128) + j % 128
    kept = torch.ones(Tn, k, dtype=torch.bool)
    if capacity > 0:
        for t in range(Tn):
            for s in range(k):
                same = idx == idx[t, s]
                kept[t, s] = int((same & (w > w[t, s])).sum()) < capacity
        assert not bool(kept.all())
    rows = []
    for t in range(Tn):
        acc = torch.zeros(H, dtype=torch.float64)
        for s in range(k):
            if kept[t, s]:
                e = int(idx[t, s])
                gt = gu64[e, gate_rows] @ x64[t]
                up = gu64[e, gate_rows + 128] @ x64[t]
                acc = acc + w64[t, s] * (d64[e] @ (torch.nn.functional.silu(gt) * up))
        rows.append(acc)
    out64 = torch.stack(rows)
    out64.backward(d_out.double())
    assert _rel(out.detach(), out64.detach()) < 1e-2
    for a, b in zip(leaves, ref):
        assert _rel(a.grad, b.grad) < 1e-2
