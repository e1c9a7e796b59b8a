"""GPU parity of the MoE pieces: comm-quant (moe.py:79-143), its wire format,
and the grouped per-expert GEMM over a token-offset table."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import assert_bits_equal, rel_fro_bf16, seeded, to_np32
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _ref_comm(x: torch.Tensor, granularity: str, rounding: int, bits: int, seed: int, offset: int):
    """Oracle dq with the reference's group choice, then the reference STE in torch CPU ops."""
    xn = to_np32(x).reshape(-1, x.shape[-1]) if x.dim() >= 2 else to_np32(x).reshape(1, -1)
    R, K = xn.shape
    if granularity in ("tile_1x128", "block_128x128"):
        gr, gc = R, 128
    elif granularity == "channel" and x.dim() >= 2:
        gr, gc = R, 1
    else:
        gr, gc = R, K
    _, _, _, dq = O.quant_grouped(xn, gr, gc, bits=bits, rounding=rounding, seed=seed, offset=offset,
                                  scale_rule=O.SCALE_BEFORE_DIVIDE)
    xc = x.detach().cpu()
    dqt = torch.from_numpy(dq).reshape(x.shape).to(x.dtype)
    return xc + (dqt - xc)


@pytest.mark.parametrize("granularity", ["block_128x128", "tile_1x128", "channel", "tensor"])
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
@pytest.mark.parametrize("shape,dtype", [((7, 257), torch.float32), ((64, 1024), torch.bfloat16),
                                         ((3, 5, 300), torch.bfloat16)])
def test_comm_quant_dequant_parity(gpu_device, granularity, rounding, shape, dtype):
    from lowbit import moe

    x = seeded(shape, seed=20260401, dtype=dtype, outliers=0.01).to(gpu_device).requires_grad_(True)
    out = moe.comm_quant_dequant(x, granularity=granularity, rounding_mode=rounding, bits=8, seed=9, offset=4)
    rc = O.ROUND_STOCHASTIC if rounding == "stochastic" else O.ROUND_NEAREST
    ref = _ref_comm(x, granularity, rc, 8, 9, 4)
    assert out.shape == x.shape and out.dtype == x.dtype
    assert_bits_equal(out.detach().float().cpu().numpy(), ref.float().numpy(), "comm dq")
    out.float().sum().backward()  # straight-through gradient
    assert x.grad is not None and torch.equal(x.grad, torch.ones_like(x))


def test_comm_quant_dequant_special_values(gpu_device):
    from lowbit import moe

    x = torch.zeros(4, 256)
    x[0, 3] = float("inf")
    x[1, 130] = float("nan")
    x[2, :2] = torch.tensor([1e-45, -1e-45])
    x = x.to(gpu_device)
    for g in ("block_128x128", "tensor", "channel"):
        out = moe.comm_quant_dequant(x, granularity=g, rounding_mode="nearest", seed=1, offset=1)
        ref = _ref_comm(x, g, O.ROUND_NEAREST, 8, 1, 1)
        assert_bits_equal(out.float().cpu().numpy(), ref.float().numpy(), f"comm dq {g}")


@pytest.mark.parametrize("fmt,grid", [("e4m3", O.GRID_E4M3), ("int_grid", O.GRID_INT)])
def test_comm_wire_format_round_trip(gpu_device, fmt, grid):
    from lowbit import moe

    x = seeded((300, 7168 // 4), seed=20260402, outliers=0.01).to(gpu_device)
    payload = moe.comm_quant(x, fmt=fmt)
    y = moe.comm_dequant(payload)
    codes, scales, _, dq = O.quant_tile_1x128(to_np32(x), grid=grid)
    assert_bits_equal(payload.q.codes.cpu().numpy(), codes, "wire codes")
    assert_bits_equal(payload.q.scales.cpu().numpy(), scales, "wire scales")
    expect = torch.from_numpy(dq).to(x.dtype).float().numpy()
    if grid == O.GRID_E4M3:
        assert_bits_equal(to_np32(y), expect, "received tokens")
    else:
        # int8 codes have no -0: a negative value that rounds to zero arrives as +0
        got = to_np32(y)
        assert np.array_equal(got, expect)
        nz = expect != 0
        assert_bits_equal(got[nz], expect[nz], "received tokens (nonzero)")
    assert payload.nbytes == x.numel() + scales.size * 4


def _routing(T, E, k, seed, device):
    from lowbit import workloads

    return workloads.zipf_topk_routing(T, E, k, seed=seed, device=device)


@pytest.mark.parametrize("fmt,grid", [("e4m3", O.GRID_E4M3), ("int_grid", O.GRID_INT)])
@pytest.mark.parametrize("T,E,k,H,I", [(64, 4, 2, 256, 256), (300, 8, 3, 384, 128), (5, 16, 2, 128, 256)])
def test_grouped_linear_matches_per_expert_oracle(gpu_device, fmt, grid, T, E, k, H, I):
    from lowbit import moe

    tokens = seeded((T, H), seed=20260403).to(gpu_device)
    routing = _routing(T, E, k, 20260404, gpu_device)
    w = seeded((E, I, H), seed=20260405, std=0.02).to(gpu_device)
    order, tok_idx, offsets = moe.sort_by_expert(routing, E)
    xs = tokens[tok_idx]
    wc, ws, wn = moe.quantize_expert_weights(w, fmt=fmt)
    y = moe.grouped_linear(xs, offsets, wc, ws, fmt=fmt, w_nan_rows=wn)
    torch.cuda.synchronize()
    off = offsets.cpu().numpy()
    xs_n = to_np32(xs)
    _, _, _, xdq = O.quant_tile_1x128(xs_n, grid=grid)
    ref = np.zeros((xs_n.shape[0], I))
    for e in range(E):
        lo, hi = off[e], off[e + 1]
        if hi == lo:
            continue
        _, _, _, wdq = O.quant_block_128x128(to_np32(w[e]), grid=grid)
        ref[lo:hi] = O.gemm_ref(xdq[lo:hi], wdq)
    assert rel_fro_bf16(y, ref) <= 1e-3


def test_sort_by_expert_offsets(gpu_device):
    from lowbit import moe

    routing = _routing(1000, 32, 8, 7, gpu_device)
    order, tok_idx, offsets = moe.sort_by_expert(routing, 32)
    flat = routing.reshape(-1).cpu()
    off = offsets.cpu()
    assert off[0] == 0 and off[-1] == flat.numel()
    sorted_ids = flat[order.cpu()]
    for e in range(32):
        assert (sorted_ids[off[e]:off[e + 1]] == e).all()
    # distinct experts per token (top-k without replacement)
    assert all(len(set(r.tolist())) == 8 for r in routing.cpu())


def test_c4_grouped_up_projection_full_size_sampled(gpu_device):
    """4096 tokens, top-8 of 32 experts, W_up [2048, 7168]."""
    from lowbit import moe, workloads

    tokens, routing, w_up, _ = workloads.c4_inputs(device="cpu")
    tokens, routing = tokens.to(gpu_device), routing.to(gpu_device)
    w_up = w_up.to(gpu_device)
    order, tok_idx, offsets = moe.sort_by_expert(routing, 32)
    xs = tokens[tok_idx]
    wc, ws, wn = moe.quantize_expert_weights(w_up, fmt="e4m3")
    y = moe.grouped_linear(xs, offsets, wc, ws, fmt="e4m3", w_nan_rows=wn)
    torch.cuda.synchronize()
    assert y.shape == (32768, 2048)
    off = offsets.cpu().numpy()
    rng = np.random.default_rng(3)
    for e in rng.choice(32, 4, replace=False):
        lo, hi = off[e], off[e + 1]
        if hi == lo:
            continue
        rows = np.arange(lo, hi)[:64]
        _, _, _, xdq = O.quant_tile_1x128(to_np32(xs[rows]), grid=O.GRID_E4M3)
        _, _, _, wdq = O.quant_block_128x128(to_np32(w_up[e]), grid=O.GRID_E4M3)
        assert rel_fro_bf16(y[rows], O.gemm_ref(xdq, wdq)) <= 1e-3
