"""GPU parity of the blockwise-scaled GEMM against the fp32-dequantize-then-float64
matmul oracle.  The bar: relative Frobenius error <= 1e-3, both
sides rounded to bf16."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import rel_fro_bf16, seeded, to_np32
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
GRIDS = [("int_grid", O.GRID_INT), ("e4m3", O.GRID_E4M3)]


def _oracle_operands(x, w, grid, bits=8):
    xn, wn = to_np32(x).reshape(-1, x.shape[-1]), to_np32(w)
    _, _, _, xdq = O.quant_tile_1x128(xn, grid=grid, bits=bits)
    _, _, _, wdq = O.quant_block_128x128(wn, grid=grid, bits=bits)
    return xdq, wdq


@pytest.mark.parametrize("mnk", [(128, 128, 128), (512, 1024, 1024), (3, 129, 257), (200, 300, 520),
                                 (1, 7, 128), (257, 640, 384)])
@pytest.mark.parametrize("fmt,grid", GRIDS)
def test_gemm_forward_parity(gpu_device, mnk, fmt, grid):
    from lowbit import ops

    M, N, K = mnk
    x = seeded((M, K), seed=20260101, outliers=0.01).to(gpu_device)
    w = seeded((N, K), seed=20260102, std=0.02).to(gpu_device)
    qx = ops.quant_tile_1x128(x, fmt=fmt)
    qw, _ = ops.quant_block_128x128(w, fmt=fmt)
    y = ops.gemm_blockscaled(qx, qw, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    xdq, wdq = _oracle_operands(x, w, grid)
    err = rel_fro_bf16(y, O.gemm_ref(xdq, wdq))
    assert err <= TOL, err


@pytest.mark.parametrize("fmt,grid", GRIDS)
def test_gemm_bias_fp32_out_and_row_scales(gpu_device, fmt, grid):
    """fp32 output, a bias, and per-row (tile) scales on B instead of blocks."""
    from lowbit import ops

    M, N, K = 96, 200, 384
    x = seeded((M, K), seed=7, dtype=torch.float32).to(gpu_device)
    w = seeded((N, K), seed=8, dtype=torch.float32, std=0.05).to(gpu_device)
    b = seeded((N,), seed=9, dtype=torch.float32).to(gpu_device)
    qx = ops.quant_tile_1x128(x, fmt=fmt)
    qw = ops.quant_tile_1x128(w, fmt=fmt)
    y = ops.gemm_blockscaled(qx, qw, bias=b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    _, _, _, xdq = O.quant_tile_1x128(to_np32(x), grid=grid)
    _, _, _, wdq = O.quant_tile_1x128(to_np32(w), grid=grid)
    ref = O.gemm_ref(xdq, wdq, to_np32(b))
    err = O.rel_frobenius(y.cpu().numpy(), ref)
    assert err <= 1e-5, err


def test_gemm_tensor_scales(gpu_device):
    """The non-recipe default: one scale per tensor on both operands."""
    from lowbit import ops
    from lowbit.ops import QTensor

    M, N, K = 64, 96, 256
    x = seeded((M, K), seed=10).to(gpu_device)
    w = seeded((N, K), seed=11, std=0.02).to(gpu_device)
    cx, sx, _, _ = ops.quant_grouped(x, M, K, ldc=256)
    cw, sw, _, _ = ops.quant_grouped(w, N, K, ldc=256)
    qx = QTensor(cx, sx, 0, 0, 0, O.GRID_INT, M, K)
    qw = QTensor(cw, sw, 0, 0, 0, O.GRID_INT, N, K)
    y = ops.gemm_blockscaled(qx, qw)
    torch.cuda.synchronize()
    _, _, _, xdq = O.quant_grouped(to_np32(x), M, K)
    _, _, _, wdq = O.quant_grouped(to_np32(w), N, K)
    assert rel_fro_bf16(y, O.gemm_ref(xdq, wdq)) <= TOL


def test_gemm_nan_rows_propagate(gpu_device):
    from lowbit import ops

    M, N, K = 64, 64, 256
    x = seeded((M, K), seed=12).to(gpu_device)
    w = seeded((N, K), seed=13, std=0.02).to(gpu_device)
    x[5, 17] = float("nan")
    w[9, 200] = float("nan")
    qx = ops.quant_tile_1x128(x, want_nan_rows=True)
    qw, _ = ops.quant_block_128x128(w, want_nan_rows=True)
    y = ops.gemm_blockscaled(qx, qw).float().cpu()
    nan = torch.isnan(y)
    assert nan[5].all() and nan[:, 9].all()
    assert nan.sum() == M + N - 1


@pytest.mark.parametrize("fmt,grid", GRIDS)
def test_gemm_full_size_c2_sampled(gpu_device, fmt, grid):
    """Config 2 at full size; the oracle checks a 64-row x 512-column sample."""
    from lowbit import ops

    M, N, K = 8192, 18432, 7168
    x = seeded((M, K), seed=20260201, heavy_channels=True).to(gpu_device)
    w = seeded((N, K), seed=20260202, std=0.006).to(gpu_device)
    qx = ops.quant_tile_1x128(x, fmt=fmt)
    qw, _ = ops.quant_block_128x128(w, fmt=fmt)
    y = ops.gemm_blockscaled(qx, qw)
    torch.cuda.synchronize()
    rows = np.random.default_rng(0).choice(M, 64, replace=False)
    cols = np.random.default_rng(1).choice(N, 512, replace=False)
    _, _, _, xdq = O.quant_tile_1x128(to_np32(x[rows]), grid=grid)
    wdq_full = O.quant_block_128x128(to_np32(w), grid=grid)[3]
    ref = O.gemm_ref(xdq, wdq_full[cols])
    err = rel_fro_bf16(y[rows][:, cols], ref)
    assert err <= TOL, err
