"""GPU parity of the split-K tail of the blockwise-scaled GEMM.

Tiles past the last whole wave are computed as K-range partials and summed in
a fixed order by the last range to finish.  The split result is checked
against the oracle (the 1e-3 bf16 bar), against the unsplit kernel in fp32
(only the summation order differs), and for determinism and for the
workspace's self-reset across calls and shapes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import rel_fro_bf16, seeded, to_np32
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
# fp32 accumulation of the same products in another association
REASSOC = 1e-5


def _operands(M, N, K, fmt, device, seed):
    from lowbit import ops

    x = seeded((M, K), seed=seed, outliers=0.01).to(device)
    w = seeded((N, K), seed=seed + 1, std=0.02).to(device)
    return x, w, ops.quant_tile_1x128(x, fmt=fmt), ops.quant_block_128x128(w, fmt=fmt)[0]


def _splits(M, N, Kp):
    from lowbit import _lib

    return int(_lib.lib().ntlb_gemm_workspace_bytes(M, N, Kp)) > 0


@pytest.mark.parametrize("mnk", [(512, 1024, 2304), (256, 512, 2432), (200, 300, 2360), (640, 768, 4608)])
@pytest.mark.parametrize("fmt,grid", [("int_grid", O.GRID_INT), ("e4m3", O.GRID_E4M3)])
def test_split_matches_oracle_and_unsplit(gpu_device, mnk, fmt, grid):
    from lowbit import ops

    M, N, K = mnk
    x, w, qx, qw = _operands(M, N, K, fmt, gpu_device, 20261101)
    assert _splits(M, N, qx.Kp), "shape chosen to take the split path"
    y = ops.gemm_blockscaled(qx, qw, out_dtype=torch.float32)
    y0 = ops.gemm_blockscaled(qx, qw, out_dtype=torch.float32, split_tail=False)
    yb = ops.gemm_blockscaled(qx, qw)
    torch.cuda.synchronize()
    assert O.rel_frobenius(y.cpu().numpy(), y0.cpu().numpy().astype(np.float64)) <= REASSOC
    xdq = O.quant_tile_1x128(to_np32(x), grid=grid)[3]
    wdq = O.quant_block_128x128(to_np32(w), grid=grid)[3]
    assert rel_fro_bf16(yb, O.gemm_ref(xdq, wdq)) <= TOL


def test_short_k_runs_unsplit():
    """K of 2048 or less (16 blocks) takes no split: two 8-block ranges lose to
    the partial tiles' round trip."""
    assert not _splits(512, 1024, 1024) and not _splits(512, 1024, 2048)
    assert _splits(512, 1024, 2304)


def test_split_deterministic_and_workspace_resets(gpu_device):
    """Repeated calls give identical bits; a smaller shape in between, on the
    same workspace, leaves it ready for the larger one again."""
    from lowbit import ops

    _, _, qx, qw = _operands(512, 1024, 2304, "e4m3", gpu_device, 20261102)
    _, _, qx2, qw2 = _operands(256, 512, 2432, "e4m3", gpu_device, 20261103)
    first = ops.gemm_blockscaled(qx, qw, out_dtype=torch.float32)
    small0 = ops.gemm_blockscaled(qx2, qw2, out_dtype=torch.float32, split_tail=False)
    for _ in range(3):
        small = ops.gemm_blockscaled(qx2, qw2, out_dtype=torch.float32)
        again = ops.gemm_blockscaled(qx, qw, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int32), first.view(torch.int32))
        assert O.rel_frobenius(small.cpu().numpy(), small0.cpu().numpy().astype(np.float64)) <= REASSOC


def test_split_bias_nan_rows_and_short_workspace(gpu_device):
    """Bias and NaN row flags go through the fixup's epilogue; a workspace
    shorter than the shape needs runs the unsplit kernel (same bits)."""
    from lowbit import _lib, ops

    M, N, K = 512, 768, 2304
    x = seeded((M, K), seed=20261104).to(gpu_device)
    w = seeded((N, K), seed=20261105, std=0.02).to(gpu_device)
    b = seeded((N,), seed=20261106, dtype=torch.float32).to(gpu_device)
    x[300, 17] = float("nan")
    w[700, 5] = float("nan")
    qx = ops.quant_tile_1x128(x, want_nan_rows=True)
    qw, _ = ops.quant_block_128x128(w, want_nan_rows=True)
    assert _splits(M, N, qx.Kp)
    y = ops.gemm_blockscaled(qx, qw, bias=b, out_dtype=torch.float32)
    y0 = ops.gemm_blockscaled(qx, qw, bias=b, out_dtype=torch.float32, split_tail=False)
    torch.cuda.synchronize()
    nan = torch.isnan(y)
    assert torch.equal(nan, torch.isnan(y0))
    assert nan[300].all() and nan[:, 700].all() and int(nan.sum()) == M + N - 1
    fin = ~nan
    assert O.rel_frobenius(y[fin].cpu().numpy(), y0[fin].cpu().numpy().astype(np.float64)) <= REASSOC

    need = int(_lib.lib().ntlb_gemm_workspace_bytes(M, N, qx.Kp))
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu_device)
    out = torch.empty((M, N), dtype=torch.float32, device=gpu_device)
    _lib.call("ntlb_gemm_blockscaled_ws", qx.grid, qx.codes.data_ptr(), qx.codes.stride(0), qx.scales.data_ptr(),
              qx.s_row, qx.s_col, qx.shift, qw.codes.data_ptr(), qw.codes.stride(0), qw.scales.data_ptr(), qw.s_row,
              qw.s_col, qw.shift, M, N, qx.Kp, b.data_ptr(), ops._dtype_code(b.dtype), out.data_ptr(),
              ops._dtype_code(out.dtype), out.stride(0), qx.nan_rows.data_ptr(), qw.nan_rows.data_ptr(),
              ws.data_ptr(), need - 1, ops._stream())
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), y0.view(torch.int32))
    assert int(ws.count_nonzero()) == 0  # never touched
    with pytest.raises(ValueError, match="256-byte aligned"):
        _lib.call("ntlb_gemm_blockscaled_ws", qx.grid, qx.codes.data_ptr(), qx.codes.stride(0),
                  qx.scales.data_ptr(), qx.s_row, qx.s_col, qx.shift, qw.codes.data_ptr(), qw.codes.stride(0),
                  qw.scales.data_ptr(), qw.s_row, qw.s_col, qw.shift, M, N, qx.Kp, None, 0, out.data_ptr(),
                  ops._dtype_code(out.dtype), out.stride(0), None, None, ws.data_ptr() + 64, need, ops._stream())


def test_split_full_size_c3_dgrad(gpu_device):
    """Config 3's dgrad shape (M 8192, N 7168, K 18432: 896 tiles, 128 split in
    two): split against unsplit over the whole output, and the oracle on a
    sample of rows in the split tiles."""
    from lowbit import ops

    M, N, K = 8192, 7168, 18432
    assert _splits(M, N, K)
    x = seeded((M, K), seed=20261107, heavy_channels=True).to(gpu_device)
    w = seeded((N, K), seed=20261108, std=0.006).to(gpu_device)
    qx = ops.quant_tile_1x128(x, fmt="e4m3")
    qw, _ = ops.quant_block_128x128(w, fmt="e4m3")
    y = ops.gemm_blockscaled(qx, qw, out_dtype=torch.float32)
    y0 = ops.gemm_blockscaled(qx, qw, out_dtype=torch.float32, split_tail=False)
    yb = ops.gemm_blockscaled(qx, qw)
    torch.cuda.synchronize()
    d = (y.double() - y0.double()).norm() / y0.double().norm()
    assert float(d) <= REASSOC, float(d)
    # the split tiles are the last 128 of the grouped raster: row tiles 24..31
    rows = np.random.default_rng(2).choice(np.arange(6144, M), 48, replace=False)
    cols = np.random.default_rng(3).choice(N, 384, replace=False)
    xdq = O.quant_tile_1x128(to_np32(x[rows]), grid=O.GRID_E4M3)[3]
    wdq = O.quant_block_128x128(to_np32(w), grid=O.GRID_E4M3)[3]
    err = rel_fro_bf16(yb[rows][:, cols], O.gemm_ref(xdq, wdq[cols]))
    assert err <= TOL, err


def test_split_workspace_shared_across_plans(gpu_device):
    """One workspace serves plans with different tail counts: a plan with 100
    split tiles (counters past the first 256 bytes), then one with 8, then the
    first again; every result matches the unsplit kernel."""
    from lowbit import ops

    big = _operands(2560, 2560, 2304, "e4m3", gpu_device, 20261109)[2:]
    small = _operands(512, 1024, 2304, "e4m3", gpu_device, 20261110)[2:]
    assert _splits(2560, 2560, 2304) and _splits(512, 1024, 2304)
    stream = torch.cuda.Stream(device=gpu_device)  # its own workspace
    stream.wait_stream(torch.cuda.current_stream())  # the operands were quantized there
    with torch.cuda.stream(stream):
        ref_big = ops.gemm_blockscaled(*big, out_dtype=torch.float32, split_tail=False)
        ref_small = ops.gemm_blockscaled(*small, out_dtype=torch.float32, split_tail=False)
        outs = [ops.gemm_blockscaled(*q, out_dtype=torch.float32) for q in (big, small, big, small, big)]
    stream.synchronize()
    for out, ref in zip(outs, (ref_big, ref_small, ref_big, ref_small, ref_big)):
        assert O.rel_frobenius(out.cpu().numpy(), ref.cpu().numpy().astype(np.float64)) <= REASSOC
