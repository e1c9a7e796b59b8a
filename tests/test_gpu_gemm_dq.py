"""GPU parity of the dequantized-operand GEMMs (csrc/gemm_dq.hip).

The reference multiplies operands rounded to the input dtype
(te_backend.py:173-202: `(q * scale).to(dtype=x.dtype)`) in an fp32 F.linear
(te_backend.py:253-259), and its straight-through backward multiplies the
same operands with the unquantized dY.  The oracle here is that computation
in float64 over the oracle's codes: round_bf16(dq) operands, bf16-to-bf16 at
the 1e-3 bar.  A tighter 2.5e-4 check separates these operands from the fp32
q * s ones (1.8e-3 to 2.3e-3 away), so a decode that skipped the bf16
rounding would fail it.  One-hot products check the in-kernel decode of
every code bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import bf16_bits, rel_fro_bf16, seeded, to_np32
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GRIDS = {"int_grid": O.GRID_INT, "e4m3": O.GRID_E4M3}
SHAPES = [(512, 1024, 1024), (300, 200, 384), (256, 256, 128), (77, 129, 257), (1024, 768, 2048)]


def _ops():
    from lowbit import ops

    return ops


def _bf16_oracle_operands(x: torch.Tensor, w: torch.Tensor, grid: int):
    xd = O.round_bf16(O.quant_tile_1x128(to_np32(x), grid=grid)[3])
    wd = O.round_bf16(O.quant_block_128x128(to_np32(w), grid=grid)[3])
    return xd, wd


@pytest.mark.parametrize("fmt", list(GRIDS))
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_dq_forward_matches_bf16_operand_oracle(gpu_device, fmt, M, N, K):
    ops = _ops()
    x = seeded((M, K), seed=20262001 + K, outliers=0.01).to(gpu_device)
    w = seeded((N, K), seed=20262002 + N, std=0.02).to(gpu_device)
    b = seeded((N,), seed=20262003).to(gpu_device)
    qx = ops.quant_tile_1x128(x, fmt=fmt)
    qw, _ = ops.quant_block_128x128(w, fmt=fmt)
    y = ops.gemm_dq_forward(qx, qw, bias=b, out_dtype=torch.bfloat16, op_dtype=torch.bfloat16)
    xd, wd = _bf16_oracle_operands(x, w, GRIDS[fmt])
    err = rel_fro_bf16(y, O.gemm_ref(xd, wd, to_np32(b)))
    assert err <= 1e-3 and err <= 2.5e-4, err


@pytest.mark.parametrize("fmt", list(GRIDS))
def test_dq_forward_fp32_operands(gpu_device, fmt):
    """fp32 inputs: the reference's operands are fp32 q * s (no rounding), on fp32 MFMA."""
    ops = _ops()
    x = seeded((200, 384), seed=20262011, dtype=torch.float32).to(gpu_device)
    w = seeded((160, 384), seed=20262012, dtype=torch.float32, std=0.05).to(gpu_device)
    qx = ops.quant_tile_1x128(x, fmt=fmt)
    qw, _ = ops.quant_block_128x128(w, fmt=fmt)
    y = ops.gemm_dq_forward(qx, qw, out_dtype=torch.float32, op_dtype=torch.float32)
    xd = O.quant_tile_1x128(to_np32(x), grid=GRIDS[fmt])[3]
    wd = O.quant_block_128x128(to_np32(w), grid=GRIDS[fmt])[3]
    assert O.rel_frobenius(y.cpu().numpy(), O.gemm_ref(xd, wd)) <= 1e-5


def _exhaustive_codes(grid: int, rows: int, cols: int) -> np.ndarray:
    """codes[r, c] = (r + c) % 256 with the NaN codes replaced by 0, so every
    row holds every finite code (and a one-hot product picks values exactly)."""
    c = ((np.arange(rows)[:, None] + np.arange(cols)[None, :]) % 256).astype(np.uint8)
    nan = (c == 0x80) if grid == O.GRID_INT else ((c & 0x7F) == 0x7F)
    c[nan] = 0
    return c


def _block_scales(nb: int, tb: int) -> np.ndarray:
    """distinct 128x128 block scales, including very small and large ones
    (2^-126: the products of codes below 1 are fp32 subnormals)"""
    base = np.array([1.0, 2.0 ** -126, 0.37, 1.7e3, 2.0 ** -20, 3.0 ** 7, 0.0123, 5.5], dtype=np.float32)
    return np.resize(base, nb * tb).reshape(nb, tb).astype(np.float32)


def _product_bits(dq: np.ndarray) -> np.ndarray:
    """bf16 bits of a one-hot product's result: the dequantized value, except
    that -0 (e4m3 code 0x80) sums with the +0 products to +0, as in any fp32
    GEMM"""
    b = O.to_bf16_bits(dq)
    b[b == 0x8000] = 0
    return b


@pytest.mark.parametrize("fmt", list(GRIDS))
def test_ste_dgrad_decodes_every_code_exactly(gpu_device, fmt):
    """dY one-hot (dY[m, n] = [m == n]) makes dX = the bf16 weight operand:
    every finite code times its block scale, rounded to bf16, bit for bit."""
    ops = _ops()
    grid = GRIDS[fmt]
    N, K = 256, 384
    codes = _exhaustive_codes(grid, N, K)
    sc = _block_scales(2, 3)
    qw = ops.QTensor(torch.from_numpy(codes).to(gpu_device), torch.from_numpy(sc).to(gpu_device), 3, 1, 7,
                     ops.grid_code(fmt), N, K)
    dy = torch.eye(N, dtype=torch.bfloat16, device=gpu_device)
    dx = ops.ste_dgrad(dy, qw, out_dtype=torch.bfloat16)
    want = _product_bits(O.dequant_grouped(codes, sc, K, 128, 128, grid))
    assert np.array_equal(bf16_bits(dx), want)


@pytest.mark.parametrize("fmt", list(GRIDS))
def test_ste_wgrad_decodes_every_code_exactly(gpu_device, fmt):
    """dY one-hot makes dW = the bf16 activation operand (1x128 tile scales,
    tile-major, one per row and 128 columns)."""
    ops = _ops()
    grid = GRIDS[fmt]
    M, K = 256, 256
    codes = _exhaustive_codes(grid, M, K)
    sc_rm = np.resize(_block_scales(2, 4).reshape(-1), M * 2).reshape(M, 2).astype(np.float32)  # [M, T]
    tile_major = np.zeros((2, M), dtype=np.float32)
    tile_major[:, :] = sc_rm.T
    qx = ops.QTensor(torch.from_numpy(codes).to(gpu_device), torch.from_numpy(tile_major).to(gpu_device), 1, M, 0,
                     ops.grid_code(fmt), M, K)
    dy = torch.eye(M, dtype=torch.bfloat16, device=gpu_device)
    dw = ops.ste_wgrad(dy, qx, out_dtype=torch.bfloat16)
    want = _product_bits(O.dequant_grouped(codes, sc_rm, K, 1, 128, grid))
    assert np.array_equal(bf16_bits(dw), want)


@pytest.mark.parametrize("fmt", list(GRIDS))
def test_dq_forward_decodes_every_code_exactly(gpu_device, fmt):
    """X one-hot (code of 1.0 at column m of row m, scale 1) makes Y = W_q^T."""
    ops = _ops()
    grid = GRIDS[fmt]
    N, K = 256, 256
    wcodes = _exhaustive_codes(grid, N, K)
    wsc = _block_scales(2, 2)
    one = 1 if grid == O.GRID_INT else 0x38  # e4m3 0x38 = 1.0
    xcodes = (np.eye(K, dtype=np.uint8) * one)
    xsc = np.ones((2, K), dtype=np.float32)  # tile-major [T, rows]
    qx = ops.QTensor(torch.from_numpy(xcodes).to(gpu_device), torch.from_numpy(xsc).to(gpu_device), 1, K, 0,
                     ops.grid_code(fmt), K, K)
    qw = ops.QTensor(torch.from_numpy(wcodes).to(gpu_device), torch.from_numpy(wsc).to(gpu_device), 2, 1, 7,
                     ops.grid_code(fmt), N, K)
    y = ops.gemm_dq_forward(qx, qw, out_dtype=torch.bfloat16, op_dtype=torch.bfloat16)
    want = _product_bits(O.dequant_grouped(wcodes, wsc, K, 128, 128, grid)).T
    assert np.array_equal(bf16_bits(y), np.ascontiguousarray(want))


def test_nan_codes_propagate_like_the_fp32_gemm(gpu_device):
    """An int-grid NaN code (-128) in W makes every dX of its column NaN and
    nothing else, as NaN in the reference's fp32 GEMM does."""
    ops = _ops()
    w = seeded((256, 256), seed=20262031, std=0.02)
    w[5, 17] = float("nan")
    w[200, 130] = float("nan")
    qw, _ = ops.quant_block_128x128(w.to(gpu_device), fmt="int_grid")
    dy = seeded((64, 256), seed=20262032, std=1e-3).to(gpu_device)
    dx = ops.ste_dgrad(dy, qw, out_dtype=torch.bfloat16).float().cpu()
    nan_cols = set(torch.nonzero(torch.isnan(dx).any(0)).flatten().tolist())
    assert nan_cols == {17, 130}
    assert torch.isnan(dx[:, [17, 130]]).all()


@pytest.mark.parametrize("fmt", list(GRIDS))
@pytest.mark.parametrize("M,N,K", [(256, 384, 512), (300, 200, 384), (77, 129, 257), (1000, 640, 1152)])
def test_ste_dgrad_wgrad_match_oracle(gpu_device, fmt, M, N, K):
    """dX = dY @ bf16(W_dq), dW = dY^T @ bf16(X_dq) (te_backend.py:250-259 under autograd)."""
    ops = _ops()
    x = seeded((M, K), seed=20262041, outliers=0.01).to(gpu_device)
    w = seeded((N, K), seed=20262042, std=0.02).to(gpu_device)
    dy = seeded((M, N), seed=20262043, std=1e-3).to(gpu_device)
    qx = ops.quant_tile_1x128(x, fmt=fmt)
    qw, _ = ops.quant_block_128x128(w, fmt=fmt)
    dx = ops.ste_dgrad(dy, qw, out_dtype=torch.bfloat16)
    dw = ops.ste_wgrad(dy, qx, out_dtype=torch.bfloat16)
    xd, wd = _bf16_oracle_operands(x, w, GRIDS[fmt])
    dyn = to_np32(dy).astype(np.float64)
    e1 = rel_fro_bf16(dx, dyn @ wd.astype(np.float64))
    e2 = rel_fro_bf16(dw, dyn.T @ xd.astype(np.float64))
    assert e1 <= 1e-3 and e2 <= 1e-3, (e1, e2)


@pytest.mark.parametrize("fmt", list(GRIDS))
@pytest.mark.parametrize("which", ["dgrad", "wgrad"])
def test_per_row_scales_past_the_last_contraction_row_add_nothing(gpu_device, fmt, which):
    """An operand with per-row 1x128 scales (X in wgrad, a 1x128-scaled W in
    dgrad) is contracted over its 97 rows in steps of 64: the scale slots of
    rows 97-127 are the tile-major array's padding (set to NaN here) and the
    first rows of the next 128-column block, whose row 0 is given a NaN
    scale here.  Their codes are zero and they must add nothing: NaN comes
    out in that tile's 128 columns and nowhere else."""
    ops = _ops()
    R, C, K = 97, 256, 384
    t = seeded((R, K), seed=20262045, outliers=0.01).to(gpu_device)
    q = ops.quant_tile_1x128(t, fmt=fmt)
    q.scales[:, R:] = float("nan")  # the padding slots of every 128-column block
    q.scales[1, 0] = float("nan")  # row 0's tile of columns 128-255: all its values NaN
    other = seeded((R, C), seed=20262046, std=1e-3).to(gpu_device)
    # dgrad: dX = other^T . bf16(dq(t)); wgrad: dW = other^T . bf16(dq(t)); the same product
    out = ops.ste_dgrad(other.t().contiguous(), q, out_dtype=torch.bfloat16) if which == "dgrad" else \
        ops.ste_wgrad(other, q, out_dtype=torch.bfloat16)
    out = out.float().cpu()
    nan_cols = torch.isnan(out).any(0)
    assert nan_cols[128:256].all() and not nan_cols[:128].any() and not nan_cols[256:].any()
    td = O.round_bf16(O.quant_tile_1x128(to_np32(t), grid=GRIDS[fmt])[3]).astype(np.float64)
    ref = to_np32(other).astype(np.float64).T @ td
    keep = np.r_[0:128, 256:K]
    assert rel_fro_bf16(out[:, keep], ref[:, keep]) <= 1e-3


@pytest.mark.parametrize("gran", ["tensor", "channel"])
def test_ste_dgrad_wgrad_tensor_and_channel_scales(gpu_device, gran):
    """Weight scales per tensor or per output row, activation scales per
    tensor (the shared-scale and per-contraction-row scale loads)."""
    ops = _ops()
    M, N, K = 320, 256, 384
    x = seeded((M, K), seed=20262051).to(gpu_device)
    w = seeded((N, K), seed=20262052, std=0.02).to(gpu_device)
    dy = seeded((M, N), seed=20262053, std=1e-3).to(gpu_device)
    gw = (1, K) if gran == "channel" else (N, K)
    wc, ws, _, _ = ops.quant_grouped(w, *gw, ldc=384, fmt="int_grid")
    qw = ops.QTensor(wc, ws, 1 if gran == "channel" else 0, 0, 0, 0, N, K)
    xc, xs, _, _ = ops.quant_grouped(x, M, K, ldc=384, fmt="int_grid")
    qx = ops.QTensor(xc, xs, 0, 0, 0, 0, M, K)
    dx = ops.ste_dgrad(dy, qw, out_dtype=torch.bfloat16)
    dw = ops.ste_wgrad(dy, qx, out_dtype=torch.bfloat16)
    wd = O.round_bf16(O.quant_grouped(to_np32(w), *gw)[3])
    xd = O.round_bf16(O.quant_grouped(to_np32(x), M, K)[3])
    dyn = to_np32(dy).astype(np.float64)
    assert rel_fro_bf16(dx, dyn @ wd.astype(np.float64)) <= 1e-3
    assert rel_fro_bf16(dw, dyn.T @ xd.astype(np.float64)) <= 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("b_transposed", [False, True])
def test_gemm_dense_matches_float64(gpu_device, dtype, b_transposed):
    ops = _ops()
    M, N, K = 300, 200, 200  # K not a multiple of the K step: zero padding inside the wrapper
    a = seeded((M, K), seed=20262061, dtype=dtype).to(gpu_device)
    b = seeded((K, N) if b_transposed else (N, K), seed=20262062, dtype=dtype).to(gpu_device)
    bias = seeded((N,), seed=20262063, dtype=dtype).to(gpu_device)
    out_dt = torch.float32 if dtype == torch.float32 else torch.bfloat16
    y = ops.gemm_dense(a, b, b_transposed=b_transposed, bias=bias, out_dtype=out_dt)
    bn = to_np32(b).astype(np.float64)
    ref = to_np32(a).astype(np.float64) @ (bn if b_transposed else bn.T) + to_np32(bias).astype(np.float64)
    if dtype == torch.float32:
        assert O.rel_frobenius(y.cpu().numpy(), ref) <= 1e-5
    else:
        assert rel_fro_bf16(y, ref) <= 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_dense_tn_matches_float64(gpu_device, dtype):
    ops = _ops()
    K, M, N = 333, 200, 136
    a = seeded((K, M), seed=20262071, dtype=dtype).to(gpu_device)
    b = seeded((K, N), seed=20262072, dtype=dtype).to(gpu_device)
    y = ops.gemm_dense_tn(a, b, out_dtype=torch.float32)
    ref = to_np32(a).astype(np.float64).T @ to_np32(b).astype(np.float64)
    assert O.rel_frobenius(y.cpu().numpy(), ref) <= 1e-5


@pytest.mark.parametrize("M,N", [(1, 5), (300, 200), (1000, 1037), (8192, 513)])
def test_colsum_matches_float64(gpu_device, M, N):
    ops = _ops()
    x = seeded((M, N), seed=20262081 + M, std=1e-3).to(gpu_device)
    s32 = ops.colsum(x, out_dtype=torch.float32).cpu().numpy()
    xn = to_np32(x).astype(np.float64)
    ref = xn.sum(0)
    # any fp32 summation order is within a few units of 2^-24 * sum |x| of
    # the exact sum; a dropped or repeated chunk is off by orders more
    assert np.all(np.abs(s32 - ref) <= 16 * 2.0 ** -24 * np.abs(xn).sum(0) + 1e-30)
    s16 = ops.colsum(x, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(O.round_bf16(s32), s16)  # the fp32 sum rounded once
    again = ops.colsum(x, out_dtype=torch.float32).cpu().numpy()
    assert np.array_equal(s32.view(np.uint32), again.view(np.uint32))  # fixed order


def test_dq_forward_c2_full_size_sampled(gpu_device):
    """benchmark config 2 at full size: the reference-exact forward against the
    bf16-operand oracle on sampled rows and columns."""
    from lowbit import workloads

    ops = _ops()
    x, w = workloads.c2_inputs(device="cpu")
    qx = ops.quant_tile_1x128(x.to(gpu_device), fmt="e4m3")
    qw, _ = ops.quant_block_128x128(w.to(gpu_device), fmt="e4m3")
    y = ops.gemm_dq_forward(qx, qw, out_dtype=torch.bfloat16, op_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    rows = np.random.default_rng(3).choice(8192, 24, replace=False)
    cols = np.random.default_rng(4).choice(18432, 160, replace=False)
    xd = O.round_bf16(O.quant_tile_1x128(x.float().numpy()[rows], grid=O.GRID_E4M3)[3])
    wd = O.round_bf16(O.quant_block_128x128(w.float().numpy(), grid=O.GRID_E4M3)[3])[cols]
    err = rel_fro_bf16(y[rows][:, cols], O.gemm_ref(xd, wd))
    assert err <= 1e-3 and err <= 2.5e-4, err


def test_ste_backward_c3_full_size_sampled(gpu_device):
    """benchmark config 3 shapes with the reference's straight-through backward:
    dX = dY @ bf16(W_dq) and dW = dY^T @ bf16(X_dq) from the forward's e4m3
    codes, on sampled rows / columns against the oracle."""
    from lowbit import workloads

    ops = _ops()
    x, w = workloads.c2_inputs(device="cpu")
    dy = workloads.c3_grad(device="cpu")
    qx = ops.quant_tile_1x128(x.to(gpu_device), fmt="e4m3")
    qw, _ = ops.quant_block_128x128(w.to(gpu_device), fmt="e4m3")
    dyg = dy.to(gpu_device)
    dx = ops.ste_dgrad(dyg, qw, out_dtype=torch.bfloat16)
    dw = ops.ste_wgrad(dyg, qx, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    rows = np.random.default_rng(5).choice(8192, 16, replace=False)
    kcols = np.random.default_rng(6).choice(7168, 128, replace=False)
    ncols = np.random.default_rng(7).choice(18432, 16, replace=False)
    wd = O.round_bf16(O.quant_block_128x128(w.float().numpy(), grid=O.GRID_E4M3)[3])
    dyn = dy.float().numpy()
    e1 = rel_fro_bf16(dx[rows][:, kcols], dyn[rows].astype(np.float64) @ wd[:, kcols].astype(np.float64))
    del wd
    xd = O.round_bf16(O.quant_tile_1x128(x.float().numpy(), grid=O.GRID_E4M3)[3])
    e2 = rel_fro_bf16(dw[ncols][:, kcols], dyn[:, ncols].T.astype(np.float64) @ xd[:, kcols].astype(np.float64))
    assert e1 <= 1e-3 and e2 <= 1e-3, (e1, e2)


@pytest.mark.parametrize("fmt", list(GRIDS))
@pytest.mark.parametrize("wscale,K", [("block", 2304), ("tile", 2304), ("tile", 2300), ("block", 2300)])
def test_ste_dgrad_split_tail_matches_unsplit(gpu_device, fmt, wscale, K):
    """dX [8192, K] (288 output tiles: one whole wave of 256 compute units
    plus a 32-tile tail) with the split-K workspace: the tail tiles' K ranges
    summed in a fixed order equal the unsplit product up to fp32 summation
    order and repeat bit for bit; a NaN code's column stays NaN through the
    split.  W's scales are 128x128 blocks (one scale per wave) or 1x128 tiles
    (contiguous per-row scales), and K = 2300 leaves the last tile column
    ragged.  (The oracle bar itself is checked by the tests above.)"""
    ops = _ops()
    from lowbit import _lib
    from lowbit._lib import call

    M, N = 8192, 4096  # contraction 4096: 64 K steps, split seven ways
    tiles = (M // 256) * (-(-K // 256))
    assert int(_lib.lib().ntlb_gemm_dq_workspace_bytes(_lib.BF16, M, K, N)) > 0, "the shape should split"
    w = seeded((N, K), seed=20262051, std=0.02)
    nan_col = 2299
    if fmt == "int_grid":
        w[3, nan_col] = float("nan")  # a column of the last (split) tile column
    if wscale == "block":
        qw, _ = ops.quant_block_128x128(w.to(gpu_device), fmt=fmt)
    else:
        qw = ops.quant_tile_1x128(w.to(gpu_device), fmt=fmt)
    dy = seeded((M, N), seed=20262052, std=1e-3).to(gpu_device)
    dx = ops.ste_dgrad(dy, qw, out_dtype=torch.float32)
    dx2 = ops.ste_dgrad(dy, qw, out_dtype=torch.float32)
    ref = torch.empty_like(dx)
    call("ntlb_gemm_ste_dgrad", _lib.BF16, dy.data_ptr(), dy.stride(0), M, N, qw.grid, qw.codes.data_ptr(),
         qw.codes.stride(0), qw.scales.data_ptr(), qw.s_row, qw.s_col, qw.shift, qw.K, ref.data_ptr(),
         ops._dtype_code(torch.float32), ref.stride(0), ops._stream())
    torch.cuda.synchronize()
    assert tiles == 288
    assert torch.equal(dx.view(torch.int32), dx2.view(torch.int32)), "split results must repeat bit for bit"
    nan = torch.isnan(ref)
    assert torch.equal(nan, torch.isnan(dx))
    if fmt == "int_grid":
        assert nan[:, nan_col].all() and nan.any(0).sum() == 1
    a, b = dx[~nan].double(), ref[~nan].double()
    assert float((a - b).norm() / b.norm()) <= 1e-6
    # the tail tiles lie in row tiles 28-31 (the last group of the grouped
    # raster); every tile above them runs whole in both calls, bit for bit
    assert torch.equal(dx[:7168].view(torch.int32), ref[:7168].view(torch.int32))


# M = 1 and 65: a contraction of one row, and one row past a K step (the
# transposing-load copies read zeros past the last row)
@pytest.mark.parametrize("M,N,K", [(300, 200, 384), (1000, 640, 1152), (77, 129, 257), (4096, 2304, 512),
                                   (1, 136, 128), (65, 264, 384)])
def test_ste_wgrad_with_db_matches_colsum(gpu_device, M, N, K):
    """The e4m3 straight-through wgrad that also forms db from its staged dY
    tiles (dY transposed in registers): dW bit-identical to the wgrad without
    db (dY through the transposing LDS loads), db within fp32
    reassociation of float64's column sums of dY (and of the separate
    column-sum pass), repeats bit-identical; the int grid refuses db."""
    ops = _ops()
    from lowbit._lib import LowBitKernelError

    x = seeded((M, K), seed=20262651, outliers=0.01).to(gpu_device)
    dy = seeded((M, N), seed=20262652, std=1e-2).to(gpu_device)
    qx = ops.quant_tile_1x128(x, fmt="e4m3")
    dw0 = ops.ste_wgrad(dy, qx, out_dtype=torch.bfloat16)
    dw1, db1 = ops.ste_wgrad(dy, qx, out_dtype=torch.bfloat16, db_dtype=torch.float32)
    dw2, db2 = ops.ste_wgrad(dy, qx, out_dtype=torch.bfloat16, db_dtype=torch.float32)
    _, db16 = ops.ste_wgrad(dy, qx, out_dtype=torch.bfloat16, db_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(dw0.view(torch.int16), dw1.view(torch.int16))
    assert torch.equal(db1, db2) and torch.equal(dw1.view(torch.int16), dw2.view(torch.int16))
    ref = to_np32(dy).astype(np.float64).sum(0)
    err = np.abs(db1.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 1e-6, err
    sep = ops.colsum(dy, out_dtype=torch.float32).cpu().numpy()
    assert np.abs(db1.cpu().numpy() - sep).max() <= 1e-6 * np.abs(ref).max()
    assert np.array_equal(bf16_bits(db16), O.to_bf16_bits(db1.cpu().numpy()))
    qi = ops.quant_tile_1x128(x, fmt="int_grid")
    with pytest.raises((LowBitKernelError, ValueError, RuntimeError)):
        ops.ste_wgrad(dy, qi, out_dtype=torch.bfloat16, db_dtype=torch.float32)
