"""GPU parity of the quantizers against the CPU oracle: codes, scales, dq and
NaN row flags must be bit-exact on identical seeded inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import (assert_bits_equal, oracle_128x1_t_cols, oracle_tile_1x128_rows, scales_row_major, seeded,
                       to_np32)
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GRIDS = [("int_grid", O.GRID_INT), ("e4m3", O.GRID_E4M3)]
ROUNDS = [("nearest", O.ROUND_NEAREST), ("stochastic", O.ROUND_STOCHASTIC)]
SHAPES = [(3, 257), (64, 1024), (130, 300), (512, 1024), (1, 8), (5, 4)]


def _check_tile(x, fmt, grid, rname, rcode, bits=8, seed=0, offset=0):
    from lowbit import ops

    R, K = x.reshape(-1, x.shape[-1]).shape
    q = ops.quant_tile_1x128(x, fmt=fmt, bits=bits, rounding=rname, seed=seed, offset=offset, want_dq=True,
                             want_nan_rows=True)
    torch.cuda.synchronize()
    xn = to_np32(x).reshape(R, K)
    codes, scales, qv, dq = O.quant_tile_1x128(xn, grid=grid, bits=bits, rounding=rcode, seed=seed, offset=offset)
    assert_bits_equal(q.codes.cpu().numpy(), codes, "codes")
    assert_bits_equal(scales_row_major(q, R, scales.shape[1]), scales, "scales")
    dq_ref = torch.from_numpy(dq).to(x.dtype).float().numpy()
    assert_bits_equal(to_np32(q.dq), dq_ref, "dq")
    nan_ref = np.isnan(qv).any(axis=1).astype(np.int32)
    assert np.array_equal(q.nan_rows.cpu().numpy(), nan_ref)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("fmt,grid", GRIDS)
@pytest.mark.parametrize("rname,rcode", ROUNDS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_tile_1x128_parity(gpu_device, shape, fmt, grid, rname, rcode, dtype):
    x = seeded(shape, seed=20260101, dtype=dtype, outliers=0.01).to(gpu_device)
    _check_tile(x, fmt, grid, rname, rcode, seed=1234, offset=7)


def test_tile_1x128_fp4_mode_and_3d(gpu_device):
    # bits=4 (the fp4 emulated mode, qmax 7) on a 3-D activation
    x = seeded((2, 3, 257), seed=20260102, dtype=torch.bfloat16).to(gpu_device)
    _check_tile(x, "int_grid", O.GRID_INT, "nearest", O.ROUND_NEAREST, bits=4)


def test_tile_1x128_special_values(gpu_device):
    x = torch.zeros(6, 256)
    x[1, :3] = torch.tensor([float("inf"), 2.6, -300.0])
    x[2, :3] = torch.tensor([float("nan"), 2.6, -300.0])
    x[3, :2] = torch.tensor([1e-45, -1e-45])
    x[4, 130] = -0.0
    x[5] = torch.linspace(-3, 3, 256)
    for dtype in (torch.float32, torch.bfloat16):
        for fmt, grid in GRIDS:
            for rname, rcode in ROUNDS:
                _check_tile(x.to(dtype).to(gpu_device), fmt, grid, rname, rcode, seed=5)


@pytest.mark.parametrize("shape", [(300, 260), (128, 128), (1024, 1024), (129, 520)])
@pytest.mark.parametrize("fmt,grid", GRIDS)
@pytest.mark.parametrize("rname,rcode", ROUNDS)
def test_block_128x128_parity(gpu_device, shape, fmt, grid, rname, rcode):
    from lowbit import ops

    w = seeded(shape, seed=20260103, std=0.02).to(gpu_device)
    q, qt = ops.quant_block_128x128(w, fmt=fmt, rounding=rname, seed=99, offset=3, want_transposed=True,
                                    want_dq=True)
    torch.cuda.synchronize()
    N, K = shape
    codes, scales, qv, dq = O.quant_block_128x128(to_np32(w), grid=grid, rounding=rcode, seed=99, offset=3)
    assert_bits_equal(q.codes.cpu().numpy(), codes, "codes")
    assert_bits_equal(q.scales.cpu().numpy(), scales, "scales")
    assert_bits_equal(to_np32(q.dq), torch.from_numpy(dq).to(w.dtype).float().numpy(), "dq")
    NB = -(-N // 128)
    ct = np.zeros((K, NB * 128), dtype=np.uint8)
    ct[:, :N] = codes[:, :K].T
    assert_bits_equal(qt.codes.cpu().numpy(), ct, "codes_t")


@pytest.mark.parametrize("shape", [(300, 70), (256, 1024), (130, 257)])
@pytest.mark.parametrize("fmt,grid", GRIDS)
@pytest.mark.parametrize("rname,rcode", ROUNDS)
def test_tile_128x1_transposed_parity(gpu_device, shape, fmt, grid, rname, rcode):
    from lowbit import ops

    x = seeded(shape, seed=20260104, std=1e-3).to(gpu_device)
    q = ops.quant_tile_128x1_t(x, fmt=fmt, rounding=rname, seed=17, offset=11, want_dq=True)
    torch.cuda.synchronize()
    R, K = shape
    ct, st, qv, dq = O.quant_tile_128x1_t(to_np32(x), grid=grid, rounding=rcode, seed=17, offset=11)
    assert_bits_equal(q.codes.cpu().numpy(), ct, "codes_t")
    assert_bits_equal(scales_row_major(q, K, st.shape[1]), st, "scales")
    assert_bits_equal(to_np32(q.dq), torch.from_numpy(dq).to(x.dtype).float().numpy(), "dq")


@pytest.mark.parametrize("shape", [(300, 136), (1000, 384), (128, 8), (2, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("fmt,grid", GRIDS)
@pytest.mark.parametrize("rname,rcode", ROUNDS)
@pytest.mark.parametrize("want_dq", [False, True])
def test_tile_128x1_fast_path_special_columns(gpu_device, shape, dtype, fmt, grid, rname, rcode, want_dq):
    """The 8-aligned path of the 128x1 quantizer: ragged R, both input dtypes,
    columns holding a NaN, an inf, all zeros and subnormals; NaN flags land on
    the transposed rows (source columns) that hold the NaN."""
    from lowbit import ops

    R, K = shape
    x = seeded(shape, seed=20260110, std=1e-2, outliers=0.02).float()
    if K >= 8:
        x[R // 2, 1] = float("nan")
        x[0, 3] = float("inf")
        x[:, 5] = 0.0
        x[:, 6] = 1e-39
        x[R - 1, 7] = -float("inf")
    x = x.to(dtype).to(gpu_device)
    q = ops.quant_tile_128x1_t(x, fmt=fmt, rounding=rname, seed=5, offset=7, want_dq=want_dq, want_nan_rows=True)
    torch.cuda.synchronize()
    ct, st, qv, dq = O.quant_tile_128x1_t(to_np32(x), grid=grid, rounding=rcode, seed=5, offset=7)
    assert_bits_equal(q.codes.cpu().numpy(), ct, "codes_t")
    assert_bits_equal(scales_row_major(q, K, st.shape[1]), st, "scales")
    if want_dq:
        assert_bits_equal(to_np32(q.dq), torch.from_numpy(dq).to(x.dtype).float().numpy(), "dq")
    nan_ref = np.isnan(to_np32(x)).any(axis=0).astype(np.int32)
    assert np.array_equal(q.nan_rows.cpu().numpy(), nan_ref)


@pytest.mark.parametrize("shape", [(300, 136), (1000, 384), (128, 8), (2, 264)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("fmt,grid", GRIDS)
@pytest.mark.parametrize("rname,rcode", ROUNDS)
@pytest.mark.parametrize("o_cols", [3, 2])
def test_dual_1x128_128x1_parity(gpu_device, shape, dtype, fmt, grid, rname, rcode, o_cols):
    """The one-pass dY quantizer writes exactly the 1x128 and the 128x1
    outputs of the oracle (and of the two single-output kernels), with the
    two layouts keyed at different offsets, or at one offset, where the
    stochastic-rounding pass draws each word once for both."""
    from lowbit import ops

    R, K = shape
    x = seeded(shape, seed=20260111, std=1e-3, outliers=0.02).float()
    x[R // 2, 1] = float("nan")
    x[0, 3] = float("inf")
    x[:, 5] = 0.0
    x = x.to(dtype).to(gpu_device)
    qr, qc = ops.quant_dual_1x128_128x1(x, fmt=fmt, rounding=rname, seed=9, offset_rows=2, offset_cols=o_cols,
                                        want_nan_rows=True)
    torch.cuda.synchronize()
    xn = to_np32(x)
    codes, scales, qv, _ = O.quant_tile_1x128(xn, grid=grid, rounding=rcode, seed=9, offset=2)
    assert_bits_equal(qr.codes.cpu().numpy(), codes, "1x128 codes")
    assert_bits_equal(scales_row_major(qr, R, scales.shape[1]), scales, "1x128 scales")
    assert np.array_equal(qr.nan_rows.cpu().numpy(), np.isnan(qv).any(axis=1).astype(np.int32))
    ct, st, _, _ = O.quant_tile_128x1_t(xn, grid=grid, rounding=rcode, seed=9, offset=o_cols)
    assert_bits_equal(qc.codes.cpu().numpy(), ct, "128x1 codes_t")
    assert_bits_equal(scales_row_major(qc, K, st.shape[1]), st, "128x1 scales")
    assert np.array_equal(qc.nan_rows.cpu().numpy(), np.isnan(xn).any(axis=0).astype(np.int32))
    q1 = ops.quant_tile_1x128(x, fmt=fmt, rounding=rname, seed=9, offset=2)
    q2 = ops.quant_tile_128x1_t(x, fmt=fmt, rounding=rname, seed=9, offset=o_cols)
    assert torch.equal(q1.codes, qr.codes) and torch.equal(q2.codes, qc.codes)
    # tile-major scale arrays pad rows to a multiple of 4; compare what is written
    assert torch.equal(q1.scales[:, :R], qr.scales[:, :R]) and torch.equal(q2.scales[:, :K], qc.scales[:, :K])


def test_c3_dy_128x1_full_size(gpu_device):
    """benchmark config 3: dY [8192, 18432] 128x1 tiles (the wgrad operand dY^T)."""
    from lowbit import ops, workloads

    dy = workloads.c3_grad(device="cpu")
    q = ops.quant_tile_128x1_t(dy.to(gpu_device), fmt="e4m3")
    torch.cuda.synchronize()
    ct, st, _, _ = O.quant_tile_128x1_t(dy.float().numpy(), grid=O.GRID_E4M3)
    assert_bits_equal(q.codes.cpu().numpy(), ct, "codes_t")
    assert_bits_equal(scales_row_major(q, dy.shape[1], st.shape[1]), st, "scales")


@pytest.mark.parametrize("fmt,grid", GRIDS)
def test_c3_dy_full_size_stochastic_rounding(gpu_device, fmt, grid):
    """benchmark config 3 with its seeded stochastic rounding, at full size:
    dY [8192, 18432] per 1x128 tile (the dgrad operand) and per 128x1 tile
    (dY^T for wgrad), single passes and the dual pass, codes and scales bit
    for bit against the oracle.  The offsets use the Philox counter's high
    offset word (offset >= 2^32)."""
    from lowbit import ops, workloads

    dy = workloads.c3_grad(device="cpu")
    dyn = dy.float().numpy()
    dyg = dy.to(gpu_device)
    o_rows, o_cols = (1 << 32) + 2, (1 << 32) + 3
    kw = dict(grid=grid, rounding=O.ROUND_STOCHASTIC, seed=3)
    q1 = ops.quant_tile_1x128(dyg, fmt=fmt, rounding="stochastic", seed=3, offset=o_rows, tile_major_scales=False)
    torch.cuda.synchronize()
    c, s = oracle_tile_1x128_rows(dyn, offset=o_rows, **kw)
    assert_bits_equal(q1.codes.cpu().numpy(), c, "dY 1x128 codes")
    assert_bits_equal(q1.scales.cpu().numpy(), s, "dY 1x128 scales")
    del c, s
    q2 = ops.quant_tile_128x1_t(dyg, fmt=fmt, rounding="stochastic", seed=3, offset=o_cols)
    torch.cuda.synchronize()
    ct, st = oracle_128x1_t_cols(dyn, offset=o_cols, **kw)
    assert_bits_equal(q2.codes.cpu().numpy(), ct, "dY 128x1 codes")
    assert_bits_equal(scales_row_major(q2, dy.shape[1], st.shape[1]), st, "dY 128x1 scales")
    del ct, st
    qd, qdt = ops.quant_dual_1x128_128x1(dyg, fmt=fmt, rounding="stochastic", seed=3, offset_rows=o_rows,
                                         offset_cols=o_cols)
    torch.cuda.synchronize()
    assert torch.equal(qd.codes, q1.codes) and torch.equal(qdt.codes, q2.codes)
    R, K = dy.shape
    assert torch.equal(qd.scales[:, :R].t(), q1.scales) and torch.equal(qdt.scales[:, :K], q2.scales[:, :K])
    del qd, qdt, q2
    # one offset for both layouts (the recipe backward's keying): the dual
    # pass draws each word once and matches the single passes at that offset
    qd, qdt = ops.quant_dual_1x128_128x1(dyg, fmt=fmt, rounding="stochastic", seed=3, offset_rows=o_rows,
                                         offset_cols=o_rows)
    q3 = ops.quant_tile_128x1_t(dyg, fmt=fmt, rounding="stochastic", seed=3, offset=o_rows)
    torch.cuda.synchronize()
    assert torch.equal(qd.codes, q1.codes) and torch.equal(qdt.codes, q3.codes)
    assert torch.equal(qdt.scales[:, :K], q3.scales[:, :K])


@pytest.mark.parametrize("fmt,grid", GRIDS)
def test_sr_uses_both_high_counter_words(gpu_device, fmt, grid):
    """Stochastic rounding with every word of the Philox counter in play:
    offset >= 2^32 (counter word 3) and element indices >= 2^34, i.e.
    element/4 >= 2^32 (counter word 1).  x is [2^24 + 64, 1024] bf16 (32 GiB);
    its last 64 rows, whose element indices all pass 2^34, carry seeded data
    and are checked bit for bit against the oracle keyed at their place."""
    from lowbit import ops

    R, K = (1 << 24) + 64, 1024
    tail = seeded((64, K), seed=20260311, outliers=0.01)
    x = torch.zeros((R, K), dtype=torch.bfloat16, device=gpu_device)
    x[R - 64:] = tail.to(gpu_device)
    seed, offset = 0x123456789ABC, (1 << 33) + 7
    q = ops.quant_tile_1x128(x, fmt=fmt, rounding="stochastic", seed=seed, offset=offset, tile_major_scales=False)
    torch.cuda.synchronize()
    codes, scales = q.codes[R - 64:].cpu().numpy(), q.scales[R - 64:].cpu().numpy()
    del q, x
    torch.cuda.empty_cache()
    assert (R - 64) * K >= 1 << 34
    c, s, _, _ = O.quant_tile_1x128(tail.float().numpy(), grid=grid, rounding=O.ROUND_STOCHASTIC, seed=seed,
                                    offset=offset, elem_base=(R - 64) * K)
    assert_bits_equal(codes, c, "codes at element index >= 2^34")
    assert_bits_equal(scales, s, "scales")


def _clamp_hits(seed: int, offset: int, idx: np.ndarray) -> np.ndarray:
    """Which source indices draw u >= 1 - 2^-18, the draws for which
    qmax + u rounds to qmax + 1 in fp32."""
    words = O.sr_bits(seed, offset, 0, int(idx.max()) + 1)[idx]
    return (words >> 8) >= (1 << 24) - 64


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_sr_clamps_after_rounding_at_the_tile_amax(gpu_device, sign):
    """Regression: the reference clamps after rounding (te_backend.py:102-106).
    With a tile amax of 127 the scale is 1 and the amax element's v is
    exactly +-127; where its draw u >= 1 - 2^-18, +-127 + u rounds to +-128
    in fp32 and must clamp back to +-127 (int grid), not wrap to the NaN
    code -128.  Elements with such draws are found with the oracle's SR bits
    and given the amax, in 1x128 tiles (each row's element 0) and in 128x1
    tiles (one row per column)."""
    from lowbit import ops

    seed, offset = 77, 5
    # 1x128: rows of 8; element 0 of row r has source index 8r
    R = 1 << 20
    hit_rows = np.nonzero(_clamp_hits(seed, offset, np.arange(R) * 8))[0]
    assert len(hit_rows) > 0
    x = torch.full((R, 8), 0.5)
    x[:, 0] = 127.0 * sign
    xg = x.to(torch.bfloat16).to(gpu_device)
    q = ops.quant_tile_1x128(xg, fmt="int_grid", rounding="stochastic", seed=seed, offset=offset)
    torch.cuda.synchronize()
    codes = q.codes.cpu().numpy()
    assert np.all(codes[hit_rows, 0] == (127 if sign > 0 else 0x81))
    c_ref = O.quant_tile_1x128(x.numpy(), rounding=O.ROUND_STOCHASTIC, seed=seed, offset=offset)[0]
    assert_bits_equal(codes, c_ref, "1x128 codes")
    # 128x1: column k's amax at a row m whose index m*K + k draws such a u
    K = 8192
    m_idx = np.arange(128)[:, None] * K + np.arange(K)[None, :]
    hits = _clamp_hits(seed, offset, m_idx.reshape(-1)).reshape(128, K)
    cols = np.nonzero(hits.any(axis=0))[0]
    assert len(cols) > 0
    rows_at = np.where(hits.any(axis=0), hits.argmax(axis=0), 0)
    xt = torch.full((128, K), 0.5)
    xt[rows_at, np.arange(K)] = 127.0 * sign
    qt = ops.quant_tile_128x1_t(xt.to(torch.bfloat16).to(gpu_device), fmt="int_grid", rounding="stochastic",
                                seed=seed, offset=offset)
    torch.cuda.synchronize()
    ct = qt.codes.cpu().numpy()
    assert np.all(ct[cols, rows_at[cols]] == (127 if sign > 0 else 0x81))
    ct_ref = O.quant_tile_128x1_t(xt.numpy(), rounding=O.ROUND_STOCHASTIC, seed=seed, offset=offset)[0]
    assert_bits_equal(ct, ct_ref, "128x1 codes")


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_e4m3_sr_clamps_after_rounding_at_448(gpu_device, sign):
    """The e4m3 counterpart: with every element at +-448 the scale is 1 and
    v = +-448 = 1.75 * 2^8 sits on a code, so the 20 bits below its spacing
    are zero and no word carries it up, not even one with r >> 12 = 2^20 - 1:
    every code is 0x7E / 0xFE, never the NaN code 0x7F.  Checked in 1x128
    tiles (2^24 elements, several such words with this seed) and in 128x1
    tiles (128 x 65536) against the oracle."""
    from lowbit import ops

    seed, offset = 77, 5
    code = 0x7E if sign > 0 else 0xFE
    R = 1 << 21
    words = O.sr_bits(seed, offset, 0, R * 8)
    assert int(((words >> 12) == (1 << 20) - 1).sum()) > 0
    x = torch.full((R, 8), 448.0 * sign)
    q = ops.quant_tile_1x128(x.to(torch.bfloat16).to(gpu_device), fmt="e4m3", rounding="stochastic", seed=seed,
                             offset=offset)
    torch.cuda.synchronize()
    codes = q.codes.cpu().numpy()[:, :8]
    assert np.all(codes == code)
    c_ref = O.quant_tile_1x128(x.numpy(), grid=O.GRID_E4M3, rounding=O.ROUND_STOCHASTIC, seed=seed,
                               offset=offset)[0]
    assert_bits_equal(codes, c_ref[:, :8], "1x128 codes")
    K = 65536
    words = O.sr_bits(seed, offset, 0, 128 * K)
    assert int(((words >> 12) == (1 << 20) - 1).sum()) > 0
    xt = torch.full((128, K), 448.0 * sign)
    qt = ops.quant_tile_128x1_t(xt.to(torch.bfloat16).to(gpu_device), fmt="e4m3", rounding="stochastic",
                                seed=seed, offset=offset)
    torch.cuda.synchronize()
    ct = qt.codes.cpu().numpy()
    assert np.all(ct == code)
    ct_ref = O.quant_tile_128x1_t(xt.numpy(), grid=O.GRID_E4M3, rounding=O.ROUND_STOCHASTIC, seed=seed,
                                  offset=offset)[0]
    assert_bits_equal(ct, ct_ref, "128x1 codes")


@pytest.mark.parametrize("kind", ["tensor", "channel_last", "channel_rows", "strip"])
@pytest.mark.parametrize("fmt,grid", GRIDS)
@pytest.mark.parametrize("rname,rcode", ROUNDS)
def test_grouped_parity(gpu_device, kind, fmt, grid, rname, rcode):
    from lowbit import ops

    R, K = 300, 520
    x = seeded((R, K), seed=20260105, outliers=0.01).to(gpu_device)
    gr, gc, rule = {
        "tensor": (R, K, O.SCALE_AFTER_DIVIDE),
        "channel_last": (R, 1, O.SCALE_AFTER_DIVIDE),
        "channel_rows": (1, K, O.SCALE_AFTER_DIVIDE),
        "strip": (R, 128, O.SCALE_BEFORE_DIVIDE),
    }[kind]
    codes, scales, dq, nan_rows = ops.quant_grouped(x, gr, gc, fmt=fmt, rounding=rname, seed=3, offset=1,
                                                    scale_rule=rule, want_dq=True, want_nan_rows=True)
    torch.cuda.synchronize()
    c2, s2, q2, d2 = O.quant_grouped(to_np32(x), gr, gc, grid=grid, rounding=rcode, seed=3, offset=1, scale_rule=rule)
    assert_bits_equal(codes.cpu().numpy(), c2, "codes")
    assert_bits_equal(scales.cpu().numpy(), s2, "scales")
    assert_bits_equal(to_np32(dq), torch.from_numpy(d2).to(x.dtype).float().numpy(), "dq")


@pytest.mark.parametrize("R,K,gr,gc", [(300, 520, 128, 1), (300, 520, 7, 3), (70000, 8, 1, 1)])
@pytest.mark.parametrize("rname,rcode", ROUNDS)
def test_grouped_parity_narrow_column_groups(gpu_device, R, K, gr, gc, rname, rcode):
    """Column groups narrower than 8 (one scale per column, or per 3) take
    the workgroup-reduced amax pass, whose workgroups each cover one row
    group: 128-row groups (the last ragged), 7-row groups, and 70000 one-row
    groups, more than that pass launches, which fall back to the
    wide-group pass.  Codes, scales and dq bit-exact against the oracle."""
    from lowbit import ops

    x = seeded((R, K), seed=20260107, outliers=0.01).to(gpu_device)
    x[5, 2] = float("nan")
    x[:, 1] = 0.0
    codes, scales, dq, _ = ops.quant_grouped(x, gr, gc, fmt="int_grid", rounding=rname, seed=3, offset=1,
                                             scale_rule=O.SCALE_BEFORE_DIVIDE, want_dq=True)
    torch.cuda.synchronize()
    c2, s2, q2, d2 = O.quant_grouped(to_np32(x), gr, gc, grid=O.GRID_INT, rounding=rcode, seed=3, offset=1,
                                     scale_rule=O.SCALE_BEFORE_DIVIDE)
    assert_bits_equal(codes.cpu().numpy(), c2, "codes")
    assert_bits_equal(scales.cpu().numpy(), s2, "scales")
    assert_bits_equal(to_np32(dq), torch.from_numpy(d2).to(x.dtype).float().numpy(), "dq")


def test_strip_subnormal_amax_rule(gpu_device):
    from lowbit import ops

    x = torch.zeros(4, 128)
    x[0, :2] = torch.tensor([1e-45, -1e-45])
    x = x.to(gpu_device)
    codes, scales, dq, _ = ops.quant_grouped(x, 4, 128, scale_rule=O.SCALE_BEFORE_DIVIDE, want_dq=True)
    c2, s2, q2, d2 = O.quant_grouped(to_np32(x), 4, 128, scale_rule=O.SCALE_BEFORE_DIVIDE)
    assert_bits_equal(codes.cpu().numpy(), c2, "codes")
    assert_bits_equal(scales.cpu().numpy(), s2, "scales")
    assert_bits_equal(to_np32(dq), d2, "dq")


@pytest.mark.parametrize("fmt,grid", GRIDS)
def test_full_size_c2_activation_and_weight(gpu_device, fmt, grid):
    """Bit-exact at the DeepSeek-V3 MLP shapes of benchmark config 2."""
    from lowbit import ops

    x = seeded((8192, 7168), seed=20260201, heavy_channels=True).to(gpu_device)
    q = ops.quant_tile_1x128(x, fmt=fmt, tile_major_scales=False)
    torch.cuda.synchronize()
    codes, scales, _, _ = O.quant_tile_1x128(to_np32(x), grid=grid)
    assert_bits_equal(q.codes.cpu().numpy(), codes, "X codes")
    assert_bits_equal(q.scales.cpu().numpy(), scales, "X scales")
    del q, x
    w = seeded((18432, 7168), seed=20260202, std=0.006).to(gpu_device)
    qw, _ = ops.quant_block_128x128(w, fmt=fmt)
    torch.cuda.synchronize()
    codes, scales, _, _ = O.quant_block_128x128(to_np32(w), grid=grid)
    assert_bits_equal(qw.codes.cpu().numpy(), codes, "W codes")
    assert_bits_equal(qw.scales.cpu().numpy(), scales, "W scales")
