"""Pins for the CPU oracle (oracle/lowbit_oracle.c + oracle/oracle.py).

The reference holds no numeric fixtures for this path, so each oracle function
is pinned here by an independent source: published known-answer vectors
(Philox), a library routine (torch's float8_e4m3fn cast, numpy argmin, Python's
round-half-even), closed forms built into the inputs (per-tile amax values
that fix every scale exactly), or the format's specification table (OCP e2m1).
Each pin is chosen so that a plausible mistake (a dropped /qmax, a transposed
block index, a wrong tie rule, swapped nibbles) fails it.  The published and
library tables live in tests/golden/ (written by tests/golden/make_fixtures.py).
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O


# ---------------------------------------------------------------------------
# Philox4x32-10: known-answer vectors of Random123 (Salmon et al., SC'11),
# kept in tests/golden/philox4x32_10_kat.json
# ---------------------------------------------------------------------------
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    with open(os.path.join(GOLDEN, name)) as fh:
        return json.load(fh)


@pytest.mark.parametrize("vec", _golden("philox4x32_10_kat.json")["vectors"])
def test_philox_known_answers(vec):
    assert list(O.philox4x32_10(vec["ctr"], vec["key"])) == vec["out"]


def test_sr_bits_contract_layout():
    seed, offset = 0x1234_5678_9ABC_DEF0, 0x0000_0002_0000_0007
    bits = O.sr_bits(seed, offset, 40, 8)
    for j in range(8):
        e = 40 + j
        g = e // 4
        ctr = [g & 0xFFFFFFFF, g >> 32, offset & 0xFFFFFFFF, offset >> 32]
        key = [seed & 0xFFFFFFFF, seed >> 32]
        assert bits[j] == O.philox4x32_10(ctr, key)[e % 4]


def test_sr_uniform_statistics():
    bits = O.sr_bits(7, 3, 0, 1 << 16)
    u = (bits >> 8).astype(np.float64) * 2.0**-24
    assert abs(u.mean() - 0.5) < 0.01
    assert abs(u.var() - 1 / 12) < 0.005


# ---------------------------------------------------------------------------
# e4m3: torch's float8_e4m3fn cast is the library oracle
# ---------------------------------------------------------------------------
def test_e4m3_encode_matches_torch_on_all_bf16():
    f = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    mine = O.e4m3_encode(f)
    ref = torch.from_numpy(f.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(mine, ref)


def test_e4m3_encode_matches_torch_on_random_fp32():
    rng = np.random.default_rng(1)
    f = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    # concentrate on the e4m3 range and its rounding boundaries as well
    g = (rng.standard_normal(1_000_000) * 100).astype(np.float32)
    for arr in (f, g):
        mine = O.e4m3_encode(arr)
        ref = torch.from_numpy(arr.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(mine, ref)


def test_e4m3_decode_matches_golden_table():
    """Every code against tests/golden/e4m3fn_codes.json (torch's decoding)."""
    want = np.array([int(b, 16) for b in _golden("e4m3fn_codes.json")["f32_bits"]], dtype=np.uint32).view(np.float32)
    mine = O.decode_codes(np.arange(256, dtype=np.uint8), O.GRID_E4M3).astype(np.float32)
    np.testing.assert_array_equal(np.isnan(mine), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(mine[ok].view(np.uint32), want[ok].view(np.uint32))


def test_e4m3_decode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    mine = O.decode_codes(codes, O.GRID_E4M3)
    ref = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(mine), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(mine[ok].view(np.uint32), ref[ok].view(np.uint32))


# ---------------------------------------------------------------------------
# int grid, round to nearest: te_backend.py:82-110
# ---------------------------------------------------------------------------
def test_round_half_even_textbook():
    # amax = 127 makes the scale exactly 1.0, so q = round-half-even(x)
    vals = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -125.5, 3.4999998, 0.49999997, 127.0]
    x = np.zeros((1, 128), dtype=np.float32)
    x[0, : len(vals)] = vals
    codes, scales, q, dq = O.quant_tile_1x128(x)
    assert scales[0, 0] == np.float32(1.0)
    expect = [round(v) for v in vals]  # Python rounds half to even
    assert list(q[0, : len(vals)]) == expect
    assert list(codes[0, : len(vals)].view(np.int8)) == expect
    assert np.array_equal(dq, q)


def test_tile_scales_follow_tile_index():
    # tile (r, t) holds amax a_rt = 10*(r+1) + t at a known column; every other
    # element is smaller.  A transposed tile index or a dropped /qmax fails.
    R, K = 3, 300
    rng = np.random.default_rng(2)
    x = (rng.uniform(-1, 1, size=(R, K))).astype(np.float32)
    T = 3
    for r in range(R):
        for t in range(T):
            col = t * 128 + (17 * r + 5 * t) % min(128, K - t * 128)
            x[r, col] = -(10.0 * (r + 1) + t) if (r + t) % 2 else 10.0 * (r + 1) + t
    codes, scales, q, dq = O.quant_tile_1x128(x)
    assert codes.shape == (R, 384)
    for r in range(R):
        for t in range(T):
            assert scales[r, t] == np.float32(10.0 * (r + 1) + t) / np.float32(127.0)
    # padding columns are zero codes; the amax element lands on +-127
    assert not codes[:, 300:].any()
    assert np.abs(q).max() == 127


def test_block_scales_follow_block_index():
    N, K = 300, 260  # 3 x 3 blocks, partial last row and column blocks
    rng = np.random.default_rng(3)
    w = rng.uniform(-0.5, 0.5, size=(N, K)).astype(np.float32)
    for nb in range(3):
        for kb in range(3):
            r = nb * 128 + (31 * kb + 7 * nb) % min(128, N - nb * 128)
            c = kb * 128 + (13 * nb + 3 * kb) % min(128, K - kb * 128)
            w[r, c] = 1.0 + 7 * nb + kb
    codes, scales, q, dq = O.quant_block_128x128(w)
    for nb in range(3):
        for kb in range(3):
            assert scales[nb, kb] == np.float32(1.0 + 7 * nb + kb) / np.float32(127.0)
    assert codes.shape == (N, 384) and not codes[:, 260:].any()


def test_rn_reconstruction_invariants():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((64, 512)) * np.exp(rng.uniform(-3, 3, size=(64, 1)))).astype(np.float32)
    codes, scales, q, dq = O.quant_tile_1x128(x)
    s = np.repeat(scales, 128, axis=1)
    assert np.all(np.abs(x - dq) <= s * 0.5000001)
    assert np.all(np.abs(q).reshape(64, 4, 128).max(axis=2) == 127)


def test_special_values():
    x = np.zeros((4, 128), dtype=np.float32)
    x[1, :3] = [np.inf, 2.6, -300.0]
    x[2, :3] = [np.nan, 2.6, -300.0]
    x[3, :2] = [1e-45, -1e-45]  # subnormal amax
    codes, scales, q, dq = O.quant_tile_1x128(x)
    # zero tile: scale 1 (te_backend.py:74-79 applied after the division)
    assert scales[0, 0] == 1.0 and not codes[0].any()
    # inf: amax/127 = inf -> scale 1, inf clamps to 127, the rest round(x) clamped
    assert scales[1, 0] == 1.0 and list(q[1, :3]) == [127.0, 3.0, -127.0]
    # NaN: amax NaN -> scale 1, NaN code -128, dq NaN
    assert scales[2, 0] == 1.0 and codes[2, 0] == 0x80 and np.isnan(dq[2, 0])
    assert list(q[2, 1:3]) == [3.0, -127.0]
    # subnormal amax: amax/127 underflows to 0 -> scale 1 under the te_backend rule
    assert scales[3, 0] == 1.0 and list(q[3, :2]) == [0.0, -0.0]
    # the moe.py:94-98 rule checks amax > 0 first: scale = amax/127 = 0 -> x/0
    _, s2, q2, _ = O.quant_grouped(x[3:4], 1, 128, scale_rule=O.SCALE_BEFORE_DIVIDE)
    assert s2[0, 0] == 0.0 and q2[0, 0] == 127.0 and q2[0, 1] == -127.0 and np.isnan(q2[0, 2])


def test_negative_zero_kept_in_q():
    x = np.zeros((1, 128), dtype=np.float32)
    x[0, 0] = 127.0
    x[0, 1] = -0.3
    _, _, q, dq = O.quant_tile_1x128(x)
    assert np.signbit(q[0, 1]) and np.signbit(dq[0, 1])


# ---------------------------------------------------------------------------
# stochastic rounding
# ---------------------------------------------------------------------------
def test_sr_int_grid_brackets_and_is_unbiased():
    x = np.zeros((1, 128), dtype=np.float32)
    x[0, 0] = 127.0  # scale 1
    x[0, 1:6] = [2.25, -2.25, 5.0, -7.0, 0.75]
    acc = np.zeros(6)
    draws = 4000
    for s in range(draws):
        _, _, q, _ = O.quant_tile_1x128(x, rounding=O.ROUND_STOCHASTIC, seed=s, offset=9)
        v = x[0, 1:6]
        assert np.all((q[0, 1:6] == np.floor(v)) | (q[0, 1:6] == np.ceil(v)))
        assert q[0, 3] == 5.0 and q[0, 4] == -7.0  # integers are exact
        acc[:5] += q[0, 1:6]
    mean = acc[:5] / draws
    assert abs(mean[0] - 2.25) < 0.03 and abs(mean[1] + 2.25) < 0.03 and abs(mean[4] - 0.75) < 0.03


def test_sr_uses_contract_bits():
    # floor(v + u) with u from the Philox contract, element index r*K + k
    x = np.full((2, 131), 0.5, dtype=np.float32)
    x[:, 0] = 127.0  # both tiles get scale 1
    x[:, 128] = 127.0
    _, _, q, _ = O.quant_tile_1x128(x, rounding=O.ROUND_STOCHASTIC, seed=11, offset=5)
    bits = O.sr_bits(11, 5, 0, 2 * 131).reshape(2, 131)
    u = (bits >> 8).astype(np.float32) * np.float32(2.0**-24)
    expect = np.floor(np.float32(0.5) + u)
    cols = [c for c in range(131) if c not in (0, 128)]
    assert np.array_equal(q[:, cols], expect[:, cols])
    assert 0 < q[:, cols].mean() < 1


def test_sr_e4m3_brackets_and_is_unbiased():
    v = np.array([1.1, -3.3, 0.004, 300.0, -0.017], dtype=np.float32)
    n = 20000
    bits = O.sr_bits(3, 1, 0, n * v.size).reshape(n, v.size)
    codes = O.e4m3_sr_encode(np.broadcast_to(v, (n, v.size)), bits)
    vals = O.decode_codes(codes, O.GRID_E4M3)
    lo = O.decode_codes(O.e4m3_encode(v), O.GRID_E4M3)
    for j in range(v.size):
        uniq = np.unique(vals[:, j])
        assert len(uniq) <= 2
        assert lo[j] in uniq or len(uniq) == 1
        assert abs(vals[:, j].mean() - v[j]) < abs(v[j]) * 0.01 + 2e-4


def test_e4m3_grid_scale_and_range():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((8, 256)) * 3).astype(np.float32)
    codes, scales, q, dq = O.quant_tile_1x128(x, grid=O.GRID_E4M3)
    amax = np.abs(x).reshape(8, 2, 128).max(axis=2)
    assert np.array_equal(scales, amax / np.float32(448.0))
    assert np.abs(q).max() == 448.0
    ref = torch.from_numpy((x / np.repeat(scales, 128, axis=1)).clip(-448, 448)).to(torch.float8_e4m3fn)
    assert np.array_equal(codes, ref.view(torch.uint8).numpy())


# ---------------------------------------------------------------------------
# grouped granularities: tensor / channel / strip (te_backend.py:165-185, moe.py:123-140)
# ---------------------------------------------------------------------------
def test_grouped_scales_follow_groups():
    R, K = 5, 260
    rng = np.random.default_rng(6)
    x = rng.uniform(-1, 1, size=(R, K)).astype(np.float32)
    x[3, 200] = 9.0
    # tensor
    _, s, _, _ = O.quant_grouped(x, R, K)
    assert s.shape == (1, 1) and s[0, 0] == np.float32(9.0) / np.float32(127)
    # channel along the last axis: one scale per column over all rows
    _, s, _, _ = O.quant_grouped(x, R, 1)
    assert s.shape == (1, K)
    assert np.array_equal(s[0], np.abs(x).max(axis=0) / np.float32(127))
    # channel along axis 0: one scale per row
    _, s, _, _ = O.quant_grouped(x, 1, K)
    assert np.array_equal(s[:, 0], np.abs(x).max(axis=1) / np.float32(127))
    # comm strip: one scale per 128 columns over all rows
    _, s, _, _ = O.quant_grouped(x, R, 128, scale_rule=O.SCALE_BEFORE_DIVIDE)
    expect = [np.abs(x[:, i : i + 128]).max() / np.float32(127) for i in (0, 128, 256)]
    assert list(s[0]) == expect


def test_tile_128x1_is_tile_of_transpose():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((300, 70)).astype(np.float32)
    ct, st, q, dq = O.quant_tile_128x1_t(x)
    c2, s2, q2, dq2 = O.quant_tile_1x128(np.ascontiguousarray(x.T))
    assert np.array_equal(ct, c2) and np.array_equal(st, s2)
    assert np.array_equal(dq, dq2.T)


# ---------------------------------------------------------------------------
# GEMM oracle: exact integer arithmetic when the scales are powers of two
# ---------------------------------------------------------------------------
def test_gemm_oracle_exact_on_power_of_two_scales():
    rng = np.random.default_rng(8)
    M, N, K = 37, 45, 256
    qa = rng.integers(-127, 128, size=(M, K))
    qb = rng.integers(-127, 128, size=(N, K))
    sa = 2.0 ** rng.integers(-6, 6, size=(M, 2))
    sb = 2.0 ** rng.integers(-6, 6, size=(1, 2))
    a_dq = O.dequant_grouped(qa.astype(np.int8).view(np.uint8), sa.astype(np.float32), K, 1, 128, O.GRID_INT)
    b_dq = O.dequant_grouped(qb.astype(np.int8).view(np.uint8), sb.astype(np.float32), K, 128, 128, O.GRID_INT)
    y = O.gemm_ref(a_dq, b_dq)
    exact = np.zeros((M, N))
    for kb in range(2):
        part = qa[:, kb * 128 : (kb + 1) * 128] @ qb[:, kb * 128 : (kb + 1) * 128].T
        exact += part * sa[:, kb : kb + 1] * sb[0, kb]
    assert np.array_equal(y, exact)


def test_bf16_rounding_helper_matches_torch():
    rng = np.random.default_rng(9)
    f = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    mine = O.to_bf16_bits(f)
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ok = ~np.isnan(f)
    assert np.array_equal(mine[ok], ref[ok])


# ---------------------------------------------------------------------------
# NF4 (layers.py:60-184): numpy argmin (first minimum) is the library oracle
# ---------------------------------------------------------------------------
def test_nf4_indices_match_numpy_argmin():
    rng = np.random.default_rng(10)
    w = (rng.standard_normal(4096) * 0.02).astype(np.float32)
    w[5] = np.nan
    for block in (64, 4096):
        packed, scales = O.nf4_quant(w, block)
        idx = np.empty(w.size, dtype=np.int64)
        idx[0::2] = packed & 15
        idx[1::2] = packed >> 4
        s = np.repeat(scales, block)[: w.size]
        c = np.clip(w / s, -1.0, 1.0).astype(np.float32)
        d = np.abs(c[:, None] - O.NF4_CODEBOOK[None, :])
        expect = np.where(np.isnan(c), 0, np.nanargmin(np.where(np.isnan(d), np.inf, d), axis=1))
        assert np.array_equal(idx, expect)


def test_nf4_ties_pick_lower_index_and_pack_low_nibble_first():
    cb = O.NF4_CODEBOOK
    mids = [(cb[i] + cb[i + 1]) / np.float32(2) for i in range(15)]
    w = np.array([1.0] + mids, dtype=np.float32)  # amax 1 -> scale 1, normalized = w
    packed, scales = O.nf4_quant(w, w.size)
    assert scales[0] == 1.0
    idx = np.empty(16, dtype=np.int64)
    idx[0::2] = packed & 15
    idx[1::2] = packed >> 4
    assert idx[0] == 15
    for i in range(15):
        m = np.float32(mids[i])
        dl, dh = abs(m - cb[i]), abs(m - cb[i + 1])
        assert idx[i + 1] == (i if dl <= dh else i + 1)
    # nibble order on a hand-built example
    w2 = np.array([-1.0, 1.0, 0.0], dtype=np.float32)
    p2, _ = O.nf4_quant(w2, 3)
    assert list(p2) == [0x0 | (0xF << 4), 0x7]


def test_nf4_dequant_round_trip_error_bound():
    rng = np.random.default_rng(11)
    w = (rng.standard_normal(64 * 100) * 0.02).astype(np.float32)
    packed, scales = O.nf4_quant(w, 64)
    d = O.nf4_dequant(packed, scales, w.size, 64)
    gap = np.max(np.diff(O.NF4_CODEBOOK))
    assert np.all(np.abs(d - w) <= np.repeat(scales, 64) * gap / 2 + 1e-7)


# ---------------------------------------------------------------------------
# MXFP4 (OCP MX v1.0): e2m1 table and the shared-exponent rule
# ---------------------------------------------------------------------------
def test_e2m1_table():
    vals = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=np.float32)
    codes = np.arange(16, dtype=np.uint8)
    dec = np.array([O.decode_codes(np.array([0]), 0)[0]])  # warm the lib
    del dec
    enc = O.e2m1_encode(np.concatenate([vals, -vals]))
    assert list(enc) == list(range(8)) + [8 | i for i in range(8)]
    # midpoints round to the even code; above 6 saturates
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.9, 100.0], dtype=np.float32)
    assert list(O.e2m1_encode(mids)) == [0, 2, 2, 4, 4, 6, 6, 7, 7]
    assert codes.size == 16


def test_mxfp4_shared_exponent():
    w = np.zeros(64, dtype=np.float32)
    w[0] = 6.0  # floor(log2 6) = 2 -> X = 2^0
    w[32] = 1.0  # floor(log2 1) = 0 -> X = 2^-2, 1.0 -> e2m1 4.0
    w[33] = 0.3  # 0.3 / 0.25 = 1.2 -> 1.0
    packed, scales = O.mxfp4_quant(w)
    assert list(scales) == [127, 125]
    d = O.mxfp4_dequant(packed, scales, 64)
    assert d[0] == 6.0 and d[32] == 1.0 and d[33] == 0.25
    w2 = np.full(32, np.nan, dtype=np.float32)
    p2, s2 = O.mxfp4_quant(w2)
    assert s2[0] == 0xFF and np.isnan(O.mxfp4_dequant(p2, s2, 32)).all()


def test_fp8_persistent_matches_torch_formula():
    # layers.py:104-117 evaluated with torch ops is the library oracle here
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((16, 64)) * 0.02).astype(np.float32)
    codes, scales = O.fp8_persistent_quant(w, 64)
    t = torch.from_numpy(w)
    s = t.abs().amax(dim=1, keepdim=True)
    ref = (t / s).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy().reshape(-1)
    assert np.array_equal(codes, ref) and np.array_equal(scales, s.numpy().reshape(-1))


def test_ep_dispatch_oracle_hand_example():
    """_build_send_partitions / _dispatch_tokens order on a hand-worked case:
    2 ranks, 2 experts per rank, top-2.  Rank 0's assignments (token, slot,
    expert): (0,0,3) (0,1,0) (1,0,1) (1,1,2) (2,0,0) (2,1,3) go to ranks
    1 0 0 1 0 1; rank 1's: (0,0,2) (0,1,1) (1,0,0) (1,1,3) go to 1 0 0 1."""
    top0 = np.array([[3, 0], [1, 2], [0, 3]])
    top1 = np.array([[2, 1], [0, 3]])
    w0 = np.array([[0.1, 0.2], [0.3, 0.4], [0.5, 0.6]], dtype=np.float32)
    w1 = np.array([[0.7, 0.8], [0.9, 1.0]], dtype=np.float32)
    order, counts = O.ep_send_order(top0, 2, 2)
    assert order.tolist() == [1, 2, 4, 0, 3, 5] and counts.tolist() == [3, 3]
    recv = O.ep_dispatch([top0, top1], [w0, w1], 2, 2)
    r0 = recv[0]
    assert r0["src_rank"].tolist() == [0, 0, 0, 1, 1]
    assert r0["token_idx"].tolist() == [0, 1, 2, 0, 1]
    assert r0["slot_idx"].tolist() == [1, 0, 0, 1, 0]
    assert r0["local_expert"].tolist() == [0, 1, 0, 1, 0]
    np.testing.assert_array_equal(r0["sort_weight"], np.array([0.2, 0.3, 0.5, 0.8, 0.9], dtype=np.float32))
    r1 = recv[1]
    assert r1["src_rank"].tolist() == [0, 0, 0, 1, 1]
    assert r1["token_idx"].tolist() == [0, 1, 2, 0, 1]
    assert r1["slot_idx"].tolist() == [0, 1, 1, 0, 1]
    assert r1["local_expert"].tolist() == [1, 0, 1, 0, 1]
    # local expert 0 first, each in arrival order
    assert O.ep_expert_order(r0["local_expert"], 2).tolist() == [0, 2, 4, 1, 3]
    assert O.ep_expert_order(r1["local_expert"], 2).tolist() == [1, 3, 0, 2, 4]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ep_combine_oracle_matches_torch_index_add(dtype):
    """The combine oracle against the reference's own op: index_add_ into
    zeros on the CPU (moe.py:1021-1027) over returned rows in the order an
    expert-parallel exchange delivers them (expert id major, then token), with
    some assignments dropped by a capacity limit."""
    g = torch.Generator().manual_seed(20261260)
    T, K, E, H = 40, 4, 8, 64
    topk = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    w = torch.rand((T, K), generator=g).to(dtype)
    tok = torch.arange(T).repeat_interleave(K)
    slot = torch.arange(K).repeat(T)
    keep = torch.rand(T * K, generator=g) > 0.15
    expert = topk.reshape(-1)
    arrival = sorted([i for i in range(T * K) if keep[i]], key=lambda i: (int(expert[i]), int(tok[i])))
    tok_a, slot_a = tok[arrival], slot[arrival]
    feat = (torch.randn((len(arrival), H), generator=g) * 3).to(dtype)
    ref = torch.zeros((T, H), dtype=dtype)
    ref.index_add_(0, tok_a, feat * w[tok_a, slot_a].unsqueeze(-1))
    got = O.ep_combine(feat.float().numpy(), tok_a.numpy(), slot_a.numpy(), topk.numpy(), w.float().numpy(), T,
                       bf16=dtype == torch.bfloat16)
    want = ref.float().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a plausible misreading -- rounding every partial sum to bf16 -- differs
    if dtype == torch.bfloat16:
        loose = O.ep_combine(feat.float().numpy(), tok_a.numpy(), slot_a.numpy(), topk.numpy(), w.float().numpy(), T,
                             per_add_rounding=True)
        assert not np.array_equal(loose.view(np.uint32), want.view(np.uint32))


def test_slice_index_base_reproduces_rows_and_columns_under_sr():
    """quant_grouped(elem_base, elem_row) on a slice draws the stochastic-
    rounding bits of the slice's place in the full matrix: a row slice and a
    column slice reproduce the full matrix's codes, and the bits do move with
    the base (a slice quantized as if it started at 0 differs)."""
    rng = np.random.default_rng(20263101)
    x = rng.standard_normal((256, 300)).astype(np.float32)
    kw = dict(grid=O.GRID_E4M3, rounding=O.ROUND_STOCHASTIC, seed=5, offset=(1 << 33) + 9)
    full = O.quant_tile_1x128(x, **kw)
    rows = O.quant_tile_1x128(x[17:31], elem_base=17 * 300, **kw)
    assert np.array_equal(rows[0], full[0][17:31]) and np.array_equal(rows[1], full[1][17:31])
    assert not np.array_equal(O.quant_tile_1x128(x[17:31], **kw)[0], full[0][17:31])
    full_t = O.quant_tile_128x1_t(x, **kw)
    cols = O.quant_tile_128x1_t(np.ascontiguousarray(x[:, 40:45]), elem_base=40, elem_row=300, **kw)
    assert np.array_equal(cols[0], full_t[0][40:45]) and np.array_equal(cols[1], full_t[1][40:45])


def test_sr_e4m3_rule_against_exact_rationals():
    """The oracle's e4m3 stochastic rounding, pinned against the rule stated
    with exact rationals: x = |v| / spacing (spacing 2^(e-3) for |v| in
    [2^e, 2^(e+1)), 2^-9 below 2^-6), f20 = floor(frac(x) * 2^20); the code
    rounds away from zero iff f20 + (r >> 12) >= 2^20.  Random |v| over the
    whole e4m3 range (subnormals, tiny values, up to 448), random words, and
    the words at and just below each carry threshold."""
    from fractions import Fraction

    rng = np.random.default_rng(20262501)
    n = 3000
    e = rng.uniform(-40, np.log2(448.0), size=n)
    v = (np.exp2(e) * rng.choice([-1.0, 1.0], size=n)).astype(np.float32)
    v = np.clip(v, np.float32(-448.0), np.float32(448.0))
    r = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)

    def parts(x):
        a = Fraction(abs(float(x)))
        spacing = Fraction(1, 512)
        if a >= Fraction(1, 64):
            ex = 0
            while Fraction(2) ** ex > a:
                ex -= 1
            while Fraction(2) ** (ex + 1) <= a:
                ex += 1
            spacing = Fraction(2) ** (ex - 3)
        q = a / spacing
        k = q.numerator // q.denominator
        return k, ((q - k) * (1 << 20)).__floor__(), spacing

    cases = []
    for x, w in zip(v, r):
        _, f20, _ = parts(x)
        at = (((1 << 20) - f20) % (1 << 20)) << 12
        cases += [(x, int(w)), (x, at)] + ([(x, at - 4096)] if at >= 4096 else [])
    vs = np.array([c[0] for c in cases], dtype=np.float32)
    ws = np.array([c[1] for c in cases], dtype=np.uint32)
    codes = O.e4m3_sr_encode(vs, ws)
    vals = O.decode_codes(codes, O.GRID_E4M3)
    ups = 0
    for x, w, c, val in zip(vs, ws, codes, vals):
        k, f20, spacing = parts(x)
        up = f20 + (int(w) >> 12) >= (1 << 20)
        ups += up
        assert Fraction(abs(float(val))) == (k + up) * spacing, (float(x), hex(int(w)), hex(int(c)))
        if k + up:
            assert bool(c & 0x80) == bool(np.signbit(x))
    assert 0 < ups < len(cases)
