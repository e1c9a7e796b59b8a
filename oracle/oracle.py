"""CPU oracle for the nano-train low-bit linear hot path (numpy + the C restatement).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline).  The product package under
``nano-train_amd/`` never imports it.

The element-level arithmetic (scales, rounding, code bytes, Philox bits, NF4,
MXFP4, e4m3) lives in ``lowbit_oracle.c`` (plain C, IEEE fp32, no FMA
contraction); this module wraps it with numpy and adds the GEMM oracle:
dequantize in fp32 (q * scale, te_backend.py:106) and multiply in float64, so
the result is the exact dequantize-then-matmul value before the bf16 output
rounding.  Citations are to lastweek/nano-train (``src/runtime/te_backend.py``,
``src/models/moe.py``, ``src/layers.py``).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblowbit_oracle.so")

GRID_INT = 0
GRID_E4M3 = 1
ROUND_NEAREST = 0
ROUND_STOCHASTIC = 1
SCALE_AFTER_DIVIDE = 0  # te_backend.py:74-79, :99-100
SCALE_BEFORE_DIVIDE = 1  # moe.py:94-98

NF4_CODEBOOK = np.array(
    [
        -1.0, -0.6961928, -0.52507305, -0.3949175, -0.28444138, -0.18477343,
        -0.09105004, 0.0, 0.0795803, 0.1609302, 0.2461123, 0.33791524,
        0.44070983, 0.562617, 0.72295684, 1.0,
    ],
    dtype=np.float32,
)  # layers.py:62-82

_lib = None


def build() -> str:
    """Compile the C oracle with the committed Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64, u64, i32 = ctypes.c_int64, ctypes.c_uint64, ctypes.c_int
        L.ntlo_philox4x32_10.argtypes = [P, P, P]
        L.ntlo_sr_bits_fill.argtypes = [u64, u64, u64, i64, P]
        L.ntlo_e4m3_encode_array.argtypes = [P, i64, P]
        L.ntlo_e4m3_sr_encode_array.argtypes = [P, P, i64, P]
        L.ntlo_code_decode_array.argtypes = [P, i64, i32, P]
        L.ntlo_e2m1_encode_array.argtypes = [P, i64, P]
        L.ntlo_quant_grouped.argtypes = [P, i64, i64, i64, i64, i32, i32, i32, i32, u64, u64, P, i64, P, P, P]
        L.ntlo_quant_grouped.restype = i32
        L.ntlo_quant_grouped_at.argtypes = [P, i64, i64, i64, i64, i32, i32, i32, i32, u64, u64, P, i64, P, P, P,
                                            u64, u64]
        L.ntlo_quant_grouped_at.restype = i32
        L.ntlo_nf4_quant.argtypes = [P, i64, i64, P, P]
        L.ntlo_nf4_quant.restype = i32
        L.ntlo_nf4_dequant.argtypes = [P, P, i64, i64, P]
        L.ntlo_nf4_dequant.restype = i32
        L.ntlo_mxfp4_quant.argtypes = [P, i64, P, P]
        L.ntlo_mxfp4_quant.restype = i32
        L.ntlo_mxfp4_dequant.argtypes = [P, P, i64, P]
        L.ntlo_mxfp4_dequant.restype = i32
        L.ntlo_fp8_persistent_quant.argtypes = [P, i64, i64, P, P]
        L.ntlo_fp8_persistent_quant.restype = i32
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ----------------------------------------------------------------------------
# random bits
# ----------------------------------------------------------------------------

def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(np.asarray(ctr, dtype=np.uint32))
    k = np.ascontiguousarray(np.asarray(key, dtype=np.uint32))
    out = np.zeros(4, dtype=np.uint32)
    lib().ntlo_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return out


def sr_bits(seed: int, offset: int, start: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().ntlo_sr_bits_fill(seed, offset, start, n, _ptr(out))
    return out


# ----------------------------------------------------------------------------
# code formats
# ----------------------------------------------------------------------------

def e4m3_encode(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint8)
    lib().ntlo_e4m3_encode_array(_ptr(v), v.size, _ptr(out))
    return out


def e4m3_sr_encode(v: np.ndarray, bits: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    r = np.ascontiguousarray(bits, dtype=np.uint32)
    out = np.empty(v.shape, dtype=np.uint8)
    lib().ntlo_e4m3_sr_encode_array(_ptr(v), _ptr(r), v.size, _ptr(out))
    return out


def decode_codes(codes: np.ndarray, grid: int) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(c.shape, dtype=np.float32)
    lib().ntlo_code_decode_array(_ptr(c), c.size, grid, _ptr(out))
    return out


def e2m1_encode(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint8)
    lib().ntlo_e2m1_encode_array(_ptr(v), v.size, _ptr(out))
    return out


# ----------------------------------------------------------------------------
# quantizers
# ----------------------------------------------------------------------------

def qmax_for_bits(bits: int) -> int:
    return (1 << (bits - 1)) - 1  # te_backend.py:98


def quant_grouped(
    x: np.ndarray,
    gr: int,
    gc: int,
    *,
    grid: int = GRID_INT,
    bits: int = 8,
    rounding: int = ROUND_NEAREST,
    scale_rule: int = SCALE_AFTER_DIVIDE,
    seed: int = 0,
    offset: int = 0,
    ldc: Optional[int] = None,
    elem_base: int = 0,
    elem_row: int = 0,
):
    """Quantize a [R, K] fp32 matrix with one scale per (gr x gc) group.

    Returns (codes uint8 [R, ldc], scales fp32 [ceil(R/gr), ceil(K/gc)],
    q fp32 [R, K], dq fp32 [R, K]).  When x is a slice of a larger matrix,
    element (i, k) draws the stochastic-rounding bits of source index
    elem_base + i * elem_row + k (elem_row 0 = K): rows [r0, r1) of an
    [R', K'] matrix use elem_base = r0 * K', columns [c0, c1) use
    elem_base = c0 and elem_row = K'.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.ndim == 2
    R, K = x.shape
    ldc = K if ldc is None else ldc
    gr = max(1, min(gr, max(R, 1)))
    gc = max(1, min(gc, max(K, 1)))
    nsr, nsc = -(-R // gr), -(-K // gc)
    codes = np.zeros((R, ldc), dtype=np.uint8)
    scales = np.zeros((nsr, nsc), dtype=np.float32)
    q = np.zeros((R, K), dtype=np.float32)
    dq = np.zeros((R, K), dtype=np.float32)
    rc = lib().ntlo_quant_grouped_at(
        _ptr(x), R, K, gr, gc, grid, qmax_for_bits(bits), rounding, scale_rule,
        seed, offset, _ptr(codes), ldc, _ptr(scales), _ptr(q), _ptr(dq), elem_base, elem_row,
    )
    if rc != 0:
        raise ValueError(f"ntlo_quant_grouped failed rc={rc}")
    return codes, scales, q, dq


def round_up(v: int, m: int) -> int:
    return -(-v // m) * m


def quant_tile_1x128(x2d, **kw):
    """te_backend.py:82-110 on a [R, K] matrix; codes padded to ceil(K/128)*128."""
    R, K = x2d.shape
    return quant_grouped(x2d, 1, 128, ldc=round_up(K, 128), **kw)


def quant_block_128x128(w2d, **kw):
    """te_backend.py:113-149 on a 2-D [N, K] weight."""
    N, K = w2d.shape
    return quant_grouped(w2d, 128, 128, ldc=round_up(K, 128), **kw)


def quant_tile_128x1_t(x2d, **kw):
    """128x1 tiles (per column, 128 rows) with transposed codes [K, ceil(R/128)*128].

    SR bits are keyed by the source element index r*K + k, as in quant_grouped.
    Returns (codesT, scalesT [K, ceil(R/128)], q, dq)."""
    R, K = x2d.shape
    codes, scales, q, dq = quant_grouped(x2d, 128, 1, ldc=K, **kw)
    Rp = round_up(R, 128)
    codesT = np.zeros((K, Rp), dtype=np.uint8)
    codesT[:, :R] = codes.T
    return codesT, np.ascontiguousarray(scales.T), q, dq


# ----------------------------------------------------------------------------
# GEMM oracle: fp32 dequantize then float64 matmul
# ----------------------------------------------------------------------------

def dequant_grouped(codes: np.ndarray, scales: np.ndarray, K: int, gr: int, gc: int, grid: int) -> np.ndarray:
    """q * scale in fp32 for a [R, ldc] code matrix (columns >= K dropped)."""
    R = codes.shape[0]
    q = decode_codes(codes[:, :K], grid)
    s = np.repeat(np.repeat(scales, gr, axis=0)[:R], gc, axis=1)[:, :K]
    return (q * s).astype(np.float32)


def gemm_ref(a_dq: np.ndarray, b_dq: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """Y = A_dq @ B_dq^T (+ bias) in float64 (te_backend.py:253-259 math)."""
    y = a_dq.astype(np.float64) @ b_dq.astype(np.float64).T
    if bias is not None:
        y = y + bias.astype(np.float64)[None, :]
    return y


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32/float64 values to bfloat16 (nearest even); returns uint16 bits."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(to_bf16_bits(x))


def rel_frobenius(a: np.ndarray, b: np.ndarray) -> float:
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


# ----------------------------------------------------------------------------
# persistent formats
# ----------------------------------------------------------------------------

def nf4_quant(w: np.ndarray, block: int):
    """layers.py:156-169 with one scale per `block` consecutive elements."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    n = w.size
    packed = np.zeros((n + 1) // 2, dtype=np.uint8)
    scales = np.zeros(-(-n // block) if n else 0, dtype=np.float32)
    rc = lib().ntlo_nf4_quant(_ptr(w), n, block, _ptr(packed), _ptr(scales))
    if rc != 0:
        raise ValueError("nf4 quant failed")
    return packed, scales


def nf4_dequant(packed: np.ndarray, scales: np.ndarray, n: int, block: int) -> np.ndarray:
    """layers.py:172-184 before the dtype cast."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.float32)
    out = np.empty(n, dtype=np.float32)
    lib().ntlo_nf4_dequant(_ptr(p), _ptr(s), n, block, _ptr(out))
    return out


def mxfp4_quant(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    n = w.size
    packed = np.zeros((n + 1) // 2, dtype=np.uint8)
    scales = np.zeros(-(-n // 32), dtype=np.uint8)
    lib().ntlo_mxfp4_quant(_ptr(w), n, _ptr(packed), _ptr(scales))
    return packed, scales


def mxfp4_dequant(packed: np.ndarray, scales: np.ndarray, n: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    lib().ntlo_mxfp4_dequant(_ptr(p), _ptr(s), n, _ptr(out))
    return out


def fp8_persistent_quant(w: np.ndarray, block: int):
    """layers.py:104-117: scale = amax per block, codes = e4m3(clamp(w/s))."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    n = w.size
    codes = np.zeros(n, dtype=np.uint8)
    scales = np.zeros(-(-n // block) if n else 0, dtype=np.float32)
    lib().ntlo_fp8_persistent_quant(_ptr(w), n, block, _ptr(codes), _ptr(scales))
    return codes, scales


# ----------------------------------------------------------------------------
# the reference emulated linear forward (te_backend.py:229-260), numpy port
# ----------------------------------------------------------------------------

def emulated_linear_forward(x2d: np.ndarray, w: np.ndarray, *, grid: int = GRID_INT, bits: int = 8,
                            rounding: int = ROUND_NEAREST, seed: int = 0, offset: int = 0,
                            bias: Optional[np.ndarray] = None, out_dtype=np.float32) -> np.ndarray:
    """Quantize X per 1x128 tile and W per 128x128 block, dequantize in fp32 and
    multiply in fp32 (F.linear in float32).  This is the timed CPU baseline."""
    _, _, _, xdq = quant_tile_1x128(x2d, grid=grid, bits=bits, rounding=rounding, seed=seed, offset=offset)
    _, _, _, wdq = quant_block_128x128(w, grid=grid, bits=bits, rounding=rounding, seed=seed, offset=offset + 1)
    y = xdq @ wdq.T
    if bias is not None:
        y = y + bias.astype(np.float32)[None, :]
    return y.astype(out_dtype)


# ----------------------------------------------------------------------------
# expert-parallel dispatch (moe.py:670-717 _build_send_partitions,
# :795-863 _dispatch_tokens, :905-923 the receive-side expert selection)
# ----------------------------------------------------------------------------

def ep_send_order(topk_idx: np.ndarray, experts_per_rank: int, ep_size: int):
    """Assignment indices a = t*K + k in send order: destination rank
    expert // experts_per_rank major, assignment order within a rank (the
    reference's boolean masks over the flattened assignments, moe.py:698-706).
    Returns (order, counts per destination)."""
    e = np.asarray(topk_idx).reshape(-1)
    dest = e // experts_per_rank
    order = np.concatenate([np.nonzero(dest == r)[0] for r in range(ep_size)]) if e.size else np.zeros(0, np.int64)
    counts = np.array([int((dest == r).sum()) for r in range(ep_size)], dtype=np.int64)
    return order.astype(np.int64), counts


def ep_dispatch(topk_by_rank, weights_by_rank, experts_per_rank: int, ep_size: int):
    """What every rank receives from _dispatch_tokens, per receiving rank r:
    dict with src_rank, token_idx, slot_idx, local_expert, sort_weight (each
    [N_recv]) in arrival order (sources in rank order, the split order of
    all_to_all_single), plus src_row (the sender's assignment index)."""
    out = []
    sends = [ep_send_order(t, experts_per_rank, ep_size) for t in topk_by_rank]
    for r in range(ep_size):
        parts = {k: [] for k in ("src_rank", "token_idx", "slot_idx", "local_expert", "sort_weight", "src_row")}
        for s, (order, counts) in enumerate(sends):
            K = np.asarray(topk_by_rank[s]).shape[1]
            e = np.asarray(topk_by_rank[s]).reshape(-1)
            w = np.asarray(weights_by_rank[s], dtype=np.float32).reshape(-1)
            start = int(counts[:r].sum())
            sel = order[start:start + int(counts[r])]
            parts["src_rank"].append(np.full(sel.size, s, dtype=np.int64))
            parts["token_idx"].append(sel // K)
            parts["slot_idx"].append(sel % K)
            parts["local_expert"].append(e[sel] % experts_per_rank)
            parts["sort_weight"].append(w[sel])
            parts["src_row"].append(sel)
        out.append({k: np.concatenate(v) for k, v in parts.items()})
    return out


def ep_expert_order(local_expert: np.ndarray, local_experts: int):
    """The receive-side selection of _run_local_experts without capacity drop:
    for each local expert in order, its received rows in arrival order
    ((recv_local_expert_idx == e).nonzero(), moe.py:905-909)."""
    le = np.asarray(local_expert).reshape(-1)
    return np.concatenate([np.nonzero(le == e)[0] for e in range(local_experts)]) if le.size else np.zeros(0, np.int64)


def ep_combine(feat: np.ndarray, token_idx: np.ndarray, slot_idx: np.ndarray, topk_idx: np.ndarray,
               topk_w: np.ndarray, T: int, *, bf16: bool = True, per_add_rounding: bool = False) -> np.ndarray:
    """The source side of _combine_remote_outputs (moe.py:1021-1027):
    output_tokens = zeros; output_tokens.index_add_(0, token_idx, feat *
    topk_w[token_idx, slot_idx]) on the CPU, with feat the returned rows in the
    output dtype.  The product is a tensor op of the output dtype (each
    element rounded to it); index_add_ on the CPU sums the rows in fp32 in
    arrival order -- for one token, ascending expert id -- and rounds once
    (bf16, or fp32 with bf16=False).  per_add_rounding rounds every partial
    sum instead, the plausible misreading the tests rule out.  Returns fp32
    [T, H] holding output-dtype values."""
    rnd = round_bf16 if bf16 else (lambda v: np.asarray(v, dtype=np.float32))
    feat = rnd(np.asarray(feat, dtype=np.float32))
    token_idx = np.asarray(token_idx, dtype=np.int64)
    slot_idx = np.asarray(slot_idx, dtype=np.int64)
    w = rnd(np.asarray(topk_w, dtype=np.float32))
    expert = np.asarray(topk_idx)[token_idx, slot_idx]
    out = np.zeros((T, feat.shape[1]), dtype=np.float32)
    for r in np.lexsort((expert, token_idx)):  # per token, ascending expert id
        t = token_idx[r]
        out[t] = out[t] + rnd(feat[r] * w[t, slot_idx[r]])
        if per_add_rounding:
            out[t] = rnd(out[t])
    return rnd(out)
