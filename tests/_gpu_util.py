"""Helpers for the GPU parity tests: seeded inputs and oracle comparisons."""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O


def to_np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def seeded(shape, *, seed: int, dtype=torch.bfloat16, std: float = 1.0, outliers: float = 0.0,
           heavy_channels: bool = False) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * std
    if outliers:
        mask = torch.rand(*shape, generator=g) < outliers
        x = torch.where(mask, x * 50.0, x)
    if heavy_channels:
        c = torch.exp(torch.empty(shape[-1]).uniform_(np.log(0.1), np.log(20.0), generator=g))
        x = x * c
    return x.to(dtype)


def scales_row_major(q, rows: int, ncol: int) -> np.ndarray:
    """Return the scales of a QTensor as [rows-groups, ncol] row-major numpy."""
    s = q.scales.detach().cpu().numpy().reshape(-1)
    out = np.empty((rows, ncol), dtype=np.float32)
    for i in range(rows):
        idx = i * q.s_row + np.arange(ncol) * q.s_col
        out[i] = s[idx]
    return out


def assert_bits_equal(a: np.ndarray, b: np.ndarray, what: str) -> None:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if a.dtype == np.float32:
        av, bv = a.view(np.uint32), b.view(np.uint32)
        nan = np.isnan(a) & np.isnan(b)
        bad = (av != bv) & ~nan
    else:
        bad = a != b
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {int(bad.sum())} mismatches, first at {idx.tolist()}: "
                             f"{a[tuple(idx[0])]} vs {b[tuple(idx[0])]}")


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def rel_fro_bf16(y_gpu: torch.Tensor, y_ref64: np.ndarray) -> float:
    """relative Frobenius error, both sides rounded to bf16 (the bar of the path)."""
    a = y_gpu.detach().float().cpu().numpy()
    b = O.round_bf16(y_ref64.astype(np.float32))
    return O.rel_frobenius(a, b)


def _pool_size() -> int:
    import os

    return max(1, min(16, os.cpu_count() or 1))  # the GPU box's CPU share


def oracle_tile_1x128_rows(x: np.ndarray, **kw):
    """O.quant_tile_1x128 of a large [R, K] matrix, row chunks in parallel
    threads (ctypes releases the GIL), each keyed at its place in x.
    Returns (codes, scales)."""
    from concurrent.futures import ThreadPoolExecutor

    R, K = x.shape
    step = -(-R // _pool_size())
    chunks = [(r0, min(R, r0 + step)) for r0 in range(0, R, step)]

    def run(c):
        r0, r1 = c
        out = O.quant_tile_1x128(np.ascontiguousarray(x[r0:r1]), elem_base=r0 * K, **kw)
        return out[0], out[1]

    with ThreadPoolExecutor(len(chunks)) as ex:
        parts = list(ex.map(run, chunks))
    return np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts])


def oracle_128x1_t_cols(x: np.ndarray, cols=None, **kw):
    """O.quant_tile_128x1_t of the columns `cols` (all when None) of a large
    [R, K] matrix, column chunks in parallel threads, each keyed at its place
    in x.  Returns (codes_t [len(cols), ceil(R/128)*128], scales_t)."""
    from concurrent.futures import ThreadPoolExecutor

    R, K = x.shape
    cols = np.arange(K) if cols is None else np.asarray(cols)
    # runs of consecutive columns, cut into pool-sized chunks
    runs, start = [], 0
    for i in range(1, len(cols) + 1):
        if i == len(cols) or cols[i] != cols[i - 1] + 1:
            runs.append((int(cols[start]), int(cols[i - 1]) + 1))
            start = i
    step = max(1, -(-len(cols) // _pool_size()))
    chunks = [(c0 + j, min(c1, c0 + j + step)) for c0, c1 in runs for j in range(0, c1 - c0, step)]

    def run(c):
        c0, c1 = c
        out = O.quant_tile_128x1_t(np.ascontiguousarray(x[:, c0:c1]), elem_base=c0, elem_row=K, **kw)
        return out[0], out[1]

    with ThreadPoolExecutor(min(len(chunks), _pool_size())) as ex:
        parts = list(ex.map(run, chunks))
    return np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts])
