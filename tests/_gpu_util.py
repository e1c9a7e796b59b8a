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
