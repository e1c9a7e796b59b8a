"""Tensor-level wrappers of the gfx950 low-bit kernels.

Every function here takes and returns torch tensors on a ROCm device, allocates
outputs with torch's caching allocator, and launches on torch's current HIP
stream through the C-ABI in ``include/ntlowbit.h``.  Nothing here computes on
the CPU: a CPU tensor is an error.

Quantized operands are carried as :class:`QTensor` (codes + scales + how the
scales are indexed), which is exactly what the blockwise GEMM consumes.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import call

_DTYPE_CODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError as exc:
        raise TypeError(f"unsupported dtype {dt}; expected float32, bfloat16 or float16") from exc


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_device(*ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                "the MI355X low-bit kernels need tensors on a ROCm device "
                f"(got {t.device}); there is no CPU path"
            )


def _as_2d(x: torch.Tensor) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1]) if x.dim() != 2 else x
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def grid_code(fmt: str) -> int:
    if fmt in ("int", "int_grid", "grid"):
        return _lib.GRID_INT
    if fmt == "e4m3":
        return _lib.GRID_E4M3
    raise ValueError(f"unknown code format {fmt!r}; expected 'int_grid' or 'e4m3'")


def rounding_code(mode: str) -> int:
    if mode == "nearest":
        return _lib.ROUND_NEAREST
    if mode == "stochastic":
        return _lib.ROUND_STOCHASTIC
    raise ValueError(f"unknown rounding mode {mode!r}")


@dataclass
class QTensor:
    """Codes plus scales of a quantized [rows, K] matrix.

    scale(i, kb) = scales.flatten()[(i >> shift) * s_row + kb * s_col]
    (kb = 128-column block; shift 7 = one scale per 128 rows).
    """

    codes: torch.Tensor  # uint8 [rows, ldc]
    scales: torch.Tensor  # fp32, flat indexing through s_row / s_col
    s_row: int
    s_col: int
    shift: int
    grid: int
    rows: int
    K: int
    nan_rows: Optional[torch.Tensor] = None
    dq: Optional[torch.Tensor] = None

    @property
    def Kp(self) -> int:
        return cdiv(self.K, 128) * 128


def quant_tile_1x128(
    x: torch.Tensor,
    *,
    fmt: str = "int_grid",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
    scale_rule: int = _lib.SCALE_AFTER_DIVIDE,
    tile_major_scales: bool = True,
    want_dq: bool = False,
    dq_dtype: Optional[torch.dtype] = None,
    want_nan_rows: bool = False,
) -> QTensor:
    """te_backend.py:82-110 on x viewed as [R, K] (leading dims flattened)."""
    _require_device(x)
    x2 = _as_2d(x)
    R, K = x2.shape
    T = cdiv(K, 128)
    ldc = T * 128
    dev = x.device
    codes = torch.empty((R, ldc), dtype=torch.uint8, device=dev)
    if tile_major_scales:
        rp = cdiv(max(R, 1), 4) * 4
        scales = torch.empty((T, rp), dtype=torch.float32, device=dev)
        s_row, s_col = 1, rp
    else:
        scales = torch.empty((R, T), dtype=torch.float32, device=dev)
        s_row, s_col = T, 1
    dq = None
    if want_dq:
        dq = torch.empty((R, K), dtype=dq_dtype or x.dtype, device=dev)
    nan_rows = torch.zeros(R, dtype=torch.int32, device=dev) if want_nan_rows else None
    call(
        "ntlb_quant_tile_1x128", x2.data_ptr(), _dtype_code(x2.dtype), R, K, x2.stride(0), grid_code(fmt),
        (1 << (bits - 1)) - 1, rounding_code(rounding), scale_rule, seed, offset, codes.data_ptr(), ldc,
        scales.data_ptr(), s_row, s_col, _ptr(dq), _dtype_code(dq.dtype) if dq is not None else 0,
        dq.stride(0) if dq is not None else 0, _ptr(nan_rows), _stream(),
    )
    return QTensor(codes, scales, s_row, s_col, 0, grid_code(fmt), R, K, nan_rows, dq)


def quant_tile_1x128_fanout(
    x: torch.Tensor,
    pos: torch.Tensor,
    fan_k: int,
    rows: int,
    *,
    fmt: str = "int_grid",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
    scale_rule: int = _lib.SCALE_AFTER_DIVIDE,
    want_nan_rows: bool = False,
) -> QTensor:
    """quant_tile_1x128 of the rows of x [T, K] gathered by expert, without the
    gathered copy: row pos[r*fan_k + f] of the result is token row r (the
    gather tokens[token_indices] of moe.py:1081 / :484 fused into the
    quantizer).  pos is int32 [T*fan_k] (ep.partition of topk_idx with divisor
    1); codes, tile-major scales and SR bits equal quant_tile_1x128 of the
    gathered [rows, K] matrix.  A negative pos entry writes nothing, so the
    rows it would have named hold no codes."""
    _require_device(x)
    if x.dim() != 2:
        raise ValueError("x must be [T, K]")
    if pos.dtype != torch.int32 or pos.numel() != x.shape[0] * fan_k:
        raise ValueError(f"pos must be int32 with T*fan_k = {x.shape[0] * fan_k} entries")
    x2 = x if x.stride(-1) == 1 else x.contiguous()
    pos = pos.contiguous()
    T_in, K = x2.shape
    T = cdiv(K, 128)
    ldc = T * 128
    dev = x.device
    codes = torch.empty((rows, ldc), dtype=torch.uint8, device=dev)
    rp = cdiv(max(rows, 1), 4) * 4
    scales = torch.empty((T, rp), dtype=torch.float32, device=dev)
    nan_rows = torch.zeros(rows, dtype=torch.int32, device=dev) if want_nan_rows else None
    call(
        "ntlb_quant_tile_1x128_fanout", x2.data_ptr(), _dtype_code(x2.dtype), T_in, K, x2.stride(0), pos.data_ptr(),
        fan_k, rows, grid_code(fmt), (1 << (bits - 1)) - 1, rounding_code(rounding), scale_rule, seed, offset,
        codes.data_ptr(), ldc, scales.data_ptr(), 1, rp, _ptr(nan_rows), _stream(),
    )
    return QTensor(codes, scales, 1, rp, 0, grid_code(fmt), rows, K, nan_rows, None)


def quant_block_128x128(
    w: torch.Tensor,
    *,
    fmt: str = "int_grid",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
    scale_rule: int = _lib.SCALE_AFTER_DIVIDE,
    want_transposed: bool = False,
    want_dq: bool = False,
    dq_dtype: Optional[torch.dtype] = None,
    want_nan_rows: bool = False,
):
    """te_backend.py:113-149 for a 2-D weight [N, K].

    Returns (QTensor, QTensor-of-W^T or None).  The transposed operand shares
    the scale tensor (block (nb, kb) of W is block (kb, nb) of W^T)."""
    _require_device(w)
    if w.dim() != 2:
        raise ValueError("block_128x128 needs a 2-D weight")
    w2 = w if w.stride(-1) == 1 else w.contiguous()
    N, K = w2.shape
    T, NB = cdiv(K, 128), cdiv(N, 128)
    ldc = T * 128
    dev = w.device
    codes = torch.empty((N, ldc), dtype=torch.uint8, device=dev)
    scales = torch.empty((NB, T), dtype=torch.float32, device=dev)
    codes_t = torch.empty((K, NB * 128), dtype=torch.uint8, device=dev) if want_transposed else None
    dq = torch.empty((N, K), dtype=dq_dtype or w.dtype, device=dev) if want_dq else None
    nan_rows = torch.zeros(N, dtype=torch.int32, device=dev) if want_nan_rows else None
    call(
        "ntlb_quant_block_128x128", w2.data_ptr(), _dtype_code(w2.dtype), N, K, w2.stride(0), grid_code(fmt),
        (1 << (bits - 1)) - 1, rounding_code(rounding), scale_rule, seed, offset, codes.data_ptr(), ldc,
        _ptr(codes_t), NB * 128 if codes_t is not None else 0, scales.data_ptr(), T, 1, _ptr(dq),
        _dtype_code(dq.dtype) if dq is not None else 0, dq.stride(0) if dq is not None else 0, _ptr(nan_rows),
        _stream(),
    )
    q = QTensor(codes, scales, T, 1, 7, grid_code(fmt), N, K, nan_rows, dq)
    qt = None
    if codes_t is not None:
        qt = QTensor(codes_t, scales, 1, T, 7, grid_code(fmt), K, N, None, None)
    return q, qt


def quant_tile_128x1_t(
    x: torch.Tensor,
    *,
    fmt: str = "int_grid",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
    scale_rule: int = _lib.SCALE_AFTER_DIVIDE,
    want_dq: bool = False,
    dq_dtype: Optional[torch.dtype] = None,
    want_nan_rows: bool = False,
) -> QTensor:
    """128x1 tiles of x [R, K] with transposed codes: a QTensor of x^T [K, R].

    nan_rows, when requested, flags the rows of x^T (columns of x) that hold a NaN."""
    _require_device(x)
    x2 = _as_2d(x)
    R, K = x2.shape
    MB = cdiv(R, 128)
    ldct = MB * 128
    dev = x.device
    codes_t = torch.empty((K, ldct), dtype=torch.uint8, device=dev)
    kp = cdiv(max(K, 1), 4) * 4
    scales = torch.empty((MB, kp), dtype=torch.float32, device=dev)  # tile-major for the GEMM
    dq = torch.empty((R, K), dtype=dq_dtype or x.dtype, device=dev) if want_dq else None
    nan = torch.zeros((K,), dtype=torch.int32, device=dev) if want_nan_rows else None
    call(
        "ntlb_quant_tile_128x1_t", x2.data_ptr(), _dtype_code(x2.dtype), R, K, x2.stride(0), grid_code(fmt),
        (1 << (bits - 1)) - 1, rounding_code(rounding), scale_rule, seed, offset, codes_t.data_ptr(), ldct,
        scales.data_ptr(), 1, kp, _ptr(dq), _dtype_code(dq.dtype) if dq is not None else 0,
        dq.stride(0) if dq is not None else 0, _ptr(nan), _stream(),
    )
    return QTensor(codes_t, scales, 1, kp, 0, grid_code(fmt), K, R, nan, dq)


def quant_dual_1x128_128x1(
    x: torch.Tensor,
    *,
    fmt: str = "int_grid",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset_rows: int = 0,
    offset_cols: int = 0,
    scale_rule: int = _lib.SCALE_AFTER_DIVIDE,
    want_nan_rows: bool = False,
):
    """One pass over x [R, K] giving (quant_tile_1x128(x), quant_tile_128x1_t(x)).

    The two QTensors equal those of the two single-output calls with the same
    arguments (SR offsets offset_rows and offset_cols).  Shapes the fused pass
    does not take (K % 8 != 0, fp16 input, unaligned rows) run the two calls."""
    _require_device(x)
    x2 = _as_2d(x)
    R, K = x2.shape
    common = dict(fmt=fmt, bits=bits, rounding=rounding, seed=seed, scale_rule=scale_rule)
    fused = (K % 8 == 0 and x2.stride(0) % 8 == 0 and x2.data_ptr() % 16 == 0
             and x2.dtype in (torch.bfloat16, torch.float32))
    if not fused or R * K == 0:
        return (quant_tile_1x128(x2, offset=offset_rows, want_nan_rows=want_nan_rows, **common),
                quant_tile_128x1_t(x2, offset=offset_cols, want_nan_rows=want_nan_rows, **common))
    dev = x.device
    T = cdiv(K, 128)
    ldc = T * 128
    rp = cdiv(R, 4) * 4
    codes = torch.empty((R, ldc), dtype=torch.uint8, device=dev)
    scales = torch.empty((T, rp), dtype=torch.float32, device=dev)
    MB = cdiv(R, 128)
    ldct = MB * 128
    kp = cdiv(K, 4) * 4
    codes_t = torch.empty((K, ldct), dtype=torch.uint8, device=dev)
    scales_t = torch.empty((MB, kp), dtype=torch.float32, device=dev)
    nan_r = torch.zeros(R, dtype=torch.int32, device=dev) if want_nan_rows else None
    nan_c = torch.zeros(K, dtype=torch.int32, device=dev) if want_nan_rows else None
    call(
        "ntlb_quant_dual_1x128_128x1", x2.data_ptr(), _dtype_code(x2.dtype), R, K, x2.stride(0), grid_code(fmt),
        (1 << (bits - 1)) - 1, rounding_code(rounding), scale_rule, seed, offset_rows, offset_cols,
        codes.data_ptr(), ldc, scales.data_ptr(), 1, rp, _ptr(nan_r), codes_t.data_ptr(), ldct, scales_t.data_ptr(),
        1, kp, _ptr(nan_c), _stream(),
    )
    return (QTensor(codes, scales, 1, rp, 0, grid_code(fmt), R, K, nan_r, None),
            QTensor(codes_t, scales_t, 1, kp, 0, grid_code(fmt), K, R, nan_c, None))


def quant_grouped(
    x: torch.Tensor,
    gr: int,
    gc: int,
    *,
    fmt: str = "int_grid",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
    scale_rule: int = _lib.SCALE_AFTER_DIVIDE,
    ldc: Optional[int] = None,
    want_dq: bool = False,
    dq_dtype: Optional[torch.dtype] = None,
    want_nan_rows: bool = False,
):
    """One scale per (gr x gc) group of x viewed as [R, K].

    Returns (codes [R, ldc], scales [ceil(R/gr), ceil(K/gc)], dq, nan_rows)."""
    _require_device(x)
    x2 = _as_2d(x)
    R, K = x2.shape
    gr = max(1, min(gr, max(R, 1)))
    gc = max(1, min(gc, max(K, 1)))
    ldc = K if ldc is None else ldc
    dev = x.device
    ngr, ngc = cdiv(R, gr), cdiv(K, gc)
    amax = torch.zeros((ngr, ngc), dtype=torch.int32, device=dev)
    codes = torch.zeros((R, ldc), dtype=torch.uint8, device=dev)
    scales = torch.empty((ngr, ngc), dtype=torch.float32, device=dev)
    dq = torch.empty((R, K), dtype=dq_dtype or x.dtype, device=dev) if want_dq else None
    nan_rows = torch.zeros(R, dtype=torch.int32, device=dev) if want_nan_rows else None
    xc = _dtype_code(x2.dtype)
    call("ntlb_amax_grouped", x2.data_ptr(), xc, R, K, x2.stride(0), gr, gc, amax.data_ptr(), _stream())
    call(
        "ntlb_quant_grouped", x2.data_ptr(), xc, R, K, x2.stride(0), gr, gc, amax.data_ptr(), grid_code(fmt),
        (1 << (bits - 1)) - 1, rounding_code(rounding), scale_rule, seed, offset, codes.data_ptr(), ldc,
        scales.data_ptr(), _ptr(dq), _dtype_code(dq.dtype) if dq is not None else 0,
        dq.stride(0) if dq is not None else 0, _ptr(nan_rows), _stream(),
    )
    return codes, scales, dq, nan_rows


_workspaces: dict = {}


def gemm_workspace(M: int, N: int, Kp: int, device: torch.device) -> Optional[torch.Tensor]:
    """The zeroed split-K workspace of the current stream on `device`, grown to
    what an (M, N, Kp) blockwise-scaled product needs; None when that shape
    runs unsplit."""
    return split_workspace(int(_lib.lib().ntlb_gemm_workspace_bytes(M, N, Kp)), device)


def split_workspace(need: int, device: torch.device) -> Optional[torch.Tensor]:
    """The zeroed split-K workspace of the current stream on `device`, grown
    to `need` bytes; None when need is 0.  Every split-K GEMM (the
    blockwise-scaled and the dequant-fused ones) leaves it zeroed with its
    tile counters at one fixed place, and calls on one stream never overlap,
    so one buffer per stream serves every GEMM issued there."""
    if need <= 0:
        return None
    key = (device.index, _stream())
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def gemm_blockscaled(
    a: QTensor,
    b: QTensor,
    *,
    bias: Optional[torch.Tensor] = None,
    out_dtype: torch.dtype = torch.bfloat16,
    out: Optional[torch.Tensor] = None,
    split_tail: bool = True,
) -> torch.Tensor:
    """Y[M, N] = dequant(a) @ dequant(b)^T (+ bias), fp32 accumulation.

    split_tail lets the tiles past the last whole wave run as K-split
    partials summed in a fixed order (results are deterministic, and equal
    the unsplit ones up to fp32 summation order)."""
    _require_device(a.codes, b.codes, bias)
    if a.grid != b.grid:
        raise ValueError("operands must share a code format")
    if a.K != b.K:
        raise ValueError(f"contraction mismatch: {a.K} vs {b.K}")
    M, N, Kp = a.rows, b.rows, a.Kp
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.codes.device)
    if bias is not None and bias.stride(-1) != 1:
        bias = bias.contiguous()
    ws = gemm_workspace(M, N, Kp, a.codes.device) if split_tail else None
    call(
        "ntlb_gemm_blockscaled_ws", a.grid, a.codes.data_ptr(), a.codes.stride(0), a.scales.data_ptr(), a.s_row,
        a.s_col, a.shift, b.codes.data_ptr(), b.codes.stride(0), b.scales.data_ptr(), b.s_row, b.s_col, b.shift,
        M, N, Kp, _ptr(bias), _dtype_code(bias.dtype) if bias is not None else 0, out.data_ptr(),
        _dtype_code(out.dtype), out.stride(0), _ptr(a.nan_rows), _ptr(b.nan_rows), _ptr(ws),
        ws.numel() if ws is not None else 0, _stream(),
    )
    return out


def dequant(q: QTensor, *, out_dtype: torch.dtype = torch.bfloat16, r_shift: Optional[int] = None,
            c_shift: int = 7) -> torch.Tensor:
    """value(code) * scale for a QTensor (codes [rows, >=K]) -> [rows, K]."""
    _require_device(q.codes)
    rows, K = q.rows, q.K
    out = torch.empty((rows, K), dtype=out_dtype, device=q.codes.device)
    call("ntlb_dequant", q.grid, q.codes.data_ptr(), q.codes.stride(0), q.scales.data_ptr(), q.s_row, q.s_col,
         q.shift if r_shift is None else r_shift, c_shift, rows, K, out.data_ptr(), _dtype_code(out_dtype),
         out.stride(0), _stream())
    return out


def dequant_raw(grid: int, codes: torch.Tensor, scales: torch.Tensor, *, K: int, s_row: int, s_col: int,
                r_shift: int, c_shift: int, out_dtype: torch.dtype) -> torch.Tensor:
    """ntlb_dequant over explicit scale indexing (strips, channels, tensors)."""
    _require_device(codes, scales)
    rows = codes.shape[0]
    out = torch.empty((rows, K), dtype=out_dtype, device=codes.device)
    call("ntlb_dequant", grid, codes.data_ptr(), codes.stride(0), scales.data_ptr(), s_row, s_col, r_shift, c_shift,
         rows, K, out.data_ptr(), _dtype_code(out_dtype), out.stride(0), _stream())
    return out


def gemm_grouped_blockscaled(
    a: QTensor,
    b_codes: torch.Tensor,
    b_scales: torch.Tensor,
    offsets: torch.Tensor,
    *,
    N: int,
    out_dtype: torch.dtype = torch.bfloat16,
    b_nan_rows: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Per-expert GEMM over rows sorted by expert.

    a        QTensor of the sorted rows [M_total, K] (1x128 tiles)
    b_codes  [E, N, Kp] uint8 weight codes (128x128 blocks)
    b_scales [E, ceil(N/128), Kp/128] fp32
    offsets  int32 [E+1] on the device, offsets[E] == M_total
    """
    _require_device(a.codes, b_codes, b_scales, offsets)
    if offsets.dtype != torch.int32:
        raise TypeError("offsets must be int32")
    E = b_codes.shape[0]
    if offsets.numel() != E + 1:
        raise ValueError(f"offsets has {offsets.numel()} entries for {E} experts")
    if b_codes.shape[1] != N or b_codes.shape[2] < a.Kp:
        raise ValueError(f"expert codes {tuple(b_codes.shape)} do not match N={N}, Kp={a.Kp}")
    b_codes = b_codes.contiguous()
    b_scales = b_scales.contiguous()
    M = a.rows
    out = torch.empty((M, N), dtype=out_dtype, device=a.codes.device)
    nb, tb = b_scales.shape[1], b_scales.shape[2]
    call(
        "ntlb_gemm_grouped_blockscaled", a.grid, a.codes.data_ptr(), a.codes.stride(0), a.scales.data_ptr(), a.s_row,
        a.s_col, a.shift, b_codes.data_ptr(), b_codes.stride(1), b_codes.stride(0), b_scales.data_ptr(), tb, 1, 7,
        nb * tb, offsets.data_ptr(), E, M, N, a.Kp, out.data_ptr(), _dtype_code(out_dtype), out.stride(0),
        _ptr(a.nan_rows), _ptr(b_nan_rows), _stream(),
    )
    return out


def gemm_swiglu_quant(
    a: QTensor,
    b_codes: torch.Tensor,
    b_scales: torch.Tensor,
    *,
    offsets: Optional[torch.Tensor] = None,
    fmt: str = "int_grid",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
    scale_rule: int = _lib.SCALE_AFTER_DIVIDE,
    want_h: bool = True,
    want_nan_rows: bool = False,
    b_nan_rows: Optional[torch.Tensor] = None,
    gu_out: Optional[torch.Tensor] = None,
):
    """h = silu(X W_gate^T) * (X W_up^T) and its 1x128 quantization, in one GEMM.

    b_codes / b_scales hold the gate and up weights interleaved in 128-row
    blocks (moe.interleave_gate_up): [2I, Kp] and [2I/128, Kp/128], or per
    expert [E, 2I, Kp] and [E, 2I/128, Kp/128] with rows of a sorted by expert
    and offsets int32 [E+1].  gu_out (grouped only), bf16 [M, 2I], receives
    the two projections' bf16 outputs in that interleaved column order.
    Returns (h bf16 [M, I] or None, QTensor of h)."""
    _require_device(a.codes, b_codes, b_scales)
    grouped = offsets is not None
    if grouped:
        _require_device(offsets)
        if offsets.dtype != torch.int32:
            raise TypeError("offsets must be int32")
        if b_codes.dim() != 3 or offsets.numel() != b_codes.shape[0] + 1:
            raise ValueError("grouped weights must be [E, 2I, Kp] with offsets of E+1 entries")
    elif b_codes.dim() != 2:
        raise ValueError("dense weights must be [2I, Kp]")
    N = b_codes.shape[-2]
    if N % 256:
        raise ValueError(f"2I = {N} must be a multiple of 256")
    if b_codes.shape[-1] < a.Kp:
        raise ValueError(f"weight codes {tuple(b_codes.shape)} are narrower than Kp={a.Kp}")
    b_codes = b_codes.contiguous()
    b_scales = b_scales.contiguous()
    I = N // 2
    M = a.rows
    dev = a.codes.device
    rp = cdiv(max(M, 1), 4) * 4
    h = torch.empty((M, I), dtype=torch.bfloat16, device=dev) if want_h else None
    hc = torch.empty((M, I), dtype=torch.uint8, device=dev)
    hs = torch.empty((I // 128, rp), dtype=torch.float32, device=dev)
    hn = torch.zeros(M, dtype=torch.int32, device=dev) if want_nan_rows else None
    qmax = (1 << (bits - 1)) - 1
    tail = (_ptr(a.nan_rows), _ptr(b_nan_rows), _ptr(h), I, hc.data_ptr(), I, hs.data_ptr(), 1, rp, _ptr(hn), qmax,
            rounding_code(rounding), scale_rule, seed, offset, _stream())
    if grouped:
        E = b_codes.shape[0]
        nb, tb = b_scales.shape[1], b_scales.shape[2]
        if gu_out is not None:
            _require_device(gu_out)
            if gu_out.dtype != torch.bfloat16 or gu_out.shape != (M, N) or gu_out.stride(-1) != 1:
                raise ValueError(f"gu_out must be a row-major bf16 [{M}, {N}] tensor")
        call("ntlb_gemm_grouped_swiglu_quant_gu", a.grid, a.codes.data_ptr(), a.codes.stride(0), a.scales.data_ptr(),
             a.s_row, a.s_col, a.shift, b_codes.data_ptr(), b_codes.stride(1), b_codes.stride(0),
             b_scales.data_ptr(), tb, 1, nb * tb, offsets.data_ptr(), E, M, N, a.Kp, *tail[:-1], _ptr(gu_out),
             gu_out.stride(0) if gu_out is not None else 0, _stream())
    else:
        if gu_out is not None:
            raise ValueError("gu_out needs the grouped (per-expert) form")
        tb = b_scales.shape[1]
        call("ntlb_gemm_swiglu_quant", a.grid, a.codes.data_ptr(), a.codes.stride(0), a.scales.data_ptr(), a.s_row,
             a.s_col, a.shift, b_codes.data_ptr(), b_codes.stride(0), b_scales.data_ptr(), tb, 1, M, N, a.Kp, *tail)
    return h, QTensor(hc, hs, 1, rp, 0, a.grid, M, I, hn, None)


# ---------------------------------------------------------------------------
# GEMMs over the operands the reference multiplies: bf16(q * s) (or fp32)
# decoded inside the GEMM, plus plain GEMMs over dequantized tensors
# ---------------------------------------------------------------------------
_OP_DTYPES = {torch.bfloat16: _lib.BF16, torch.float32: _lib.F32}


def op_dtype_code(dt: torch.dtype) -> int:
    """The MFMA operand type for a reference dtype: bf16 or fp32 only."""
    try:
        return _OP_DTYPES[dt]
    except KeyError as exc:
        raise TypeError(f"the dequantized-operand GEMMs take bfloat16 or float32 operands, not {dt}") from exc


def _kstep(op_dtype: torch.dtype) -> int:
    return 64 if op_dtype == torch.bfloat16 else 32


def _pad_cols(t: torch.Tensor, mult: int) -> torch.Tensor:
    """t [R, C] with C rounded up to `mult` (zero columns) and 16-byte rows."""
    R, C = t.shape
    Cp = cdiv(max(C, 1), mult) * mult
    if Cp == C and t.stride(-1) == 1 and (t.stride(0) * t.element_size()) % 16 == 0 and t.data_ptr() % 16 == 0:
        return t
    out = torch.zeros((R, Cp), dtype=t.dtype, device=t.device)
    out[:, :C] = t
    return out


def gemm_dq_forward(a: QTensor, b: QTensor, *, bias: Optional[torch.Tensor] = None,
                    out_dtype: torch.dtype = torch.bfloat16, op_dtype: torch.dtype = torch.bfloat16,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Y[M, N] = op(dq(a)) @ op(dq(b))^T + bias with op = rounding to op_dtype
    (te_backend.py:229-260 as the reference runs it: each dequantized operand
    cast to the input dtype, then an fp32 GEMM)."""
    _require_device(a.codes, b.codes, bias)
    if a.grid != b.grid:
        raise ValueError("operands must share a code format")
    if a.K != b.K:
        raise ValueError(f"contraction mismatch: {a.K} vs {b.K}")
    M, N, Kp = a.rows, b.rows, a.Kp
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.codes.device)
    if bias is not None and bias.stride(-1) != 1:
        bias = bias.contiguous()
    call("ntlb_gemm_dq_forward", op_dtype_code(op_dtype), a.grid, a.codes.data_ptr(), a.codes.stride(0),
         a.scales.data_ptr(), a.s_row, a.s_col, a.shift, b.codes.data_ptr(), b.codes.stride(0), b.scales.data_ptr(),
         b.s_row, b.s_col, b.shift, M, N, Kp, _ptr(bias), _dtype_code(bias.dtype) if bias is not None else 0,
         out.data_ptr(), _dtype_code(out.dtype), out.stride(0), _stream())
    return out


def ste_dgrad(dy: torch.Tensor, w: QTensor, *, out_dtype: torch.dtype) -> torch.Tensor:
    """dX[M, K] = dY[M, N] @ bf16(dq(w))[N, K] (the straight-through input
    gradient of te_backend.py:250-259), decoded from the forward's weight codes."""
    _require_device(dy, w.codes)
    if dy.dtype != torch.bfloat16:
        raise TypeError("ste_dgrad takes a bfloat16 dY")
    M, N = dy.shape
    if N != w.rows:
        raise ValueError(f"dY has {N} columns, the weight {w.rows} rows")
    dyp = _pad_cols(dy, 64)
    out = torch.empty((M, w.K), dtype=out_dtype, device=dy.device)
    # the tiles past the last whole wave run as summed K ranges (split-K tail)
    ws = split_workspace(int(_lib.lib().ntlb_gemm_dq_workspace_bytes(_lib.BF16, M, w.K, N)), dy.device)
    call("ntlb_gemm_ste_dgrad_ws", _lib.BF16, dyp.data_ptr(), dyp.stride(0), M, N, w.grid, w.codes.data_ptr(),
         w.codes.stride(0), w.scales.data_ptr(), w.s_row, w.s_col, w.shift, w.K, out.data_ptr(),
         _dtype_code(out_dtype), out.stride(0), _ptr(ws), ws.numel() if ws is not None else 0, _stream())
    return out


def ste_wgrad(dy: torch.Tensor, x: QTensor, *, out_dtype: torch.dtype, db_dtype: Optional[torch.dtype] = None):
    """dW[N, K] = dY[M, N]^T @ bf16(dq(x))[M, K] (the straight-through weight
    gradient), decoded from the forward's activation codes.  With db_dtype,
    returns (dW, db): db[N] = dY summed over its rows in fp32 (the bias
    gradient), formed by the same kernel from the dY tiles it stages."""
    _require_device(dy, x.codes)
    if dy.dtype != torch.bfloat16:
        raise TypeError("ste_wgrad takes a bfloat16 dY")
    M, N = dy.shape
    if M != x.rows:
        raise ValueError(f"dY has {M} rows, the activation {x.rows}")
    if dy.stride(-1) != 1 or dy.stride(0) % 8 or dy.data_ptr() % 16:
        dy = _pad_cols(dy, 8)
    out = torch.empty((N, x.K), dtype=out_dtype, device=dy.device)
    db = torch.empty((N,), dtype=db_dtype, device=dy.device) if db_dtype is not None else None
    call("ntlb_gemm_ste_wgrad_db", _lib.BF16, dy.data_ptr(), dy.stride(0), M, N, x.grid, x.codes.data_ptr(),
         x.codes.stride(0), x.scales.data_ptr(), x.s_row, x.s_col, x.shift, x.K, out.data_ptr(),
         _dtype_code(out_dtype), out.stride(0), _ptr(db), _dtype_code(db_dtype) if db is not None else 0, _stream())
    return out if db is None else (out, db)


def grouped_ste_dgrad(dy: torch.Tensor, offsets: torch.Tensor, w_codes: torch.Tensor, w_scales: torch.Tensor, *,
                      grid: int, K: int, out_dtype: torch.dtype) -> torch.Tensor:
    """dX[rows of e] = dY[rows of e] @ bf16(dq(W_e)) for rows sorted by expert
    (offsets int32 [E+1]); W_e the 128x128-block codes [E, N, Kp] and scales
    [E, N/128, Kp/128] of moe.quantize_expert_weights.  dX [R, K]."""
    _require_device(dy, offsets, w_codes, w_scales)
    if dy.dtype != torch.bfloat16:
        raise TypeError("grouped_ste_dgrad takes a bfloat16 dY")
    E, N, ldw = w_codes.shape
    if dy.shape[1] != N or offsets.numel() != E + 1 or offsets.dtype != torch.int32:
        raise ValueError("dY columns must match the weights' rows and offsets must be int32 [E+1]")
    w_codes, w_scales = w_codes.contiguous(), w_scales.contiguous()
    R = dy.shape[0]
    dyp = _pad_cols(dy, 64)
    out = torch.empty((R, K), dtype=out_dtype, device=dy.device)
    tb = w_scales.shape[2]
    call("ntlb_gemm_grouped_ste_dgrad", _lib.BF16, dyp.data_ptr(), dyp.stride(0), R, N, offsets.data_ptr(), E, grid,
         w_codes.data_ptr(), ldw, w_codes.stride(0), w_scales.data_ptr(), tb, 1, 7, w_scales.stride(0), K,
         out.data_ptr(), _dtype_code(out_dtype), out.stride(0), _stream())
    return out


def grouped_ste_dgrad_gate_up(d_gu: torch.Tensor, offsets: torch.Tensor, w_codes: torch.Tensor,
                              w_scales: torch.Tensor, *, grid: int, K: int) -> torch.Tensor:
    """The gate and up Linears' summed input gradient of every expert:
    bf16(dX_gate) + bf16(dX_up) added in bf16, over the interleaved gate/up
    layout (d_gu bf16 [R, 2I], codes [E, 2I, Kp], scales [E, 2I/128, Kp/128]).
    dX bf16 [R, K]."""
    _require_device(d_gu, offsets, w_codes, w_scales)
    if d_gu.dtype != torch.bfloat16:
        raise TypeError("grouped_ste_dgrad_gate_up takes a bfloat16 d_gate_up")
    E, N2, ldw = w_codes.shape
    R = d_gu.shape[0]
    if d_gu.shape[1] != N2 or offsets.numel() != E + 1 or offsets.dtype != torch.int32:
        raise ValueError("d_gate_up columns must match the weights' rows and offsets must be int32 [E+1]")
    w_codes, w_scales = w_codes.contiguous(), w_scales.contiguous()
    d_gu = _pad_cols(d_gu, 64)
    out = torch.empty((R, K), dtype=torch.bfloat16, device=d_gu.device)
    call("ntlb_gemm_grouped_ste_dgrad_gate_up", _lib.BF16, d_gu.data_ptr(), d_gu.stride(0), R, N2 // 2,
         offsets.data_ptr(), E, grid, w_codes.data_ptr(), ldw, w_codes.stride(0), w_scales.data_ptr(),
         w_scales.shape[2], 1, w_scales.stride(0), K, out.data_ptr(), out.stride(0), _stream())
    return out


def grouped_ste_wgrad(dy: torch.Tensor, offsets: torch.Tensor, x: QTensor, n_experts: int, *,
                      out_dtype: torch.dtype) -> torch.Tensor:
    """dW[e] = dY[rows of e]^T @ bf16(dq(X[rows of e])) for every expert (zero
    for an expert without rows); X's codes carry per-row 1x128 tile-major
    scales.  dW [E, N, K]."""
    _require_device(dy, offsets, x.codes)
    if dy.dtype != torch.bfloat16:
        raise TypeError("grouped_ste_wgrad takes a bfloat16 dY")
    R, N = dy.shape
    if R != x.rows or offsets.numel() != n_experts + 1 or offsets.dtype != torch.int32:
        raise ValueError("dY and X must have the same rows and offsets must be int32 [E+1]")
    if dy.stride(-1) != 1 or dy.stride(0) % 8 or dy.data_ptr() % 16:
        dy = _pad_cols(dy, 8)
    out = torch.empty((n_experts, N, x.K), dtype=out_dtype, device=dy.device)
    call("ntlb_gemm_grouped_ste_wgrad", _lib.BF16, dy.data_ptr(), dy.stride(0), R, N, offsets.data_ptr(), n_experts,
         x.grid, x.codes.data_ptr(), x.codes.stride(0), x.scales.data_ptr(), x.s_row, x.s_col, x.shift, x.K,
         out.data_ptr(), _dtype_code(out_dtype), out.stride(1), out.stride(0) * out.element_size(), _stream())
    return out


def grouped_dgrad_dense(dy: torch.Tensor, offsets: torch.Tensor, w: torch.Tensor, *,
                        out_dtype: torch.dtype) -> torch.Tensor:
    """dX[rows of e] = dY[rows of e] @ w[e] for rows sorted by expert, w bf16
    [E, N, K] (the straight-through operands of the experts' weights)."""
    _require_device(dy, offsets, w)
    if dy.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise TypeError("grouped_dgrad_dense takes bf16 operands")
    E, N, K = w.shape
    if dy.shape[1] != N or offsets.numel() != E + 1 or offsets.dtype != torch.int32:
        raise ValueError("dY columns must match the weights' rows and offsets must be int32 [E+1]")
    w = w if (w.is_contiguous() and K % 4 == 0) else _pad_cols(w.reshape(E * N, K), 4).reshape(E, N, -1)
    R = dy.shape[0]
    dyp = _pad_cols(dy, 64)
    out = torch.empty((R, K), dtype=out_dtype, device=dy.device)
    call("ntlb_gemm_grouped_dgrad_dense", _lib.BF16, dyp.data_ptr(), dyp.stride(0), R, N, offsets.data_ptr(), E,
         w.data_ptr(), w.stride(1), w.stride(0), K, out.data_ptr(), _dtype_code(out_dtype), out.stride(0), _stream())
    return out


def grouped_dgrad_dense_gate_up(d_gu: torch.Tensor, offsets: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """grouped_ste_dgrad_gate_up over dense bf16 gate/up operands w [E, 2I, H]
    (128-row blocks alternating gate and up): bf16(dX_gate) + bf16(dX_up)."""
    _require_device(d_gu, offsets, w)
    if d_gu.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise TypeError("grouped_dgrad_dense_gate_up takes bf16 operands")
    E, N2, H = w.shape
    if d_gu.shape[1] != N2 or offsets.numel() != E + 1 or offsets.dtype != torch.int32:
        raise ValueError("d_gate_up columns must match the weights' rows and offsets must be int32 [E+1]")
    w = w if (w.is_contiguous() and H % 4 == 0) else _pad_cols(w.reshape(E * N2, H), 4).reshape(E, N2, -1)
    R = d_gu.shape[0]
    d_gu = _pad_cols(d_gu, 64)
    out = torch.empty((R, H), dtype=torch.bfloat16, device=d_gu.device)
    call("ntlb_gemm_grouped_dgrad_dense_gate_up", _lib.BF16, d_gu.data_ptr(), d_gu.stride(0), R, N2 // 2,
         offsets.data_ptr(), E, w.data_ptr(), w.stride(1), w.stride(0), H, out.data_ptr(), out.stride(0), _stream())
    return out


def grouped_wgrad_dense(dy: torch.Tensor, offsets: torch.Tensor, x: torch.Tensor, n_experts: int, *,
                        out_dtype: torch.dtype) -> torch.Tensor:
    """dW[e] = dY[rows of e]^T @ x[rows of e] over dense bf16 rows (zero for an
    expert without rows).  dW [E, N, K]."""
    _require_device(dy, offsets, x)
    if dy.dtype != torch.bfloat16 or x.dtype != torch.bfloat16:
        raise TypeError("grouped_wgrad_dense takes bf16 operands")
    R, N = dy.shape
    K = x.shape[1]
    if x.shape[0] != R or offsets.numel() != n_experts + 1 or offsets.dtype != torch.int32:
        raise ValueError("dY and x must have the same rows and offsets must be int32 [E+1]")
    dy = dy if (dy.stride(-1) == 1 and dy.stride(0) % 4 == 0 and dy.data_ptr() % 16 == 0) else _pad_cols(dy, 4)
    x = x if (x.stride(-1) == 1 and x.stride(0) % 4 == 0 and x.data_ptr() % 16 == 0) else _pad_cols(x, 4)
    out = torch.empty((n_experts, N, K), dtype=out_dtype, device=dy.device)
    call("ntlb_gemm_grouped_wgrad_dense", _lib.BF16, dy.data_ptr(), dy.stride(0), R, N, offsets.data_ptr(),
         n_experts, x.data_ptr(), x.stride(0), K, out.data_ptr(), _dtype_code(out_dtype), out.stride(1),
         out.stride(0) * out.element_size(), _stream())
    return out


def gemm_dense(a: torch.Tensor, b: torch.Tensor, *, b_transposed: bool = False, bias: Optional[torch.Tensor] = None,
               out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Y = a @ b^T (b [N, K]) or a @ b (b_transposed: b [K, N]) + bias over
    bf16 or fp32 matrices of one dtype, fp32 accumulation."""
    _require_device(a, b, bias)
    if a.dtype != b.dtype:
        raise TypeError(f"operand dtypes differ: {a.dtype} vs {b.dtype}")
    code = op_dtype_code(a.dtype)
    M, K = a.shape
    step = _kstep(a.dtype)
    ap = _pad_cols(a, step)
    if b_transposed:
        if b.shape[0] != K:
            raise ValueError(f"contraction mismatch: {K} vs {b.shape[0]}")
        N = b.shape[1]
        bp = _pad_cols(b, 16 // b.element_size())
        # rows of B past K are zero inside the kernel; A's pad columns are zero
        bp_rows = torch.zeros((ap.shape[1], bp.shape[1]), dtype=b.dtype, device=b.device) if ap.shape[1] != K else bp
        if bp_rows is not bp:
            bp_rows[:K] = bp
        bp = bp_rows
    else:
        if b.shape[1] != K:
            raise ValueError(f"contraction mismatch: {K} vs {b.shape[1]}")
        N = b.shape[0]
        bp = _pad_cols(b, step)
    if bias is not None and bias.stride(-1) != 1:
        bias = bias.contiguous()
    out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    call("ntlb_gemm_dense", code, ap.data_ptr(), ap.stride(0), 0, bp.data_ptr(), bp.stride(0), int(b_transposed), M, N,
         ap.shape[1], _ptr(bias), _dtype_code(bias.dtype) if bias is not None else 0, out.data_ptr(),
         _dtype_code(out_dtype), out.stride(0), _stream())
    return out


def gemm_dense_tn(a: torch.Tensor, b: torch.Tensor, *, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Y[M, N] = a^T @ b for a [K, M], b [K, N] (the weight gradient over
    dequantized tensors), fp32 accumulation."""
    _require_device(a, b)
    if a.dtype != b.dtype:
        raise TypeError(f"operand dtypes differ: {a.dtype} vs {b.dtype}")
    code = op_dtype_code(a.dtype)
    K, M = a.shape
    if b.shape[0] != K:
        raise ValueError(f"contraction mismatch: {K} vs {b.shape[0]}")
    N = b.shape[1]
    mult = 16 // a.element_size()
    ap, bp = _pad_cols(a, mult), _pad_cols(b, mult)
    out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    call("ntlb_gemm_dense_tn", code, ap.data_ptr(), ap.stride(0), bp.data_ptr(), bp.stride(0), M, N, K,
         out.data_ptr(), _dtype_code(out_dtype), out.stride(0), _stream())
    return out


_colsum_ws: dict = {}


def ste_value(t: torch.Tensor, t_dq: torch.Tensor) -> torch.Tensor:
    """t + (t_dq - t) in t's dtype (te_backend.py:250-251): the operand the
    reference multiplies; it differs from t_dq only under stochastic rounding."""
    _require_device(t, t_dq)
    if t.dtype != t_dq.dtype or t.shape != t_dq.shape:
        raise ValueError(f"ste_value operands differ: {t.dtype}{tuple(t.shape)} vs {t_dq.dtype}{tuple(t_dq.shape)}")
    t, t_dq = t.contiguous(), t_dq.contiguous()
    out = torch.empty_like(t)
    call("ntlb_ste_value", _dtype_code(t.dtype), t.data_ptr(), t_dq.data_ptr(), out.data_ptr(), t.numel(), _stream())
    return out


def colsum(x: torch.Tensor, *, out_dtype: torch.dtype) -> torch.Tensor:
    """sum over rows of x [M, N] in fp32, cast to out_dtype (F.linear's bias
    gradient), in a fixed order."""
    _require_device(x)
    x2 = _as_2d(x)
    M, N = x2.shape
    out = torch.empty((N,), dtype=out_dtype, device=x.device)
    need = int(_lib.lib().ntlb_colsum_workspace_bytes(M, N))
    key = (x.device.index, _stream())
    ws = _colsum_ws.get(key)
    if ws is None or ws.numel() * 4 < max(need, 4):
        ws = torch.empty((max(need, 4) + 3) // 4, dtype=torch.float32, device=x.device)
        _colsum_ws[key] = ws
    call("ntlb_colsum", x2.data_ptr(), _dtype_code(x2.dtype), M, N, x2.stride(0), ws.data_ptr(), ws.numel() * 4,
         out.data_ptr(), _dtype_code(out_dtype), _stream())
    return out
