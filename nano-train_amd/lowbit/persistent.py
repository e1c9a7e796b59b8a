"""Persistent low-bit weights on the MI355X kernels.

Drop-ins for the persistent-parameter helpers of nano-train's src/layers.py,
with the same signatures, buffer dtypes and scale shapes (so checkpoints keep
the `_persistent_fp4_codes` uint8 packed nibbles, `_persistent_fp8_weight`
float8_e4m3fn values and `_persistent_scale` fp32 layout, layers.py:235-246):

  nf4_codebook                  layers.py:60-83
  quantize_nf4_persistent       layers.py:156-169 (+ _pack_nibbles :130-139)
  dequantize_nf4_persistent     layers.py:172-184 (+ _unpack_nibbles :142-153)
  quantize_fp8_persistent       layers.py:104-117
  dequantize_fp8_persistent     layers.py:120-127

plus the benchmark config 5 formats that have no reference function: NF4 with
one scale per 64 elements, MXFP4 (e2m1 + e8m0 per 32), and the GEMMs with the
dequantization fused into the weight-tile prologue (linear_nf4, linear_mxfp4,
and linear_fp8p for the persistent FP8 weight).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib, ops
from ._lib import call

NF4_CODEBOOK = (
    -1.0, -0.6961928, -0.52507305, -0.3949175, -0.28444138, -0.18477343, -0.09105004, 0.0,
    0.0795803, 0.1609302, 0.2461123, 0.33791524, 0.44070983, 0.562617, 0.72295684, 1.0,
)


def nf4_codebook(device: torch.device) -> torch.Tensor:
    return torch.tensor(NF4_CODEBOOK, dtype=torch.float32, device=device)


def _block_and_scale_shape(tensor: torch.Tensor, granularity: str):
    """Scale grouping of layers.py:86-101: per_channel reduces over dims 1..,
    per_tensor over everything (and so does per_channel on a 1-D tensor)."""
    if granularity == "per_channel" and tensor.dim() > 1:
        block = tensor.numel() // tensor.shape[0]
        shape = (tensor.shape[0],) + (1,) * (tensor.dim() - 1)
    else:
        block = tensor.numel()
        shape = ()
    return max(block, 1), shape


def _flat(t: torch.Tensor) -> torch.Tensor:
    ops._require_device(t)
    return t.detach().reshape(-1) if t.is_contiguous() else t.detach().contiguous().reshape(-1)


def quantize_nf4_blocks(tensor: torch.Tensor, block: int):
    """NF4 codes with one scale per `block` consecutive elements: (packed, scales[ceil(n/block)])."""
    flat = _flat(tensor)
    n = flat.numel()
    nb = ops.cdiv(n, block) if n else 0
    packed = torch.empty((n + 1) // 2, dtype=torch.uint8, device=flat.device)
    scales = torch.empty(nb, dtype=torch.float32, device=flat.device)
    ws = torch.zeros(max(nb, 1), dtype=torch.int32, device=flat.device)
    call("ntlb_nf4_quant", flat.data_ptr(), ops._dtype_code(flat.dtype), n, block, ws.data_ptr(), packed.data_ptr(),
         scales.data_ptr(), ops._stream())
    return packed, scales


def quantize_nf4_persistent(tensor: torch.Tensor, *, granularity: str):
    """(packed codes, scale) exactly as _quantize_nf4_persistent (layers.py:156-169)."""
    block, shape = _block_and_scale_shape(tensor, granularity)
    packed, scales = quantize_nf4_blocks(tensor, block)
    return packed, scales.reshape(shape)


def dequantize_nf4_blocks(packed: torch.Tensor, scales: torch.Tensor, *, num_values: int, block: int,
                          target_dtype: torch.dtype) -> torch.Tensor:
    ops._require_device(packed, scales)
    out = torch.empty(num_values, dtype=target_dtype, device=packed.device)
    sc = scales.reshape(-1).contiguous().float()
    call("ntlb_nf4_dequant", packed.data_ptr(), sc.data_ptr(), num_values, block, out.data_ptr(),
         ops._dtype_code(target_dtype), ops._stream())
    return out


def dequantize_nf4_persistent(packed_codes: torch.Tensor, scale: torch.Tensor, *, num_values: int,
                              target_shape: torch.Size, target_dtype: torch.dtype) -> torch.Tensor:
    """_dequantize_nf4_persistent (layers.py:172-184)."""
    nscale = max(scale.numel(), 1)
    block = max(num_values // nscale, 1) if num_values else 1
    out = dequantize_nf4_blocks(packed_codes, scale, num_values=num_values, block=block, target_dtype=target_dtype)
    return out.reshape(target_shape)


def quantize_fp8_persistent(tensor: torch.Tensor, *, granularity: str):
    """(float8_e4m3fn values, scale) exactly as _quantize_fp8_persistent (layers.py:104-117)."""
    block, shape = _block_and_scale_shape(tensor, granularity)
    flat = _flat(tensor)
    n = flat.numel()
    nb = ops.cdiv(n, block) if n else 0
    codes = torch.empty(n, dtype=torch.uint8, device=flat.device)
    scales = torch.empty(nb, dtype=torch.float32, device=flat.device)
    ws = torch.zeros(max(nb, 1), dtype=torch.int32, device=flat.device)
    call("ntlb_fp8_persistent_quant", flat.data_ptr(), ops._dtype_code(flat.dtype), n, block, ws.data_ptr(),
         codes.data_ptr(), scales.data_ptr(), ops._stream())
    return codes.view(torch.float8_e4m3fn).reshape(tensor.shape), scales.reshape(shape)


def dequantize_fp8_persistent(fp8_values: torch.Tensor, scale: torch.Tensor, *,
                              target_dtype: torch.dtype) -> torch.Tensor:
    """_dequantize_fp8_persistent (layers.py:120-127)."""
    ops._require_device(fp8_values, scale)
    codes = fp8_values.contiguous().view(torch.uint8).reshape(-1)
    n = codes.numel()
    nscale = max(scale.numel(), 1)
    block = max(n // nscale, 1) if n else 1
    out = torch.empty(n, dtype=target_dtype, device=codes.device)
    sc = scale.reshape(-1).contiguous().float()
    call("ntlb_fp8_persistent_dequant", codes.data_ptr(), sc.data_ptr(), n, block, out.data_ptr(),
         ops._dtype_code(target_dtype), ops._stream())
    return out.reshape(fp8_values.shape)


def quantize_mxfp4(tensor: torch.Tensor):
    """MXFP4 codes: (packed [ceil(n/2)] uint8, e8m0 scales [ceil(n/32)] uint8)."""
    flat = _flat(tensor)
    n = flat.numel()
    packed = torch.empty((n + 1) // 2, dtype=torch.uint8, device=flat.device)
    scales = torch.empty(ops.cdiv(n, 32), dtype=torch.uint8, device=flat.device)
    call("ntlb_mxfp4_quant", flat.data_ptr(), ops._dtype_code(flat.dtype), n, packed.data_ptr(), scales.data_ptr(),
         ops._stream())
    return packed, scales


def dequantize_mxfp4(packed: torch.Tensor, scales: torch.Tensor, *, num_values: int,
                     target_dtype: torch.dtype) -> torch.Tensor:
    ops._require_device(packed, scales)
    out = torch.empty(num_values, dtype=target_dtype, device=packed.device)
    call("ntlb_mxfp4_dequant", packed.data_ptr(), scales.data_ptr(), num_values, out.data_ptr(),
         ops._dtype_code(target_dtype), ops._stream())
    return out


def _x2(x: torch.Tensor, K: int) -> torch.Tensor:
    ops._require_device(x)
    if x.dtype != torch.bfloat16:
        raise TypeError("the fused low-bit GEMMs take bf16 activations")
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


_LOWBIT_NF4, _LOWBIT_MXFP4, _LOWBIT_FP8P = 0, 1, 2


def _fused(fmt: int, x2: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, block: int, bias, M: int, N: int,
           K: int, out_dtype) -> torch.Tensor:
    """ntlb_gemm_lowbit_ws with the current stream's split-K workspace."""
    if bias is not None:
        ops._require_device(bias)
        if bias.numel() != N:
            raise ValueError(f"bias must have {N} entries, got {bias.numel()}")
        bias = bias.reshape(-1).contiguous()
    y = torch.empty((M, N), dtype=out_dtype or torch.bfloat16, device=x2.device)
    ws = ops.split_workspace(int(_lib.lib().ntlb_gemm_lowbit_workspace_bytes(M, N, K)), x2.device)
    call("ntlb_gemm_lowbit_ws", fmt, x2.data_ptr(), x2.stride(0), w.data_ptr(), scales.data_ptr(), block,
         ops._ptr(bias), ops._dtype_code(bias.dtype) if bias is not None else 0, M, N, K, y.data_ptr(),
         ops._dtype_code(y.dtype), y.stride(0), ops._ptr(ws), ws.numel() if ws is not None else 0, ops._stream())
    return y


def _dq_forward(fmt: int, x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, block: int, bias, N: int, K: int,
                out_dtype) -> torch.Tensor:
    """ntlb_gemm_lowbit_dq_forward_ws: the weight decoded into the dequantized-
    operand GEMM (bf16 or fp32 activations, K % 4 == 0, one scale per row or
    one for all)."""
    ops._require_device(x, w, scales, bias)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("the persistent-weight GEMM takes bf16 or fp32 activations")
    x2 = ops._pad_cols(x.reshape(-1, K), 64 if x.dtype == torch.bfloat16 else 32)
    M = x2.shape[0]
    if bias is not None:
        if bias.numel() != N:
            raise ValueError(f"bias must have {N} entries, got {bias.numel()}")
        bias = bias.reshape(-1).contiguous()
    y = torch.empty((M, N), dtype=out_dtype or x.dtype, device=x.device)
    op = _lib.BF16 if x.dtype == torch.bfloat16 else _lib.F32
    ws = ops.split_workspace(int(_lib.lib().ntlb_gemm_dq_workspace_bytes(op, M, N, K)), x.device)
    call("ntlb_gemm_lowbit_dq_forward_ws", fmt, op, x2.data_ptr(), x2.stride(0), M, w.data_ptr(), scales.data_ptr(),
         block, N, K, ops._ptr(bias), ops._dtype_code(bias.dtype) if bias is not None else 0, y.data_ptr(),
         ops._dtype_code(y.dtype), y.stride(0), ops._ptr(ws), ws.numel() if ws is not None else 0, ops._stream())
    return y


def _fused_kernel_fits(x: torch.Tensor, K: int) -> bool:
    """the dequant-fused kernel: bf16 activations and K % 64 == 0; otherwise the
    dequantized-operand GEMM decodes the weight (fp32 activations, ragged K)"""
    return x.dtype == torch.bfloat16 and K % 64 == 0


def linear_nf4(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, *, out_features: int, block: int,
               bias: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Y = x @ deq(W)^T (+ bias) with W [out_features, K] in NF4, dequantized inside the GEMM.

    block: elements per scale (K for per_channel, 0 or numel for per_tensor, 64...).  bf16 x with
    K % 64 == 0 runs the dequant-fused kernel; fp32 x, or K % 64 != 0 (K % 4 == 0), the
    dequantized-operand GEMM, which takes per-row or per-tensor scales."""
    K = x.shape[-1]
    N = out_features
    blk = 0 if block >= N * K else block
    sc = scales.reshape(-1).contiguous()
    if not _fused_kernel_fits(x, K):
        y = _dq_forward(_LOWBIT_NF4, x, packed, sc.float(), blk, bias, N, K, out_dtype)
        return y.reshape(*x.shape[:-1], N)
    x2 = _x2(x, K)
    M = x2.shape[0]
    y = _fused(_LOWBIT_NF4, x2, packed, sc, blk, bias, M, N, K, out_dtype)
    return y.reshape(*x.shape[:-1], N)


def linear_fp8p(x: torch.Tensor, fp8_values: torch.Tensor, scale: torch.Tensor, *,
                bias: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Y = x @ deq(W)^T (+ bias) with W the persistent FP8 weight [N, K]
    (float8_e4m3fn values and a per_channel [N, 1] or per_tensor scale),
    dequantized inside the GEMM as _dequantize_fp8_persistent does
    (layers.py:120-127)."""
    ops._require_device(fp8_values, scale)
    N, K = fp8_values.shape
    codes = fp8_values.contiguous().view(torch.uint8)
    sc = scale.reshape(-1).contiguous().float()
    block = 0 if sc.numel() <= 1 else K
    if block and sc.numel() != N:
        raise ValueError(f"scale must be per_tensor or one per row, got {tuple(scale.shape)}")
    if not _fused_kernel_fits(x, K):
        y = _dq_forward(_LOWBIT_FP8P, x, codes, sc, block, bias, N, K, out_dtype)
        return y.reshape(*x.shape[:-1], N)
    x2 = _x2(x, K)
    M = x2.shape[0]
    y = _fused(_LOWBIT_FP8P, x2, codes, sc, block, bias, M, N, K, out_dtype)
    return y.reshape(*x.shape[:-1], N)


def dgrad(dy: torch.Tensor, codes: torch.Tensor, scale: torch.Tensor, *, fmt: str, out_features: int,
          in_features: int, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """dX [M, K] = dY [M, N] @ deq(W) for a persistent weight W [N, K], decoded
    inside the GEMM (ntlb_gemm_lowbit_dgrad_ws): the straight-through input
    gradient of the persistent layers (layers.py:409-436), with no dequantized
    copy of W.  fmt "nf4" (packed nibbles, per_channel [N, 1] or per_tensor
    scale) or "fp8" (float8_e4m3fn values [N, K]).  dY bf16 multiplies the
    bf16-rounded weight values on bf16 MFMA, dY fp32 the fp32 values."""
    ops._require_device(dy, codes, scale)
    N, K = out_features, in_features
    if dy.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("dgrad takes a bf16 or fp32 dY")
    dy2 = dy.reshape(-1, N)
    M = dy2.shape[0]
    dy2 = ops._pad_cols(dy2, 64 if dy.dtype == torch.bfloat16 else 32)
    sc = scale.reshape(-1).float().contiguous()
    if sc.numel() not in (1, N):
        raise ValueError(f"scale must be per_tensor or one per row, got {tuple(scale.shape)}")
    block = K if sc.numel() == N and N > 1 else 0
    w = codes.contiguous().view(torch.uint8)
    f = _LOWBIT_NF4 if fmt == "nf4" else _LOWBIT_FP8P
    dx = torch.empty((M, K), dtype=out_dtype or dy.dtype, device=dy.device)
    op = _lib.BF16 if dy.dtype == torch.bfloat16 else _lib.F32
    ws = ops.split_workspace(int(_lib.lib().ntlb_gemm_dq_workspace_bytes(op, M, K, N)), dy.device)
    call("ntlb_gemm_lowbit_dgrad_ws", f, op, dy2.data_ptr(), dy2.stride(0), M, N, w.data_ptr(), sc.data_ptr(), block,
         K, dx.data_ptr(), ops._dtype_code(dx.dtype), dx.stride(0), ops._ptr(ws), ws.numel() if ws is not None else 0,
         ops._stream())
    return dx.reshape(*dy.shape[:-1], K)


def linear_mxfp4(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, *, out_features: int,
                 bias: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Y = x @ deq(W)^T (+ bias) with W [out_features, K] in MXFP4, dequantized inside the GEMM."""
    K = x.shape[-1]
    x2 = _x2(x, K)
    M, N = x2.shape[0], out_features
    y = _fused(_LOWBIT_MXFP4, x2, packed, scales, 32, bias, M, N, K, out_dtype)
    return y.reshape(*x.shape[:-1], N)
