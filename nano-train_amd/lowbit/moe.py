"""MoE side of the low-bit path: comm-quant of the dispatch payload and the
grouped per-expert GEMM, mirroring src/models/moe.py of nano-train.

comm_quant_dequant() is the drop-in for _comm_quant_dequant (moe.py:79-143):
same arguments, same granularities (one scale per tensor; per column;
per 128-column strip over all rows for both 'tile_1x128' and
'block_128x128'), the same before-division scale rule (moe.py:94-98), the int
grid with qmax = 2^(bits-1)-1, and the same straight-through estimator
`tensor + (dq - tensor).detach()` (moe.py:107-143).  Stochastic rounding draws
its bits from the Philox contract of the C-ABI instead of torch.rand_like
(moe.py:72-76).

comm_quant() / comm_dequant() are the wire format a real expert-parallel
all-to-all would carry (codes plus per-row 1x128 scales, e4m3 or int grid);
the reference has no counterpart (it all-to-alls the dequantized bf16 tensor,
moe.py:787-793).

route_by_expert() orders the (token, slot) assignments by expert with one
stable counting sort on the GPU (ntlb_ep_partition), which gives the rows of
each expert in the order the reference's per-expert nonzero() selects them
(moe.py:1077, :478) and the token-offset table.  local_moe_forward() is the
single-rank expert loop (moe.py:1062-1093, LocalRoutedMoE :476-491) on HIP
kernels only: the routing sort, the 1x128 quantization of the token rows
gathered by expert (one read per token), the gate/up GEMM with SwiGLU and
h's quantization in its epilogue, the down GEMM, and the weighted combine into
token order.  grouped_linear() runs one Linear per expert over rows already
sorted by expert.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from . import ops
from .ops import QTensor

_comm_calls = itertools.count()


def _comm_seed_offset(seed: Optional[int], offset: Optional[int]):
    if seed is None:
        seed = torch.initial_seed() & 0xFFFFFFFFFFFFFFFF
    if offset is None:
        offset = (1 << 40) + next(_comm_calls)  # a stream of its own, apart from the Linear backends
    return seed, offset


def comm_quant_dequant(
    tensor: torch.Tensor,
    *,
    granularity: str,
    rounding_mode: str,
    bits: int = 8,
    seed: Optional[int] = None,
    offset: Optional[int] = None,
) -> torch.Tensor:
    """Fake quant-dequant of a comm payload preserving autograd (moe.py:79-143)."""
    if tensor.numel() == 0:
        return tensor
    if tensor.device.type != "cuda":
        raise RuntimeError("comm_quant_dequant runs on a ROCm device only; there is no CPU path")
    seed, offset = _comm_seed_offset(seed, offset)
    x2 = tensor.reshape(-1, tensor.shape[-1]) if tensor.dim() >= 2 else tensor.reshape(1, -1)
    R, K = x2.shape
    if granularity in ("tile_1x128", "block_128x128") and tensor.dim() >= 1:
        gr, gc = R, 128  # one scale per 128-column strip over all rows (moe.py:123-140)
    elif granularity == "channel" and tensor.dim() >= 2:
        gr, gc = R, 1  # one scale per column (moe.py:112-121)
    else:
        gr, gc = R, K  # tensor, 1-D channel, or anything else (moe.py:107-110, :141-143)
    rounding = "stochastic" if rounding_mode == "stochastic" else "nearest"
    x2 = x2.detach()
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    gr, gc = max(1, min(gr, R)), max(1, min(gc, K))
    amax = torch.zeros(ops.cdiv(R, gr) * ops.cdiv(K, gc), dtype=torch.int32, device=tensor.device)
    out = torch.empty((R, K), dtype=tensor.dtype, device=tensor.device)
    xc = ops._dtype_code(x2.dtype)
    _lib.call("ntlb_amax_grouped", x2.data_ptr(), xc, R, K, x2.stride(0), gr, gc, amax.data_ptr(), ops._stream())
    # the kernel writes tensor + (dq - tensor) as the reference evaluates it
    _lib.call("ntlb_comm_quant_dequant", x2.data_ptr(), xc, R, K, x2.stride(0), gr, gc, amax.data_ptr(),
              ops.grid_code("int_grid"), (1 << (bits - 1)) - 1, ops.rounding_code(rounding),
              _lib.SCALE_BEFORE_DIVIDE, seed, offset, out.data_ptr(), K, ops._stream())
    return _StraightThrough.apply(tensor, out.reshape(tensor.shape))


class _StraightThrough(torch.autograd.Function):
    """The value of tensor + (dq - tensor).detach() with its gradient: the
    identity to tensor (moe.py:110, :121, :141, :143)."""

    @staticmethod
    def forward(ctx, tensor, value):
        return value

    @staticmethod
    def backward(ctx, grad):
        return grad, None


@dataclass
class CommPayload:
    """Quantized dispatch payload: codes [rows, Kp] plus 1x128 scales."""

    q: QTensor
    shape: tuple
    dtype: torch.dtype

    @property
    def nbytes(self) -> int:
        return self.q.codes.numel() + self.q.scales.numel() * 4


def comm_quant(
    tensor: torch.Tensor,
    *,
    fmt: str = "e4m3",
    rounding_mode: str = "nearest",
    bits: int = 8,
    seed: Optional[int] = None,
    offset: Optional[int] = None,
) -> CommPayload:
    """Quantize a payload [..., H] per 1x128 tile of each row (the DeepSeek-V3 wire format)."""
    seed, offset = _comm_seed_offset(seed, offset)
    rounding = "stochastic" if rounding_mode == "stochastic" else "nearest"
    q = ops.quant_tile_1x128(tensor, fmt=fmt, bits=bits, rounding=rounding, seed=seed, offset=offset,
                             tile_major_scales=False)
    return CommPayload(q, tuple(tensor.shape), tensor.dtype)


def comm_dequant(payload: CommPayload, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """The receiver's dequantize back to the token dtype."""
    out = ops.dequant(payload.q, out_dtype=dtype or payload.dtype, r_shift=0, c_shift=7)
    return out.reshape(payload.shape)


@dataclass
class ExpertRouting:
    """The (token, slot) assignments of top-k routing ordered by expert.

    pos[a] is assignment a's row in expert order (a = token * top_k + slot),
    inv[row] the assignment of a row; rows of one expert keep assignment
    order, as the reference's (topk_indices == e).nonzero() lists them.
    offsets int32 [E+1] is the token-offset table of the grouped GEMMs."""

    pos: torch.Tensor  # int32 [T*top_k]
    inv: torch.Tensor  # int32 [T*top_k]
    counts: torch.Tensor  # int64 [E]
    offsets: torch.Tensor  # int32 [E+1]
    top_k: int

    @property
    def rows(self) -> int:
        return self.pos.numel()


def route_by_expert(expert_ids: torch.Tensor, n_experts: int) -> ExpertRouting:
    """One stable counting sort of expert_ids [T, k] (int32 or int64) by
    expert on the GPU (ntlb_ep_partition: three kernels, no host sync)."""
    from . import ep

    if expert_ids.dim() != 2:
        raise ValueError("expert_ids must be [tokens, top_k]")
    pos, inv, counts, offsets = ep.partition(expert_ids.reshape(-1), divisor=1, buckets=n_experts)
    return ExpertRouting(pos, inv, counts, offsets, expert_ids.shape[1])


def sort_by_expert(expert_ids: torch.Tensor, n_experts: int):
    """Token-offset table for top-k routing.

    expert_ids [T, k] int -> (order [T*k] int64 indices into the flattened
    (token, slot) pairs sorted by expert, stable; token_index [T*k] the source
    token of each sorted row; offsets int32 [E+1]).  route_by_expert() holds
    the same order without the int64 index tensors."""
    r = route_by_expert(expert_ids, n_experts)
    order = r.inv.to(torch.int64)
    return order, order // expert_ids.shape[1], r.offsets


def quantize_expert_weights(w: torch.Tensor, *, fmt: str = "e4m3", bits: int = 8, rounding: str = "nearest",
                            seed: int = 0, offset: int = 0):
    """128x128 block codes of stacked expert weights [E, N, K] (N % 128 == 0,
    so no block straddles two experts): codes [E, N, Kp], scales [E, N/128, Kp/128]."""
    E, N, K = w.shape
    if N % 128:
        raise ValueError("expert weights need N % 128 == 0 for per-expert 128x128 blocks")
    q, _ = ops.quant_block_128x128(w.reshape(E * N, K), fmt=fmt, bits=bits, rounding=rounding, seed=seed,
                                   offset=offset, want_nan_rows=True)
    codes = q.codes.reshape(E, N, -1)
    scales = q.scales.reshape(E, N // 128, -1)
    return codes, scales, q.nan_rows.reshape(E, N)


def grouped_linear(
    x_sorted: torch.Tensor,
    offsets: torch.Tensor,
    w_codes: torch.Tensor,
    w_scales: torch.Tensor,
    *,
    fmt: str = "e4m3",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
    out_dtype: Optional[torch.dtype] = None,
    w_nan_rows: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Y[rows of expert e] = X_dq[rows] @ W_dq[e]^T for rows sorted by expert.

    X is quantized per 1x128 tile over all rows at once; the experts' codes
    come from quantize_expert_weights()."""
    if isinstance(x_sorted, ops.QTensor):
        qx = x_sorted
        out_dtype = out_dtype or torch.bfloat16
    else:
        qx = ops.quant_tile_1x128(x_sorted, fmt=fmt, bits=bits, rounding=rounding, seed=seed, offset=offset,
                                  want_nan_rows=True)
        out_dtype = out_dtype or x_sorted.dtype
    return ops.gemm_grouped_blockscaled(qx, w_codes, w_scales, offsets, N=w_codes.shape[1],
                                        out_dtype=out_dtype or x_sorted.dtype, b_nan_rows=w_nan_rows)


def interleave_gate_up(gate_codes: torch.Tensor, gate_scales: torch.Tensor, up_codes: torch.Tensor,
                       up_scales: torch.Tensor, gate_nan: Optional[torch.Tensor] = None,
                       up_nan: Optional[torch.Tensor] = None):
    """Gate and up weight codes of the SwiGLU MLP (moe.py:160-177) interleaved in
    128-row blocks, the B operand of ops.gemm_swiglu_quant.

    Works on one expert ([I, Kp] codes, [I/128, Kp/128] scales) or a stack
    ([E, I, Kp], [E, I/128, Kp/128]); 128x128 blocks move whole, so the block
    scales stay valid.  Returns (codes, scales, nan_rows or None)."""
    if gate_codes.shape != up_codes.shape or gate_scales.shape != up_scales.shape:
        raise ValueError("gate and up weights must have the same shape")
    I, Kp = gate_codes.shape[-2], gate_codes.shape[-1]
    if I % 128:
        raise ValueError(f"intermediate size {I} must be a multiple of 128")
    lead = gate_codes.shape[:-2]
    nb = I // 128
    codes = torch.stack([gate_codes.reshape(*lead, nb, 128, Kp), up_codes.reshape(*lead, nb, 128, Kp)],
                        dim=-3).reshape(*lead, 2 * I, Kp)
    tb = gate_scales.shape[-1]
    scales = torch.stack([gate_scales.reshape(*lead, nb, tb), up_scales.reshape(*lead, nb, tb)],
                         dim=-2).reshape(*lead, 2 * nb, tb)
    nan = None
    if gate_nan is not None or up_nan is not None:
        gn = gate_nan if gate_nan is not None else torch.zeros_like(up_nan)
        un = up_nan if up_nan is not None else torch.zeros_like(gate_nan)
        nan = torch.stack([gn.reshape(*lead, nb, 128), un.reshape(*lead, nb, 128)], dim=-2).reshape(*lead, 2 * I)
    return codes.contiguous(), scales.contiguous(), nan


def expert_mlp(
    x_sorted: torch.Tensor,
    offsets: torch.Tensor,
    gate_up,
    down,
    *,
    fmt: str = "e4m3",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
    want_h: bool = False,
    out_dtype: torch.dtype = None,
):
    """ExpertMLP.forward (moe.py:190-193) for all local experts at once.

    x_sorted [T, H] rows sorted by expert, or those rows already as 1x128
    codes (a QTensor with tile-major scales, e.g. the received rows of
    ep.unpack_dispatch; out_dtype then defaults to bf16), offsets int32 [E+1];
    gate_up is
    interleave_gate_up()'s (codes, scales, nan) of [E, 2I, Kp], down is
    quantize_expert_weights()'s (codes, scales, nan) of [E, H, Ip].  Three
    kernels: the 1x128 quantization of x, the gate/up GEMM with SwiGLU and the
    1x128 quantization of h in its epilogue, the down GEMM.  Both projections
    read one quantization of x (the reference quantizes x once per Linear;
    with round to nearest the codes are the same).  Returns out [T, H] (and h
    when want_h)."""
    gu_codes, gu_scales, gu_nan = gate_up
    d_codes, d_scales, d_nan = down
    if isinstance(x_sorted, ops.QTensor):
        qx = x_sorted
        out_dtype = out_dtype or torch.bfloat16
    else:
        qx = ops.quant_tile_1x128(x_sorted, fmt=fmt, bits=bits, rounding=rounding, seed=seed, offset=offset,
                                  want_nan_rows=True)
        out_dtype = out_dtype or x_sorted.dtype
    h, qh = ops.gemm_swiglu_quant(qx, gu_codes, gu_scales, offsets=offsets, fmt=fmt, bits=bits, rounding=rounding,
                                  seed=seed, offset=offset + 1, want_h=want_h, want_nan_rows=True,
                                  b_nan_rows=gu_nan)
    out = ops.gemm_grouped_blockscaled(qh, d_codes, d_scales, offsets, N=d_codes.shape[1], out_dtype=out_dtype,
                                       b_nan_rows=d_nan)
    return (out, h) if want_h else out


def combine_rows(y: torch.Tensor, routing: ExpertRouting, expert_ids: torch.Tensor, topk_w: torch.Tensor,
                 n_tokens: int) -> torch.Tensor:
    """out[t] = sum over token t's slots, in ascending expert id, of
    y[pos[t*k + s]] * topk_w[t, s], formed as the reference's expert loop forms
    it (moe.py:1087-1088, :489-490: `output[token_indices] += expert_out *
    weights`, each product and each sum rounded to its torch dtype).  y [rows,
    H] holds the expert outputs in expert order, in the output dtype."""
    ops._require_device(y)
    if y.dim() != 2 or y.stride(-1) != 1:
        raise ValueError("y must be a row-major [rows, H] tensor")
    if expert_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError("expert_ids must be int32 or int64")
    k = routing.top_k
    if expert_ids.numel() != n_tokens * k or topk_w.numel() != n_tokens * k:
        raise ValueError("expert_ids and topk_w must be [tokens, top_k]")
    H = y.shape[1]
    out = torch.empty((n_tokens, H), dtype=y.dtype, device=y.device)
    ids = expert_ids.contiguous()
    w = topk_w.contiguous()
    _lib.call("ntlb_moe_combine_rows", y.data_ptr(), y.stride(0), y.shape[0], routing.pos.data_ptr(), ids.data_ptr(),
              1 if ids.dtype == torch.int64 else 0, w.data_ptr(), ops._dtype_code(w.dtype), n_tokens, k, H,
              out.data_ptr(), ops._dtype_code(out.dtype), out.stride(0), ops._stream())
    return out


def local_moe_forward(
    tokens: torch.Tensor,
    expert_ids: torch.Tensor,
    topk_w: torch.Tensor,
    gate_up,
    down,
    *,
    n_experts: int,
    fmt: str = "e4m3",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
    routing: Optional[ExpertRouting] = None,
):
    """The single-rank routed expert loop (moe.py:1062-1093, LocalRoutedMoE
    :476-491 without capacity drop) for all local experts at once: returns
    the token outputs [T, H] in tokens.dtype.

    Kernels: the routing sort (skipped when `routing` is given), the 1x128
    quantization of the token rows gathered by expert (each token row read
    once), the gate/up GEMM with SwiGLU and h's 1x128 quantization in its
    epilogue, the down GEMM, and the weighted combine into token order.  gate_up
    and down are as for expert_mlp()."""
    if routing is None:
        routing = route_by_expert(expert_ids, n_experts)
    qx = ops.quant_tile_1x128_fanout(tokens, routing.pos, routing.top_k, routing.rows, fmt=fmt, bits=bits,
                                     rounding=rounding, seed=seed, offset=offset, want_nan_rows=True)
    y = expert_mlp(qx, routing.offsets, gate_up, down, fmt=fmt, bits=bits, rounding=rounding, seed=seed,
                   offset=offset, out_dtype=tokens.dtype)
    return combine_rows(y, routing, expert_ids, topk_w, tokens.shape[0])
