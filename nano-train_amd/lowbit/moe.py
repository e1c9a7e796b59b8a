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
import math
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
    or -1 when a capacity dropped it; inv[row] the assignment of a row; rows
    of one expert keep assignment order, as the reference's
    (topk_indices == e).nonzero() lists them, or under a capacity the kept
    rows highest routing weight first (torch.topk(sorted=True)).  offsets
    int32 [E+1] is the token-offset table of the grouped GEMMs; counts int64
    [E] the rows per expert (the reference's token_counts / local_counts).
    Buffers over rows are sized for every assignment (`rows`); under a
    capacity the rows past offsets[E] are unused, so no host sync is needed."""

    pos: torch.Tensor  # int32 [T*top_k]
    inv: torch.Tensor  # int32 [T*top_k]
    counts: torch.Tensor  # int64 [E]
    offsets: torch.Tensor  # int32 [E+1]
    top_k: int
    capacity: int = 0

    @property
    def rows(self) -> int:
        return self.pos.numel()

    def dropped(self) -> int:
        """Assignments a capacity dropped (moe.py:1082; a device-to-host read)."""
        return self.rows - int(self.counts.sum().item())


def compute_capacity(capacity_factor: float, num_tokens: int, top_k: int, num_experts: int) -> int:
    """Per-expert capacity of LocalRoutedMoE._compute_capacity (moe.py:432-439):
    ceil(capacity_factor * tokens * top_k / experts), at least 1; 0 tokens -> 0."""
    if capacity_factor <= 0:
        raise ValueError("capacity_factor must be positive")
    if num_tokens <= 0:
        return 0
    expected = (num_tokens * top_k) / float(num_experts)
    return max(int(math.ceil(capacity_factor * expected)), 1)


def route_by_expert(expert_ids: torch.Tensor, n_experts: int, *, capacity: int = 0,
                    topk_w: Optional[torch.Tensor] = None) -> ExpertRouting:
    """One stable counting sort of expert_ids [T, k] (int32 or int64) by
    expert on the GPU (ntlb_ep_partition: three kernels, no host sync).

    capacity > 0 keeps, per expert with more rows than that, the `capacity`
    rows of highest routing weight topk_w [T, k], highest first
    (ntlb_moe_capacity_keep: moe.py:1077-1081 / :482-486,
    torch.topk(sort_weights, k=capacity, sorted=True); equal weights keep
    row order)."""
    from . import ep

    if expert_ids.dim() != 2:
        raise ValueError("expert_ids must be [tokens, top_k]")
    pos, inv, counts, offsets = ep.partition(expert_ids.reshape(-1), divisor=1, buckets=n_experts)
    k = expert_ids.shape[1]
    if capacity <= 0:
        return ExpertRouting(pos, inv, counts, offsets, k)
    if topk_w is None or topk_w.shape != expert_ids.shape:
        raise ValueError("a capacity needs the routing weights topk_w [tokens, top_k]")
    ops._require_device(topk_w)
    w = topk_w.detach().contiguous()
    n = pos.numel()
    pos2 = torch.empty_like(pos)
    inv2 = torch.empty_like(inv)
    offsets2 = torch.empty_like(offsets)
    counts2 = torch.empty_like(counts)
    _lib.call("ntlb_moe_capacity_keep", inv.data_ptr(), offsets.data_ptr(), n_experts, n, n, w.data_ptr(),
              ops._dtype_code(w.dtype), capacity, pos2.data_ptr(), inv2.data_ptr(), offsets2.data_ptr(),
              counts2.data_ptr(), ops._stream())
    return ExpertRouting(pos2, inv2, counts2, offsets2, k, capacity)


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
    capacity: int = 0,
):
    """The single-rank routed expert loop (moe.py:1062-1093, LocalRoutedMoE
    :476-491) for all local experts at once, forward only: returns the token
    outputs [T, H] in tokens.dtype.  capacity > 0 drops, per expert, all but
    the `capacity` rows of highest routing weight (route_by_expert).

    Kernels: the routing sort (skipped when `routing` is given), the 1x128
    quantization of the token rows gathered by expert (each token row read
    once), the gate/up GEMM with SwiGLU and h's 1x128 quantization in its
    epilogue, the down GEMM, and the weighted combine into token order.  gate_up
    and down are as for expert_mlp()."""
    if routing is None:
        routing = route_by_expert(expert_ids, n_experts, capacity=capacity, topk_w=topk_w)
    qx = ops.quant_tile_1x128_fanout(tokens, routing.pos, routing.top_k, routing.rows, fmt=fmt, bits=bits,
                                     rounding=rounding, seed=seed, offset=offset, want_nan_rows=True)
    y = expert_mlp(qx, routing.offsets, gate_up, down, fmt=fmt, bits=bits, rounding=rounding, seed=seed,
                   offset=offset, out_dtype=tokens.dtype)
    return combine_rows(y, routing, expert_ids, topk_w, tokens.shape[0])


def stack_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """Gate and up weights [E, I, H] (the experts' gate_proj / up_proj,
    moe.py:160-177) as the one [E, 2I, H] tensor that local_moe() trains:
    128-row blocks alternating gate block t and up block t, the row order of
    interleave_gate_up()'s codes.  A copy; split_gate_up() gives the two back
    as views."""
    if w_gate.shape != w_up.shape or w_gate.dim() != 3:
        raise ValueError("gate and up weights must both be [E, I, H]")
    E, I, H = w_gate.shape
    if I % 128:
        raise ValueError(f"intermediate size {I} must be a multiple of 128")
    nb = I // 128
    return torch.stack([w_gate.reshape(E, nb, 128, H), w_up.reshape(E, nb, 128, H)], dim=2).reshape(E, 2 * I, H)


def split_gate_up(w_gate_up: torch.Tensor):
    """(gate, up) views [E, I/128, 128, H] of stack_gate_up()'s layout."""
    E, N2, H = w_gate_up.shape
    v = w_gate_up.reshape(E, N2 // 256, 2, 128, H)
    return v[:, :, 0], v[:, :, 1]


def _dequant_experts(codes: torch.Tensor, scales: torch.Tensor, grid: int, K: int) -> torch.Tensor:
    """bf16(q * s) of quantize_expert_weights' codes [E, N, Kp] and 128x128
    block scales [E, N/128, Kp/128], as [E, N, K]"""
    E, N, Kp = codes.shape
    q = QTensor(codes.reshape(E * N, Kp), scales.reshape(-1).contiguous(), scales.shape[2], 1, 7, grid, E * N, K,
                None, None)
    return ops.dequant(q, out_dtype=torch.bfloat16).reshape(E, N, K)


class _LocalMoE(torch.autograd.Function):
    """The single-rank expert loop with its backward on HIP kernels.

    Forward: local_moe_forward's kernels, with the two projections' bf16
    outputs kept for the SwiGLU backward.  Backward, the autograd of the
    reference's loop (moe.py:1062-1093: tokens[token_indices] -> ExpertMLP ->
    `output[token_indices] += expert_out * weights`, each expert Linear the
    straight-through estimator of te_backend.py:250-259):
      ntlb_moe_combine_backward   dY rows = d_out[token] * w, and the
                                  routing-weight gradient sum_H d_out * y;
      ntlb_gemm_grouped_ste_dgrad dH = dY . bf16(dq(W_down[e])) per expert;
      ntlb_swiglu_backward        d_gate, d_up through F.silu(gate) * up;
      ntlb_gemm_grouped_ste_dgrad_gate_up  dX rows = bf16(d_gate . W_gate_q) +
                                  bf16(d_up . W_up_q), added in bf16 (x feeds
                                  both Linears);
      ntlb_moe_token_grad         the token gradient: each token's rows in
                                  descending expert id, each add rounded
                                  (autograd's order over the loop);
      ntlb_gemm_grouped_ste_wgrad dW_down[e] = dY^T . bf16(dq(h)), dW_gate_up[e]
                                  = [d_gate | d_up]^T . bf16(dq(x)) over the
                                  expert's rows only."""

    @staticmethod
    def forward(ctx, tokens, topk_w, w_gate_up, w_down, expert_ids, n_experts, capacity, cfg):
        fmt, bits, rounding, seed, offset = cfg
        T, H = tokens.shape
        E, N2, _ = w_gate_up.shape
        I = N2 // 2
        routing = route_by_expert(expert_ids, n_experts, capacity=capacity, topk_w=topk_w)
        gu_codes, gu_scales, gu_nan = quantize_expert_weights(w_gate_up.detach(), fmt=fmt, bits=bits,
                                                              rounding=rounding, seed=seed, offset=offset + 2)
        d_codes, d_scales, d_nan = quantize_expert_weights(w_down.detach(), fmt=fmt, bits=bits, rounding=rounding,
                                                           seed=seed, offset=offset + 3)
        qx = ops.quant_tile_1x128_fanout(tokens.detach(), routing.pos, routing.top_k, routing.rows, fmt=fmt,
                                         bits=bits, rounding=rounding, seed=seed, offset=offset, want_nan_rows=True)
        train = any(ctx.needs_input_grad[:4])
        # stochastic rounding: the backward multiplies the reference's operands
        # t + (t_dq - t), which differ from bf16(q * s) (te_backend.py:250-251)
        sr = train and rounding == "stochastic"
        gu = torch.empty((routing.rows, N2), dtype=torch.bfloat16, device=tokens.device) if train else None
        h, qh = ops.gemm_swiglu_quant(qx, gu_codes, gu_scales, offsets=routing.offsets, fmt=fmt, bits=bits,
                                      rounding=rounding, seed=seed, offset=offset + 1, want_h=sr,
                                      want_nan_rows=True, b_nan_rows=gu_nan, gu_out=gu)
        y = ops.gemm_grouped_blockscaled(qh, d_codes, d_scales, routing.offsets, N=H, out_dtype=tokens.dtype,
                                         b_nan_rows=d_nan)
        out = combine_rows(y, routing, expert_ids, topk_w.detach(), T)
        ctx.meta = (T, H, E, I, routing.top_k, routing.rows, qx.grid, qx.s_col, qh.s_col, tokens.dtype,
                    w_gate_up.dtype, w_down.dtype)
        ctx.sr = sr
        if sr:
            bf = torch.bfloat16
            # row -> token (the rows past the kept count hold -1: any in-range
            # token serves them, the GEMMs never read those rows)
            rows_tok = (routing.inv.clamp(0, T * routing.top_k - 1) // routing.top_k).long()
            xq = ops.ste_value(tokens.detach().index_select(0, rows_tok), ops.dequant(qx, out_dtype=bf))
            hq = ops.ste_value(h, ops.dequant(qh, out_dtype=bf))
            wguq = ops.ste_value(w_gate_up.detach(), _dequant_experts(gu_codes, gu_scales, qx.grid, H))
            wdq = ops.ste_value(w_down.detach(), _dequant_experts(d_codes, d_scales, qx.grid, I))
            ctx.save_for_backward(routing.pos, routing.inv, routing.counts, routing.offsets, expert_ids,
                                  topk_w.detach(), xq, gu, hq, y, wguq, wdq)
        else:
            ctx.save_for_backward(routing.pos, routing.inv, routing.counts, routing.offsets, expert_ids,
                                  topk_w.detach(), qx.codes, qx.scales, gu, qh.codes, qh.scales, y, gu_codes,
                                  gu_scales, d_codes, d_scales)
        return out

    @staticmethod
    def backward(ctx, d_out):
        T, H, E, I, k, R, grid, x_rp, h_rp, tdt, gudt, ddt = ctx.meta
        if ctx.sr:
            pos, inv, counts, offsets, expert_ids, topk_w, xq, gu, hq, y, wguq, wdq = ctx.saved_tensors
        else:
            (pos, inv, counts, offsets, expert_ids, topk_w, xc, xs, gu, hc, hs, y, gu_codes, gu_scales, d_codes,
             d_scales) = ctx.saved_tensors
        d_out = d_out.contiguous()
        dev = d_out.device
        routing = ExpertRouting(pos, inv, counts, offsets, k)
        # combine: dY rows (y's dtype) and the routing-weight gradient
        ld = ops.cdiv(H, 64) * 64  # the dgrad reads whole 64-column K steps: zero pad columns
        dyr = (torch.zeros if ld != H else torch.empty)((R, ld), dtype=y.dtype, device=dev)
        d_w = torch.empty(topk_w.shape, dtype=topk_w.dtype, device=dev)
        _lib.call("ntlb_moe_combine_backward", d_out.data_ptr(), d_out.stride(0), y.data_ptr(), y.stride(0),
                  ops._dtype_code(y.dtype), pos.data_ptr(), topk_w.data_ptr(), ops._dtype_code(topk_w.dtype), T, k, H,
                  dyr.data_ptr(), ld, d_w.data_ptr(), ops._stream())
        dyr = dyr[:, :H]
        # down projection, then the SwiGLU
        if ctx.sr:
            dh = ops.grouped_dgrad_dense(dyr, offsets, wdq, out_dtype=torch.bfloat16)
        else:
            dh = ops.grouped_ste_dgrad(dyr, offsets, d_codes, d_scales, grid=grid, K=I, out_dtype=torch.bfloat16)
        d_gu = torch.empty((R, 2 * I), dtype=torch.bfloat16, device=dev)
        _lib.call("ntlb_swiglu_backward", dh.data_ptr(), dh.stride(0), gu.data_ptr(), gu.stride(0), R, I,
                  d_gu.data_ptr(), d_gu.stride(0), ops._stream())
        d_tok = dw_gu = dw_down = None
        if ctx.needs_input_grad[0]:
            if ctx.sr:
                dxr = ops.grouped_dgrad_dense_gate_up(d_gu, offsets, wguq)
            else:
                dxr = ops.grouped_ste_dgrad_gate_up(d_gu, offsets, gu_codes, gu_scales, grid=grid, K=H)
            d_tok = torch.empty((T, H), dtype=tdt, device=dev)
            ids = expert_ids.contiguous()
            _lib.call("ntlb_moe_token_grad", dxr.data_ptr(), dxr.stride(0), ops._dtype_code(dxr.dtype),
                      pos.data_ptr(), ids.data_ptr(), 1 if ids.dtype == torch.int64 else 0, T, k, H,
                      d_tok.data_ptr(), d_tok.stride(0), ops._stream())
        if ctx.needs_input_grad[3]:
            if ctx.sr:
                dw_down = ops.grouped_wgrad_dense(dyr, offsets, hq, E, out_dtype=ddt)
            else:
                qh = QTensor(hc, hs, 1, h_rp, 0, grid, R, I, None, None)
                dw_down = ops.grouped_ste_wgrad(dyr, offsets, qh, E, out_dtype=ddt)
        if ctx.needs_input_grad[2]:
            if ctx.sr:
                dw_gu = ops.grouped_wgrad_dense(d_gu, offsets, xq, E, out_dtype=gudt)
            else:
                qx = QTensor(xc, xs, 1, x_rp, 0, grid, R, H, None, None)
                dw_gu = ops.grouped_ste_wgrad(d_gu, offsets, qx, E, out_dtype=gudt)
        return d_tok, (d_w if ctx.needs_input_grad[1] else None), dw_gu, dw_down, None, None, None, None


def local_moe(
    tokens: torch.Tensor,
    expert_ids: torch.Tensor,
    topk_w: torch.Tensor,
    w_gate_up: torch.Tensor,
    w_down: torch.Tensor,
    *,
    capacity: int = 0,
    fmt: str = "e4m3",
    bits: int = 8,
    rounding: str = "nearest",
    seed: int = 0,
    offset: int = 0,
) -> torch.Tensor:
    """The single-rank routed expert loop, trainable (moe.py:1062-1093,
    LocalRoutedMoE.forward :476-491, ExpertMLP.forward :190-193): returns the
    token outputs [T, H] and, under autograd, the gradients of the tokens,
    the routing weights and the expert weights.

    tokens bf16 [T, H]; expert_ids [T, k] int32/int64 and topk_w [T, k] (the
    router's topk_indices / topk_weights); w_gate_up bf16 [E, 2I, H] in
    stack_gate_up()'s row order; w_down bf16 [E, H, I]; I and H multiples of
    128.  capacity > 0 keeps per expert the `capacity` rows of highest
    routing weight (compute_capacity() gives the reference's value); the
    dropped assignments add nothing and get a zero routing-weight gradient.
    Forward arithmetic: the blockwise-scaled GEMMs (fp32 q * s operands);
    backward: the straight-through gradients over the reference's operands,
    t + (t_dq - t) in bf16 (te_backend.py:250-251): bf16(q * s), decoded from
    the codes inside the GEMMs, under round to nearest; under stochastic
    rounding, where the two differ, the operands themselves (ntlb_ste_value)
    on the grouped bf16 GEMMs.  Stochastic rounding quantizes x once for the
    gate and up projections (the reference's two Linears draw twice).  An
    expert that receives no rows gets a zero weight gradient (the reference's
    separate Linears would get none)."""
    if tokens.dim() != 2 or expert_ids.dim() != 2 or topk_w.shape != expert_ids.shape:
        raise ValueError("tokens must be [T, H], expert_ids and topk_w [T, k]")
    if tokens.dtype != torch.bfloat16 or w_gate_up.dtype != torch.bfloat16 or w_down.dtype != torch.bfloat16:
        raise TypeError("local_moe trains bf16 tokens and bf16 expert weights")
    E, N2, H = w_gate_up.shape
    if H != tokens.shape[1] or w_down.shape != (E, H, N2 // 2) or N2 % 256:
        raise ValueError(f"weights must be w_gate_up [E, 2I, H] (2I % 256 == 0) and w_down [E, H, I]; got "
                         f"{tuple(w_gate_up.shape)}, {tuple(w_down.shape)}")
    if expert_ids.shape[1] > 8:
        raise ValueError("local_moe supports top_k <= 8")
    return _LocalMoE.apply(tokens, topk_w, w_gate_up, w_down, expert_ids, E, int(capacity),
                           (fmt, bits, rounding, seed, offset))
