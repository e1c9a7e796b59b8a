"""Expert-parallel dispatch wire format on the MI355X kernels.

nano-train's _dispatch_tokens (src/models/moe.py:795-863) sends, per
destination rank, the comm-quantized token rows (dequantized to bf16 before
the exchange), then token index, slot index, local expert index and routing
weight, each with its own all_to_all after a count exchange
(_build_send_partitions, moe.py:670-717).  Here every routed (token, slot)
assignment becomes one fixed-size record holding the row's 1x128 codes and
fp32 tile scales and its metadata (layout: include/ntlowbit.h,
ntlb_ep_record_bytes), so the exchange is one count all_to_all plus one byte
all_to_all, and the receiver hands the codes to the grouped GEMM without a
dequantize/re-quantize round trip.

  pack_dispatch     sender: destination order + records (kernels ntlb_ep_partition,
                    ntlb_ep_pack_records_grouped)
  exchange          the two all_to_alls (torch.distributed; one process per GPU)
  unpack_dispatch   receiver: rows grouped by local expert in arrival order, as
                    _run_local_experts selects them (moe.py:905-923), as a QTensor
                    for ops.gemm_grouped_blockscaled plus the metadata of
                    _DispatchedTokens (moe.py:49-58)
  pack_return       expert side of the combine: the expert outputs as records
                    back to their source ranks (ntlb_ep_pack_return)
  combine           source side: the returned records summed into the token
                    outputs with the routing weights (ntlb_ep_combine)

Capacity dropping (moe.py:919-923) keeps the top-capacity rows of an expert by
routing weight: capacity_order selects them, and unpack_dispatch gathers that
explicit record order.

Value records (wire="values", the only wire of the reference's `channel`
comm-quant, whose one scale per column a record's tile scales cannot hold)
carry the reference's wire values themselves: _comm_quant_dequant of the send
buffer, tensor + (dq - tensor) in the tokens' dtype, written by
ntlb_ep_pack_values / ntlb_ep_pack_return_values, gathered by
ntlb_ep_unpack_values into dense rows (ExpertRows.values) and summed by
ntlb_ep_combine_values.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch

from . import ops
from . import _lib
from ._lib import call, lib
from .ops import QTensor, cdiv

KEY_INT32, KEY_INT64 = 0, 1


def record_layout(H: int):
    """(record bytes, scale offset, metadata offset) of a row of H values."""
    R = int(lib().ntlb_ep_record_bytes(H))
    s_off = cdiv(H, 128) * 128  # whole tiles of codes, zero past H
    return R, s_off, R - 32


def value_record_layout(H: int, dtype: torch.dtype):
    """(record bytes, metadata offset) of a value record of H values of dtype."""
    R = int(lib().ntlb_ep_value_record_bytes(H, ops._dtype_code(dtype)))
    return R, R - 32


def partition(keys: torch.Tensor, *, divisor: int, buckets: int):
    """Stable counting sort of keys // divisor into buckets.

    Returns (pos, inv, counts, offsets): pos[i] = place of i in bucket order,
    inv[pos[i]] = i, counts int64 [buckets], offsets int32 [buckets + 1]."""
    ops._require_device(keys)
    if keys.dtype not in (torch.int32, torch.int64):
        raise TypeError("keys must be int32 or int64")
    keys = keys.contiguous().reshape(-1)
    kd = KEY_INT64 if keys.dtype == torch.int64 else KEY_INT32
    return _partition(keys.data_ptr(), kd, keys.element_size(), keys.numel(), divisor, buckets, keys.device)


def _partition(ptr: int, key_dtype: int, key_stride: int, n: int, divisor: int, buckets: int, dev):
    pos = torch.empty(n, dtype=torch.int32, device=dev)
    inv = torch.empty(n, dtype=torch.int32, device=dev)
    counts = torch.empty(buckets, dtype=torch.int64, device=dev)
    offsets = torch.empty(buckets + 1, dtype=torch.int32, device=dev)
    ws = torch.empty(max(cdiv(n, 256) * buckets, 1), dtype=torch.int32, device=dev)
    call("ntlb_ep_partition", ptr, key_dtype, key_stride, n, divisor, buckets, pos.data_ptr(), inv.data_ptr(),
         counts.data_ptr(), offsets.data_ptr(), ws.data_ptr(), ws.numel(), ops._stream())
    return pos, inv, counts, offsets


@dataclass
class SendBuffer:
    records: torch.Tensor  # uint8 [T*K, R], destination-major
    counts: torch.Tensor  # int64 [ep_size] (device)
    H: int
    value_dtype: Optional[torch.dtype] = None  # value records of this dtype; None: code records


def _payload_mode(granularity: Optional[str], fmt: Optional[str], scale_rule: Optional[int], H: int,
                  wire: Optional[str] = None):
    """(grid code, scale rule, group columns or None, value records?) of a
    record payload.

    granularity None: per-row 1x128 tiles (fmt e4m3 by default) in code
    records.  Otherwise the reference's comm-quant granularity
    (moe.py:107-140): tile_1x128 and block_128x128 give one scale per
    128-column strip over all rows, tensor one scale, channel one per column;
    the reference quantizes on the int grid with the scale rule that checks
    the amax before dividing.  wire "codes" (the default but for channel)
    sends codes and tile scales, "values" (the default and only wire for
    channel) the reference's wire values."""
    if wire not in (None, "codes", "values"):
        raise ValueError(f"wire {wire!r}: 'codes' or 'values'")
    if granularity is None:
        if wire == "values":
            raise ValueError("value records carry the reference's comm-quant: name its granularity")
        return ops.grid_code(fmt or "e4m3"), (0 if scale_rule is None else scale_rule), None, False
    if granularity in ("tile_1x128", "block_128x128"):
        gc = 128
    elif granularity == "tensor":
        gc = H
    elif granularity == "channel":
        if wire == "codes":
            raise ValueError("granularity 'channel': one scale per column does not fit a code record's tile "
                             "scales; use wire='values'")
        gc, wire = 1, "values"
    else:
        raise ValueError(f"granularity {granularity!r}: tile_1x128, block_128x128, tensor or channel")
    rule = _lib.SCALE_BEFORE_DIVIDE if scale_rule is None else scale_rule
    return ops.grid_code(fmt or "int_grid"), rule, gc, wire == "values"


def _group_amax(x: torch.Tensor, gc: Optional[int]):
    """Per-group |x| maxima (int32 bits) over all rows of x [n, H], or None."""
    if gc is None or x.shape[0] == 0:
        return None
    n, H = x.shape
    amax = torch.zeros(cdiv(H, gc), dtype=torch.int32, device=x.device)
    call("ntlb_amax_grouped", x.data_ptr(), ops._dtype_code(x.dtype), n, H, x.stride(0), n, gc, amax.data_ptr(),
         ops._stream())
    return amax


def pack_dispatch(tokens: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor, *, experts_per_rank: int,
                  ep_size: int, fmt: Optional[str] = None, bits: int = 8, rounding: str = "nearest", seed: int = 0,
                  offset: int = 0, scale_rule: Optional[int] = None, granularity: Optional[str] = None,
                  wire: Optional[str] = None) -> SendBuffer:
    """The send side of _dispatch_tokens (moe.py:795-814) as records.

    Assignment a = t*K + k goes to rank topk_idx[t, k] // experts_per_rank;
    within a rank, assignments keep their order (the reference's boolean
    masks).  Each record carries token t's row quantized with the
    stochastic-rounding element index p*H + column of its send position p,
    and (t, k, local expert, weight).  The payload is per-row 1x128 tiles
    (granularity None, e4m3 by default), or the reference's own comm-quant of
    the send buffer (granularity tile_1x128 / block_128x128 / tensor: int-grid
    codes with strip or tensor scales, the codes and scales
    _comm_quant_dequant computes; with wire="values", and always for
    channel, value records holding the values _comm_quant_dequant returns)."""
    ops._require_device(tokens, topk_idx, topk_w)
    if tokens.dim() != 2 or topk_idx.shape != topk_w.shape or topk_idx.dim() != 2 \
            or topk_idx.shape[0] != tokens.shape[0]:
        raise ValueError("tokens [T, H], topk_idx and topk_w [T, K]")
    T, H = tokens.shape
    K = topk_idx.shape[1]
    idx = topk_idx.contiguous()
    w = topk_w.contiguous()
    if tokens.stride(-1) != 1 or tokens.stride(0) % 8 or tokens.data_ptr() % 16:
        tokens = tokens.contiguous()
    grid, rule, gc, values = _payload_mode(granularity, fmt, scale_rule, H, wire)
    pos, _, counts, _ = partition(idx, divisor=experts_per_rank, buckets=ep_size)
    amax = _group_amax(tokens, gc)
    if values:
        R, _ = value_record_layout(H, tokens.dtype)
        records = torch.empty((T * K, R), dtype=torch.uint8, device=tokens.device)
        if T * K:
            call("ntlb_ep_pack_values", tokens.data_ptr(), ops._dtype_code(tokens.dtype), T, H, tokens.stride(0),
                 pos.data_ptr(), idx.data_ptr(), KEY_INT64 if idx.dtype == torch.int64 else KEY_INT32, w.data_ptr(),
                 ops._dtype_code(w.dtype), K, experts_per_rank, amax.data_ptr(), gc, grid, (1 << (bits - 1)) - 1,
                 ops.rounding_code(rounding), rule, seed, offset, records.data_ptr(), ops._stream())
        return SendBuffer(records, counts, H, tokens.dtype)
    R, _, _ = record_layout(H)
    records = torch.empty((T * K, R), dtype=torch.uint8, device=tokens.device)
    call("ntlb_ep_pack_records_grouped", tokens.data_ptr(), ops._dtype_code(tokens.dtype), T, H, tokens.stride(0),
         pos.data_ptr(), idx.data_ptr(), KEY_INT64 if idx.dtype == torch.int64 else KEY_INT32, w.data_ptr(),
         ops._dtype_code(w.dtype), K, experts_per_rank, None if amax is None else amax.data_ptr(), gc or 0, grid,
         (1 << (bits - 1)) - 1, ops.rounding_code(rounding), rule, seed, offset, records.data_ptr(), ops._stream())
    return SendBuffer(records, counts, H)


def exchange(send: SendBuffer, group=None):
    """One count all_to_all and one byte all_to_all (replacing the 1 + 1 + 4
    collectives of moe.py:720-863).  Returns (received records, counts per
    source rank)."""
    import torch.distributed as dist

    R = send.records.shape[1]
    recv_counts = torch.empty_like(send.counts)
    dist.all_to_all_single(recv_counts, send.counts, group=group)
    sc = [int(c) for c in send.counts.tolist()]
    rc = [int(c) for c in recv_counts.tolist()]
    recv = torch.empty((sum(rc), R), dtype=torch.uint8, device=send.records.device)
    dist.all_to_all_single(recv.view(-1), send.records.view(-1), output_split_sizes=[c * R for c in rc],
                           input_split_sizes=[c * R for c in sc], group=group)
    return recv, rc


@dataclass
class ExpertRows:
    """Received rows in expert order: the operand of the grouped GEMM and the
    per-row metadata of _DispatchedTokens."""

    q: Optional[QTensor]  # codes [n, ldc] + tile-major 1x128 scales, nan_rows (code records)
    offsets: torch.Tensor  # int32 [local_experts + 1]
    counts: torch.Tensor  # int64 [local_experts]
    token_idx: torch.Tensor  # int32 [n]
    slot_idx: torch.Tensor  # int32 [n]
    src_rank: torch.Tensor  # int32 [n]
    weight: torch.Tensor  # fp32 [n]
    order: torch.Tensor  # int32 [n]: received record of each row
    values: Optional[torch.Tensor] = None  # [n, H] in the records' dtype (value records)


def unpack_dispatch(records: torch.Tensor, recv_counts: Sequence[int], *, H: int, local_experts: int,
                    fmt: str = "e4m3", order: Optional[torch.Tensor] = None,
                    order_counts: Optional[Sequence[int]] = None,
                    value_dtype: Optional[torch.dtype] = None) -> ExpertRows:
    """Group the received records by local expert (stable in arrival order),
    or take the given record order (rows of expert e next to each other,
    order_counts[e] of them, e.g. from capacity_order), into codes + scales
    for the grouped GEMM, or, for value records of value_dtype, into the
    dense rows the reference's experts receive (recv_tokens, moe.py:816-824)."""
    ops._require_device(records)
    if value_dtype is not None:
        R, m_off = value_record_layout(H, value_dtype)
    else:
        R, _, m_off = record_layout(H)
    if records.dim() != 2 or records.shape[1] != R or records.dtype != torch.uint8:
        raise ValueError(f"records must be uint8 [n, {R}]")
    n = records.shape[0]
    if sum(int(c) for c in recv_counts) != n:
        raise ValueError("recv_counts must add up to the number of records")
    dev = records.device
    records = records.contiguous()
    if order is None:
        # keys: each record's local-expert int32, R bytes apart
        _, order, counts, offsets = _partition(records.data_ptr() + m_off + 8, KEY_INT32, R, n, 1, local_experts, dev)
    else:
        order = order.to(device=dev, dtype=torch.int32).contiguous()
        counts = offsets = None
        if order_counts is not None:
            if len(order_counts) != local_experts or sum(int(c) for c in order_counts) != order.numel():
                raise ValueError("order_counts needs one count per local expert, adding up to len(order)")
            counts = torch.tensor([int(c) for c in order_counts], dtype=torch.int64).to(dev, non_blocking=True)
            offsets = torch.tensor([0] + _cumsum(order_counts), dtype=torch.int32).to(dev, non_blocking=True)
    rows = order.numel()
    token_idx = torch.empty(rows, dtype=torch.int32, device=dev)
    slot_idx = torch.empty(rows, dtype=torch.int32, device=dev)
    src_rank = torch.empty(rows, dtype=torch.int32, device=dev)
    weight = torch.empty(rows, dtype=torch.float32, device=dev)
    # host memory: the entry point reads the prefix at the call (no copy to the device)
    recv_offsets = (ctypes.c_int64 * (len(recv_counts) + 1))(0, *_cumsum(recv_counts))
    if value_dtype is not None:
        values = torch.empty((rows, H), dtype=value_dtype, device=dev)
        call("ntlb_ep_unpack_values", records.data_ptr(), n, H, ops._dtype_code(value_dtype), order.data_ptr(), rows,
             ctypes.addressof(recv_offsets), len(recv_counts), values.data_ptr(), H, token_idx.data_ptr(),
             slot_idx.data_ptr(), src_rank.data_ptr(), weight.data_ptr(), ops._stream())
        return ExpertRows(None, offsets, counts, token_idx, slot_idx, src_rank, weight, order, values)
    T = cdiv(H, 128)
    ldc = T * 128
    rp = cdiv(max(rows, 1), 4) * 4
    codes = torch.empty((rows, ldc), dtype=torch.uint8, device=dev)  # whole tiles come from the records
    scales = torch.empty((T, rp), dtype=torch.float32, device=dev)
    nan_rows = torch.empty(rows, dtype=torch.int32, device=dev)
    call("ntlb_ep_unpack_records", records.data_ptr(), n, H, order.data_ptr(), rows, ctypes.addressof(recv_offsets),
         len(recv_counts), codes.data_ptr(), ldc, scales.data_ptr(), 1, rp, nan_rows.data_ptr(),
         token_idx.data_ptr(), slot_idx.data_ptr(), src_rank.data_ptr(), weight.data_ptr(), ops._stream())
    q = QTensor(codes, scales, 1, rp, 0, ops.grid_code(fmt), rows, H, nan_rows)
    return ExpertRows(q, offsets, counts, token_idx, slot_idx, src_rank, weight, order)


def pack_return(expert_out: torch.Tensor, rows: ExpertRows, *, ep_size: int, fmt: Optional[str] = None, bits: int = 8,
                rounding: str = "nearest", seed: int = 0, offset: int = 0, scale_rule: Optional[int] = None,
                granularity: Optional[str] = None, wire: Optional[str] = None) -> SendBuffer:
    """The expert side of the combine (moe.py:926-962) as records: row i of
    expert_out [n, H] (the rows of `rows`, in their order) goes back to rank
    rows.src_rank[i]; each destination's records keep the rows' order, which
    is expert order as send_back_features_parts builds it.  Records carry
    (token, slot, weight) and the payload as in pack_dispatch (granularity:
    the reference's comm-quant of send_back_features, over all n rows; value
    records for wire="values" and channel)."""
    ops._require_device(expert_out)
    if expert_out.dim() != 2 or expert_out.shape[0] != rows.token_idx.numel():
        raise ValueError("expert_out must be [rows, H], one row per received row")
    n, H = expert_out.shape
    if expert_out.stride(-1) != 1 or expert_out.stride(0) % 8 or expert_out.data_ptr() % 16:
        expert_out = expert_out.contiguous()
    grid, rule, gc, values = _payload_mode(granularity, fmt, scale_rule, H, wire)
    dev = expert_out.device
    src = rows.src_rank.to(dtype=torch.int32).contiguous()
    pos, _, counts, _ = _partition(src.data_ptr(), KEY_INT32, 4, n, 1, ep_size, dev)
    amax = _group_amax(expert_out, gc)
    if values:
        R, _ = value_record_layout(H, expert_out.dtype)
        records = torch.empty((n, R), dtype=torch.uint8, device=dev)
        if n:
            call("ntlb_ep_pack_return_values", expert_out.data_ptr(), ops._dtype_code(expert_out.dtype), n, H,
                 expert_out.stride(0), pos.data_ptr(), rows.token_idx.data_ptr(), rows.slot_idx.data_ptr(), None,
                 rows.weight.data_ptr(), amax.data_ptr(), gc, grid, (1 << (bits - 1)) - 1,
                 ops.rounding_code(rounding), rule, seed, offset, records.data_ptr(), ops._stream())
        return SendBuffer(records, counts, H, expert_out.dtype)
    R, _, _ = record_layout(H)
    records = torch.empty((n, R), dtype=torch.uint8, device=dev)
    call("ntlb_ep_pack_return", expert_out.data_ptr(), ops._dtype_code(expert_out.dtype), n, H, expert_out.stride(0),
         pos.data_ptr(), rows.token_idx.data_ptr(), rows.slot_idx.data_ptr(), None, rows.weight.data_ptr(),
         None if amax is None else amax.data_ptr(), gc or 0, grid, (1 << (bits - 1)) - 1,
         ops.rounding_code(rounding), rule, seed, offset, records.data_ptr(), ops._stream())
    return SendBuffer(records, counts, H)


def combine(records: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor, *, H: int, fmt: str = "e4m3",
            out_dtype: torch.dtype = torch.bfloat16, value_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """The source side of the combine (moe.py:1021-1027): the returned
    records summed into the token outputs [T, H] with their routing weights,
    as index_add_ into zeros sums them on the CPU (each product rounded to
    out_dtype, the products added in fp32 in ascending expert id per token,
    the sum rounded once).  fmt names the records'
    code grid (int_grid for the reference's comm-quant granularities);
    value_dtype marks value records of that dtype, each value rounded to
    out_dtype first (recv_back_features.to(tokens.dtype), moe.py:998-999)."""
    ops._require_device(records, topk_idx, topk_w)
    if value_dtype is not None:
        R, _ = value_record_layout(H, value_dtype)
    else:
        R, _, _ = record_layout(H)
    if records.dim() != 2 or records.shape[1] != R or records.dtype != torch.uint8:
        raise ValueError(f"records must be uint8 [n, {R}]")
    if topk_idx.dim() != 2 or topk_idx.shape != topk_w.shape:
        raise ValueError("topk_idx and topk_w [T, K]")
    T, K = topk_idx.shape
    idx = topk_idx.contiguous()
    w = topk_w.contiguous()
    records = records.contiguous()
    out = torch.empty((T, H), dtype=out_dtype, device=records.device)
    slot_map = torch.empty(max(T * K, 1), dtype=torch.int32, device=records.device)
    if value_dtype is not None:
        call("ntlb_ep_combine_values", records.data_ptr(), records.shape[0], H, ops._dtype_code(value_dtype),
             idx.data_ptr(), KEY_INT64 if idx.dtype == torch.int64 else KEY_INT32, w.data_ptr(),
             ops._dtype_code(w.dtype), T, K, out.data_ptr(), ops._dtype_code(out_dtype), H, slot_map.data_ptr(),
             ops._stream())
        return out
    call("ntlb_ep_combine", records.data_ptr(), records.shape[0], H, idx.data_ptr(),
         KEY_INT64 if idx.dtype == torch.int64 else KEY_INT32, w.data_ptr(), ops._dtype_code(w.dtype), T, K,
         ops.grid_code(fmt), out.data_ptr(), ops._dtype_code(out_dtype), H, slot_map.data_ptr(), ops._stream())
    return out


def capacity_order(rows: ExpertRows, capacity: int):
    """The rows _run_local_experts keeps under an expert capacity
    (moe.py:919-923): per local expert, the `capacity` rows of highest routing
    weight, highest first (torch.topk, sorted), or all rows in arrival order
    when there are no more than `capacity` (or capacity <= 0).  Returns (record
    order, kept count per expert) for unpack_dispatch(order=, order_counts=)."""
    if rows.offsets is None:
        raise ValueError("capacity_order needs rows grouped by unpack_dispatch (offsets known)")
    offs = [int(v) for v in rows.offsets.tolist()]
    parts, kept = [], []
    for e in range(len(offs) - 1):
        a, b = offs[e], offs[e + 1]
        sel = rows.order[a:b]
        if 0 < capacity < b - a:
            sel = sel[torch.topk(rows.weight[a:b], k=capacity, sorted=True).indices]
        parts.append(sel)
        kept.append(int(sel.numel()))
    order = torch.cat(parts) if parts else rows.order[:0]
    return order, kept


def _cumsum(xs: Sequence[int]) -> List[int]:
    out, acc = [], 0
    for x in xs:
        acc += int(x)
        out.append(acc)
    return out
