"""The reference's emulated low-bit linear as torch CPU ops: test infrastructure.

This module is a CPU restatement of nano-train's emulated backend, written as
the torch op sequence the reference runs, so that `bench.py` can time that
path on the host's cores next to the GPU figures (its `cpu_baseline`) and
tests can compare it with the C oracle.  Nothing in the product package
imports it.

Restated:
  _round_values / _stochastic_round   te_backend.py:61-71
  _safe_scale                         te_backend.py:74-79
  _tile_quant_dequant                 te_backend.py:82-110   (gr=1, gc=128)
  _block_quant_dequant                te_backend.py:113-149  (gr=gc=128; tiles for non-2-D)
  _quantize_dequantize_with_granularity  te_backend.py:152-204
  _ste_fake_quantize                  te_backend.py:40-58
  EmulatedLowBitBackend.linear        te_backend.py:229-260 (forward; autograd gives the STE backward)
  _dequantize_nf4_persistent          layers.py:142-184 (codebook gather, scale, cast)

Every granularity is one "grouped" fake quantization: the 2-D operand, zero
padded to whole groups, viewed as [R/gr, gr, K/gc, gc]; the amax over each
(gr x gc) group, scale = safe(amax / qmax), q = clamp(round(x / scale)), dq =
q * scale.  The values are those of the reference's reshapes (a group's
amax, divide, round, clamp and multiply do not depend on how the group is
laid out).  Stochastic rounding draws from torch.rand_like, as the reference
does (its own unseeded stream, not the seeded Philox contract of the
kernels): use it for timing; parity pins use round to nearest.

Pinned by tests/test_torch_emulated_pins.py against the C oracle: codes-equivalent
dequantized values bit for bit for every granularity (with NaN, inf, zero
tiles and ragged shapes), and the linear forward and its autograd gradients
against float64 products of those values.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F


def _qmax(bits: int) -> int:
    return (1 << (bits - 1)) - 1  # te_backend.py:98


def _round(v: torch.Tensor, rounding: str) -> torch.Tensor:
    if rounding == "stochastic":
        u = torch.rand_like(v)
        return torch.where(v >= 0, torch.floor(v + u), torch.ceil(v - u))
    return torch.round(v)


def grouped_qdq(x_f: torch.Tensor, *, bits: int, gr: int, gc: int, rounding: str = "nearest") -> torch.Tensor:
    """fp32 dq of a 2-D fp32 tensor with one scale per (gr x gc) group."""
    R, K = x_f.shape
    gr = max(1, min(gr, max(R, 1)))
    gc = max(1, min(gc, max(K, 1)))
    Rp, Kp = -(-R // gr) * gr, -(-K // gc) * gc
    xp = F.pad(x_f, (0, Kp - K, 0, Rp - R)) if (Rp, Kp) != (R, K) else x_f
    g = xp.reshape(Rp // gr, gr, Kp // gc, gc)
    qmax = _qmax(bits)
    scale = g.abs().amax(dim=(1, 3), keepdim=True) / float(qmax)
    scale = torch.where(torch.isfinite(scale) & (scale > 0), scale, torch.ones_like(scale))
    q = torch.clamp(_round(g / scale, rounding), min=-qmax, max=qmax)
    dq = (q * scale).reshape(Rp, Kp)
    return dq[:R, :K] if (Rp, Kp) != (R, K) else dq


def _tensor_scale_first(x_f: torch.Tensor, bits: int) -> torch.Tensor:
    """_ste_fake_quantize's dq: per tensor, amax checked before the divide, round to nearest."""
    qmax = _qmax(bits)
    amax = x_f.abs().amax()
    scale = amax / float(qmax) if bool(torch.isfinite(amax)) and float(amax) > 0 else x_f.new_tensor(1.0)
    return torch.clamp(torch.round(x_f / scale), min=-qmax, max=qmax) * scale


def quantize_dequantize(x: torch.Tensor, *, bits: int, granularity: str, rounding: str,
                        channel_axis: int) -> torch.Tensor:
    """te_backend.py:152-204: the dequantized operand, cast back to x.dtype."""
    if x.numel() == 0:
        return x
    x_f = x.float()
    if granularity == "tensor":
        x2 = x_f.reshape(1, -1)
        dq = grouped_qdq(x2, bits=bits, gr=1, gc=x2.shape[1], rounding=rounding)
    elif granularity == "channel":
        axis = channel_axis if channel_axis >= 0 else x_f.dim() + channel_axis
        xm = x_f.movedim(axis, 0).reshape(x_f.shape[axis], -1)  # one row per channel
        dq = grouped_qdq(xm, bits=bits, gr=1, gc=xm.shape[1], rounding=rounding)
        dq = dq.reshape(x_f.movedim(axis, 0).shape).movedim(0, axis)
    elif granularity == "tile_1x128" or (granularity == "block_128x128" and x_f.dim() != 2):
        x2 = x_f.reshape(-1, x_f.shape[-1])
        dq = grouped_qdq(x2, bits=bits, gr=1, gc=128, rounding=rounding)
    elif granularity == "block_128x128":
        dq = grouped_qdq(x_f, bits=bits, gr=128, gc=128, rounding=rounding)
    else:
        dq = _tensor_scale_first(x_f, bits)
    return dq.reshape(x.shape).to(dtype=x.dtype)


def emulated_linear(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor], *, bits: int = 8,
                    act: str = "tile_1x128", wgt: str = "block_128x128", rounding: str = "nearest") -> torch.Tensor:
    """te_backend.py:229-260: straight-through fake quantization of both
    operands, then an fp32 F.linear cast back to x.dtype.  Differentiable:
    its autograd is the reference's STE backward."""
    x_dq = quantize_dequantize(x, bits=bits, granularity=act, rounding=rounding, channel_axis=-1)
    w_dq = quantize_dequantize(w, bits=bits, granularity=wgt, rounding=rounding, channel_axis=0)
    x_q = x + (x_dq - x).detach()
    w_q = w + (w_dq - w).detach()
    y = F.linear(x_q.to(torch.float32), w_q.to(torch.float32), None if b is None else b.to(torch.float32))
    return y.to(dtype=x.dtype)


def nf4_dequantize(packed: torch.Tensor, scales: torch.Tensor, *, numel: int, block: int,
                   dtype: torch.dtype) -> torch.Tensor:
    """layers.py:142-184: unpack the nibbles (even element low), codebook value
    times its block's fp32 scale, cast to dtype."""
    lo = packed & 0x0F
    hi = packed >> 4
    idx = torch.stack((lo, hi), dim=-1).reshape(-1)[:numel].long()
    from oracle.oracle import NF4_CODEBOOK  # the codebook of layers.py:62-82

    cb = torch.from_numpy(NF4_CODEBOOK.astype("float32"))
    vals = cb[idx] * scales.reshape(-1).repeat_interleave(block)[:numel]
    return vals.to(dtype)


class _LinearFwd32Ste(torch.autograd.Function):
    """A Linear whose forward multiplies fp32 q * s operands (the blockwise
    GEMM's numerics) and whose backward is the reference's straight-through
    gradient over its bf16(q * s) operands (te_backend.py:250-259 under
    autograd): dX = dY . W_q, dW = dY^T . X_q, in fp32, cast to the input dtypes."""

    @staticmethod
    def forward(ctx, x, w, x_dq32, w_dq32, x_q, w_q):
        ctx.save_for_backward(x_q, w_q)
        ctx.dts = (x.dtype, w.dtype)
        return F.linear(x_dq32, w_dq32).to(x.dtype)

    @staticmethod
    def backward(ctx, dy):
        x_q, w_q = ctx.saved_tensors
        dyf = dy.float()
        dx = (dyf @ w_q.float()).to(ctx.dts[0])
        dw = (dyf.t() @ x_q.float()).to(ctx.dts[1])
        return dx, dw, None, None, None, None


def _linear_for_moe(x: torch.Tensor, w: torch.Tensor, *, forward: str, qdq) -> torch.Tensor:
    """One expert Linear: x quantized per 1x128 tile, w per 128x128 block
    (qdq(t_fp32, gr, gc) gives the fp32 dq values)."""
    x32 = qdq(x.float(), 1, 128)
    w32 = qdq(w.float(), 128, 128)
    x_q = x + (x32.to(x.dtype) - x).detach()
    w_q = w + (w32.to(w.dtype) - w).detach()
    if forward == "reference":
        # te_backend.py:250-260
        return F.linear(x_q.to(torch.float32), w_q.to(torch.float32)).to(x.dtype)
    return _LinearFwd32Ste.apply(x, w, x32, w32, x_q.detach(), w_q.detach())


class _ValueOf(torch.autograd.Function):
    """`value` in the forward, the gradient of `computed` in the backward."""

    @staticmethod
    def forward(ctx, computed, value):
        return value.clone()

    @staticmethod
    def backward(ctx, grad):
        return grad, None


def local_moe_loop(tokens: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor, w_gate_up: torch.Tensor,
                   w_down: torch.Tensor, *, capacity: int = 0, forward: str = "reference", bits: int = 8,
                   qdq=None, gate_up_values=None) -> torch.Tensor:
    """The reference's single-rank routed expert loop as torch CPU ops, with
    autograd: moe.py:1062-1093 (LocalRoutedMoE.forward :476-491), each expert
    an ExpertMLP (moe.py:146-193: silu(gate_proj(x)) * up_proj(x) -> down_proj)
    of emulated low-bit Linears, round to nearest.

    w_gate_up [E, 2I, H] holds each expert's gate and up weights in 128-row
    blocks, alternating (gate block t, up block t); w_down [E, H, I].
    forward="reference": each Linear is EmulatedLowBitBackend.linear (bf16(q*s)
    operands, te_backend.py:229-260) with 1x128 activation tiles and 128x128
    weight blocks; forward="fp32_dq": the forward multiplies fp32 q * s
    operands (the blockwise-scaled GEMM's numerics) while the backward keeps
    the reference's straight-through gradients.  qdq(t_fp32_2d, gr, gc)
    quantizes with one scale per (gr x gc) group and returns the fp32 dq
    values; the default is the reference's int grid (grouped_qdq).
    gate_up_values(e) -> (gate, up) replaces the forward values of expert e's
    two projections (its rows in the loop's order) while their gradients stay
    those of the Linears: the same bf16 projections as another implementation
    whose fp32 sums run in another order, so that the re-quantization of h
    does not turn their last-bit differences into whole code steps."""
    if qdq is None:
        qdq = lambda t, gr, gc: grouped_qdq(t, bits=bits, gr=gr, gc=gc)
    T, H = tokens.shape
    E, N2, _ = w_gate_up.shape
    I = N2 // 2
    output = torch.zeros_like(tokens)
    v = w_gate_up.reshape(E, I // 128, 2, 128, H)
    for e in range(E):
        selected = (topk_idx == e).nonzero(as_tuple=False)
        if selected.numel() == 0:
            continue
        token_indices = selected[:, 0]
        slot_indices = selected[:, 1]
        sort_weights = topk_w[token_indices, slot_indices].detach()
        if capacity > 0 and token_indices.numel() > capacity:
            keep_rel = torch.topk(sort_weights, k=capacity, sorted=True).indices
            token_indices = token_indices[keep_rel]
            slot_indices = slot_indices[keep_rel]
        x = tokens[token_indices]
        wg = v[e, :, 0].reshape(I, H)
        wu = v[e, :, 1].reshape(I, H)
        lin = lambda a, b: _linear_for_moe(a, b, forward=forward, qdq=qdq)
        g, u = lin(x, wg), lin(x, wu)
        if gate_up_values is not None:
            gv, uv = gate_up_values(e)
            g, u = _ValueOf.apply(g, gv), _ValueOf.apply(u, uv)
        gated = F.silu(g) * u
        expert_out = lin(gated, w_down[e])
        weights = topk_w[token_indices, slot_indices].unsqueeze(-1)
        output[token_indices] += expert_out * weights
    return output
