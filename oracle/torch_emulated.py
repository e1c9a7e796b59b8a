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
