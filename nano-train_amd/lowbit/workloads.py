"""Synthetic inputs of the five benchmark configurations of this path.

Seeds follow s = 20260000 + config_id*100 + tensor_id, so every consumer
(tests, bench, CPU baseline) draws identical tensors for a (config, tensor).

  c1  X [512, 1024] ~ N(0,1), 1% of entries x50;  W [1024, 1024] ~ N(0, 0.02)
  c2  X [8192, 7168] ~ N(0,1) * c_k, c_k log-uniform in [0.1, 20] per channel;
      W [18432, 7168] ~ N(0, 0.006)
  c3  dY [8192, 18432] ~ N(0, 1e-3) with the X, W of c2
  c4  tokens [4096, 7168] ~ N(0,1), top-8 of 32 experts with Zipf(1.2)
      popularity (Gumbel top-k on log-weights); W_up [E, 2048, 7168],
      W_down [E, 7168, 2048] ~ N(0, 0.006)
  c5  W [14336, 4096] ~ N(0, 0.02);  X [4096, 4096] ~ N(0, 1)
"""

from __future__ import annotations

import math
from typing import Optional

import torch

SHAPES = {
    1: dict(M=512, N=1024, K=1024),
    2: dict(M=8192, N=18432, K=7168),
    3: dict(M=8192, N=18432, K=7168),
    4: dict(tokens=4096, hidden=7168, inter=2048, experts=32, top_k=8),
    5: dict(M=4096, N=14336, K=4096),
}


def seed_for(config_id: int, tensor_id: int) -> int:
    return 20260000 + config_id * 100 + tensor_id


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def normal(shape, *, std: float, seed: int, device="cpu", dtype=torch.bfloat16) -> torch.Tensor:
    g = _gen(device, seed)
    return (torch.randn(*shape, generator=g, device=device) * std).to(dtype)


def c1_inputs(device="cpu", dtype=torch.bfloat16):
    s = SHAPES[1]
    g = _gen(device, seed_for(1, 0))
    x = torch.randn(s["M"], s["K"], generator=g, device=device)
    mask = torch.rand(s["M"], s["K"], generator=g, device=device) < 0.01
    x = torch.where(mask, x * 50.0, x).to(dtype)
    w = normal((s["N"], s["K"]), std=0.02, seed=seed_for(1, 1), device=device, dtype=dtype)
    return x, w


def heavy_tailed_activation(rows: int, cols: int, *, seed: int, device="cpu", dtype=torch.bfloat16,
                            row_offset: int = 0) -> torch.Tensor:
    """N(0,1) rows times a per-channel scale drawn log-uniform in [0.1, 20].

    The channel scales come from their own generator so that a row slice
    (row_offset, rows) of the full matrix can be rebuilt on its own."""
    gc = _gen("cpu", seed + 50)
    c = torch.exp(torch.empty(cols).uniform_(math.log(0.1), math.log(20.0), generator=gc)).to(device)
    g = _gen(device, seed)
    if row_offset:
        torch.randn(row_offset, cols, generator=g, device=device)  # advance the stream
    return (torch.randn(rows, cols, generator=g, device=device) * c).to(dtype)


def c2_inputs(device="cpu", dtype=torch.bfloat16, rows: Optional[int] = None):
    s = SHAPES[2]
    x = heavy_tailed_activation(rows or s["M"], s["K"], seed=seed_for(2, 0), device=device, dtype=dtype)
    w = normal((s["N"], s["K"]), std=0.006, seed=seed_for(2, 1), device=device, dtype=dtype)
    return x, w


def c3_grad(device="cpu", dtype=torch.bfloat16):
    s = SHAPES[3]
    return normal((s["M"], s["N"]), std=1e-3, seed=seed_for(3, 2), device=device, dtype=dtype)


def zipf_topk_routing(tokens: int, experts: int, top_k: int, *, s: float = 1.2, seed: int, device="cpu"):
    """Distinct top-k experts per token, expert popularity ~ Zipf(s), by
    Gumbel-top-k on the log popularity.  Returns (expert_ids [T, k] int64)."""
    g = _gen("cpu", seed)
    ranks = torch.arange(1, experts + 1, dtype=torch.float64)
    logp = -s * torch.log(ranks)
    u = torch.rand(tokens, experts, generator=g, dtype=torch.float64).clamp_(1e-12, 1 - 1e-12)
    gumbel = -torch.log(-torch.log(u))
    idx = torch.topk(logp[None, :] + gumbel, top_k, dim=1).indices
    return idx.to(device)


def c4_inputs(device="cpu", dtype=torch.bfloat16, experts: Optional[int] = None):
    """experts: generate only the first `experts` experts' weights (the same
    values as the full tensors' leading slices: generation runs in order)."""
    s = SHAPES[4]
    ne = s["experts"] if experts is None else experts
    tokens = normal((s["tokens"], s["hidden"]), std=1.0, seed=seed_for(4, 0), device=device, dtype=dtype)
    routing = zipf_topk_routing(s["tokens"], s["experts"], s["top_k"], seed=seed_for(4, 1), device=device)
    w_up = normal((ne, s["inter"], s["hidden"]), std=0.006, seed=seed_for(4, 2), device=device, dtype=dtype)
    w_down = normal((ne, s["hidden"], s["inter"]), std=0.006, seed=seed_for(4, 3), device=device, dtype=dtype)
    return tokens, routing, w_up, w_down


def c4_gate(device="cpu", dtype=torch.bfloat16, experts: Optional[int] = None):
    """The SwiGLU gate weight of config 4's experts (same shape and law as W_up)."""
    s = SHAPES[4]
    ne = s["experts"] if experts is None else experts
    return normal((ne, s["inter"], s["hidden"]), std=0.006, seed=seed_for(4, 4), device=device, dtype=dtype)


def c5_inputs(device="cpu", dtype=torch.bfloat16):
    s = SHAPES[5]
    w = normal((s["N"], s["K"]), std=0.02, seed=seed_for(5, 0), device=device, dtype=dtype)
    x = normal((s["M"], s["K"]), std=1.0, seed=seed_for(5, 1), device=device, dtype=dtype)
    return x, w
