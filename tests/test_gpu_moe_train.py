"""GPU tests of the trainable single-rank expert loop (lowbit.moe.local_moe)
against the reference's per-expert loop run with autograd on the CPU
(oracle/torch_emulated.local_moe_loop: moe.py:1062-1093, LocalRoutedMoE
:476-491, ExpertMLP :190-193, capacity keep :482-486):

- the kept rows under a capacity equal the reference's torch.topk selection,
  row for row and in order;
- the token outputs and the gradients of the tokens, the routing weights and
  both expert weight stacks, within 1e-3 relative Frobenius (bf16-rounded on
  both sides), at small shapes with and without a capacity, both code
  formats, and at config 4 sampled (two experts' weight gradients, a sample
  of tokens).

The oracle loop's forward multiplies fp32 q * s operands (the blockwise
GEMM's numerics, forward="fp32_dq") and its backward is the reference's
straight-through estimator over bf16(q * s); both are the kernels' contract.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import rel_fro_bf16, to_np32
from oracle import oracle as O
from oracle import torch_emulated as TE

pytestmark = pytest.mark.gpu


def _problem(T, H, I, E, k, seed, skew=1.2):
    g = torch.Generator().manual_seed(seed)
    tokens = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ranks = torch.arange(1, E + 1, dtype=torch.float64)
    logp = -skew * torch.log(ranks)
    u = torch.rand(T, E, generator=g, dtype=torch.float64).clamp_(1e-12, 1 - 1e-12)
    idx = torch.topk(logp[None, :] + (-torch.log(-torch.log(u))), k, dim=1).indices
    w = torch.softmax(torch.randn(T, k, generator=g), dim=-1)
    w_gu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    w_d = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    d_out = (torch.randn(T, H, generator=g) * 1e-2).to(torch.bfloat16)
    return tokens, idx, w, w_gu, w_d, d_out


def _run_gpu(tokens, idx, w, w_gu, w_d, d_out, dev, **kw):
    from lowbit import moe

    leaves = [t.to(dev).requires_grad_(True) for t in (tokens, w, w_gu, w_d)]
    out = moe.local_moe(leaves[0], idx.to(dev), leaves[1], leaves[2], leaves[3], **kw)
    out.backward(d_out.to(dev))
    torch.cuda.synchronize()
    return out.detach().cpu(), [t.grad.detach().cpu() for t in leaves]


def _c_oracle_qdq(grid):
    """fp32 dq values of the C oracle's quantizer (one scale per gr x gc group)"""
    def qdq(t, gr, gc):
        return torch.from_numpy(O.quant_grouped(t.detach().numpy(), gr, gc, grid=grid)[3])
    return qdq


def _run_oracle(tokens, idx, w, w_gu, w_d, d_out, *, fmt, **kw):
    grid = O.GRID_E4M3 if fmt == "e4m3" else O.GRID_INT
    leaves = [t.clone().requires_grad_(True) for t in (tokens, w, w_gu, w_d)]
    out = TE.local_moe_loop(leaves[0], idx, leaves[1], leaves[2], leaves[3], forward="fp32_dq",
                            qdq=_c_oracle_qdq(grid), **kw)
    out.backward(d_out)
    return out.detach(), [t.grad for t in leaves]


def _gpu_gate_up(tokens, idx, w, w_gu, dev, *, capacity, fmt):
    """The fused forward's bf16 gate / up projections (the values local_moe
    keeps for its backward), rows in expert order, and the offset table."""
    from lowbit import moe, ops

    r = moe.route_by_expert(idx.to(dev), w_gu.shape[0], capacity=capacity, topk_w=w.to(dev))
    c, s_, nan = moe.quantize_expert_weights(w_gu.to(dev), fmt=fmt)
    qx = ops.quant_tile_1x128_fanout(tokens.to(dev), r.pos, r.top_k, r.rows, fmt=fmt, want_nan_rows=True)
    gu = torch.empty((r.rows, w_gu.shape[1]), dtype=torch.bfloat16, device=dev)
    ops.gemm_swiglu_quant(qx, c, s_, offsets=r.offsets, fmt=fmt, want_h=False, b_nan_rows=nan, gu_out=gu)
    return gu.cpu(), r.offsets.cpu().tolist()


def _split_rows(gu_rows: torch.Tensor):
    n, N2 = gu_rows.shape
    v = gu_rows.reshape(n, N2 // 256, 2, 128)
    return v[:, :, 0].reshape(n, N2 // 2), v[:, :, 1].reshape(n, N2 // 2)


def _grad_or_zero(g, like):
    return torch.zeros_like(like) if g is None else g


@pytest.mark.parametrize("capacity", [0, 40])
@pytest.mark.parametrize("fmt", ["e4m3", "int_grid"])
def test_local_moe_forward_and_gradients_match_reference_loop(gpu_device, capacity, fmt):
    T, H, I, E, k = 96, 256, 256, 6, 3
    tokens, idx, w, w_gu, w_d, d_out = _problem(T, H, I, E, k, seed=20262401)
    out, grads = _run_gpu(tokens, idx, w, w_gu, w_d, d_out, gpu_device, capacity=capacity, fmt=fmt)
    counts = torch.bincount(idx.reshape(-1), minlength=E)
    if capacity:
        assert int(counts.max()) > capacity, "the test should drop rows"
    # end to end: the bf16 projections differ from the oracle's in the last
    # bit on about 1% of values (fp32 summation order), and the 8-bit
    # re-quantization of h turns some of those into whole code steps
    ref_out, _ = _run_oracle(tokens, idx, w, w_gu, w_d, d_out, capacity=capacity, fmt=fmt)
    assert rel_fro_bf16(out, ref_out.double().numpy()) <= 5e-3
    # staged at the one-GEMM bar: the oracle loop takes the kernels' bf16
    # projections as its forward values (its gradients stay its own)
    gu, offs = _gpu_gate_up(tokens, idx, w, w_gu, gpu_device, capacity=capacity, fmt=fmt)
    values = lambda e: _split_rows(gu[offs[e]:offs[e + 1]])  # noqa: E731
    ref_out, ref_grads = _run_oracle(tokens, idx, w, w_gu, w_d, d_out, capacity=capacity, fmt=fmt,
                                     gate_up_values=values)
    assert rel_fro_bf16(out, ref_out.double().numpy()) <= 1e-3
    names = ["tokens", "topk_w", "w_gate_up", "w_down"]
    for name, g, r in zip(names, grads, ref_grads):
        r = _grad_or_zero(r, g)
        if name == "topk_w":
            err = O.rel_frobenius(to_np32(g), to_np32(r))
        else:
            err = rel_fro_bf16(g, r.double().numpy())
        assert err <= 1e-3, (name, err)


def test_capacity_keeps_the_reference_rows_in_order(gpu_device):
    """route_by_expert(capacity=C) keeps, per expert, the rows
    torch.topk(sort_weights, k=C, sorted=True) keeps, in that order."""
    from lowbit import moe

    T, E, k, C = 777, 9, 3, 130
    g = torch.Generator().manual_seed(20262411)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    idx[:300, 0] = 0  # one crowded expert
    idx[:300, 1:] = torch.stack([torch.randperm(E - 1, generator=g)[:k - 1] + 1 for _ in range(300)])
    w = torch.softmax(torch.randn(T, k, generator=g), dim=-1)
    r = moe.route_by_expert(idx.to(gpu_device), E, capacity=C, topk_w=w.to(gpu_device))
    offs = r.offsets.cpu().tolist()
    inv = r.inv.cpu()
    pos = r.pos.cpu()
    assert r.counts.cpu().tolist() == [min(int((idx == e).sum()), C) for e in range(E)]
    for e in range(E):
        sel = (idx == e).nonzero(as_tuple=False)
        tok, slot = sel[:, 0], sel[:, 1]
        if tok.numel() > C:
            keep = torch.topk(w[tok, slot], k=C, sorted=True).indices
            tok, slot = tok[keep], slot[keep]
        got = inv[offs[e]:offs[e + 1]]
        assert torch.equal(got, (tok * k + slot).to(torch.int32)), e
    kept = set(inv[:offs[-1]].tolist())
    for a in range(T * k):
        assert (int(pos[a]) >= 0) == (a in kept)
    assert bool((inv[offs[-1]:] == -1).all())  # no stale row -> assignment entries past the kept rows
    assert r.dropped() == T * k - offs[-1] > 0


def _torch_e4m3_qdq(t32: torch.Tensor, gr: int, gc: int) -> torch.Tensor:
    """fp32 dq of the e4m3 blockwise quantizer as torch ops (scale = amax / 448,
    1 where that is zero or not finite; code = the float8_e4m3fn cast of the
    clamped quotient), one scale per (gr x gc) group.  Both divisions are the
    correctly rounded fp32 quotients, formed in float64 and rounded once
    (torch's GPU division by a scalar multiplies by its reciprocal instead,
    which is a last-bit away for some amax)."""
    R, K = t32.shape
    Rp, Kp = -(-R // gr) * gr, -(-K // gc) * gc
    xp = torch.nn.functional.pad(t32, (0, Kp - K, 0, Rp - R))
    g = xp.reshape(Rp // gr, gr, Kp // gc, gc)
    s = (g.abs().amax(dim=(1, 3), keepdim=True).double() / 448.0).float()
    s = torch.where(torch.isfinite(s) & (s > 0), s, torch.ones_like(s))
    q = (g.double() / s.double()).float().clamp(-448.0, 448.0).to(torch.float8_e4m3fn).float()
    return (q * s).reshape(Rp, Kp)[:R, :K]


def _interleave(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    n, I = a.shape
    return torch.stack([a.reshape(n, I // 128, 128), b.reshape(n, I // 128, 128)], dim=2).reshape(n, 2 * I)


def test_local_moe_config4_sampled(gpu_device):
    """Config 4's shapes (4096 tokens, hidden 7168, 32 experts of 2048, top-8,
    Zipf routing): the weight gradients of two experts in full and the token
    and routing-weight gradients of a sample of tokens, against the reference
    loop's per-row math restated in float64 torch ops on the GPU (its own
    e4m3 quantization, F.silu and mul in bf16, its roundings of each Linear's
    output and input gradient to bf16)."""
    from lowbit import moe, workloads

    tokens, routing_ids, w_up, w_down = workloads.c4_inputs(device=gpu_device)
    w_gate = workloads.c4_gate(device=gpu_device)
    w_gu = moe.stack_gate_up(w_gate, w_up)
    del w_gate, w_up
    T, H = tokens.shape
    E, I = w_gu.shape[0], w_gu.shape[1] // 2
    k = routing_ids.shape[1]
    g = torch.Generator(device=gpu_device).manual_seed(20262421)
    topk_w = torch.softmax(torch.randn(T, k, generator=g, device=gpu_device), dim=-1)
    d_out = (torch.randn(T, H, generator=g, device=gpu_device) * 1e-2).to(torch.bfloat16)
    leaves = [t.clone().requires_grad_(True) for t in (tokens, topk_w, w_gu, w_down)]
    out = moe.local_moe(leaves[0], routing_ids, leaves[1], leaves[2], leaves[3])
    out.backward(d_out)
    torch.cuda.synchronize()
    d_tok, d_w, d_wgu, d_wd = [t.grad for t in leaves]
    del leaves, out

    # the fused forward's bf16 projections (see the small-shape test: their
    # last bits depend on the fp32 summation order)
    from lowbit import ops
    r = moe.route_by_expert(routing_ids, E)
    c, s_, nan = moe.quantize_expert_weights(w_gu)
    qx = ops.quant_tile_1x128_fanout(tokens, r.pos, r.top_k, r.rows, fmt="e4m3", want_nan_rows=True)
    gu_all = torch.empty((r.rows, 2 * I), dtype=torch.bfloat16, device=gpu_device)
    ops.gemm_swiglu_quant(qx, c, s_, offsets=r.offsets, fmt="e4m3", want_h=False, b_nan_rows=nan, gu_out=gu_all)
    del c, s_, qx
    pos = r.pos.long()

    def expert_backward(e, t_idx, s_idx):
        x32 = _torch_e4m3_qdq(tokens[t_idx].float(), 1, 128)
        wgu32 = _torch_e4m3_qdq(w_gu[e].float(), 128, 128)
        gu = gu_all[pos[t_idx * k + s_idx]]
        v = gu.reshape(-1, I // 128, 2, 128)
        gate = v[:, :, 0].reshape(-1, I).clone().requires_grad_(True)
        up = v[:, :, 1].reshape(-1, I).clone().requires_grad_(True)
        h = torch.nn.functional.silu(gate) * up
        h32 = _torch_e4m3_qdq(h.detach().float(), 1, 128)
        wd32 = _torch_e4m3_qdq(w_down[e].float(), 128, 128)
        y = (h32.double() @ wd32.double().t()).float().to(torch.bfloat16)
        wrow = topk_w[t_idx, s_idx].float()[:, None]
        dy = (d_out[t_idx].float() * wrow).to(torch.bfloat16)
        dw_route = (d_out[t_idx].double() * y.double()).sum(1)
        dh = (dy.double() @ wd32.to(torch.bfloat16).double()).float().to(torch.bfloat16)
        h.backward(dh)
        dgu = _interleave(gate.grad, up.grad).double()
        # x feeds the gate and the up Linear: each input gradient rounds to
        # bf16, and autograd adds the two in bf16
        wv = wgu32.to(torch.bfloat16).double().reshape(I // 128, 2, 128, H)
        dxg = (gate.grad.double() @ wv[:, 0].reshape(I, H)).float().to(torch.bfloat16)
        dxu = (up.grad.double() @ wv[:, 1].reshape(I, H)).float().to(torch.bfloat16)
        dx = dxg + dxu
        dWd = dy.double().t() @ h32.to(torch.bfloat16).double()
        dWgu = dgu.t() @ x32.to(torch.bfloat16).double()
        return dx, dw_route, dWd, dWgu

    ids = routing_ids
    cnt = torch.bincount(ids.reshape(-1), minlength=E).cpu()
    for e in torch.argsort(cnt)[:2].tolist():
        t_idx, s_idx = (ids == e).nonzero(as_tuple=True)
        _, _, dWd, dWgu = expert_backward(e, t_idx, s_idx)
        assert rel_fro_bf16(d_wd[e], dWd.cpu().numpy()) <= 1e-3, ("w_down", e)
        assert rel_fro_bf16(d_wgu[e], dWgu.cpu().numpy()) <= 1e-3, ("w_gate_up", e)
    sample = torch.from_numpy(np.random.default_rng(20262422).choice(T, 6, replace=False)).to(gpu_device)
    # each token's rows added in descending expert id, each add rounded to
    # bf16: the order in which autograd accumulates the gathered rows
    dx_ref = torch.zeros((len(sample), H), dtype=torch.bfloat16, device=gpu_device)
    dwr_ref = torch.zeros((len(sample), k), dtype=torch.float64, device=gpu_device)
    for j, t in enumerate(sample.tolist()):
        acc = None
        for s in sorted(range(k), key=lambda q: -int(ids[t, q])):
            tt = torch.tensor([t], device=gpu_device)
            ss = torch.tensor([s], device=gpu_device)
            dx, dwr, _, _ = expert_backward(int(ids[t, s]), tt, ss)
            acc = dx[0] if acc is None else acc + dx[0]
            dwr_ref[j, s] = dwr[0]
        dx_ref[j] = acc
    assert rel_fro_bf16(d_tok[sample], dx_ref.double().cpu().numpy()) <= 1e-3
    assert O.rel_frobenius(to_np32(d_w[sample]), dwr_ref.cpu().numpy()) <= 1e-3


def _sr_qdq_from_gpu(tokens, idx, w, w_gu, w_d, dev, *, capacity, fmt, seed, offset):
    """The stochastic-rounding dq values local_moe draws (x at `offset`, h at
    +1, gate/up weights at +2, down weights at +3), served to the oracle loop
    in the order it quantizes: per expert with rows, x and the gate weight,
    x and the up weight, h and the down weight.  Also the kernels' bf16
    gate / up projections (rows in expert order) and the offsets."""
    from lowbit import moe, ops

    E, N2, H = w_gu.shape
    I = N2 // 2
    kw = dict(fmt=fmt, rounding="stochastic", seed=seed)
    r = moe.route_by_expert(idx.to(dev), E, capacity=capacity, topk_w=w.to(dev))
    gc, gs, gn = moe.quantize_expert_weights(w_gu.to(dev), offset=offset + 2, **kw)
    dc, ds, _ = moe.quantize_expert_weights(w_d.to(dev), offset=offset + 3, **kw)
    qx = ops.quant_tile_1x128_fanout(tokens.to(dev), r.pos, r.top_k, r.rows, offset=offset, want_nan_rows=True,
                                     **kw)
    gu = torch.empty((r.rows, N2), dtype=torch.bfloat16, device=dev)
    _, qh = ops.gemm_swiglu_quant(qx, gc, gs, offsets=r.offsets, offset=offset + 1, want_h=False, b_nan_rows=gn,
                                  gu_out=gu, **kw)

    def deq_experts(c, s_, K):
        En, Nn, Kp = c.shape
        q = ops.QTensor(c.reshape(En * Nn, Kp), s_.reshape(-1).contiguous(), s_.shape[2], 1, 7, qx.grid, En * Nn, K)
        return ops.dequant(q, out_dtype=torch.float32).reshape(En, Nn, K).cpu()

    xd = ops.dequant(qx, out_dtype=torch.float32).cpu()
    hd = ops.dequant(qh, out_dtype=torch.float32).cpu()
    wgu_d = deq_experts(gc, gs, H).reshape(E, I // 128, 2, 128, H)
    wd_d = deq_experts(dc, ds, I)
    offs = r.offsets.cpu().tolist()
    order = []
    for e in range(E):
        lo, hi = offs[e], offs[e + 1]
        if hi > lo:
            order += [xd[lo:hi], wgu_d[e, :, 0].reshape(I, H), xd[lo:hi], wgu_d[e, :, 1].reshape(I, H), hd[lo:hi],
                      wd_d[e]]
    it = iter(order)

    def qdq(t, gr, gc_):
        v = next(it)
        assert v.shape == t.shape
        return v

    return qdq, gu.cpu(), offs


@pytest.mark.parametrize("capacity", [0, 40])
def test_local_moe_stochastic_rounding_gradients_match_reference_loop(gpu_device, capacity):
    """Under stochastic rounding the expert loop's backward multiplies the
    reference's straight-through operands t + (t_dq - t) (which differ from
    bf16(q * s) there) on the grouped bf16 GEMMs: the gradients of tokens,
    routing weights and both weight stacks against the reference loop's
    autograd fed the same stochastic dq values (the ones the kernels draw)
    and the kernels' bf16 projections, within 1e-3."""
    T, H, I, E, k = 96, 256, 256, 6, 3
    seed, offset = 4242, 16
    tokens, idx, w, w_gu, w_d, d_out = _problem(T, H, I, E, k, seed=20262571)
    out, grads = _run_gpu(tokens, idx, w, w_gu, w_d, d_out, gpu_device, capacity=capacity, fmt="e4m3",
                          rounding="stochastic", seed=seed, offset=offset)
    qdq, gu, offs = _sr_qdq_from_gpu(tokens, idx, w, w_gu, w_d, gpu_device, capacity=capacity, fmt="e4m3", seed=seed,
                                     offset=offset)
    leaves = [t.clone().requires_grad_(True) for t in (tokens, w, w_gu, w_d)]
    values = lambda e: _split_rows(gu[offs[e]:offs[e + 1]])  # noqa: E731
    ref = TE.local_moe_loop(leaves[0], idx, leaves[1], leaves[2], leaves[3], capacity=capacity, forward="fp32_dq",
                            qdq=qdq, gate_up_values=values)
    ref.backward(d_out)
    assert rel_fro_bf16(out, ref.detach().double().numpy()) <= 1e-3
    for name, g, r in zip(["tokens", "topk_w", "w_gate_up", "w_down"], grads, [t.grad for t in leaves]):
        r = _grad_or_zero(r, g)
        err = O.rel_frobenius(to_np32(g), to_np32(r)) if name == "topk_w" else rel_fro_bf16(g, r.double().numpy())
        assert err <= 1e-3, (name, err)
