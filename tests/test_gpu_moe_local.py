"""GPU parity of the single-rank expert loop on HIP kernels (moe.py:1062-1093,
LocalRoutedMoE :456-510): the routing sort, the 1x128 quantization of the
token rows gathered by expert, and the weighted combine back into token order.

The gather+quantize kernel is held bit for bit to the tile quantizer applied to
the gathered rows (itself pinned to the oracle in test_gpu_quant.py).  The
combine is held bit for bit to the reference's own op sequence
(`output[token_indices] += expert_out * weights`, once per expert in ascending
id) run in torch on the CPU."""

from __future__ import annotations

import pytest
import torch

from _gpu_util import seeded

pytestmark = pytest.mark.gpu


def _routing(T: int, E: int, k: int, seed: int, device, dtype=torch.int64):
    """Top-k of distinct experts per token from seeded scores."""
    g = torch.Generator().manual_seed(seed)
    scores = torch.rand((T, E), generator=g)
    return torch.topk(scores, k, dim=1).indices.to(dtype).to(device)


def _reference_combine(y_rows: torch.Tensor, pos: torch.Tensor, ids: torch.Tensor, w: torch.Tensor, E: int,
                       out_dtype: torch.dtype) -> torch.Tensor:
    """moe.py:1073-1088 on the CPU: for each expert in ascending id, the
    tokens routed to it (nonzero order), `output[token_indices] += expert_out *
    weights`.  Expert output of assignment a is y_rows[pos[a]]; pos < 0 is an
    assignment that was dropped."""
    ids, w, pos, y_rows = ids.cpu(), w.cpu(), pos.cpu().long(), y_rows.cpu()
    T, k = ids.shape
    output = torch.zeros((T, y_rows.shape[1]), dtype=out_dtype)
    for e in range(E):
        selected = (ids == e).nonzero(as_tuple=False)
        if selected.numel() == 0:
            continue
        token_indices, slot_indices = selected[:, 0], selected[:, 1]
        p = pos[token_indices * k + slot_indices]
        keep = p >= 0
        token_indices, slot_indices, p = token_indices[keep], slot_indices[keep], p[keep]
        if p.numel() == 0:
            continue
        expert_out = y_rows[p]
        weights = w[token_indices, slot_indices].unsqueeze(-1)
        output[token_indices] += expert_out * weights
    return output


def test_route_by_expert_is_the_stable_sort(gpu_device):
    from lowbit import moe

    ids = _routing(1000, 32, 8, 11, gpu_device)
    r = moe.route_by_expert(ids, 32)
    flat = ids.reshape(-1).cpu()
    order = torch.sort(flat, stable=True).indices
    assert torch.equal(r.inv.cpu().long(), order)
    pos = r.pos.cpu().long()
    assert torch.equal(pos[order], torch.arange(flat.numel()))
    counts = torch.bincount(flat, minlength=32)
    assert torch.equal(r.counts.cpu(), counts)
    assert torch.equal(r.offsets.cpu().long(), torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]))
    # the int32 routing of another caller gives the same order
    r32 = moe.route_by_expert(ids.to(torch.int32), 32)
    assert torch.equal(r32.pos.cpu(), r.pos.cpu())


@pytest.mark.parametrize("fmt", ["e4m3", "int_grid"])
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
@pytest.mark.parametrize("T,K,E,k,dtype", [(37, 1000, 5, 3, torch.bfloat16), (64, 7168, 32, 8, torch.bfloat16),
                                           (50, 264, 6, 2, torch.float32)])
def test_fanout_equals_gather_then_quantize(gpu_device, fmt, rounding, T, K, E, k, dtype):
    from lowbit import moe, ops

    x = seeded((T, K), seed=20260901, dtype=dtype, outliers=0.01).to(gpu_device)
    x[3, 17] = float("nan")  # one token row with a NaN: all its k rows are flagged
    x[5, :130] = 0.0  # a zero tile
    ids = _routing(T, E, k, 20260902, gpu_device)
    r = moe.route_by_expert(ids, E)
    kw = dict(fmt=fmt, rounding=rounding, seed=9, offset=4, want_nan_rows=True)
    got = ops.quant_tile_1x128_fanout(x, r.pos, k, r.rows, **kw)
    ref = ops.quant_tile_1x128(x[r.inv.long() // k], **kw)
    torch.cuda.synchronize()
    assert got.s_row == ref.s_row and got.s_col == ref.s_col
    assert torch.equal(got.codes, ref.codes)
    assert torch.equal(got.scales[:, :r.rows], ref.scales[:, :r.rows])
    assert torch.equal(got.nan_rows, ref.nan_rows)
    assert int(got.nan_rows.sum()) == k


def test_fanout_negative_positions_write_nothing(gpu_device):
    from lowbit import moe, ops

    T, K, E, k = 40, 512, 4, 2
    x = seeded((T, K), seed=20260903).to(gpu_device)
    ids = _routing(T, E, k, 20260904, gpu_device)
    r = moe.route_by_expert(ids, E)
    pos = r.pos.clone()
    dropped = torch.tensor([0, 7, 33, 79], device=gpu_device)
    pos[dropped] = -1
    got = ops.quant_tile_1x128_fanout(x, pos, k, r.rows, fmt="e4m3", want_nan_rows=True)
    ref = ops.quant_tile_1x128(x[r.inv.long() // k], fmt="e4m3")
    torch.cuda.synchronize()
    kept = torch.ones(r.rows, dtype=torch.bool, device=gpu_device)
    kept[r.pos[dropped].long()] = False
    assert torch.equal(got.codes[kept], ref.codes[kept])
    assert torch.equal(got.scales[:, :r.rows][:, kept], ref.scales[:, :r.rows][:, kept])


@pytest.mark.parametrize("out_dtype,w_dtype", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                               (torch.float32, torch.bfloat16), (torch.float16, torch.float16)])
@pytest.mark.parametrize("T,H,E,k", [(64, 256, 8, 2), (33, 1000, 5, 3), (17, 2056, 32, 8)])
def test_combine_rows_matches_the_reference_loop(gpu_device, out_dtype, w_dtype, T, H, E, k):
    from lowbit import moe

    ids = _routing(T, E, k, 20260905 + H, gpu_device)
    r = moe.route_by_expert(ids, E)
    y = seeded((r.rows, H), seed=20260906, dtype=out_dtype).to(gpu_device)
    w = torch.rand((T, k), generator=torch.Generator().manual_seed(20260907)).to(w_dtype).to(gpu_device)
    got = moe.combine_rows(y, r, ids, w, T)
    ref = _reference_combine(y, r.pos, ids, w, E, out_dtype)
    torch.cuda.synchronize()
    assert got.dtype == out_dtype
    assert torch.equal(got.cpu().view(torch.int16 if out_dtype != torch.float32 else torch.int32),
                       ref.view(torch.int16 if out_dtype != torch.float32 else torch.int32))


def test_combine_rows_skips_dropped_assignments(gpu_device):
    from lowbit import moe

    T, H, E, k = 50, 384, 6, 3
    ids = _routing(T, E, k, 20260908, gpu_device)
    r = moe.route_by_expert(ids, E)
    y = seeded((r.rows, H), seed=20260909).to(gpu_device)
    w = torch.rand((T, k), generator=torch.Generator().manual_seed(20260910)).to(torch.bfloat16).to(gpu_device)
    pos = r.pos.clone()
    pos[torch.tensor([1, 2, 40, 149], device=gpu_device)] = -1
    rd = moe.ExpertRouting(pos, r.inv, r.counts, r.offsets, k)
    got = moe.combine_rows(y, rd, ids, w, T)
    ref = _reference_combine(y, pos, ids, w, E, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("fmt", ["e4m3", "int_grid"])
def test_local_moe_forward_equals_its_composition(gpu_device, fmt):
    """Sort, gather+quantize, expert MLP and combine in one call equal the
    gathered rows through expert_mlp (whose GEMMs the oracle pins in
    test_gpu_moe.py) and the reference's combine loop."""
    from lowbit import moe

    T, H, I, E, k = 96, 256, 256, 4, 2
    tokens = seeded((T, H), seed=20260911).to(gpu_device)
    ids = _routing(T, E, k, 20260912, gpu_device)
    w = torch.rand((T, k), generator=torch.Generator().manual_seed(20260913)).to(torch.bfloat16).to(gpu_device)
    wg = seeded((E, I, H), seed=20260914, std=0.02).to(gpu_device)
    wu = seeded((E, I, H), seed=20260915, std=0.02).to(gpu_device)
    wd = seeded((E, H, I), seed=20260916, std=0.02).to(gpu_device)
    qg, qu = moe.quantize_expert_weights(wg, fmt=fmt), moe.quantize_expert_weights(wu, fmt=fmt)
    gate_up = moe.interleave_gate_up(qg[0], qg[1], qu[0], qu[1], qg[2], qu[2])
    down = moe.quantize_expert_weights(wd, fmt=fmt)
    out = moe.local_moe_forward(tokens, ids, w, gate_up, down, n_experts=E, fmt=fmt)
    r = moe.route_by_expert(ids, E)
    y = moe.expert_mlp(tokens[r.inv.long() // k], r.offsets, gate_up, down, fmt=fmt)
    ref = _reference_combine(y, r.pos, ids, w, E, torch.bfloat16)
    torch.cuda.synchronize()
    assert out.shape == (T, H) and out.dtype == torch.bfloat16
    assert torch.equal(out.cpu().view(torch.int16), ref.view(torch.int16))


def test_c4_fanout_and_combine_full_size(gpu_device):
    """benchmark config 4: 4096 tokens, top-8 of 32 experts, hidden 7168."""
    from lowbit import moe, ops, workloads

    tokens, routing, _, _ = workloads.c4_inputs(device="cpu", experts=1)
    tokens, routing = tokens.to(gpu_device), routing.to(gpu_device)
    r = moe.route_by_expert(routing, 32)
    got = ops.quant_tile_1x128_fanout(tokens, r.pos, 8, r.rows, fmt="e4m3", want_nan_rows=True)
    ref = ops.quant_tile_1x128(tokens[r.inv.long() // 8], fmt="e4m3", want_nan_rows=True)
    torch.cuda.synchronize()
    assert got.codes.shape == (32768, 7168)
    assert torch.equal(got.codes, ref.codes)
    assert torch.equal(got.scales[:, :r.rows], ref.scales[:, :r.rows])
    del got, ref
    w = torch.rand(routing.shape, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(gpu_device)
    y = seeded((r.rows, 7168), seed=20260917).to(gpu_device)
    out = moe.combine_rows(y, r, routing, w, 4096)
    torch.cuda.synchronize()
    tok = torch.tensor([0, 1, 2047, 4095])
    sub_ids = routing.cpu()[tok]
    rows = r.pos.cpu().long().view(4096, 8)[tok]
    # the reference loop on the sampled tokens only: their rows, renumbered
    y_sub = y.cpu()[rows.reshape(-1)]
    pos_sub = torch.arange(rows.numel(), dtype=torch.int32)
    ref = _reference_combine(y_sub, pos_sub, sub_ids, w.cpu()[tok], 32, torch.bfloat16)
    assert torch.equal(out.cpu()[tok].view(torch.int16), ref.view(torch.int16))
