"""GPU parity of the expert-parallel dispatch wire format (moe.py:670-863,
:905-923): the stable partition against numpy's stable sort, every send record
(codes, scales, metadata) bit-exact against the oracle quantizer applied to the
reference's send buffer, and an exchange between emulated ranks on one GPU
(the all_to_all replaced by slicing) against the oracle's restatement of what
_dispatch_tokens delivers, in _run_local_experts' expert order."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import assert_bits_equal, rel_fro_bf16, seeded, to_np32
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _routing(T, K, experts, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(experts, generator=g)[:K] for _ in range(T)]) if T else \
        torch.zeros((0, K), dtype=torch.int64)
    w = torch.rand((T, K), generator=g)
    return idx, w


def _decode(records: np.ndarray, H: int):
    """codes, scales, (token, slot, local expert, nan flag), weight of records."""
    from lowbit import ep

    R, s_off, m_off = ep.record_layout(H)
    T = -(-H // 128)
    rec = np.ascontiguousarray(records).reshape(-1, R)
    codes = rec[:, :H]
    scales = rec[:, s_off:s_off + 4 * T].copy().view(np.float32)
    meta = rec[:, m_off:m_off + 32].copy().view(np.int32)
    return codes, scales, meta[:, :4], meta[:, 4].copy().view(np.float32), meta[:, 5:]


@pytest.mark.parametrize("n", [0, 1, 300, 5000, 70000])
@pytest.mark.parametrize("dtype,divisor,buckets", [(torch.int32, 1, 7), (torch.int64, 4, 8), (torch.int64, 1, 512),
                                                   (torch.int32, 3, 4096)])
def test_partition_is_a_stable_sort(gpu_device, n, dtype, divisor, buckets):
    from lowbit import ep

    g = torch.Generator().manual_seed(20261201 + n)
    keys = torch.randint(0, buckets * divisor, (n,), generator=g).to(dtype)
    pos, inv, counts, offsets = ep.partition(keys.to(gpu_device), divisor=divisor, buckets=buckets)
    torch.cuda.synchronize()
    b = keys.numpy() // divisor
    want_inv = np.argsort(b, kind="stable")
    want_pos = np.empty(n, dtype=np.int64)
    want_pos[want_inv] = np.arange(n)
    want_counts = np.bincount(b, minlength=buckets)
    # np.array_equal keeps a failure report short (no element-wise diff of long lists)
    assert np.array_equal(inv.cpu().numpy(), want_inv), "inv"
    assert np.array_equal(pos.cpu().numpy(), want_pos), "pos"
    assert np.array_equal(counts.cpu().numpy(), want_counts), "counts"
    assert np.array_equal(offsets.cpu().numpy(), np.concatenate([[0], np.cumsum(want_counts)])), "offsets"


def test_partition_clamps_out_of_range_keys(gpu_device):
    from lowbit import ep

    keys = torch.tensor([5, -3, 100, 2, 2], dtype=torch.int32, device=gpu_device)
    _, inv, counts, _ = ep.partition(keys, divisor=1, buckets=4)
    torch.cuda.synchronize()
    # -3 -> bucket 0, 5 and 100 -> bucket 3
    assert counts.cpu().tolist() == [1, 0, 2, 2]
    assert inv.cpu().tolist() == [1, 3, 4, 0, 2]


@pytest.mark.parametrize("fmt,grid", [("e4m3", O.GRID_E4M3), ("int_grid", O.GRID_INT)])
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
@pytest.mark.parametrize("H", [1024, 200])
def test_pack_records_match_oracle(gpu_device, fmt, grid, rounding, H):
    from lowbit import ep

    T, K, epr, ep_size = 96, 4, 3, 4
    x = seeded((T, H), seed=20261202, outliers=0.01).to(gpu_device)
    x[7, 5] = float("nan")
    idx, w = _routing(T, K, epr * ep_size, 20261203)
    send = ep.pack_dispatch(x, idx.to(gpu_device), w.to(gpu_device), experts_per_rank=epr, ep_size=ep_size, fmt=fmt,
                            rounding=rounding, seed=77, offset=5)
    torch.cuda.synchronize()
    order, counts = O.ep_send_order(idx.numpy(), epr, ep_size)
    assert send.counts.cpu().numpy().tolist() == counts.tolist()
    codes, scales, meta, weight, reserved = _decode(send.records.cpu().numpy(), H)
    # the reference's send buffer: token rows in send order (moe.py:693, :805)
    send_rows = to_np32(x)[order // K]
    rc = O.ROUND_STOCHASTIC if rounding == "stochastic" else O.ROUND_NEAREST
    c_ref, s_ref, _, _ = O.quant_tile_1x128(send_rows, grid=grid, rounding=rc, seed=77, offset=5)
    assert_bits_equal(codes, c_ref[:, :H], "record codes")
    assert_bits_equal(scales, s_ref, "record scales")
    assert np.array_equal(meta[:, 0], order // K), "token index"
    assert np.array_equal(meta[:, 1], order % K), "slot"
    assert np.array_equal(meta[:, 2], idx.numpy().reshape(-1)[order] % epr), "local expert"
    # the flag of every record of token 7, whose row holds the NaN
    assert np.array_equal(meta[:, 3], np.isnan(send_rows).any(axis=1).astype(np.int32)), "NaN flags"
    assert_bits_equal(weight, w.numpy().reshape(-1)[order].astype(np.float32), "record weights")
    assert not reserved.any()


def _emulated_exchange(ep_size, epr, H, tokens_per_rank, K, seed, device, rounding="nearest"):
    from lowbit import ep

    xs, idxs, ws, sends = [], [], [], []
    for r, T in enumerate(tokens_per_rank):
        x = seeded((T, H), seed=seed + 10 * r).to(device)
        idx, w = _routing(T, K, epr * ep_size, seed + 10 * r + 1)
        xs.append(x), idxs.append(idx), ws.append(w)
        sends.append(ep.pack_dispatch(x, idx.to(device), w.to(device), experts_per_rank=epr, ep_size=ep_size,
                                      rounding=rounding, seed=seed, offset=r))
    # all_to_all_single: receiver r gets, from each source s in rank order, s's slice for r
    recv = []
    for r in range(ep_size):
        parts, counts = [], []
        for s in range(ep_size):
            c = sends[s].counts.cpu().tolist()
            start = sum(c[:r])
            parts.append(sends[s].records[start:start + c[r]])
            counts.append(c[r])
        recv.append((torch.cat(parts), counts))
    return xs, idxs, ws, sends, recv


def test_exchange_between_emulated_ranks(gpu_device):
    from lowbit import ep

    ep_size, epr, H, K = 4, 3, 512, 4
    tokens = [40, 0, 77, 13]  # one rank sends nothing
    xs, idxs, ws, sends, recv = _emulated_exchange(ep_size, epr, H, tokens, K, 20261210, gpu_device)
    ref = O.ep_dispatch([i.numpy() for i in idxs], [w.numpy() for w in ws], epr, ep_size)
    for r in range(ep_size):
        records, counts = recv[r]
        rows = ep.unpack_dispatch(records, counts, H=H, local_experts=epr)
        torch.cuda.synchronize()
        want = ref[r]
        order = O.ep_expert_order(want["local_expert"], epr)
        assert np.array_equal(rows.order.cpu().numpy(), order), "expert order"
        assert np.array_equal(rows.counts.cpu().numpy(), np.bincount(want["local_expert"], minlength=epr)), "counts"
        for key, got in (("src_rank", rows.src_rank), ("token_idx", rows.token_idx), ("slot_idx", rows.slot_idx)):
            assert np.array_equal(got.cpu().numpy(), want[key][order]), key
        assert_bits_equal(rows.weight.cpu().numpy(), want["sort_weight"][order], "weights")
        # payload: each row's codes and scales are those its sender quantized
        n = len(order)
        if n == 0:
            continue
        q = rows.q
        src = want["src_rank"][order]
        for s in np.unique(src):
            sel = np.nonzero(src == s)[0]
            K_s = idxs[s].shape[1]
            srow = want["src_row"][order][sel]
            c_ref, s_ref, _, _ = O.quant_tile_1x128(to_np32(xs[s])[srow // K_s], grid=O.GRID_E4M3)
            assert_bits_equal(q.codes.cpu().numpy()[sel, :H], c_ref[:, :H], "payload codes")
            got_s = q.scales.cpu().numpy()[:, sel].T
            assert_bits_equal(np.ascontiguousarray(got_s), s_ref, "payload scales")


def test_grouped_gemm_on_received_rows(gpu_device):
    """The unpacked rows feed the grouped GEMM directly (no dequantize /
    re-quantize); checked per expert against the oracle GEMM."""
    from lowbit import ep, moe, ops

    ep_size, epr, H, K, N = 2, 4, 1024, 2, 384
    xs, idxs, ws, sends, recv = _emulated_exchange(ep_size, epr, H, [200, 150], K, 20261220, gpu_device)
    records, counts = recv[0]
    rows = ep.unpack_dispatch(records, counts, H=H, local_experts=epr)
    wts = seeded((epr, N, H), seed=20261221, std=0.02).to(gpu_device)
    b_codes, b_scales, _ = moe.quantize_expert_weights(wts)
    y = ops.gemm_grouped_blockscaled(rows.q, b_codes, b_scales, rows.offsets, N=N)
    torch.cuda.synchronize()
    ref = O.ep_dispatch([i.numpy() for i in idxs], [w.numpy() for w in ws], epr, ep_size)[0]
    order = O.ep_expert_order(ref["local_expert"], epr)
    src, srow, le = ref["src_rank"][order], ref["src_row"][order], ref["local_expert"][order]
    x_rows = np.stack([to_np32(xs[s])[r // K] for s, r in zip(src, srow)])
    xdq = O.quant_tile_1x128(x_rows, grid=O.GRID_E4M3)[3]
    out = np.zeros((len(order), N))
    for e in range(epr):
        sel = le == e
        wdq = O.quant_block_128x128(to_np32(wts[e]), grid=O.GRID_E4M3)[3]
        out[sel] = O.gemm_ref(xdq[sel], wdq)
    assert rel_fro_bf16(y, out) <= 1e-3


def test_c4_size_records_feed_the_expert_path(gpu_device):
    """Config 4 (4096 tokens, hidden 7168, top-8 of 32 experts): the records
    received for all 32 experts (one rank) unpack to exactly the codes and
    scales the existing expert path quantizes from the expert-sorted tokens."""
    from lowbit import ep, moe, ops, workloads

    tokens, routing, _, _ = workloads.c4_inputs(device="cpu")
    idx = routing if isinstance(routing, torch.Tensor) else routing[0]
    x = tokens.to(gpu_device)
    w = torch.rand(idx.shape, generator=torch.Generator().manual_seed(20261230))
    send = ep.pack_dispatch(x, idx.to(gpu_device), w.to(gpu_device), experts_per_rank=32, ep_size=1)
    rows = ep.unpack_dispatch(send.records, [send.records.shape[0]], H=7168, local_experts=32)
    order, token_index, offsets = moe.sort_by_expert(idx.to(gpu_device), 32)
    qx = ops.quant_tile_1x128(x[token_index.long()], fmt="e4m3", tile_major_scales=True)
    torch.cuda.synchronize()
    assert torch.equal(rows.offsets.cpu(), offsets.cpu().to(torch.int32))
    assert torch.equal(rows.token_idx.cpu().long(), token_index.cpu().long())
    assert torch.equal(rows.q.codes, qx.codes)
    M = rows.q.rows
    assert torch.equal(rows.q.scales[:, :M], qx.scales[:, :M])
    # a sample of the send records against the oracle: each record's codes
    # and tile scales are the 1x128 quantization of its token row
    rec = send.records.cpu().numpy()
    pick = np.sort(np.random.default_rng(20261231).choice(rec.shape[0], 64, replace=False))
    codes, scales, meta, _, _ = _decode(rec[pick], 7168)
    tok = meta[:, 0]
    c_ref, s_ref, _, _ = O.quant_tile_1x128(tokens.float().numpy()[tok], grid=O.GRID_E4M3)
    assert_bits_equal(codes, c_ref[:, :7168], "sampled c4 record codes")
    assert_bits_equal(scales, s_ref, "sampled c4 record scales")


def test_capacity_drop_keeps_top_weights(gpu_device):
    """Capacity drop (moe.py:919-923): per local expert the `capacity` rows of
    highest routing weight, highest first; the kept record indices run past
    the number of kept rows, so every row must come from its own record."""
    from lowbit import ep

    ep_size, epr, H, K, cap = 2, 4, 384, 4, 9
    _, _, _, _, recv = _emulated_exchange(ep_size, epr, H, [30, 25], K, 20261240, gpu_device)
    records, counts = recv[1]
    rows = ep.unpack_dispatch(records, counts, H=H, local_experts=epr)
    order, kept = ep.capacity_order(rows, cap)
    got = ep.unpack_dispatch(records, counts, H=H, local_experts=epr, order=order, order_counts=kept)
    torch.cuda.synchronize()
    rec = records.cpu().numpy()
    codes, scales, meta, weight, _ = _decode(rec, H)
    want, want_kept = [], []
    for e in range(epr):
        sel = np.nonzero(meta[:, 2] == e)[0]  # arrival order
        if len(sel) > cap:
            sel = sel[np.argsort(-weight[sel], kind="stable")[:cap]]
        want.extend(sel.tolist())
        want_kept.append(len(sel))
    want = np.array(want)
    assert kept == want_kept and sum(kept) < len(rec) and want.max() >= len(want)
    assert np.array_equal(got.order.cpu().numpy(), want), "kept order"
    assert np.array_equal(got.offsets.cpu().numpy(), np.concatenate([[0], np.cumsum(want_kept)])), "offsets"
    assert_bits_equal(got.q.codes.cpu().numpy()[:, :H], codes[want], "kept codes")
    assert_bits_equal(np.ascontiguousarray(got.q.scales.cpu().numpy()[:, :len(want)].T), scales[want], "kept scales")
    assert np.array_equal(got.token_idx.cpu().numpy(), meta[want, 0]), "token index"
    assert_bits_equal(got.weight.cpu().numpy(), weight[want], "weights")
    src = np.searchsorted(np.cumsum(counts), want, side="right")
    assert np.array_equal(got.src_rank.cpu().numpy(), src), "source rank"


def test_unpack_rejects_bad_offsets(gpu_device):
    from lowbit import ep

    R, _, _ = ep.record_layout(256)
    records = torch.zeros((6, R), dtype=torch.uint8, device=gpu_device)
    with pytest.raises(ValueError):
        ep.unpack_dispatch(records, [2, 3], H=256, local_experts=2)  # counts add up to 5, not 6
    with pytest.raises(ValueError):
        ep.unpack_dispatch(records, [1] * 6 + [0] * 251, H=256, local_experts=2)  # more than 256 ranks


def test_expert_mlp_on_received_codes_equals_local_path(gpu_device):
    """The received codes go straight into the expert MLP (no dequantize and
    re-quantize): with round to nearest the codes are those the local path
    quantizes from the expert-sorted tokens, so the output is bit-identical."""
    from lowbit import ep, moe

    T, H, I, E, K = 512, 1024, 256, 8, 4
    x = seeded((T, H), seed=20261250, outliers=0.01).to(gpu_device)
    idx, w = _routing(T, K, E, 20261251)
    idx = idx.to(gpu_device)
    wg, wu = seeded((E, I, H), seed=20261252, std=0.02).to(gpu_device), seeded((E, I, H), seed=20261253,
                                                                                  std=0.02).to(gpu_device)
    wd = seeded((E, H, I), seed=20261254, std=0.02).to(gpu_device)
    g, u = moe.quantize_expert_weights(wg), moe.quantize_expert_weights(wu)
    gate_up = moe.interleave_gate_up(g[0], g[1], u[0], u[1], g[2], u[2])
    down = moe.quantize_expert_weights(wd)
    send = ep.pack_dispatch(x, idx, w.to(gpu_device), experts_per_rank=E, ep_size=1)
    rows = ep.unpack_dispatch(send.records, [send.records.shape[0]], H=H, local_experts=E)
    got = moe.expert_mlp(rows.q, rows.offsets, gate_up, down)
    _, token_index, offsets = moe.sort_by_expert(idx, E)
    want = moe.expert_mlp(x[token_index.long()], offsets, gate_up, down)
    torch.cuda.synchronize()
    assert torch.equal(rows.token_idx.long(), token_index.long())
    assert got.dtype == want.dtype and torch.equal(got, want)


@pytest.mark.parametrize("granularity", ["tile_1x128", "tensor"])
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
@pytest.mark.parametrize("H", [1024, 200])
def test_pack_records_with_reference_comm_quant(gpu_device, granularity, rounding, H):
    """granularity mode: the records hold exactly the codes and the strip (or
    tensor) scales of the reference's _comm_quant_dequant applied to the send
    buffer (moe.py:79-143: int grid, qmax 127, amax checked before dividing).
    The receiver's bf16(q * s) equals the value the reference puts on the
    wire, tensor + (dq - tensor) in bf16, except for the sign of zero and for
    elements where dq - tensor is inexact in bf16 (then one bf16 ulp)."""
    from lowbit import ep

    T, K, epr, ep_size = 96, 4, 3, 4
    x = seeded((T, H), seed=20261270, outliers=0.01).to(gpu_device)
    x[11, 3] = float("nan")
    idx, w = _routing(T, K, epr * ep_size, 20261271)
    send = ep.pack_dispatch(x, idx.to(gpu_device), w.to(gpu_device), experts_per_rank=epr, ep_size=ep_size,
                            granularity=granularity, rounding=rounding, seed=77, offset=5)
    torch.cuda.synchronize()
    order, counts = O.ep_send_order(idx.numpy(), epr, ep_size)
    assert send.counts.cpu().numpy().tolist() == counts.tolist()
    codes, scales, meta, weight, _ = _decode(send.records.cpu().numpy(), H)
    send_rows = to_np32(x)[order // K]
    gc = 128 if granularity == "tile_1x128" else H
    rc = O.ROUND_STOCHASTIC if rounding == "stochastic" else O.ROUND_NEAREST
    c_ref, s_ref, q_ref, _ = O.quant_grouped(send_rows, len(order), gc, grid=O.GRID_INT, rounding=rc,
                                             scale_rule=O.SCALE_BEFORE_DIVIDE, seed=77, offset=5)
    assert_bits_equal(codes, c_ref, "record codes")
    Tt = -(-H // 128)
    tile_scale = s_ref[0, np.minimum(np.arange(Tt) * 128 // gc, s_ref.shape[1] - 1)]
    assert_bits_equal(scales, np.broadcast_to(tile_scale, scales.shape), "record scales")
    assert np.array_equal(meta[:, 3], np.isnan(send_rows).any(axis=1).astype(np.int32)), "NaN flags"
    # the receiver's value against the reference's wire value
    got = O.round_bf16(O.decode_codes(codes, O.GRID_INT) * np.repeat(scales, 128, axis=1)[:, :H])
    t = torch.from_numpy(send_rows).to(torch.bfloat16)
    dq = torch.from_numpy(q_ref * np.repeat(s_ref, gc, axis=1)[:, :H]).to(torch.bfloat16)
    want = (t + (dq - t)).float().numpy()
    both_nan = np.isnan(got) & np.isnan(want)
    same = (got == want) | both_nan
    assert np.isnan(got).sum() == np.isnan(want).sum()
    bits_g = O.to_bf16_bits(got[~same]).astype(np.int32)
    bits_w = O.to_bf16_bits(want[~same]).astype(np.int32)
    assert np.all(np.abs(bits_g - bits_w) == 1), "differences beyond one bf16 ulp"
    # stochastic rounding also rounds up values far below half a step, where
    # dq - tensor needs more bits than bf16 holds; nearest rarely does
    limit = 1e-2 if rounding == "stochastic" else 1e-3
    assert (~same).mean() < limit, f"{(~same).sum()} of {same.size} elements differ by one ulp"


@pytest.mark.parametrize("mode", ["row_e4m3", "strip_int"])
@pytest.mark.parametrize("capacity", [0, 7])
def test_return_and_combine_round_trip(gpu_device, mode, capacity):
    """Dispatch between 3 emulated ranks, synthetic expert outputs, the return
    records (their codes and scales against the oracle quantizer of the
    send-back buffer in the reference's order), the emulated return exchange,
    and the combine at every source rank bit-exact against the reference's
    index_add_ on the CPU over the rows the records carry, in arrival order."""
    from lowbit import ep

    ep_size, epr, H, K = 3, 2, 384, 3
    tokens = [50, 0, 37]
    gran = None if mode == "row_e4m3" else "tile_1x128"
    fmt = "e4m3" if mode == "row_e4m3" else "int_grid"
    xs, idxs, ws, sends, recv = _emulated_exchange(ep_size, epr, H, tokens, K, 20261280, gpu_device)
    ws = [w.to(torch.bfloat16) for w in ws]  # the routing weights in the tokens' dtype, as the reference has them
    back = []  # per expert rank: the return records and their counts per source rank
    for r in range(ep_size):
        records, counts = recv[r]
        rows = ep.unpack_dispatch(records, counts, H=H, local_experts=epr)
        if capacity:
            order, kept = ep.capacity_order(rows, capacity)
            rows = ep.unpack_dispatch(records, counts, H=H, local_experts=epr, order=order, order_counts=kept)
        out_rows = seeded((rows.token_idx.numel(), H), seed=20261290 + r, std=2.0).to(gpu_device)
        sb = ep.pack_return(out_rows, rows, ep_size=ep_size, granularity=gran, fmt=fmt, seed=9, offset=r)
        torch.cuda.synchronize()
        # the reference's send-back order: per source rank, rows in expert (row) order
        src = rows.src_rank.cpu().numpy()
        ret_order = np.concatenate([np.nonzero(src == s)[0] for s in range(ep_size)])
        assert sb.counts.cpu().numpy().tolist() == np.bincount(src, minlength=ep_size).tolist()
        c, sc, meta, wt, _ = _decode(sb.records.cpu().numpy(), H)
        ref_rows = to_np32(out_rows)[ret_order]
        if gran is None:
            c_ref, s_ref, _, _ = O.quant_tile_1x128(ref_rows, grid=O.GRID_E4M3, seed=9, offset=r)
            assert_bits_equal(sc, s_ref, "return scales")
        else:
            c_ref, s_ref, _, _ = O.quant_grouped(ref_rows, len(ret_order), 128, grid=O.GRID_INT,
                                                 scale_rule=O.SCALE_BEFORE_DIVIDE, seed=9, offset=r)
            assert_bits_equal(sc, np.broadcast_to(s_ref[0], sc.shape), "return scales")
        assert_bits_equal(c[:, :H], c_ref[:, :H], "return codes")
        assert np.array_equal(meta[:, 0], rows.token_idx.cpu().numpy()[ret_order]), "token index"
        assert np.array_equal(meta[:, 1], rows.slot_idx.cpu().numpy()[ret_order]), "slot"
        back.append((sb.records, sb.counts.cpu().tolist()))
    for s in range(ep_size):
        # all_to_all_single back: source s receives, from each expert rank in order, that rank's slice for s
        parts = []
        for r in range(ep_size):
            rec, cnt = back[r]
            start = sum(cnt[:s])
            parts.append(rec[start:start + cnt[s]])
        got_rec = torch.cat(parts)
        T = tokens[s]
        out = ep.combine(got_rec, idxs[s].to(gpu_device), ws[s].to(gpu_device), H=H, fmt=fmt)
        torch.cuda.synchronize()
        assert out.shape == (T, H) and out.dtype == torch.bfloat16
        c, sc, meta, _, _ = _decode(got_rec.cpu().numpy(), H)
        feat = O.round_bf16(O.decode_codes(c[:, :H], O.GRID_E4M3 if gran is None else O.GRID_INT)
                            * np.repeat(sc, 128, axis=1)[:, :H])
        tok = torch.from_numpy(meta[:, 0].astype(np.int64))
        slot = torch.from_numpy(meta[:, 1].astype(np.int64))
        ref = torch.zeros((T, H), dtype=torch.bfloat16)
        if len(tok):
            ref.index_add_(0, tok, torch.from_numpy(feat).to(torch.bfloat16) * ws[s][tok, slot].unsqueeze(-1))
        assert_bits_equal(out.float().cpu().numpy(), ref.float().numpy(), "combined tokens")
        if T:
            assert_bits_equal(out.float().cpu().numpy(),
                              O.ep_combine(feat, meta[:, 0], meta[:, 1], idxs[s].numpy(), ws[s].float().numpy(), T),
                              "combined tokens (oracle)")


def test_combine_without_records_is_zero(gpu_device):
    """Tokens none of whose assignments came back (all dropped) stay zero, as
    index_add_ into zeros leaves them."""
    from lowbit import ep

    R, _, _ = ep.record_layout(256)
    idx, w = _routing(5, 2, 4, 20261300)
    out = ep.combine(torch.empty((0, R), dtype=torch.uint8, device=gpu_device), idx.to(gpu_device),
                     w.to(gpu_device, torch.bfloat16), H=256)
    torch.cuda.synchronize()
    assert out.shape == (5, 256) and not out.float().abs().sum().item()
    assert not torch.signbit(out.float()).any()


@pytest.mark.parametrize("fmt,grid", [("e4m3", O.GRID_E4M3), ("int_grid", O.GRID_INT)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_combine_decodes_every_code(gpu_device, fmt, grid, out_dtype):
    """All 256 codes through the combine's decode (scale 1, weight 1, a
    second all-zero record for the same token): the output is each code's
    value added to zero, NaN codes included."""
    from lowbit import ep

    H = 256
    R, s_off, m_off = ep.record_layout(H)
    rec = np.zeros((2, R), dtype=np.uint8)
    rec[0, :H] = np.arange(256, dtype=np.uint8)
    rec[:, s_off:s_off + 8] = np.frombuffer(np.array([1.0, 1.0], dtype=np.float32).tobytes(), dtype=np.uint8)
    rec[:, m_off:m_off + 8] = np.frombuffer(np.array([[0, 0], [0, 1]], dtype=np.int32).tobytes(),
                                            dtype=np.uint8).reshape(2, 8)
    idx = torch.tensor([[3, 1]], dtype=torch.int64)
    w = torch.ones((1, 2), dtype=out_dtype)
    out = ep.combine(torch.from_numpy(rec).to(gpu_device), idx.to(gpu_device), w.to(gpu_device), H=H, fmt=fmt,
                     out_dtype=out_dtype)
    torch.cuda.synchronize()
    want = O.decode_codes(np.arange(256, dtype=np.uint8), grid).astype(np.float32)
    if out_dtype == torch.bfloat16:
        want = O.round_bf16(want)
    want = np.float32(0.0) + want  # the sum starts from zero: -0 comes out as +0, as from index_add_ into zeros
    assert_bits_equal(out.float().cpu().numpy()[0], want, "decoded codes")


def _value_payload(records: np.ndarray, H: int, dtype: torch.dtype):
    """values (fp32), (token, slot, local expert, flag), weight, reserved of value records."""
    from lowbit import ep

    R, m_off = ep.value_record_layout(H, dtype)
    rec = np.ascontiguousarray(records).reshape(-1, R)
    esz = 2 if dtype == torch.bfloat16 else 4
    raw = torch.from_numpy(rec[:, :H * esz].copy())
    vals = raw.view(dtype).float().numpy() if len(rec) else np.zeros((0, H), np.float32)
    meta = rec[:, m_off:m_off + 32].copy().view(np.int32)
    return vals, meta[:, :4], meta[:, 4].copy().view(np.float32), meta[:, 5:]


def _wire_values(rows: np.ndarray, gc: int, dtype: torch.dtype, rounding: str, seed: int, offset: int):
    """The reference's wire value of a send buffer (moe.py:79-143): the
    oracle's int-grid quantizer with one scale per gc columns over all rows
    (amax checked before dividing), dq = q * scale in fp32, then tensor + (dq
    - tensor) evaluated by torch on the CPU in the tensor's dtype."""
    n, H = rows.shape
    rc = O.ROUND_STOCHASTIC if rounding == "stochastic" else O.ROUND_NEAREST
    _, _, _, dq = O.quant_grouped(rows, max(n, 1), gc, grid=O.GRID_INT, rounding=rc,
                                  scale_rule=O.SCALE_BEFORE_DIVIDE, seed=seed, offset=offset)
    t = torch.from_numpy(rows).to(dtype)
    d = torch.from_numpy(dq).to(dtype)
    return (t + (d - t)).float().numpy()


def _reference_channel_rn(rows: np.ndarray, dtype: torch.dtype):
    """_comm_quant_dequant(granularity="channel", rounding "nearest") as the
    reference's column loop forms it (moe.py:91-121), in torch on the CPU."""
    tensor = torch.from_numpy(rows).to(dtype)
    x = tensor.float()
    cols = []
    for c in range(x.shape[-1]):
        block = x[..., c:c + 1]
        scale = block.abs().amax()
        scale = block.new_tensor(1.0) if (not torch.isfinite(scale) or scale <= 0) else scale / 127.0
        cols.append(torch.clamp(torch.round(block / scale), min=-127, max=127) * scale)
    dq = torch.cat(cols, dim=-1).to(dtype)
    return (tensor + (dq - tensor)).float().numpy()


@pytest.mark.parametrize("granularity", ["channel", "tile_1x128", "tensor"])
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H", [1024, 200])
def test_value_records_hold_the_reference_wire_values(gpu_device, granularity, rounding, dtype, H):
    """Value records (the only wire of channel comm-quant): every record's
    payload bit-exact against the reference's wire value of the send buffer
    (oracle quantizer, the straight-through expression in torch on the CPU)
    and against comm_quant_dequant of the send buffer on the GPU; metadata as
    in code records.  Round to nearest with channel scales also against the
    reference's own column loop restated in torch.  A NaN element makes its
    column's (or strip's, or the tensor's) scale 1."""
    from lowbit import ep, moe

    T, K, epr, ep_size = 96, 4, 3, 4
    x = seeded((T, H), seed=20261400, outliers=0.01, dtype=dtype).to(gpu_device)
    x[11, 3] = float("nan")
    x[20, 5] = 0.0
    x[:, 7] = 0.0  # an all-zero column: scale 1
    idx, w = _routing(T, K, epr * ep_size, 20261401)
    send = ep.pack_dispatch(x, idx.to(gpu_device), w.to(gpu_device), experts_per_rank=epr, ep_size=ep_size,
                            granularity=granularity, wire="values", rounding=rounding, seed=77, offset=5)
    order, counts = O.ep_send_order(idx.numpy(), epr, ep_size)
    send_t = x[torch.from_numpy(order // K).to(gpu_device)]
    gpu_wire = moe.comm_quant_dequant(send_t, granularity=granularity, rounding_mode=rounding, seed=77, offset=5)
    torch.cuda.synchronize()
    assert send.value_dtype == dtype and send.counts.cpu().numpy().tolist() == counts.tolist()
    rec = send.records.cpu().numpy()
    R, m_off = ep.value_record_layout(H, dtype)
    assert R % 128 == 0 and m_off == R - 32 and R - 32 >= H * x.element_size()
    assert not rec[:, H * x.element_size():m_off].any(), "padding must be zero"
    vals, meta, weight, reserved = _value_payload(rec, H, dtype)
    send_rows = to_np32(x)[order // K]
    gc = {"channel": 1, "tile_1x128": 128, "tensor": H}[granularity]
    want = _wire_values(send_rows, gc, dtype, rounding, 77, 5)
    assert_bits_equal(vals, want, "record values (oracle)")
    assert_bits_equal(vals, to_np32(gpu_wire), "record values (comm_quant_dequant)")
    if granularity == "channel" and rounding == "nearest" and H == 200:
        assert_bits_equal(vals, _reference_channel_rn(send_rows, dtype), "record values (reference column loop)")
    assert np.array_equal(meta[:, 0], order // K) and np.array_equal(meta[:, 1], order % K)
    assert np.array_equal(meta[:, 2], idx.numpy().reshape(-1)[order] % epr) and not meta[:, 3].any()
    assert_bits_equal(weight, w.numpy().reshape(-1)[order].astype(np.float32), "record weights")
    assert not reserved.any()


def test_value_records_reject_what_they_cannot_carry(gpu_device):
    from lowbit import ep

    x = seeded((8, 256), seed=20261402).to(gpu_device)
    idx, w = _routing(8, 2, 4, 20261403)
    with pytest.raises(ValueError, match="channel"):
        ep.pack_dispatch(x, idx.to(gpu_device), w.to(gpu_device), experts_per_rank=2, ep_size=2,
                         granularity="channel", wire="codes")
    with pytest.raises(ValueError, match="granularity"):
        ep.pack_dispatch(x, idx.to(gpu_device), w.to(gpu_device), experts_per_rank=2, ep_size=2, wire="values")


@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
@pytest.mark.parametrize("capacity", [0, 7])
def test_channel_value_records_dispatch_return_and_combine(gpu_device, rounding, capacity):
    """The channel comm-quant end to end between 3 emulated ranks: dispatch
    value records, the receiver's rows (expert order, metadata against the
    oracle's ep_dispatch, each row the sender's wire value), a capacity drop,
    synthetic expert outputs sent back as value records (against the
    reference's wire value of the send-back buffer in its order), and the
    combine bit-exact against index_add_ on the CPU of the returned rows in
    the tokens' dtype times their weights, and against the oracle."""
    from lowbit import ep

    ep_size, epr, H, K = 3, 2, 384, 3
    tokens = [50, 0, 37]
    xs, idxs, ws, sends = [], [], [], []
    for r, T in enumerate(tokens):
        x = seeded((T, H), seed=20261410 + 10 * r, heavy_channels=True).to(gpu_device)
        idx, w = _routing(T, K, epr * ep_size, 20261411 + 10 * r)
        w = w.to(torch.bfloat16)
        xs.append(x), idxs.append(idx), ws.append(w)
        sends.append(ep.pack_dispatch(x, idx.to(gpu_device), w.to(gpu_device), experts_per_rank=epr,
                                      ep_size=ep_size, granularity="channel", rounding=rounding, seed=31, offset=r))
    torch.cuda.synchronize()
    # each sender's wire values by assignment index
    wire = []
    for s in range(ep_size):
        by_a = np.zeros((tokens[s] * K, H), np.float32)
        if tokens[s]:
            order, _ = O.ep_send_order(idxs[s].numpy(), epr, ep_size)
            by_a[order] = _wire_values(to_np32(xs[s])[order // K], 1, torch.bfloat16, rounding, 31, s)
        wire.append(by_a)
    ref = O.ep_dispatch([i.numpy() for i in idxs], [w.float().numpy() for w in ws], epr, ep_size)
    back = []
    for r in range(ep_size):
        parts, counts = [], []
        for s in range(ep_size):
            c = sends[s].counts.cpu().tolist()
            start = sum(c[:r])
            parts.append(sends[s].records[start:start + c[r]])
            counts.append(c[r])
        records = torch.cat(parts)
        rows = ep.unpack_dispatch(records, counts, H=H, local_experts=epr, value_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        want = ref[r]
        order = O.ep_expert_order(want["local_expert"], epr)
        assert rows.q is None and rows.values.dtype == torch.bfloat16
        assert np.array_equal(rows.order.cpu().numpy(), order), "expert order"
        for key, got in (("src_rank", rows.src_rank), ("token_idx", rows.token_idx), ("slot_idx", rows.slot_idx)):
            assert np.array_equal(got.cpu().numpy(), want[key][order]), key
        exp_vals = np.stack([wire[s][a] for s, a in zip(want["src_rank"][order], want["src_row"][order])]) \
            if len(order) else np.zeros((0, H), np.float32)
        assert_bits_equal(to_np32(rows.values), exp_vals, "received rows")
        if capacity:
            korder, kept = ep.capacity_order(rows, capacity)
            rows = ep.unpack_dispatch(records, counts, H=H, local_experts=epr, order=korder, order_counts=kept,
                                      value_dtype=torch.bfloat16)
            assert_bits_equal(to_np32(rows.values), _value_payload(records.cpu().numpy(), H, torch.bfloat16)[0][
                korder.cpu().numpy()], "kept rows")
        out_rows = seeded((rows.token_idx.numel(), H), seed=20261490 + r, std=2.0).to(gpu_device)
        sb = ep.pack_return(out_rows, rows, ep_size=ep_size, granularity="channel", rounding=rounding, seed=9,
                            offset=r)
        torch.cuda.synchronize()
        src = rows.src_rank.cpu().numpy()
        ret_order = np.concatenate([np.nonzero(src == s)[0] for s in range(ep_size)]) if len(src) else \
            np.zeros(0, np.int64)
        vals, meta, _, _ = _value_payload(sb.records.cpu().numpy(), H, torch.bfloat16)
        if len(ret_order):
            assert_bits_equal(vals, _wire_values(to_np32(out_rows)[ret_order], 1, torch.bfloat16, rounding, 9, r),
                              "return values")
        assert np.array_equal(meta[:, 0], rows.token_idx.cpu().numpy()[ret_order]), "token index"
        assert np.array_equal(meta[:, 1], rows.slot_idx.cpu().numpy()[ret_order]), "slot"
        back.append((sb.records, sb.counts.cpu().tolist()))
    for s in range(ep_size):
        parts = []
        for r in range(ep_size):
            rec, cnt = back[r]
            start = sum(cnt[:s])
            parts.append(rec[start:start + cnt[s]])
        got_rec = torch.cat(parts)
        T = tokens[s]
        out = ep.combine(got_rec, idxs[s].to(gpu_device), ws[s].to(gpu_device), H=H, value_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        assert out.shape == (T, H) and out.dtype == torch.bfloat16
        feat, meta, _, _ = _value_payload(got_rec.cpu().numpy(), H, torch.bfloat16)
        tok = torch.from_numpy(meta[:, 0].astype(np.int64))
        slot = torch.from_numpy(meta[:, 1].astype(np.int64))
        want = torch.zeros((T, H), dtype=torch.bfloat16)
        if len(tok):
            want.index_add_(0, tok, torch.from_numpy(feat).to(torch.bfloat16) * ws[s][tok, slot].unsqueeze(-1))
        assert_bits_equal(out.float().cpu().numpy(), want.float().numpy(), "combined tokens")
        if T:
            assert_bits_equal(out.float().cpu().numpy(),
                              O.ep_combine(feat, meta[:, 0], meta[:, 1], idxs[s].numpy(), ws[s].float().numpy(), T),
                              "combined tokens (oracle)")


@pytest.mark.parametrize("val_dtype,out_dtype", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32),
                                                 (torch.float32, torch.float32)])
def test_value_combine_rounds_each_value_to_the_output_dtype(gpu_device, val_dtype, out_dtype):
    """fp32 values combined into bf16 round to bf16 first (the reference's
    .to(tokens.dtype) after the exchange), then the product with the weight;
    bf16 values into fp32 are exact.  Against index_add_ on the CPU."""
    from lowbit import ep

    T, K, H = 9, 3, 256
    R, m_off = ep.value_record_layout(H, val_dtype)
    g = torch.Generator().manual_seed(20261420)
    idx = torch.stack([torch.randperm(8, generator=g)[:K] for _ in range(T)])
    w = torch.rand((T, K), generator=g).to(out_dtype)
    n = T * K - 2  # the last two assignments dropped
    vals = (torch.randn((n, H), generator=g) * 3).to(val_dtype)
    rec = np.zeros((n, R), dtype=np.uint8)
    esz = 2 if val_dtype == torch.bfloat16 else 4
    rec[:, :H * esz] = vals.view(torch.uint8).numpy().reshape(n, H * esz)
    perm = torch.randperm(n, generator=g).numpy()  # arrival order other than the assignment order
    a = np.arange(n)[perm]
    meta = np.zeros((n, 8), np.int32)
    meta[:, 0], meta[:, 1] = a // K, a % K
    rec[:, m_off:] = meta.view(np.uint8).reshape(n, 32)
    out = ep.combine(torch.from_numpy(rec).to(gpu_device), idx.to(gpu_device), w.to(gpu_device), H=H,
                     out_dtype=out_dtype, value_dtype=val_dtype)
    torch.cuda.synchronize()
    feat = vals.to(out_dtype)
    ref = torch.zeros((T, H), dtype=out_dtype)
    # index_add_ over the rows in ascending expert id per token: the CPU order for one token
    tok = torch.from_numpy(meta[:, 0].astype(np.int64))
    slot = torch.from_numpy(meta[:, 1].astype(np.int64))
    order = np.lexsort((idx.numpy()[meta[:, 0], meta[:, 1]], meta[:, 0]))
    o = torch.from_numpy(order)
    ref.index_add_(0, tok[o], feat[o] * w[tok[o], slot[o]].unsqueeze(-1))
    assert_bits_equal(out.float().cpu().numpy(), ref.float().numpy(), "combined values")
