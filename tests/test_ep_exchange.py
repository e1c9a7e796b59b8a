"""The host side of the expert-parallel exchange (lowbit.ep.exchange): one
count all_to_all and one byte all_to_all of fixed-size records deliver, to
every rank, each source's records for it in source-rank order -- the split
order of the reference's all_to_all_single calls (moe.py:720-863).  Three
processes over gloo on CPU tensors; the records carry (source, destination,
index) so the test sees where every byte went."""

from __future__ import annotations

import socket

import torch
import torch.multiprocessing as mp

R = 48
COUNTS = [[3, 0, 2], [1, 4, 0], [0, 2, 5]]  # COUNTS[src][dst]


def _records(src: int) -> torch.Tensor:
    rows = []
    for dst, c in enumerate(COUNTS[src]):
        for j in range(c):
            rows.append(torch.full((R,), 0, dtype=torch.uint8))
            rows[-1][0], rows[-1][1], rows[-1][2] = src, dst, j
            rows[-1][3:] = (src * 31 + dst * 7 + j) % 251
    return torch.stack(rows) if rows else torch.empty((0, R), dtype=torch.uint8)


def _worker(rank: int, world: int, port: int, queue) -> None:
    import torch.distributed as dist

    from lowbit.ep import SendBuffer, exchange

    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank, world_size=world)
    try:
        send = SendBuffer(_records(rank), torch.tensor(COUNTS[rank], dtype=torch.int64), H=0)
        recv, counts = exchange(send)
        queue.put((rank, counts, recv.clone()))
    finally:
        dist.destroy_process_group()


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def test_exchange_over_gloo():
    world = len(COUNTS)
    ctx = mp.get_context("spawn")
    queue = ctx.Queue()
    port = _free_port()
    procs = [ctx.Process(target=_worker, args=(r, world, port, queue)) for r in range(world)]
    for p in procs:
        p.start()
    results = {}
    try:
        for _ in range(world):
            rank, counts, recv = queue.get(timeout=120)
            results[rank] = (counts, recv)
    finally:
        for p in procs:
            p.join(timeout=60)
            if p.is_alive():
                p.kill()
    assert all(p.exitcode == 0 for p in procs)
    for dst in range(world):
        counts, recv = results[dst]
        assert counts == [COUNTS[src][dst] for src in range(world)]
        want = [row for src in range(world) for row in _records(src) if int(row[1]) == dst]
        want = torch.stack(want) if want else torch.empty((0, R), dtype=torch.uint8)
        assert torch.equal(recv, want)


def test_record_layouts_and_payload_modes():
    """Value records are whole 128-byte lines with the 32 metadata bytes last
    and room for the row; code records are unchanged.  The channel
    granularity takes value records (the only wire that carries one scale
    per column), and the other reference granularities take either wire."""
    import pytest

    from lowbit import _lib, ep

    for H, dt, esz in [(7168, torch.bfloat16, 2), (200, torch.bfloat16, 2), (200, torch.float32, 4), (8, torch.float32, 4)]:
        R, m_off = ep.value_record_layout(H, dt)
        assert R % 128 == 0 and m_off == R - 32 and H * esz <= m_off < H * esz + 128
    assert int(_lib.lib().ntlb_ep_value_record_bytes(0, 1)) == 0
    assert int(_lib.lib().ntlb_ep_value_record_bytes(64, 7)) == 0
    R, s_off, m_off = ep.record_layout(7168)
    assert (R, s_off, m_off) == (7424, 7168, 7392)

    assert ep._payload_mode("channel", None, None, 512)[2:] == (1, True)
    assert ep._payload_mode("tile_1x128", None, None, 512)[2:] == (128, False)
    assert ep._payload_mode("block_128x128", None, None, 512, "values")[2:] == (128, True)
    assert ep._payload_mode("tensor", None, None, 512)[2:] == (512, False)
    assert ep._payload_mode(None, None, None, 512)[2:] == (None, False)
    with pytest.raises(ValueError, match="channel"):
        ep._payload_mode("channel", None, None, 512, "codes")
    with pytest.raises(ValueError, match="granularity"):
        ep._payload_mode(None, None, None, 512, "values")
    with pytest.raises(ValueError, match="granularity"):
        ep._payload_mode("per_row", None, None, 512)
    with pytest.raises(ValueError, match="wire"):
        ep._payload_mode("tensor", None, None, 512, "bytes")
