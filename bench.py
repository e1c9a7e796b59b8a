"""Benchmark of the low-bit linear hot path on one MI355X.

One step = one emulated-FP8 Linear forward of benchmark config 2 (the
DeepSeek-V3 dense MLP up-projection): quantize X [8192, 7168] per 1x128 tile,
quantize W [18432, 7168] per 128x128 block (e4m3, amax/448 scales, round to
nearest), and the blockwise-scaled FP8 GEMM Y = X_dq W_dq^T (fp32 accumulate,
bf16 out).  Inputs are resident in HBM before the timed region; three input
sets rotate so that no step reads its inputs from the 256 MB Infinity Cache.

Before the W counted warm-up steps, the step runs untimed for SPIN_UP_S
seconds so that the timed steps see the sustained clock, not the ramp from
idle.  `value` = GEMM FLOPs per step / step time (quantizers included).  The
`roofline` object is the GEMM kernel alone, timed with HIP events on the
stream the kernels run on.  `cpu_baseline` times the reference's emulated
path as its own torch op sequence (oracle/torch_emulated.py) on the host's
cores, over a 1024-row sample of the same workload.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--format e4m3|int_grid]
                  [--rounding nearest|stochastic] [--no-cpu-baseline]
                  [--config c1|c2|c3|c4|c5] [--backward fp8|ste]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from typing import Optional

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nano-train_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0  # dense fp8 (and int8 TOP/s) of MI355X
SPIN_UP_S = 0.3  # untimed sustained load before the counted warm-up steps


def parse_args():
    global SPIN_UP_S
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--format", default="e4m3", choices=["e4m3", "int_grid"])
    p.add_argument("--rounding", default=None, choices=["nearest", "stochastic"],
                   help="default: nearest, except c3, whose dY quantizers use the seeded stochastic rounding "
                        "its benchmark configuration names")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-sample-rows", type=int, default=1024)
    p.add_argument("--calib-copy", action="store_true",
                   help="also launch a plain 1 GiB device copy (HBM counter calibration for rocprofv3 --pmc)")
    p.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"],
                   help="c2 (default) is the headline; c1/c3/c4/c5 measure the other benchmark configurations")
    p.add_argument("--no-library-compare", action="store_true",
                   help="skip the library GEMMs timed for comparison (hipBLASLt through torch.matmul), so that a "
                        "kernel trace holds this build's kernels only")
    p.add_argument("--backward", default="fp8", choices=["fp8", "ste"],
                   help="c3: fp8 = the quantized dgrad/wgrad recipe of the configuration; ste = the reference's "
                        "straight-through backward (dY unquantized, operands bf16(q*s) decoded in the GEMM)")
    p.add_argument("--spin-up-s", type=float, default=SPIN_UP_S,
                   help="seconds of untimed sustained load before the counted warm-up steps; 0 times the steps "
                        "from an idle GPU, inside the clock ramp")
    a = p.parse_args()
    SPIN_UP_S = a.spin_up_s
    if a.rounding is None:
        a.rounding = "stochastic" if a.config == "c3" else "nearest"
    return a


def _spin_up(fn, seconds: Optional[float] = None) -> None:
    """Run fn untimed for `seconds` of wall time.  From idle, the clocks take
    about 50 ms of sustained load to settle (a c2 GEMM runs 7-30% slower over
    its first launches); the timed steps should see the sustained rate that a
    training loop runs at."""
    import torch

    if seconds is None:
        seconds = SPIN_UP_S
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        fn(i)
        i += 1
        if i % 4 == 0:
            torch.cuda.synchronize()  # keep the host within a few launches of the GPU
    torch.cuda.synchronize()


def _time_ms(fn, n: int, warmup: int, stream) -> float:
    import torch

    # the full spin-up before every timed op: hipBLASLt's GEMMs (the library
    # comparisons) read up to 25% slow for the first ~0.1 s at a new shape
    _spin_up(fn, SPIN_UP_S)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record(stream)
    for i in range(n):
        fn(warmup + i)
    ev[1].record(stream)
    torch.cuda.synchronize()
    return ev[0].elapsed_time(ev[1]) / n


def _calibration_copy(dev) -> None:
    """A plain 1 GiB device copy: its FETCH_SIZE / WRITE_SIZE calibrate the HBM counters."""
    import torch

    a = torch.empty(1 << 29, dtype=torch.int16, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()


def other_config(args) -> dict:
    """One line for benchmark configs 1, 3, 4, 5 (kernel times by HIP events)."""
    import torch

    from lowbit import moe, ops, persistent, workloads

    dev = torch.device("cuda", 0)
    st = torch.cuda.current_stream()
    fmt = args.format
    res = {"metric": f"{args.config} throughput", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "data": "synthetic (seeded)",
           "cpu_baseline": None}
    if args.config == "c1":
        x, w = workloads.c1_inputs(device="cpu")
        x, w = x.to(dev), w.to(dev)
        step = lambda i: ops.gemm_blockscaled(ops.quant_tile_1x128(x, fmt=fmt), ops.quant_block_128x128(w, fmt=fmt)[0])
        ms = _time_ms(step, args.steps, args.warmup, st)
        # the same step captured in a HIP graph: the three launches replayed without the host in between
        side = torch.cuda.Stream()
        side.wait_stream(st)
        with torch.cuda.stream(side):
            step(0)
            step(0)
        st.wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(0)
        g_ms = _time_ms(lambda i: graph.replay(), args.steps, args.warmup, st)
        res.update(value=round(2 * 512 * 1024 * 1024 / (ms * 1e-3) / 1e12, 3), unit="TFLOP/s",
                   ms_per_step=round(ms, 4), graph_ms_per_step=round(g_ms, 4),
                   dtype="fp8_e4m3" if fmt == "e4m3" else "int8",
                   config={"workload": "c1 small emulated-FP8 Linear forward (latency-bound)", "M": 512, "N": 1024,
                           "K": 1024})
        return res
    if args.config == "c3":
        x, w = workloads.c2_inputs(device="cpu")
        dy = workloads.c3_grad(device="cpu")
        x, w, dy = x.to(dev), w.to(dev), dy.to(dev)
        M, K = x.shape
        N = w.shape[0]
        if args.backward == "ste":
            return _c3_ste(args, res, x, w, dy, st)
        qx_t = ops.quant_tile_128x1_t(x, fmt=fmt)
        _, qw_t = ops.quant_block_128x128(w, fmt=fmt, want_transposed=True)
        t = {}
        rnd = dict(rounding=args.rounding, seed=3)  # the recipe's dY rounding (c3: seeded stochastic by default)
        t["dy_1x128_us"] = _time_ms(lambda i: ops.quant_tile_1x128(dy, fmt=fmt, **rnd), args.steps, args.warmup,
                                    st) * 1e3
        t["dy_128x1_us"] = _time_ms(lambda i: ops.quant_tile_128x1_t(dy, fmt=fmt, **rnd), args.steps, args.warmup,
                                    st) * 1e3
        t["dy_dual_us"] = _time_ms(lambda i: ops.quant_dual_1x128_128x1(dy, fmt=fmt, **rnd), args.steps,
                                   args.warmup, st) * 1e3
        qdy = ops.quant_tile_1x128(dy, fmt=fmt, **rnd)
        qdy_t = ops.quant_tile_128x1_t(dy, fmt=fmt, **rnd)
        dg = _time_ms(lambda i: ops.gemm_blockscaled(qdy, qw_t), args.steps, args.warmup, st)
        wg = _time_ms(lambda i: ops.gemm_blockscaled(qdy_t, qx_t), args.steps, args.warmup, st)
        fl = 2.0 * M * N * K
        # HBM bytes per dgrad launch (uniform B scales: template <GRID, true, false, 0>) from the committed profile
        traffic = None
        prof = os.path.join(ROOT, "profiles", f"c3_backward_{fmt}.json")
        dg_name = f"gemm_blockscaled_kernel<{1 if fmt == 'e4m3' else 0}, true, false, 0>"
        if os.path.exists(prof):
            with open(prof) as fh:
                for kname, tv in json.load(fh).get("traffic", {}).items():
                    if dg_name in kname:
                        traffic = int(tv["total_bytes"])
        res.update(value=round(2 * fl / ((dg + wg) * 1e-3) / 1e12, 2), unit="TFLOP/s", ms_per_step=round(dg + wg, 4),
                   dtype="fp8_e4m3" if fmt == "e4m3" else "int8",
                   config={"workload": "c3 backward GEMMs (dgrad + wgrad) of the c2 layer, fp8 recipe", "M": M,
                           "N": N, "K": K, "dy_rounding": args.rounding},
                   roofline={"bound": "mfma", "kernel": "gemm_blockscaled_kernel (dgrad, split-K tail)",
                             "achieved": round(fl / (dg * 1e-3) / 1e12, 2), "peak": FP8_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(fl / (dg * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                             "traffic": traffic, "traffic_source": f"profiles/c3_backward_{fmt}.md" if traffic else None,
                             "avg_ms": round(dg, 4)},
                   dgrad_tflops=round(fl / (dg * 1e-3) / 1e12, 2), wgrad_tflops=round(fl / (wg * 1e-3) / 1e12, 2),
                   quantizers={k: round(v, 2) for k, v in t.items()},
                   dy_1x128_GBs=round((M * N * 3 + M * (N // 128) * 4) / t["dy_1x128_us"] / 1e3, 1),
                   dy_128x1_GBs=round((M * N * 3 + N * (M // 128) * 4) / t["dy_128x1_us"] / 1e3, 1),
                   dy_dual_GBs=round((M * N * 4 + M * (N // 128) * 4 + N * (M // 128) * 4) / t["dy_dual_us"] / 1e3,
                                     1))
        return res
    if args.config == "c4":
        tokens, routing, w_up, w_down = workloads.c4_inputs(device="cpu")
        w_gate = workloads.c4_gate(device="cpu")
        # the dispatched rows for the comm-quant lines, gathered on the host
        # (set-up, not a timed step)
        order = torch.sort(routing.reshape(-1), stable=True).indices
        xs = tokens[order // routing.shape[1]].to(dev)
        del order
        tokens, routing = tokens.to(dev), routing.to(dev)
        w_up, w_down, w_gate = w_up.to(dev), w_down.to(dev), w_gate.to(dev)
        route = moe.route_by_expert(routing, 32)
        offsets = route.offsets
        # routing weights in the token dtype, as the reference's router returns them
        topk_w = torch.rand(routing.shape, generator=torch.Generator().manual_seed(4), dtype=torch.float32).to(dev)
        w_b = topk_w.to(torch.bfloat16)
        R, H = xs.shape
        inter = w_up.shape[1]
        qg = moe.quantize_expert_weights(w_gate, fmt=fmt)
        qu = moe.quantize_expert_weights(w_up, fmt=fmt)
        gate_up = moe.interleave_gate_up(qg[0], qg[1], qu[0], qu[1], qg[2], qu[2])
        del qg, qu
        down = moe.quantize_expert_weights(w_down, fmt=fmt)
        w_gu = moe.stack_gate_up(w_gate, w_up)  # the trainable loop's [E, 2I, H] master weights
        del w_gate, w_up
        comm_us = _time_ms(lambda i: moe.comm_quant(xs, fmt=fmt), args.steps, args.warmup, st) * 1e3
        payload = moe.comm_quant(xs, fmt=fmt)
        dequant_us = _time_ms(lambda i: moe.comm_dequant(payload), args.steps, args.warmup, st) * 1e3
        del payload
        # the reference's own comm-quant (_comm_quant_dequant, strip granularity) as a drop-in: the amax pass,
        # then the quantize pass writing tensor + (dq - tensor)
        ref_cq_us = _time_ms(lambda i: moe.comm_quant_dequant(xs, granularity="tile_1x128", rounding_mode="nearest",
                                                              seed=1, offset=i), args.steps, args.warmup, st) * 1e3
        # the step: the single-rank expert loop's forward on HIP kernels, from
        # the token rows and the routing to the token outputs
        layer = _time_ms(lambda i: moe.local_moe_forward(tokens, routing, w_b, gate_up, down, n_experts=32, fmt=fmt),
                         args.steps, args.warmup, st)
        mlp = _time_ms(lambda i: moe.expert_mlp(xs, offsets, gate_up, down, fmt=fmt), args.steps, args.warmup, st)
        # the kernels of one step, timed alone
        route_us = _time_ms(lambda i: moe.route_by_expert(routing, 32), args.steps, args.warmup, st) * 1e3
        fan_us = _time_ms(lambda i: ops.quant_tile_1x128_fanout(tokens, route.pos, 8, route.rows, fmt=fmt,
                                                                want_nan_rows=True), args.steps, args.warmup,
                          st) * 1e3
        y_rows = moe.expert_mlp(xs, offsets, gate_up, down, fmt=fmt)
        comb_rows_us = _time_ms(lambda i: moe.combine_rows(y_rows, route, routing, w_b, tokens.shape[0]), args.steps,
                                args.warmup, st) * 1e3
        del y_rows
        qx = ops.quant_tile_1x128(xs, fmt=fmt)
        _, qh = ops.gemm_swiglu_quant(qx, gate_up[0], gate_up[1], offsets=offsets, fmt=fmt, want_h=False)
        qx_us = _time_ms(lambda i: ops.quant_tile_1x128(xs, fmt=fmt), args.steps, args.warmup, st) * 1e3
        gu_ms = _time_ms(lambda i: ops.gemm_swiglu_quant(qx, gate_up[0], gate_up[1], offsets=offsets, fmt=fmt,
                                                         want_h=False), args.steps, args.warmup, st)
        dn_ms = _time_ms(lambda i: ops.gemm_grouped_blockscaled(qh, down[0], down[1], offsets, N=H),
                         args.steps, args.warmup, st)
        # the trainable loop (moe.local_moe): quantize the bf16 expert weights,
        # forward, and the backward to the tokens, the routing weights and the
        # expert weights; and its grouped straight-through GEMMs alone
        leaves = [t.clone().requires_grad_(True) for t in (tokens, topk_w, w_gu, w_down)]
        d_out = (torch.randn(tokens.shape, generator=torch.Generator().manual_seed(6)) * 1e-2).to(dev, torch.bfloat16)

        def train_fwd(i):
            return moe.local_moe(leaves[0], routing, leaves[1], leaves[2], leaves[3], fmt=fmt)

        def train_step(i):
            for t in leaves:
                t.grad = None
            train_fwd(i).backward(d_out)

        train_ms = _time_ms(train_step, args.steps, args.warmup, st)
        train_fwd_ms = _time_ms(train_fwd, args.steps, args.warmup, st)
        for t in leaves:
            t.grad = None
        del leaves
        dyr = (torch.randn((R, H), generator=torch.Generator().manual_seed(7)) * 1e-3).to(dev, torch.bfloat16)
        d_gu = (torch.randn((R, 2 * inter), generator=torch.Generator().manual_seed(8)) * 1e-3).to(dev, torch.bfloat16)
        grid_c = ops.grid_code(fmt)
        dg_dn_ms = _time_ms(lambda i: ops.grouped_ste_dgrad(dyr, offsets, down[0], down[1], grid=grid_c, K=inter,
                                                            out_dtype=torch.bfloat16), args.steps, args.warmup, st)
        dg_gu_ms = _time_ms(lambda i: ops.grouped_ste_dgrad_gate_up(d_gu, offsets, gate_up[0], gate_up[1],
                                                                    grid=grid_c, K=H), args.steps, args.warmup, st)
        wg_dn_ms = _time_ms(lambda i: ops.grouped_ste_wgrad(dyr, offsets, qh, 32, out_dtype=torch.bfloat16),
                            args.steps, args.warmup, st)
        wg_gu_ms = _time_ms(lambda i: ops.grouped_ste_wgrad(d_gu, offsets, qx, 32, out_dtype=torch.bfloat16),
                            args.steps, args.warmup, st)
        del dyr, d_gu, w_gu
        # expert-parallel wire format, one GPU's share of an 8-rank layout (4 experts per rank):
        # pack every (token, slot) assignment into a record, unpack as many received records
        from lowbit import ep

        send = ep.pack_dispatch(tokens, routing, topk_w, experts_per_rank=4, ep_size=8, fmt=fmt)
        rcounts = send.counts.cpu().tolist()
        pack_us = _time_ms(lambda i: ep.pack_dispatch(tokens, routing, topk_w, experts_per_rank=4, ep_size=8, fmt=fmt),
                           args.steps, args.warmup, st) * 1e3
        unpack_us = _time_ms(lambda i: ep.unpack_dispatch(send.records, rcounts, H=H, local_experts=4, fmt=fmt),
                             args.steps, args.warmup, st) * 1e3
        rec_b = send.records.shape[1]
        n_rec = send.records.shape[0]
        # the return trip: every row's expert output back as a record, then the
        # weighted sum into the 4096 token outputs
        rows = ep.unpack_dispatch(send.records, rcounts, H=H, local_experts=4, fmt=fmt)
        out_rows = torch.randn((n_rec, H), generator=torch.Generator().manual_seed(5), dtype=torch.float32)
        out_rows = out_rows.to(dev, torch.bfloat16)
        ret = ep.pack_return(out_rows, rows, ep_size=8, fmt=fmt)
        ret_us = _time_ms(lambda i: ep.pack_return(out_rows, rows, ep_size=8, fmt=fmt), args.steps, args.warmup,
                          st) * 1e3
        comb_us = _time_ms(lambda i: ep.combine(ret.records, routing, w_b, H=H, fmt=fmt), args.steps, args.warmup,
                           st) * 1e3
        ret_bytes = n_rec * (H * 2 + rec_b)
        comb_bytes = n_rec * rec_b + tokens.shape[0] * H * 2
        # the reference's channel comm-quant on the same layout: value records
        # (the bf16 wire values and the metadata), both directions
        chv = dict(granularity="channel")
        send_v = ep.pack_dispatch(tokens, routing, topk_w, experts_per_rank=4, ep_size=8, **chv)
        vpack_us = _time_ms(lambda i: ep.pack_dispatch(tokens, routing, topk_w, experts_per_rank=4, ep_size=8, **chv),
                            args.steps, args.warmup, st) * 1e3
        vunpack_us = _time_ms(lambda i: ep.unpack_dispatch(send_v.records, rcounts, H=H, local_experts=4,
                                                           value_dtype=torch.bfloat16), args.steps, args.warmup,
                              st) * 1e3
        rows_v = ep.unpack_dispatch(send_v.records, rcounts, H=H, local_experts=4, value_dtype=torch.bfloat16)
        ret_v = ep.pack_return(out_rows, rows_v, ep_size=8, **chv)
        vret_us = _time_ms(lambda i: ep.pack_return(out_rows, rows_v, ep_size=8, **chv), args.steps, args.warmup,
                           st) * 1e3
        vcomb_us = _time_ms(lambda i: ep.combine(ret_v.records, routing, w_b, H=H, value_dtype=torch.bfloat16),
                            args.steps, args.warmup, st) * 1e3
        rec_v = send_v.records.shape[1]
        T_t = tokens.shape[0]
        # HBM bytes: the amax pass reads the rows once and the pack once more;
        # the unpack writes each row's values and 4 metadata words
        ep_values = {"record_bytes": rec_v, "pack_us": round(vpack_us, 2),
                     "pack_GBs": round((2 * T_t * H * 2 + n_rec * rec_v) / vpack_us / 1e3, 1),
                     "unpack_us": round(vunpack_us, 2),
                     "unpack_GBs": round(n_rec * (rec_v + H * 2 + 16) / vunpack_us / 1e3, 1),
                     "return_pack_us": round(vret_us, 2),
                     "return_pack_GBs": round(n_rec * (2 * H * 2 + rec_v) / vret_us / 1e3, 1),
                     "combine_us": round(vcomb_us, 2),
                     "combine_GBs": round((n_rec * rec_v + T_t * H * 2) / vcomb_us / 1e3, 1)}
        del rows, out_rows, ret, send_v, rows_v, ret_v
        # pack: every bf16 token row read once, one record written per assignment;
        # unpack: one record read, codes + tile scales + 5 words of metadata written per row
        pack_bytes = tokens.shape[0] * H * 2 + n_rec * rec_b
        unpack_bytes = n_rec * (rec_b + ops.cdiv(H, 128) * 128 + ops.cdiv(H, 128) * 4 + 20)
        del send
        fl = 2.0 * R * H * inter  # one projection
        comm_bytes = R * H * 3 + R * (H // 128) * 4
        T_tok = tokens.shape[0]
        # HBM bytes per gate/up launch from the committed FETCH_SIZE / WRITE_SIZE runs
        traffic = None
        prof = os.path.join(ROOT, "profiles", f"c4_moe_experts_{fmt}.json")
        gu_name = f"gemm_blockscaled_kernel<{1 if fmt == 'e4m3' else 0}, true, true, 1>"
        if os.path.exists(prof):
            with open(prof) as fh:
                for kname, tv in json.load(fh).get("traffic", {}).items():
                    if gu_name in kname:
                        traffic = int(tv["total_bytes"])
        res.update(value=round(3 * fl / (layer * 1e-3) / 1e12, 2), unit="TFLOP/s", ms_per_step=round(layer, 4),
                   dtype="fp8_e4m3" if fmt == "e4m3" else "int8",
                   config={"workload": "c4 MoE local experts, the single-rank expert loop's forward for all 32 "
                                       "experts: routing sort, 1x128 quantization of the token rows gathered by "
                                       "expert, gate+up GEMM with SwiGLU and 1x128 h in the epilogue, down GEMM, "
                                       "weighted combine into token order",
                           "tokens": T_tok, "rows": R, "hidden": H, "inter": inter, "experts": 32, "top_k": 8},
                   roofline={"bound": "mfma", "kernel": "gemm_blockscaled_kernel (gate+up with SwiGLU)",
                             "achieved": round(2 * fl / (gu_ms * 1e-3) / 1e12, 2), "peak": FP8_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(2 * fl / (gu_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                             "traffic": traffic,
                             "traffic_source": f"profiles/c4_moe_experts_{fmt}.md" if traffic else None,
                             "avg_ms": round(gu_ms, 4)},
                   expert_mlp_ms=round(mlp, 4),
                   train={"what": "moe.local_moe forward + backward (the reference loop under autograd): bf16 "
                                  "expert weights quantized each step, gradients of tokens, routing weights and "
                                  "both weight stacks",
                          "step_ms": round(train_ms, 4), "forward_ms": round(train_fwd_ms, 4),
                          "tflops": round(9 * fl / (train_ms * 1e-3) / 1e12, 2),
                          "dgrad_down_tflops": round(fl / (dg_dn_ms * 1e-3) / 1e12, 2),
                          "dgrad_gate_up_tflops": round(2 * fl / (dg_gu_ms * 1e-3) / 1e12, 2),
                          "wgrad_down_tflops": round(fl / (wg_dn_ms * 1e-3) / 1e12, 2),
                          "wgrad_gate_up_tflops": round(2 * fl / (wg_gu_ms * 1e-3) / 1e12, 2),
                          "peak_bf16_tflops": 2500.0},
                   route_us=round(route_us, 2), gather_quant_x_us=round(fan_us, 2),
                   gather_quant_x_GBs=round((T_tok * H * 2 + R * H + R * (H // 128) * 4) / fan_us / 1e3, 1),
                   combine_rows_us=round(comb_rows_us, 2),
                   combine_rows_GBs=round((R * H * 2 + T_tok * H * 2) / comb_rows_us / 1e3, 1),
                   gate_up_swiglu_tflops=round(2 * fl / (gu_ms * 1e-3) / 1e12, 2),
                   down_tflops=round(fl / (dn_ms * 1e-3) / 1e12, 2), quant_x_us=round(qx_us, 2),
                   comm_quant_us=round(comm_us, 2), comm_quant_GBs=round(comm_bytes / comm_us / 1e3, 1),
                   comm_dequant_us=round(dequant_us, 2),
                   comm_dequant_GBs=round((R * H * 3 + R * (H // 128) * 4) / dequant_us / 1e3, 1),
                   reference_comm_quant_dequant_us=round(ref_cq_us, 2),
                   reference_comm_quant_dequant_GBs=round(R * H * 2 * 3 / ref_cq_us / 1e3, 1),
                   ep_dispatch={"records": n_rec, "record_bytes": rec_b, "pack_us": round(pack_us, 2),
                                "pack_GBs": round(pack_bytes / pack_us / 1e3, 1), "unpack_us": round(unpack_us, 2),
                                "unpack_GBs": round(unpack_bytes / unpack_us / 1e3, 1),
                                "return_pack_us": round(ret_us, 2), "return_pack_GBs": round(ret_bytes / ret_us / 1e3, 1),
                                "combine_us": round(comb_us, 2), "combine_GBs": round(comb_bytes / comb_us / 1e3, 1),
                                "channel_values": ep_values})
        return res
    # c5
    x, w = workloads.c5_inputs(device="cpu")
    x, w = x.to(dev), w.to(dev)
    M, K = x.shape
    N = w.shape[0]
    pk, sc = persistent.quantize_nf4_blocks(w, 64)
    mx_packed, mx_scales = persistent.quantize_mxfp4(w)
    f8_vals, f8_scale = persistent.quantize_fp8_persistent(w, granularity="per_channel")
    # the optimizer side of the same weight: AdamW step + NF4 refresh, fused and as two passes
    from lowbit import optim

    n = N * K
    master = w.float().reshape(-1).contiguous()
    mst, vst = torch.zeros_like(master), torch.zeros_like(master)
    grad = (torch.randn(n, device=dev, dtype=torch.bfloat16) * 1e-3)
    wp = w.reshape(-1).clone()
    codes = torch.empty(n // 2, dtype=torch.uint8, device=dev)
    scl = torch.empty(n // 64, dtype=torch.float32, device=dev)
    hp = dict(lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, step=1)
    fused_ms = _time_ms(lambda i: optim.adamw_step_refresh(master, grad, mst, vst, param=wp, refresh="nf4", block=64,
                                                           codes=codes, scales=scl, **hp), args.steps, args.warmup, st)
    two_ms = _time_ms(lambda i: (optim.adamw_step_refresh(master, grad, mst, vst, param=wp, **hp),
                                 persistent.quantize_nf4_blocks(wp, 64)), args.steps, args.warmup, st)
    # grad bf16 in, fp32 master/m/v in and out, bf16 param out, NF4 codes and 64-block scales out
    opt_bytes = n * (2 + 12 + 12 + 2) + n // 2 + (n // 64) * 4
    nf4 = _time_ms(lambda i: persistent.linear_nf4(x, pk, sc, out_features=N, block=64), args.steps, args.warmup, st)
    mx = _time_ms(lambda i: persistent.linear_mxfp4(x, mx_packed, mx_scales, out_features=N), args.steps, args.warmup,
                  st)
    f8 = _time_ms(lambda i: persistent.linear_fp8p(x, f8_vals, f8_scale), args.steps, args.warmup, st)
    fl = 2.0 * M * N * K
    # HBM bytes per NF4 fused launch from the committed profile
    traffic = None
    prof = os.path.join(ROOT, "profiles", "c5_persistent_fused.json")
    if os.path.exists(prof):
        with open(prof) as fh:
            for kname, tv in json.load(fh).get("traffic", {}).items():
                if "gemm_lowbit_fused_kernel<0>" in kname:
                    traffic = int(tv["total_bytes"])
    bf = unf = None
    if not args.no_library_compare:
        bf = _time_ms(lambda i: torch.matmul(x, w.t()), args.steps, args.warmup, st)
        # the unfused alternative: the NF4 dequant kernel to a bf16 weight, then torch's bf16 matmul
        unf = _time_ms(lambda i: torch.matmul(x, persistent.dequantize_nf4_blocks(
            pk, sc, num_values=N * K, block=64, target_dtype=torch.bfloat16).view(N, K).t()), args.steps,
            args.warmup, st)
    res.update(value=round(fl / (nf4 * 1e-3) / 1e12, 2), unit="TFLOP/s", ms_per_step=round(nf4, 4), dtype="bf16",
               config={"workload": "c5 NF4 (64-element blocks) dequant-fused GEMM", "M": M, "N": N, "K": K},
               roofline={"bound": "mfma", "kernel": "gemm_lowbit_fused_kernel<NF4> (split-K tail)",
                         "achieved": round(fl / (nf4 * 1e-3) / 1e12, 2), "peak": 2500.0,
                         "unit": "TFLOP/s", "frac": round(fl / (nf4 * 1e-3) / 1e12 / 2500.0, 4), "traffic": traffic,
                         "traffic_source": "profiles/c5_persistent_fused.md" if traffic else None,
                         "avg_ms": round(nf4, 4)},
               mxfp4_tflops=round(fl / (mx * 1e-3) / 1e12, 2),
               fp8_persistent_tflops=round(fl / (f8 * 1e-3) / 1e12, 2),
               adamw_nf4_refresh={"fused_us": round(fused_ms * 1e3, 1), "two_pass_us": round(two_ms * 1e3, 1),
                                  "fused_GB/s": round(opt_bytes / (fused_ms * 1e-3) / 1e9, 1), "params": n},
               torch_bf16_matmul_tflops=None if bf is None else round(fl / (bf * 1e-3) / 1e12, 2),
               nf4_dequant_then_torch_matmul_tflops=None if unf is None else round(fl / (unf * 1e-3) / 1e12, 2))
    return res


def _c3_ste(args, res: dict, x, w, dy, st) -> dict:
    """c3 shapes with the reference's straight-through backward
    (te_backend.py:250-259 under autograd): dX = dY @ bf16(W_dq),
    dW = dY^T @ bf16(X_dq), db = sum dY, from the forward's codes."""
    import torch

    from lowbit import ops
    from lowbit.backend import HipLowBitBackend
    from lowbit.contracts import LowBitKernelSpec

    fmt = args.format
    M, K = x.shape
    N = w.shape[0]
    qx = ops.quant_tile_1x128(x, fmt=fmt)
    qw, _ = ops.quant_block_128x128(w, fmt=fmt)
    bf = torch.bfloat16
    # each kernel alone, HIP events on the stream it runs on
    dg = _time_ms(lambda i: ops.ste_dgrad(dy, qw, out_dtype=bf), args.steps, args.warmup, st)
    wg = _time_ms(lambda i: ops.ste_wgrad(dy, qx, out_dtype=bf), args.steps, args.warmup, st)
    db = _time_ms(lambda i: ops.colsum(dy, out_dtype=bf), args.steps, args.warmup, st)
    # e4m3: the wgrad variant that also forms db from its register-transposed
    # dY tiles (one launch; the layer step runs the plain wgrad and the column
    # sum, which is faster); its extra time against the plain wgrad
    wg_db = None
    if fmt == "e4m3":
        wg_db = _time_ms(lambda i: ops.ste_wgrad(dy, qx, out_dtype=bf, db_dtype=bf), args.steps, args.warmup, st)
    # the whole layer step through the backend's autograd function: both
    # quantizers, the forward GEMM, dgrad, wgrad and db
    spec = LowBitKernelSpec("linear", K, N, True, "tile_1x128", "block_128x128", "nearest")
    be = HipLowBitBackend(mode="fp8", kernel_spec=spec, code_format=fmt, seed=7)
    xg = x.detach().clone().requires_grad_(True)
    wg_ = w.detach().clone().requires_grad_(True)
    b = torch.zeros(N, device=x.device, dtype=bf, requires_grad=True)

    def layer(i):
        xg.grad = wg_.grad = b.grad = None
        be.linear(xg, wg_, b).backward(dy)

    layer_ms = _time_ms(layer, args.steps, args.warmup, st)
    fwd_ms = _time_ms(lambda i: be.linear(x, w, None), args.steps, args.warmup, st)
    fl = 2.0 * M * N * K
    tf = lambda ms: round(fl / (ms * 1e-3) / 1e12, 2)
    # HBM bytes per dgrad launch from the committed FETCH_SIZE / WRITE_SIZE runs
    traffic = None
    prof = os.path.join(ROOT, "profiles", "c3_backward_ste.json")
    if fmt == "e4m3" and os.path.exists(prof):
        with open(prof) as fh:
            for kname, tv in json.load(fh).get("traffic", {}).items():
                if "gemm_dq_kernel<0, 0, 3, 1" in kname:
                    traffic = int(tv["total_bytes"])
    lib = None
    if not args.no_library_compare:
        # the same two products as library GEMMs over dequantized bf16
        # operands (what this path replaced: hipBLASLt through torch.matmul)
        wdq = ops.dequant(qw, out_dtype=bf)
        xdq = ops.dequant(qx, out_dtype=bf)
        lib_dg = _time_ms(lambda i: torch.matmul(dy, wdq), args.steps, args.warmup, st)
        lib_wg = _time_ms(lambda i: torch.matmul(dy.t(), xdq), args.steps, args.warmup, st)
        del wdq, xdq
        lib = {"dgrad_tflops": tf(lib_dg), "wgrad_tflops": tf(lib_wg)}
    res.update(value=round(2 * fl / ((dg + wg) * 1e-3) / 1e12, 2), unit="TFLOP/s", ms_per_step=round(dg + wg, 4),
               dtype="bf16",
               config={"workload": "c3 shapes, the reference's straight-through backward: dX = dY bf16(W_dq), "
                                   "dW = dY^T bf16(X_dq) decoded from the forward's codes, db = sum dY",
                       "M": M, "N": N, "K": K, "code_format": fmt},
               roofline={"bound": "mfma", "kernel": "gemm_dq_kernel (dgrad)", "achieved": tf(dg), "peak": 2500.0,
                         "unit": "TFLOP/s", "frac": round(fl / (dg * 1e-3) / 1e12 / 2500.0, 4), "traffic": traffic,
                         "traffic_source": "profiles/c3_backward_ste.md" if traffic else None,
                         "min_hbm_bytes": M * N * 2 + N * K + M * K * 2, "avg_ms": round(dg, 4)},
               dgrad_tflops=tf(dg), wgrad_tflops=tf(wg), wgrad_frac_bf16_peak=round(tf(wg) / 2500.0, 4),
               db_colsum_us=round(db * 1e3, 2), db_colsum_GBs=round(M * N * 2 / (db * 1e-3) / 1e9, 1),
               wgrad_with_db_us=None if wg_db is None else round(wg_db * 1e3, 2),
               db_in_wgrad_extra_us=None if wg_db is None else round((wg_db - wg) * 1e3, 2),
               layer_forward_backward_ms=round(layer_ms, 4), layer_forward_ms=round(fwd_ms, 4),
               hipblaslt_on_dequantized_bf16=lib)
    return res


def _median_s(fn, runs: int = 3) -> float:
    """Median wall time of `runs` calls after one warm-up call."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def _host_threads() -> int:
    """CPU threads this process may run on (its affinity mask)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return int(os.cpu_count() or 1)


def cpu_baseline(args) -> dict:
    """The reference's emulated path as its own torch op sequence
    (oracle/torch_emulated.py restates te_backend.py:40-260 and
    layers.py:142-184) on the host's cores, over a bounded sample of the
    configuration: median of 3 timed runs after 1 warm-up.  The C oracle's
    one-thread 1x128 quantizer is reported beside it (c2)."""
    import numpy as np
    import torch

    from lowbit import moe, workloads
    from oracle import torch_emulated as T

    threads = _host_threads()
    torch.set_num_threads(threads)
    config = args.config
    extra = {}
    if config in ("c1", "c2"):
        rows = args.cpu_sample_rows
        x, w = workloads.c1_inputs(device="cpu") if config == "c1" else workloads.c2_inputs(device="cpu", rows=rows)
        rnd = args.rounding

        def run():
            with torch.no_grad():
                return T.emulated_linear(x, w, None, act="tile_1x128", wgt="block_128x128", rounding=rnd)

        flops = 2.0 * x.shape[0] * w.shape[0] * w.shape[1]
        what = (f"the reference's emulated linear (1x128 X and 128x128 W fake quantization, int grid, {rnd}, "
                f"fp32 F.linear) over X rows [0, {x.shape[0]}) of config {config[1]} with the full W "
                f"{list(w.shape)}")
        q_t = _median_s(lambda: T.quantize_dequantize(x, bits=8, granularity="tile_1x128", rounding=rnd,
                                                      channel_axis=-1))
        q_bytes = x.numel() * 3 + x.shape[0] * (x.shape[1] // 128) * 4
        extra["quantizer_GB/s"] = round(q_bytes / q_t / 1e9, 3)
        if config == "c2":
            from oracle import oracle as O

            O.lib()
            xn = x.float().numpy()
            grid = O.GRID_E4M3 if args.format == "e4m3" else O.GRID_INT
            c_t = _median_s(lambda: O.quant_tile_1x128(xn, grid=grid))
            extra["oracle_c_1thread"] = {"quantizer_GB/s": round(q_bytes / c_t / 1e9, 3),
                                         "what": "the C oracle's 1x128 quantizer on 1 thread, same rows"}
    elif config == "c3":
        rows = 512
        x, w = workloads.c2_inputs(device="cpu", rows=rows)
        dy = workloads.c3_grad(device="cpu")[:rows].contiguous()
        xg = x.clone().requires_grad_(True)
        wg = w.clone().requires_grad_(True)
        y = T.emulated_linear(xg, wg, None, act="tile_1x128", wgt="block_128x128", rounding="nearest")

        def run():
            return torch.autograd.grad(y, (xg, wg), dy, retain_graph=True)

        flops = 4.0 * rows * w.shape[0] * w.shape[1]
        what = (f"the reference's straight-through backward (autograd of the emulated linear: fp32 dX = dY W_q, "
                f"dW = dY^T X_q) over rows [0, {rows}) of config 3; the reference has no quantized-gradient "
                f"recipe, so this is its backward for both --backward modes")
    elif config == "c4":
        rows = 512
        tokens, routing, _, _ = workloads.c4_inputs(device="cpu", experts=0)
        n_exp = workloads.SHAPES[4]["experts"]
        # the rows of each expert in the reference's nonzero() order (a stable
        # sort by expert) and the offset table, on the host
        flat = routing.reshape(-1)
        tok_idx = torch.sort(flat, stable=True).indices // routing.shape[1]
        off = [0] + torch.bincount(flat, minlength=n_exp).cumsum(0).tolist()
        reach = int(np.searchsorted(np.asarray(off), rows, side="left"))
        _, _, w_up, w_down = workloads.c4_inputs(device="cpu", experts=min(reach, n_exp))
        w_gate = workloads.c4_gate(device="cpu", experts=min(reach, n_exp))
        xs = tokens[tok_idx[:rows]]
        parts = [(e, max(off[e], 0), min(off[e + 1], rows)) for e in range(len(off) - 1) if off[e] < rows]
        parts = [p for p in parts if p[2] > p[1]]

        def run():
            with torch.no_grad():
                outs = []
                for e, lo, hi in parts:  # moe.py:888-962 with ExpertMLP (moe.py:146-193) per expert
                    xe = xs[lo:hi]
                    g = T.emulated_linear(xe, w_gate[e], None)
                    u = T.emulated_linear(xe, w_up[e], None)
                    h = torch.nn.functional.silu(g) * u
                    outs.append(T.emulated_linear(h, w_down[e], None))
                return outs

        flops = 6.0 * rows * w_up.shape[2] * w_up.shape[1]
        what = (f"the reference's per-expert loop over expert-sorted rows [0, {rows}) of config 4 "
                f"({len(parts)} expert(s)): gate, up and down emulated Linears (1x128 / 128x128, int grid, "
                f"each weight quantized per call) and F.silu(gate) * up")
    else:
        rows = 256
        x, w = workloads.c5_inputs(device="cpu")
        xs = x[:rows].contiguous()
        N, K = w.shape
        from oracle import oracle as O

        packed, sc = O.nf4_quant(w.float().numpy(), 64)  # the persistent codes exist before the step
        pk, sct = torch.from_numpy(packed), torch.from_numpy(sc)

        def run():
            with torch.no_grad():
                wd = T.nf4_dequantize(pk, sct, numel=N * K, block=64, dtype=torch.bfloat16).view(N, K)
                return torch.nn.functional.linear(xs, wd)

        flops = 2.0 * rows * N * K
        what = (f"the reference's persistent NF4 forward: unpack, codebook times 64-block scale, cast to bf16 "
                f"(layers.py:142-184), then a bf16 F.linear, over X rows [0, {rows}) of config 5")
    dt = _median_s(run)
    out = {"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
           "sample": f"{what}: {dt:.3f} s, median of 3 runs after 1 warm-up; torch CPU ops on {threads} threads "
                     f"(the process's affinity; os.cpu_count() = {os.cpu_count()}); CPU {_cpu_model()}"}
    out.update(extra)
    return out


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (the kernels run on one GPU's share of a "
                                   "sharded layer); run with --gpus 1"}))
        sys.exit(2)

    import torch

    from lowbit import ops, workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.config != "c2":
        if args.calib_copy:
            _calibration_copy(dev)
        res = other_config(args)
        if not args.no_cpu_baseline:
            res["cpu_baseline"] = cpu_baseline(args)
        print(json.dumps(res))
        return
    shp = workloads.SHAPES[2]
    M, N, K = shp["M"], shp["N"], shp["K"]

    # input set 0 from the seeded CPU generators (identical to the parity tests),
    # sets 1 and 2 are device-side permutations of it at other addresses
    x0, w0 = workloads.c2_inputs(device="cpu")
    x0, w0 = x0.to(dev), w0.to(dev)
    sets = [(x0, w0), (-x0, w0.flip(0).contiguous()), (x0.flip(0).contiguous(), -w0)]
    torch.cuda.synchronize()

    rounding = args.rounding
    stream = torch.cuda.current_stream()

    def step(i, ev=None):
        x, w = sets[i % len(sets)]
        if ev is not None:
            ev[0].record(stream)
        qx = ops.quant_tile_1x128(x, fmt=args.format, rounding=rounding, seed=1, offset=2 * i)
        if ev is not None:
            ev[1].record(stream)
        qw, _ = ops.quant_block_128x128(w, fmt=args.format, rounding=rounding, seed=1, offset=2 * i + 1)
        if ev is not None:
            ev[2].record(stream)
        y = ops.gemm_blockscaled(qx, qw, out_dtype=torch.bfloat16)
        if ev is not None:
            ev[3].record(stream)
        return y

    _spin_up(step)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        y = step(args.warmup + i, events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    del y

    qx_ms = [e[0].elapsed_time(e[1]) for e in events]
    qw_ms = [e[1].elapsed_time(e[2]) for e in events]
    gm_ms = [e[2].elapsed_time(e[3]) for e in events]
    step_ms = [e[0].elapsed_time(e[3]) for e in events]
    avg = lambda v: sum(v) / len(v)
    flops = 2.0 * M * N * K
    ms_per_step = wall * 1e3 / args.steps
    value = flops / (ms_per_step * 1e-3) / 1e12

    # algorithmic bytes of the quantizers: bf16 in + 1-byte code + fp32 scale per tile/block
    qx_bytes = M * K * 2 + M * K + M * (K // 128) * 4
    qw_bytes = N * K * 2 + N * K + (N // 128) * (K // 128) * 4
    gemm_tflops = flops / (avg(gm_ms) * 1e-3) / 1e12
    # the GEMM's own minimum HBM traffic: both code matrices, their scales, bf16 out
    gemm_min_bytes = M * K + N * K + M * (K // 128) * 4 + (N // 128) * (K // 128) * 4 + M * N * 2

    # each quantizer on its own over the same rotating inputs: inside the step it
    # follows the previous GEMM, whose 0.3 GB of output is still being written back
    qx_alone = _time_ms(lambda i: ops.quant_tile_1x128(sets[i % len(sets)][0], fmt=args.format, rounding=rounding,
                                                       seed=1, offset=2 * i), args.steps, args.warmup, stream)
    qw_alone = _time_ms(lambda i: ops.quant_block_128x128(sets[i % len(sets)][1], fmt=args.format, rounding=rounding,
                                                          seed=1, offset=2 * i + 1), args.steps, args.warmup, stream)

    # the other two GEMMs of the same forward on the same inputs: the
    # reference-exact mode (bf16(q*s) operands decoded in the GEMM, bf16 MFMA)
    # and the int-grid codes of the reference's numerics on int8 MFMA
    xq0 = ops.quant_tile_1x128(sets[0][0], fmt=args.format)
    wq0, _ = ops.quant_block_128x128(sets[0][1], fmt=args.format)
    ref_ms = _time_ms(lambda i: ops.gemm_dq_forward(xq0, wq0), args.steps, args.warmup, stream)
    del xq0, wq0
    other_fmt = "int_grid" if args.format == "e4m3" else "e4m3"
    xq1 = ops.quant_tile_1x128(sets[0][0], fmt=other_fmt)
    wq1, _ = ops.quant_block_128x128(sets[0][1], fmt=other_fmt)
    other_ms = _time_ms(lambda i: ops.gemm_blockscaled(xq1, wq1), args.steps, args.warmup, stream)
    del xq1, wq1
    ref_tf = flops / (ref_ms * 1e-3) / 1e12
    other_tf = flops / (other_ms * 1e-3) / 1e12

    # library ceilings at the same shape: hipBLASLt's FP8 GEMM through
    # torch._scaled_mm with one scale per tensor and with row-wise scales (one
    # per row of X, one per row of W, applied once in the epilogue).  Blockwise
    # 1x128 / 128x128 scales inside K are not offered by the library.
    lib_fp8 = None
    if args.format == "e4m3" and not args.no_library_compare:
        lib_fp8 = {}
        xq0 = ops.quant_tile_1x128(sets[0][0], fmt="e4m3")
        wq0, _ = ops.quant_block_128x128(sets[0][1], fmt="e4m3")
        a8 = xq0.codes[:, :K].view(torch.float8_e4m3fn)
        b8 = wq0.codes[:, :K].view(torch.float8_e4m3fn).t()
        one = torch.ones((), device=dev, dtype=torch.float32)
        sa_row = torch.rand(M, 1, device=dev, dtype=torch.float32) + 0.5
        sb_col = torch.rand(1, N, device=dev, dtype=torch.float32) + 0.5
        for name, sa_, sb_ in (("tensorwise", one, one), ("rowwise", sa_row, sb_col)):
            try:
                ms = _time_ms(lambda i: torch._scaled_mm(a8, b8, scale_a=sa_, scale_b=sb_, out_dtype=torch.bfloat16),
                              args.steps, args.warmup, stream)
                lib_fp8[name] = {"tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                                 "frac_peak": round(flops / (ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                                 "avg_ms": round(ms, 4)}
            except (RuntimeError, NotImplementedError) as exc:
                lib_fp8[name] = {"error": str(exc).splitlines()[0][:160]}
        del xq0, wq0, a8, b8

    # achievable HBM rate on this box: a 1 GiB device-to-device copy (read + write)
    ca = torch.empty(1 << 29, dtype=torch.int16, device=dev)
    cb = torch.empty_like(ca)
    cb.copy_(ca)
    ce = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ce[0].record(stream)
    for _ in range(5):
        cb.copy_(ca)
    ce[1].record(stream)
    torch.cuda.synchronize()
    copy_gbs = 5 * 2 * ca.numel() * 2 / (ce[0].elapsed_time(ce[1]) * 1e-3) / 1e9
    del ca, cb

    if args.calib_copy:
        _calibration_copy(dev)

    # HBM bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE (calibrated
    # against a 1 GiB copy) for this workload, committed under profiles/
    traffic = {}
    prof = os.path.join(ROOT, "profiles", f"c2_forward_{args.format}.json")
    if rounding == "nearest" and os.path.exists(prof):
        with open(prof) as fh:
            pj = json.load(fh)
        # the kernels of this format (template argument GRID: 1 = e4m3, 0 = int
        # grid); the line also runs the other format's GEMM once
        g = 1 if args.format == "e4m3" else 0
        names = {"gemm_blockscaled_kernel": f"gemm_blockscaled_kernel<{g}, true, false, 0>",
                 "quant_tile_1x128": f"quant_tile_1x128_fast<1, {g}, false, false, false>",
                 "quant_block_128x128": f"quant_block_128x128_fast<1, {g}, false, false>"}
        for kname, tv in pj.get("traffic", {}).items():
            for short, full in names.items():
                if full in kname:
                    traffic[short] = int(tv["total_bytes"])

    result = {
        "metric": "FP8 blockwise GEMM TFLOP/s (% fp8 MFMA peak); quantizer GB/s (% HBM peak)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "spin_up_s": SPIN_UP_S,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3" if args.format == "e4m3" else "int8",
        "data": "synthetic (seeded, benchmark config 2 distributions); 3 rotating input sets",
        "config": {
            "workload": "c2 DeepSeek-V3 dense MLP up-projection forward: quant X 1x128 + quant W 128x128 + "
                        "blockwise-scaled GEMM",
            "M": M, "N": N, "K": K, "code_format": args.format, "rounding": rounding,
            "out_dtype": "bf16", "parallelism": "single-gpu",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_blockscaled_kernel",
            "achieved": round(gemm_tflops, 2),
            "peak": FP8_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / FP8_PEAK_TFLOPS, 4),
            "traffic": traffic.get("gemm_blockscaled_kernel"),
            "traffic_source": f"profiles/c2_forward_{args.format}.md" if traffic else None,
            "avg_ms": round(avg(gm_ms), 4),
            "median_ms": round(sorted(gm_ms)[len(gm_ms) // 2], 4),
            "min_hbm_bytes": gemm_min_bytes,
        },
        "quantizers": {
            "x_tile_1x128": {"avg_us": round(avg(qx_ms) * 1e3, 2), "bytes": qx_bytes,
                             "alone_us": round(qx_alone * 1e3, 2),
                             "alone_GB/s": round(qx_bytes / (qx_alone * 1e-3) / 1e9, 1),
                             "alone_frac_hbm": round(qx_bytes / (qx_alone * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                             "traffic": traffic.get("quant_tile_1x128"),
                             "GB/s": round(qx_bytes / (avg(qx_ms) * 1e-3) / 1e9, 1),
                             "frac_hbm": round(qx_bytes / (avg(qx_ms) * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
            "w_block_128x128": {"avg_us": round(avg(qw_ms) * 1e3, 2), "bytes": qw_bytes,
                                "alone_us": round(qw_alone * 1e3, 2),
                                "alone_GB/s": round(qw_bytes / (qw_alone * 1e-3) / 1e9, 1),
                                "alone_frac_hbm": round(qw_bytes / (qw_alone * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                "traffic": traffic.get("quant_block_128x128"),
                                "GB/s": round(qw_bytes / (avg(qw_ms) * 1e-3) / 1e9, 1),
                                "frac_hbm": round(qw_bytes / (avg(qw_ms) * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        },
        "reference_forward_gemm": {"kernel": "gemm_dq_kernel (codes decoded to bf16(q*s), bf16 MFMA)",
                                   "tflops": round(ref_tf, 2), "frac_bf16_peak": round(ref_tf / 2500.0, 4),
                                   "avg_ms": round(ref_ms, 4)},
        f"{other_fmt}_gemm": {"kernel": "gemm_blockscaled_kernel", "tflops": round(other_tf, 2),
                              "frac_peak": round(other_tf / FP8_PEAK_TFLOPS, 4), "avg_ms": round(other_ms, 4)},
        "hipblaslt_fp8_scaled_mm": lib_fp8,
        "hbm_copy_GB/s": round(copy_gbs, 1),
        "event_ms_per_step": round(avg(step_ms), 4),
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
