"""GPU tests of the elementwise kernels of the trainable expert loop's
backward, each against torch's autograd of the reference loop's own
expressions (moe.py:1062-1093, :476-491, ExpertMLP :190-193):

- ntlb_moe_combine_backward against the backward of
  `output[token_indices] += expert_out * weights` (torch on the CPU): the
  expert-output gradient bit for bit, the routing-weight gradient to the
  last bit of its dtype (the fp32 sum runs in another order), for
  bf16 / fp16 / fp32 outputs and bf16 / fp32 weights, with dropped slots;
- ntlb_swiglu_backward against the backward of `F.silu(gate) * up` in bf16
  (torch on the GPU, the reference's device);
- ntlb_moe_token_grad against autograd's accumulation of the gathered
  tokens' gradients over the loop (torch on the CPU), with dropped slots,
  int32 and int64 expert ids.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _routing(T: int, E: int, k: int, seed: int, capacity: int, device):
    """expert ids [T, k] (distinct per token), softmax weights, and the GPU
    routing (route_by_expert with the capacity) copied to the CPU"""
    from lowbit import moe

    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    idx[: T // 3, 0] = 0  # a crowded expert, so a capacity drops rows
    idx[: T // 3, 1:] = torch.stack([torch.randperm(E - 1, generator=g)[:k - 1] + 1 for _ in range(T // 3)])
    w = torch.softmax(torch.randn(T, k, generator=g), dim=-1)
    r = moe.route_by_expert(idx.to(device), E, capacity=capacity, topk_w=w.to(device))
    return idx, w, r, r.pos.cpu(), r.inv.cpu(), r.offsets.cpu().tolist()


def _expert_rows(inv, offs, e: int, k: int):
    a = inv[offs[e]:offs[e + 1]].long()
    return a // k, a % k, torch.arange(offs[e], offs[e + 1])


def _ulp_diff16(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """distance in units of the last place of two same-sign 16-bit float tensors"""
    ia = a.contiguous().view(torch.int16).to(torch.int32)
    ib = b.contiguous().view(torch.int16).to(torch.int32)
    return (ia - ib).abs()


@pytest.mark.parametrize("ydt,wdt", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float16, torch.float32), (torch.float32, torch.float32)])
@pytest.mark.parametrize("H,capacity", [(512, 0), (196, 40)])
def test_combine_backward_matches_autograd(gpu_device, ydt, wdt, H, capacity):
    from lowbit import _lib, ops

    T, E, k = 300, 7, 3
    idx, w, r, pos, inv, offs = _routing(T, E, k, 20262501 + H, capacity, gpu_device)
    R = offs[-1]
    g = torch.Generator().manual_seed(20262502)
    y = (torch.randn(R, H, generator=g) * torch.exp(torch.randn(R, 1, generator=g))).to(ydt)
    d_out = torch.randn(T, H, generator=g).to(ydt)
    w = w.to(wdt)
    # the reference loop's combine under autograd, on the CPU
    yr = y.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    output = torch.zeros(T, H, dtype=ydt)
    for e in range(E):
        ti, si, rows = _expert_rows(inv, offs, e, k)
        if ti.numel():
            output[ti] += yr[rows] * wr[ti, si].unsqueeze(-1)
    output.backward(d_out)
    # the kernel
    sentinel = torch.full((R + 1, H), 7.0, dtype=ydt)
    dy = sentinel.to(gpu_device)
    d_w = torch.full((T, k), 5.0, dtype=wdt, device=gpu_device)
    yg, dg, wg = y.to(gpu_device), d_out.to(gpu_device), w.to(gpu_device)
    _lib.call("ntlb_moe_combine_backward", dg.data_ptr(), H, yg.data_ptr(), H, ops._dtype_code(ydt),
              r.pos.data_ptr(), wg.data_ptr(), ops._dtype_code(wdt), T, k, H, dy.data_ptr(), H, d_w.data_ptr(),
              ops._stream())
    torch.cuda.synchronize()
    dy, d_w = dy.cpu(), d_w.cpu()
    assert torch.equal(dy[:R], yr.grad)
    assert torch.equal(dy[R], sentinel[R])  # no row past the kept ones is written
    kept = (pos >= 0).reshape(T, k)
    assert bool((d_w[~kept] == 0).all()) and bool((wr.grad[~kept] == 0).all())
    if wdt == torch.float32:
        ref = wr.grad.double()
        assert torch.allclose(d_w.double(), ref, rtol=2e-6, atol=1e-6 * float(ref.abs().max()))
    else:
        ulp = _ulp_diff16(d_w, wr.grad)
        assert int(ulp.max()) <= 1
        assert float((ulp > 0).float().mean()) < 0.05


def test_combine_backward_dw_rounds_bf16_products(gpu_device):
    """With bf16 weights the routing-weight gradient sums the bf16-rounded
    products d * y (torch's mul backward), not the exact ones.  Each token
    has d * y = 16 * 16 = 256 and (129/128) * (255/256) = 1.003875..., which
    bf16 rounds to 1: the rounded products sum to 257, a tie that bf16
    rounds to 256, while the exact sum rounds to 258."""
    from lowbit import _lib, ops

    T, k, H = 64, 1, 256
    d = torch.zeros(T, H)
    y = torch.zeros(T, H)
    d[:, 0], y[:, 0] = 16.0, 16.0
    d[:, 1], y[:, 1] = 129 / 128, 255 / 256
    d, y = d.to(torch.bfloat16), y.to(torch.bfloat16)
    pos = torch.arange(T, dtype=torch.int32, device=gpu_device)
    dg, yg = d.to(gpu_device), y.to(gpu_device)
    dy = torch.empty(T, H, dtype=torch.bfloat16, device=gpu_device)
    # the reference's expression under autograd on the CPU
    wr = torch.ones(T, k, dtype=torch.bfloat16, requires_grad=True)
    (y * wr).backward(d)
    assert bool((wr.grad == 256).all())
    for wdt, want in ((torch.bfloat16, 256.0), (torch.float32, 257.0 + 127 / 32768)):
        w = torch.ones(T, k, dtype=wdt, device=gpu_device)
        d_w = torch.empty(T, k, dtype=wdt, device=gpu_device)
        _lib.call("ntlb_moe_combine_backward", dg.data_ptr(), H, yg.data_ptr(), H, ops._dtype_code(torch.bfloat16),
                  pos.data_ptr(), w.data_ptr(), ops._dtype_code(wdt), T, k, H, dy.data_ptr(), H, d_w.data_ptr(),
                  ops._stream())
        torch.cuda.synchronize()
        assert bool((d_w.cpu().double() == want).all()), (wdt, d_w[:4, 0].tolist())


@pytest.mark.parametrize("R,I", [(1000, 256), (37, 1024)])
def test_swiglu_backward_matches_autograd(gpu_device, R, I):
    from lowbit import _lib

    g = torch.Generator().manual_seed(20262511 + R)
    gate = (torch.randn(R, I, generator=g) * 4).to(torch.bfloat16)
    gate[0, :8] = torch.tensor([0.0, -0.0, 30.0, -30.0, 90.0, -90.0, 1e-3, -1e-3]).to(torch.bfloat16)
    up = torch.randn(R, I, generator=g).to(torch.bfloat16)
    dh = torch.randn(R, I, generator=g).to(torch.bfloat16)
    gg = gate.to(gpu_device).requires_grad_(True)
    uu = up.to(gpu_device).requires_grad_(True)
    (F.silu(gg) * uu).backward(dh.to(gpu_device))
    # interleaved columns: 128-column blocks alternating gate block t, up block t
    gu = torch.stack([gate.reshape(R, I // 128, 128), up.reshape(R, I // 128, 128)], dim=2).reshape(R, 2 * I)
    gu = gu.to(gpu_device)
    dhg = dh.to(gpu_device)
    dgu = torch.empty(R, 2 * I, dtype=torch.bfloat16, device=gpu_device)
    _lib.call("ntlb_swiglu_backward", dhg.data_ptr(), I, gu.data_ptr(), 2 * I, R, I, dgu.data_ptr(), 2 * I,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    v = dgu.cpu().reshape(R, I // 128, 2, 128)
    d_gate, d_up = v[:, :, 0].reshape(R, I), v[:, :, 1].reshape(R, I)
    assert torch.equal(d_up, uu.grad.cpu())
    assert torch.equal(d_gate, gg.grad.cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("idx_dtype,capacity", [(torch.int64, 0), (torch.int32, 30)])
def test_token_grad_matches_autograd_accumulation(gpu_device, dtype, idx_dtype, capacity):
    from lowbit import _lib, ops

    T, E, k, H = 200, 9, 4, 136
    idx, w, r, pos, inv, offs = _routing(T, E, k, 20262521, capacity, gpu_device)
    R = offs[-1]
    g = torch.Generator().manual_seed(20262522)
    dx = (torch.randn(R, H, generator=g) * torch.exp(torch.randn(R, 1, generator=g) * 3)).to(dtype)

    class _Inject(torch.autograd.Function):
        """the expert's input gradient is given: dx's rows of that expert"""

        @staticmethod
        def forward(ctx, x, grad):
            ctx.save_for_backward(grad)
            return x.clone()

        @staticmethod
        def backward(ctx, d):
            return ctx.saved_tensors[0], None

    tokens = torch.zeros(T, H, dtype=dtype, requires_grad=True)
    output = torch.zeros(T, H, dtype=dtype)
    for e in range(E):  # the reference loop's gathers, in its order
        ti, si, rows = _expert_rows(inv, offs, e, k)
        if ti.numel():
            output[ti] += _Inject.apply(tokens[ti], dx[rows])
    output.backward(torch.ones(T, H, dtype=dtype))
    out = torch.full((T, H), 3.0, dtype=dtype, device=gpu_device)
    ids = idx.to(idx_dtype).to(gpu_device)
    dxg = dx.to(gpu_device)
    _lib.call("ntlb_moe_token_grad", dxg.data_ptr(), H, ops._dtype_code(dtype), r.pos.data_ptr(), ids.data_ptr(),
              1 if idx_dtype == torch.int64 else 0, T, k, H, out.data_ptr(), H, ops._stream())
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), tokens.grad)


def _offsets(counts, device):
    o = [0]
    for c in counts:
        o.append(o[-1] + c)
    return o, torch.tensor(o, dtype=torch.int32, device=device)


COUNTS = [150, 0, 333, 97, 420]  # one expert without rows


@pytest.mark.parametrize("fmt", ["e4m3", "int_grid"])
def test_grouped_ste_dgrad_equals_per_expert_dgrad(gpu_device, fmt):
    """The rows-grouped straight-through dgrad gives, on each expert's rows,
    the dense dgrad's result over that expert's weight bit for bit (the
    same K loop over the same operands)."""
    from lowbit import moe, ops

    E, N, K = len(COUNTS), 384, 700
    offs, offsets = _offsets(COUNTS, gpu_device)
    R = offs[-1]
    g = torch.Generator().manual_seed(20262541)
    w = (torch.randn(E, N, K, generator=g) * 0.05).bfloat16().to(gpu_device)
    dy = torch.randn(R, N, generator=g).bfloat16().to(gpu_device)
    codes, scales, _ = moe.quantize_expert_weights(w, fmt=fmt)
    got = ops.grouped_ste_dgrad(dy, offsets, codes, scales, grid=ops.grid_code(fmt), K=K, out_dtype=torch.bfloat16)
    for e in range(E):
        lo, hi = offs[e], offs[e + 1]
        if hi == lo:
            continue
        qw, _ = ops.quant_block_128x128(w[e], fmt=fmt)
        want = ops.ste_dgrad(dy[lo:hi], qw, out_dtype=torch.bfloat16)
        assert torch.equal(got[lo:hi], want), e


def test_grouped_ste_dgrad_gate_up_adds_the_two_rounded_halves(gpu_device):
    """The gate/up dgrad over the interleaved layout equals bf16(dX_gate) +
    bf16(dX_up) added in bf16, each half the dense dgrad over that half's
    weight, bit for bit."""
    from lowbit import moe, ops

    E, I, H = len(COUNTS), 256, 640
    offs, offsets = _offsets(COUNTS, gpu_device)
    R = offs[-1]
    g = torch.Generator().manual_seed(20262542)
    wg = (torch.randn(E, I, H, generator=g) * 0.05).bfloat16().to(gpu_device)
    wu = (torch.randn(E, I, H, generator=g) * 0.05).bfloat16().to(gpu_device)
    d_gu = torch.randn(R, 2 * I, generator=g).bfloat16().to(gpu_device)
    codes, scales, _ = moe.quantize_expert_weights(moe.stack_gate_up(wg, wu))
    got = ops.grouped_ste_dgrad_gate_up(d_gu, offsets, codes, scales, grid=ops.grid_code("e4m3"), K=H)
    j = torch.arange(I, device=gpu_device)
    gate_cols = 256 * (j // 128) + j % 128
    for e in range(E):
        lo, hi = offs[e], offs[e + 1]
        if hi == lo:
            continue
        qg, _ = ops.quant_block_128x128(wg[e], fmt="e4m3")
        qu, _ = ops.quant_block_128x128(wu[e], fmt="e4m3")
        dg = ops.ste_dgrad(d_gu[lo:hi, gate_cols].contiguous(), qg, out_dtype=torch.bfloat16)
        du = ops.ste_dgrad(d_gu[lo:hi, gate_cols + 128].contiguous(), qu, out_dtype=torch.bfloat16)
        assert torch.equal(got[lo:hi], dg + du), e


@pytest.mark.parametrize("fmt", ["e4m3", "int_grid"])
def test_grouped_ste_wgrad_equals_per_expert_wgrad(gpu_device, fmt):
    """The contraction-grouped straight-through wgrad gives each expert the
    dense wgrad over that expert's rows bit for bit, and an expert without
    rows a zero gradient."""
    from lowbit import ops

    E, N, K = len(COUNTS), 384, 700
    offs, offsets = _offsets(COUNTS, gpu_device)
    R = offs[-1]
    g = torch.Generator().manual_seed(20262543)
    x = torch.randn(R, K, generator=g).bfloat16().to(gpu_device)
    dy = torch.randn(R, N, generator=g).bfloat16().to(gpu_device)
    qx = ops.quant_tile_1x128(x, fmt=fmt)
    got = ops.grouped_ste_wgrad(dy, offsets, qx, E, out_dtype=torch.bfloat16)
    for e in range(E):
        lo, hi = offs[e], offs[e + 1]
        if hi == lo:
            assert bool((got[e] == 0).all())
            continue
        qe = ops.quant_tile_1x128(x[lo:hi], fmt=fmt)
        want = ops.ste_wgrad(dy[lo:hi], qe, out_dtype=torch.bfloat16)
        assert torch.equal(got[e], want), e


# K = 700: rows of W and x are not whole 16-byte chunks, so the grouped
# kernels transpose those operands in registers while the dense references
# (whose wrappers pad the rows) use the transposing LDS loads; K = 704: both
# use the transposing loads
@pytest.mark.parametrize("K", [700, 704])
def test_grouped_dense_gemms_equal_per_expert_dense(gpu_device, K):
    """The grouped backward GEMMs over dense bf16 operands (the stochastic-
    rounding form of the expert loop's backward) equal, on each expert's
    rows, the dense kernels over that expert's operands bit for bit: dgrad
    and the interleaved gate/up dgrad against ops.gemm_dense (W read
    transposed), wgrad against ops.gemm_dense_tn; an expert without rows gets
    a zero weight gradient."""
    from lowbit import ops

    E, N, I = len(COUNTS), 384, 256
    offs, offsets = _offsets(COUNTS, gpu_device)
    R = offs[-1]
    g = torch.Generator().manual_seed(20262561)
    w = (torch.randn(E, N, K, generator=g) * 0.05).bfloat16().to(gpu_device)
    wgu = (torch.randn(E, 2 * I, K, generator=g) * 0.05).bfloat16().to(gpu_device)
    dy = torch.randn(R, N, generator=g).bfloat16().to(gpu_device)
    dgu = torch.randn(R, 2 * I, generator=g).bfloat16().to(gpu_device)
    x = torch.randn(R, K, generator=g).bfloat16().to(gpu_device)
    dx = ops.grouped_dgrad_dense(dy, offsets, w, out_dtype=torch.bfloat16)
    dxgu = ops.grouped_dgrad_dense_gate_up(dgu, offsets, wgu)
    dw = ops.grouped_wgrad_dense(dy, offsets, x, E, out_dtype=torch.bfloat16)
    j = torch.arange(I, device=gpu_device)
    gate, up = 256 * (j // 128) + j % 128, 256 * (j // 128) + 128 + j % 128
    for e in range(E):
        lo, hi = offs[e], offs[e + 1]
        if hi == lo:
            assert bool((dw[e] == 0).all())
            continue
        want = ops.gemm_dense(dy[lo:hi], w[e], b_transposed=True, out_dtype=torch.bfloat16)
        assert torch.equal(dx[lo:hi].view(torch.int16), want.view(torch.int16)), e
        dg = ops.gemm_dense(dgu[lo:hi, gate].contiguous(), wgu[e, gate].contiguous(), b_transposed=True,
                            out_dtype=torch.bfloat16)
        du = ops.gemm_dense(dgu[lo:hi, up].contiguous(), wgu[e, up].contiguous(), b_transposed=True,
                            out_dtype=torch.bfloat16)
        assert torch.equal(dxgu[lo:hi].view(torch.int16), (dg + du).view(torch.int16)), e
        want = ops.gemm_dense_tn(dy[lo:hi].contiguous(), x[lo:hi].contiguous(), out_dtype=torch.bfloat16)
        assert torch.equal(dw[e].view(torch.int16), want.view(torch.int16)), e
