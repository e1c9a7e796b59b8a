"""GPU parity of the persistent low-bit weights: NF4 (layers.py:60-184),
persistent FP8 (layers.py:104-127), MXFP4, and the dequant-fused GEMMs.
Codes and scales bit-exact against the oracle; GEMMs within 1e-3 relative
Frobenius of the float64 matmul over the bf16-rounded dequantized weight."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu_util import assert_bits_equal, rel_fro_bf16, seeded, to_np32
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(64, 128), (129, 257), (7,), (33, 64)])
@pytest.mark.parametrize("granularity", ["per_channel", "per_tensor"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_nf4_persistent_parity(gpu_device, shape, granularity, dtype):
    from lowbit import persistent as P

    w = seeded(shape, seed=20260501, std=0.02, dtype=dtype).to(gpu_device)
    packed, scale = P.quantize_nf4_persistent(w, granularity=granularity)
    torch.cuda.synchronize()
    block = (w.numel() // shape[0]) if (granularity == "per_channel" and len(shape) > 1) else w.numel()
    p_ref, s_ref = O.nf4_quant(to_np32(w), block)
    assert packed.dtype == torch.uint8 and packed.numel() == (w.numel() + 1) // 2
    assert_bits_equal(packed.cpu().numpy(), p_ref, "nf4 packed")
    assert_bits_equal(scale.reshape(-1).cpu().numpy(), s_ref, "nf4 scale")
    expect_shape = (shape[0],) + (1,) * (len(shape) - 1) if (granularity == "per_channel" and len(shape) > 1) else ()
    assert tuple(scale.shape) == expect_shape
    deq = P.dequantize_nf4_persistent(packed, scale, num_values=w.numel(), target_shape=w.shape, target_dtype=dtype)
    d_ref = O.nf4_dequant(p_ref, s_ref, w.numel(), block)
    assert_bits_equal(to_np32(deq).reshape(-1), torch.from_numpy(d_ref).to(dtype).float().numpy(), "nf4 dequant")


def test_nf4_special_values_and_ties(gpu_device):
    from lowbit import persistent as P

    cb = O.NF4_CODEBOOK
    mids = [(cb[i] + cb[i + 1]) / np.float32(2) for i in range(15)]
    w = torch.tensor([1.0] + mids + [float("nan"), 0.0, -0.0, 1e-40], dtype=torch.float32).to(gpu_device)
    packed, scale = P.quantize_nf4_persistent(w, granularity="per_tensor")
    p_ref, s_ref = O.nf4_quant(to_np32(w), w.numel())
    assert_bits_equal(packed.cpu().numpy(), p_ref, "nf4 packed")
    assert_bits_equal(scale.reshape(-1).cpu().numpy(), s_ref, "nf4 scale")


def test_nf4_index_around_every_bracket_edge(gpu_device):
    """Every codebook entry and every midpoint between neighbours, and the 64
    floats on each side of each, with a unit scale (the tensor holds 1.0), so
    the kernel's codebook search meets each bracket boundary and each
    distance tie at float resolution; codes against the oracle's argmin."""
    from lowbit import persistent as P

    cb = O.NF4_CODEBOOK.astype(np.float32)
    edges = list(cb) + [(cb[i] + cb[i + 1]) / np.float32(2) for i in range(15)]
    vals = [np.float32(1.0)]
    for e in edges:
        up = dn = np.float32(e)
        vals.append(up)
        for _ in range(64):
            up = np.nextafter(up, np.float32(2))
            dn = np.nextafter(dn, np.float32(-2))
            vals += [up, dn]
    w = torch.from_numpy(np.clip(np.array(vals, dtype=np.float32), -1, 1)).to(gpu_device)
    packed, scale = P.quantize_nf4_persistent(w, granularity="per_tensor")
    p_ref, s_ref = O.nf4_quant(to_np32(w), w.numel())
    assert float(s_ref.reshape(-1)[0]) == 1.0
    assert_bits_equal(packed.cpu().numpy(), p_ref, "nf4 packed")
    # the 64-element block quantizer shares the search
    wb = torch.nn.functional.pad(w, (0, (-w.numel()) % 64))
    wb[::64] = 1.0
    pb, sb = P.quantize_nf4_blocks(wb, 64)
    pb_ref, sb_ref = O.nf4_quant(to_np32(wb), 64)
    assert_bits_equal(pb.cpu().numpy(), pb_ref, "nf4 blocks packed")
    assert_bits_equal(sb.reshape(-1).cpu().numpy(), sb_ref, "nf4 blocks scales")


@pytest.mark.parametrize("shape", [(64, 128), (129, 256), (8, 96)])
@pytest.mark.parametrize("granularity", ["per_channel", "per_tensor"])
def test_fp8_persistent_parity(gpu_device, shape, granularity):
    from lowbit import persistent as P

    w = seeded(shape, seed=20260502, std=0.02, dtype=torch.bfloat16).to(gpu_device)
    w[0, 0] = float("inf") if shape[0] > 8 else w[0, 0]
    vals, scale = P.quantize_fp8_persistent(w, granularity=granularity)
    torch.cuda.synchronize()
    block = shape[1] if granularity == "per_channel" else w.numel()
    c_ref, s_ref = O.fp8_persistent_quant(to_np32(w), block)
    assert vals.dtype == torch.float8_e4m3fn
    assert_bits_equal(vals.view(torch.uint8).reshape(-1).cpu().numpy(), c_ref, "fp8 codes")
    assert_bits_equal(scale.reshape(-1).cpu().numpy(), s_ref, "fp8 scale")
    deq = P.dequantize_fp8_persistent(vals, scale, target_dtype=torch.bfloat16)
    ref = (torch.from_numpy(c_ref).view(torch.float8_e4m3fn).float() * torch.from_numpy(np.repeat(s_ref, block))
           ).to(torch.bfloat16)
    assert_bits_equal(to_np32(deq).reshape(-1), ref.float().numpy(), "fp8 dequant")


@pytest.mark.parametrize("n", [64, 1000, 32 * 7 + 3])
def test_mxfp4_parity(gpu_device, n):
    from lowbit import persistent as P

    w = seeded((n,), seed=20260503, std=0.02, dtype=torch.float32).to(gpu_device)
    w[5] = 0.0
    if n > 100:
        w[40:72] = 0.0  # an all-zero block
        w[80] = float("nan")
    packed, scales = P.quantize_mxfp4(w)
    p_ref, s_ref = O.mxfp4_quant(to_np32(w))
    assert_bits_equal(scales.cpu().numpy(), s_ref, "e8m0 scales")
    assert_bits_equal(packed.cpu().numpy(), p_ref, "e2m1 codes")
    d = P.dequantize_mxfp4(packed, scales, num_values=n, target_dtype=torch.float32)
    assert_bits_equal(to_np32(d), O.mxfp4_dequant(p_ref, s_ref, n), "mxfp4 dequant")


@pytest.mark.parametrize("M,N,K,block", [(256, 256, 256, 64), (100, 300, 512, 64), (512, 384, 1024, 1024),
                                         (64, 128, 128, 0)])
def test_nf4_fused_gemm(gpu_device, M, N, K, block):
    from lowbit import persistent as P

    x = seeded((M, K), seed=20260504).to(gpu_device)
    w = seeded((N, K), seed=20260505, std=0.02).to(gpu_device)
    qb = block if block else N * K
    packed, scales = P.quantize_nf4_blocks(w, qb)
    y = P.linear_nf4(x, packed, scales, out_features=N, block=qb)
    torch.cuda.synchronize()
    p_ref, s_ref = O.nf4_quant(to_np32(w), qb)
    wdq = O.round_bf16(O.nf4_dequant(p_ref, s_ref, N * K, qb)).reshape(N, K)  # weight dtype bf16 (layers.py:184)
    assert rel_fro_bf16(y, O.gemm_ref(to_np32(x), wdq)) <= 1e-3


def _fused_unsplit(fmt, x, w, scales, block, N, out_dtype):
    """The fused GEMM through the entry points without a workspace (every
    tile whole)."""
    from lowbit import ops
    from lowbit._lib import call

    M, K = x.shape
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if fmt == "nf4":
        call("ntlb_gemm_nf4", x.data_ptr(), x.stride(0), w.data_ptr(), scales.data_ptr(), block, M, N, K,
             y.data_ptr(), ops._dtype_code(out_dtype), y.stride(0), ops._stream())
    elif fmt == "mxfp4":
        call("ntlb_gemm_mxfp4", x.data_ptr(), x.stride(0), w.data_ptr(), scales.data_ptr(), M, N, K, y.data_ptr(),
             ops._dtype_code(out_dtype), y.stride(0), ops._stream())
    else:
        call("ntlb_gemm_fp8p", x.data_ptr(), x.stride(0), w.data_ptr(), scales.data_ptr(), block, M, N, K,
             y.data_ptr(), ops._dtype_code(out_dtype), y.stride(0), ops._stream())
    return y


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4", "fp8p"])
def test_fused_gemm_split_tail_and_bias(gpu_device, fmt):
    """M 4096, N 5120, K 2048: 320 tiles on 256 compute units, so the 64 tail
    tiles run as 3 K ranges each.  The split GEMM (fp32 out, no bias) equals
    the unsplit one within fp32 reassociation, repeats bit for bit (the
    workspace counters reset), and with a bias matches the oracle."""
    from lowbit import _lib, persistent as P

    M, N, K = 4096, 5120, 2048
    if int(_lib.lib().ntlb_gemm_lowbit_workspace_bytes(M, N, K)) == 0:
        pytest.skip("this device runs the shape unsplit")
    x = seeded((M, K), seed=20260510).to(gpu_device)
    w = seeded((N, K), seed=20260511, std=0.02).to(gpu_device)
    bias = seeded((N,), seed=20260512, std=0.5).to(gpu_device)
    if fmt == "nf4":
        codes, scales = P.quantize_nf4_blocks(w, 64)
        run = lambda b, od: P.linear_nf4(x, codes, scales, out_features=N, block=64, bias=b, out_dtype=od)
        sc, blk = scales.reshape(-1).contiguous(), 64
        p_ref, s_ref = O.nf4_quant(to_np32(w), 64)
        wdq = O.round_bf16(O.nf4_dequant(p_ref, s_ref, N * K, 64)).reshape(N, K)
    elif fmt == "mxfp4":
        codes, scales = P.quantize_mxfp4(w)
        run = lambda b, od: P.linear_mxfp4(x, codes, scales, out_features=N, bias=b, out_dtype=od)
        sc, blk = scales, 32
        p_ref, s_ref = O.mxfp4_quant(to_np32(w))
        wdq = O.round_bf16(O.mxfp4_dequant(p_ref, s_ref, N * K)).reshape(N, K)
    else:
        vals, scale = P.quantize_fp8_persistent(w, granularity="per_channel")
        run = lambda b, od: P.linear_fp8p(x, vals, scale, bias=b, out_dtype=od)
        codes, sc, blk = vals.view(torch.uint8), scale.reshape(-1).contiguous().float(), K
        c, s = O.fp8_persistent_quant(to_np32(w), K)
        wdq = O.round_bf16((O.decode_codes(c, O.GRID_E4M3) * np.repeat(s, K)).reshape(N, K))
    y_split = run(None, torch.float32)
    y_again = run(None, torch.float32)
    y_whole = _fused_unsplit(fmt, x, codes, sc, blk, N, torch.float32)
    y_bias = run(bias, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(y_split, y_again)
    d = (y_split.double() - y_whole.double()).norm() / y_whole.double().norm()
    assert float(d) <= 1e-6, float(d)
    rows = np.random.default_rng(5).choice(M, 48, replace=False)
    rows[:8] = np.arange(M - 8, M)  # the last row tile is a split tail tile
    ref = O.gemm_ref(to_np32(x)[rows], wdq, to_np32(bias))
    assert rel_fro_bf16(y_bias[rows], ref) <= 1e-3


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (130, 200, 320), (512, 512, 2048)])
def test_mxfp4_fused_gemm(gpu_device, M, N, K):
    from lowbit import persistent as P

    x = seeded((M, K), seed=20260506).to(gpu_device)
    w = seeded((N, K), seed=20260507, std=0.02).to(gpu_device)
    packed, scales = P.quantize_mxfp4(w)
    y = P.linear_mxfp4(x, packed, scales, out_features=N)
    torch.cuda.synchronize()
    p_ref, s_ref = O.mxfp4_quant(to_np32(w))
    wdq = O.round_bf16(O.mxfp4_dequant(p_ref, s_ref, N * K)).reshape(N, K)
    assert rel_fro_bf16(y, O.gemm_ref(to_np32(x), wdq)) <= 1e-3


def test_c5_nf4_fused_gemm_full_size_sampled(gpu_device):
    """benchmark config 5: W [14336, 4096] NF4 (64-element blocks), X [4096, 4096]."""
    from lowbit import persistent as P, workloads

    x, w = workloads.c5_inputs(device="cpu")
    xg, wg = x.to(gpu_device), w.to(gpu_device)
    packed, scales = P.quantize_nf4_blocks(wg, 64)
    y = P.linear_nf4(xg, packed, scales, out_features=14336, block=64)
    torch.cuda.synchronize()
    p_ref, s_ref = O.nf4_quant(w.float().numpy(), 64)
    assert_bits_equal(packed.cpu().numpy(), p_ref, "c5 nf4 codes")
    rows = np.random.default_rng(0).choice(4096, 32, replace=False)
    cols = np.random.default_rng(1).choice(14336, 256, replace=False)
    wdq = O.round_bf16(O.nf4_dequant(p_ref, s_ref, 14336 * 4096, 64)).reshape(14336, 4096)
    ref = O.gemm_ref(x.float().numpy()[rows], wdq[cols])
    assert rel_fro_bf16(y[rows][:, cols], ref) <= 1e-3


def test_c5_mxfp4_fused_gemm_full_size_sampled(gpu_device):
    """benchmark config 5 as MXFP4 (32-element blocks, e8m0 scales): W
    [14336, 4096], X [4096, 4096]; codes and scales bit for bit, the fused
    GEMM on sampled rows and columns against the oracle."""
    from lowbit import persistent as P, workloads

    x, w = workloads.c5_inputs(device="cpu")
    xg, wg = x.to(gpu_device), w.to(gpu_device)
    packed, scales = P.quantize_mxfp4(wg)
    y = P.linear_mxfp4(xg, packed, scales, out_features=14336)
    torch.cuda.synchronize()
    p_ref, s_ref = O.mxfp4_quant(w.float().numpy())
    assert_bits_equal(packed.cpu().numpy(), p_ref, "c5 mxfp4 codes")
    assert_bits_equal(scales.cpu().numpy(), s_ref, "c5 mxfp4 scales")
    rows = np.random.default_rng(3).choice(4096, 32, replace=False)
    cols = np.random.default_rng(4).choice(14336, 256, replace=False)
    wdq = O.round_bf16(O.mxfp4_dequant(p_ref, s_ref, 14336 * 4096)).reshape(14336, 4096)
    ref = O.gemm_ref(x.float().numpy()[rows], wdq[cols])
    assert rel_fro_bf16(y[rows][:, cols], ref) <= 1e-3


@pytest.mark.parametrize("per_tensor", [False, True])
def test_fp8p_fused_gemm_dequant_exact_all_codes(gpu_device, per_tensor):
    """X = I makes the fused GEMM return deq(W)^T exactly (one nonzero product
    per output), so every e4m3 code's bf16(value * scale) is checked bit for
    bit against the oracle decode; rows holding a NaN code (0x7F, 0xFF) turn
    their output column NaN."""
    from lowbit import persistent as P

    K, N = 256, 96
    rng = np.random.default_rng(20260601)
    codes = np.stack([rng.permutation(256) for _ in range(N)]).astype(np.uint8)
    nan_rows = [5, 70]
    for r in range(N):
        if r not in nan_rows:
            codes[r][codes[r] == 0x7F] = 0x00
            codes[r][codes[r] == 0xFF] = 0x80
    scales = (np.exp(rng.uniform(np.log(1e-20), np.log(1e20), N))).astype(np.float32)
    if per_tensor:
        scales = scales[:1]
    x = torch.eye(K, dtype=torch.bfloat16, device=gpu_device)
    w = torch.from_numpy(codes).to(gpu_device).view(torch.float8_e4m3fn)
    s = torch.from_numpy(scales).to(gpu_device).reshape(-1, 1) if not per_tensor else \
        torch.from_numpy(scales).to(gpu_device).reshape(())
    y = P.linear_fp8p(x, w, s, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = y.cpu().numpy().T  # [N, K]
    vals = O.decode_codes(codes, O.GRID_E4M3)
    want = O.round_bf16(vals * (scales[:, None] if not per_tensor else scales[0]))
    for r in nan_rows:
        assert np.isnan(got[r]).all()
    keep = [r for r in range(N) if r not in nan_rows]
    np.testing.assert_array_equal(got[keep], want[keep])


@pytest.mark.parametrize("block", [64, 192])
def test_fp8p_fused_gemm_block_scales_exact(gpu_device, block):
    """ntlb_gemm_fp8p with a scale per block of 64 or 192 weights of a row:
    X = I returns every code's bf16(value * its block's scale) bit for bit."""
    K, N = 384, 64
    rng = np.random.default_rng(20260611 + block)
    codes = np.stack([rng.permutation(np.tile(np.arange(256), 2))[:K] for _ in range(N)]).astype(np.uint8)
    codes[codes == 0x7F] = 0x00
    codes[codes == 0xFF] = 0x80
    scales = np.exp(rng.uniform(np.log(1e-20), np.log(1e20), N * (K // block))).astype(np.float32)
    x = torch.eye(K, dtype=torch.bfloat16, device=gpu_device)
    y = _fused_unsplit("fp8p", x, torch.from_numpy(codes).to(gpu_device), torch.from_numpy(scales).to(gpu_device),
                       block, N, torch.float32)
    torch.cuda.synchronize()
    vals = O.decode_codes(codes, O.GRID_E4M3)
    want = O.round_bf16(vals * np.repeat(scales.reshape(N, K // block), block, axis=1))
    np.testing.assert_array_equal(y.cpu().numpy().T, want)


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (130, 200, 320), (512, 384, 2048), (1, 64, 64)])
@pytest.mark.parametrize("granularity", ["per_channel", "per_tensor"])
def test_fp8p_fused_gemm(gpu_device, M, N, K, granularity):
    from lowbit import persistent as P

    x = seeded((M, K), seed=20260602).to(gpu_device)
    w = seeded((N, K), seed=20260603, std=0.02).to(gpu_device)
    vals, scale = P.quantize_fp8_persistent(w, granularity=granularity)
    y = P.linear_fp8p(x, vals, scale)
    torch.cuda.synchronize()
    block = K if granularity == "per_channel" else N * K
    c_ref, s_ref = O.fp8_persistent_quant(to_np32(w), block)
    wdq = O.round_bf16(O.decode_codes(c_ref, O.GRID_E4M3) * np.repeat(s_ref, block)).reshape(N, K)
    assert rel_fro_bf16(y, O.gemm_ref(to_np32(x), wdq)) <= 1e-3


def test_c5_fp8p_fused_gemm_full_size_sampled(gpu_device):
    """The c5 shapes with the weight held as persistent FP8 (per_channel)."""
    from lowbit import persistent as P, workloads

    x, w = workloads.c5_inputs(device="cpu")
    xg, wg = x.to(gpu_device), w.to(gpu_device)
    vals, scale = P.quantize_fp8_persistent(wg, granularity="per_channel")
    y = P.linear_fp8p(xg, vals, scale)
    torch.cuda.synchronize()
    c_ref, s_ref = O.fp8_persistent_quant(w.float().numpy(), 4096)
    assert_bits_equal(vals.view(torch.uint8).reshape(-1).cpu().numpy(), c_ref, "c5 fp8 codes")
    rows = np.random.default_rng(0).choice(4096, 32, replace=False)
    cols = np.random.default_rng(1).choice(14336, 256, replace=False)
    wdq = O.round_bf16(O.decode_codes(c_ref.reshape(14336, 4096)[cols], O.GRID_E4M3) * s_ref[cols, None])
    ref = O.gemm_ref(x.float().numpy()[rows], wdq)
    assert rel_fro_bf16(y[rows][:, cols], ref) <= 1e-3


def test_fp8p_fused_gemm_rejects_bad_scale_shape(gpu_device):
    from lowbit import persistent as P

    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=gpu_device)
    w = torch.zeros(8, 64, dtype=torch.uint8, device=gpu_device).view(torch.float8_e4m3fn)
    with pytest.raises(ValueError):
        P.linear_fp8p(x, w, torch.ones(3, device=gpu_device))


# blocks of 32 * 2^p weights, of 32 * 6, one per row and one tensor-wide
@pytest.mark.parametrize("block,K", [(64, 256), (256, 256), (0, 256), (32, 256), (192, 384), (384, 384)])
def test_nf4_fused_gemm_dequant_exact_all_codes(gpu_device, block, K):
    """X = I returns deq(W)^T exactly: every NF4 code at every nibble position,
    under scales spanning many binades, against the oracle dequant (bit for
    bit, after the bf16 rounding of the weight dtype)."""
    from lowbit import persistent as P

    N = 80
    rng = np.random.default_rng(20260604)
    idx = np.stack([rng.permutation(np.tile(np.arange(16), K // 16)) for _ in range(N)]).astype(np.uint8)
    flat = idx.reshape(-1)
    packed = (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8)
    nb = (N * K) // block if block else 1
    scales = np.exp(rng.uniform(np.log(1e-30), np.log(1e30), nb)).astype(np.float32)
    x = torch.eye(K, dtype=torch.bfloat16, device=gpu_device)
    y = P.linear_nf4(x, torch.from_numpy(packed).to(gpu_device), torch.from_numpy(scales).to(gpu_device),
                     out_features=N, block=block if block else N * K, out_dtype=torch.float32)
    torch.cuda.synchronize()
    want = O.round_bf16(O.nf4_dequant(packed, scales, N * K, block if block else N * K)).reshape(N, K)
    np.testing.assert_array_equal(y.cpu().numpy().T, want)


def test_mxfp4_fused_gemm_dequant_exact_all_codes(gpu_device):
    """X = I returns deq(W)^T exactly for every e2m1 code under a range of
    e8m0 scales, the smallest ones included (bf16 subnormal weights) and the
    largest whose products stay finite; a block with scale byte 0xFF (NaN)
    turns its row's output column NaN."""
    from lowbit import persistent as P

    K, N = 256, 64
    rng = np.random.default_rng(20260605)
    idx = np.stack([rng.permutation(np.tile(np.arange(16), K // 16)) for _ in range(N)]).astype(np.uint8)
    flat = idx.reshape(-1)
    packed = (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8)
    sbytes = rng.integers(127 - 100, 127 + 100, (N * K) // 32).astype(np.uint8)
    sbytes[: 8 * (K // 32)] = np.repeat(np.array([0, 1, 2, 3, 4, 250, 251, 252], dtype=np.uint8), K // 32)
    nan_row = 9
    sbytes[nan_row * (K // 32) + 3] = 0xFF
    x = torch.eye(K, dtype=torch.bfloat16, device=gpu_device)
    y = P.linear_mxfp4(x, torch.from_numpy(packed).to(gpu_device), torch.from_numpy(sbytes).to(gpu_device),
                       out_features=N, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = y.cpu().numpy().T
    want = O.round_bf16(O.mxfp4_dequant(packed, sbytes, N * K)).reshape(N, K)
    assert np.isnan(got[nan_row]).all()
    keep = [r for r in range(N) if r != nan_row]
    np.testing.assert_array_equal(got[keep], want[keep])


# MXFP4 blocks are always 32 elements: its one size is the 64-weight case
@pytest.mark.parametrize("fmt,block", [("nf4", 64), ("nf4", 96), ("nf4", 0), ("mxfp4", 64), ("fp8p", 64),
                                       ("fp8p", 96), ("fp8p", 0)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dequant_vector_path_matches_elementwise_and_oracle(gpu_device, fmt, block, out_dtype):
    """The 16-weights-per-thread dequant (aligned output, n and block multiples
    of 16) against the element-wise kernel (the same call on an output offset
    by one element, which that path requires) and against the oracle: every
    code byte, scales across many binades, MXFP4 NaN blocks (e8m0 0xFF), a
    non-power-of-two block (96) and a tensor-wide one (0 = n)."""
    from lowbit import _lib, ops

    # whole scale blocks (and whole 32-element MXFP4 blocks), as a weight of K % block == 0 has
    n = {64: 64 * 1025, 96: 96 * 683, 0: 16 * 4099}[block]
    blk = n if block == 0 else block
    rng = np.random.default_rng(20261202 + blk)
    if fmt == "fp8p":
        codes = rng.integers(0, 256, n, dtype=np.uint8)
        nscale = n // blk
        scales = np.float32(2.0) ** rng.integers(-30, 30, nscale).astype(np.float32) * rng.uniform(
            1, 2, nscale).astype(np.float32)
        want = (torch.from_numpy(codes).view(torch.float8_e4m3fn).float() *
                torch.from_numpy(np.repeat(scales, blk))).numpy()
    else:
        codes = rng.integers(0, 256, n // 2, dtype=np.uint8)
        if fmt == "nf4":
            nscale = n // blk
            scales = np.float32(2.0) ** rng.integers(-30, 30, nscale).astype(np.float32) * rng.uniform(
                1, 2, nscale).astype(np.float32)
            want = O.nf4_dequant(codes, scales, n, blk)
        else:
            assert n % 32 == 0
            scales = rng.integers(0, 256, n // 32, dtype=np.uint8)
            scales[::17] = 0xFF
            scales[1::23] = 0
            want = O.mxfp4_dequant(codes, scales, n)
    want_t = torch.from_numpy(want).to(out_dtype)
    c_d = torch.from_numpy(codes).to(gpu_device)
    s_d = torch.from_numpy(scales).to(gpu_device)
    outs = []
    for off in (0, 1):
        buf = torch.zeros(n + 8, dtype=out_dtype, device=gpu_device)
        out = buf[off:off + n]
        st = ops._stream()
        if fmt == "nf4":
            _lib.call("ntlb_nf4_dequant", c_d.data_ptr(), s_d.data_ptr(), n, blk, out.data_ptr(),
                      ops._dtype_code(out_dtype), st)
        elif fmt == "mxfp4":
            _lib.call("ntlb_mxfp4_dequant", c_d.data_ptr(), s_d.data_ptr(), n, out.data_ptr(),
                      ops._dtype_code(out_dtype), st)
        else:
            _lib.call("ntlb_fp8_persistent_dequant", c_d.data_ptr(), s_d.data_ptr(), n, blk, out.data_ptr(),
                      ops._dtype_code(out_dtype), st)
        torch.cuda.synchronize()
        outs.append(out.cpu())
        # nothing written outside [off, off + n)
        assert not buf.cpu()[:off].any() and not buf.cpu()[off + n:].any()
    bits = torch.int32 if out_dtype == torch.float32 else torch.int16
    assert torch.equal(outs[0].view(bits), outs[1].view(bits))
    # NaNs (e4m3 codes 0x7F / 0xFF, MXFP4 NaN blocks) by position, every other value bit for bit
    nan = torch.isnan(want_t)
    assert torch.equal(torch.isnan(outs[0]), nan)
    assert torch.equal(outs[0][~nan].view(bits), want_t[~nan].view(bits))
    assert fmt == "nf4" or nan.any()


def _nf4_all_codes(N: int, K: int, rng) -> np.ndarray:
    """packed nibbles of an [N, K] weight whose rows hold every NF4 code"""
    idx = np.stack([rng.permutation(np.tile(np.arange(16), K // 16)) for _ in range(N)]).astype(np.uint8)
    flat = idx.reshape(-1)
    return (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8)


@pytest.mark.parametrize("fmt", ["nf4", "fp8"])
@pytest.mark.parametrize("per_tensor", [False, True])
@pytest.mark.parametrize("op_dtype", [torch.bfloat16, torch.float32])
def test_lowbit_dgrad_decodes_every_code_exactly(gpu_device, fmt, per_tensor, op_dtype):
    """dY = I makes dX = deq(W): every NF4 code (or every finite e4m3 code)
    times its row or tensor scale, over scales spanning many binades, bit for
    bit against the oracle's dequantization, rounded to bf16 for bf16 dY and
    exact for fp32 dY (_dequantize_*_persistent with the layer's dtype)."""
    from lowbit import persistent as P

    N, K = 192, 256
    rng = np.random.default_rng(20262601)
    scales = np.exp(rng.uniform(np.log(1e-30), np.log(1e30), 1 if per_tensor else N)).astype(np.float32)
    if fmt == "nf4":
        codes = _nf4_all_codes(N, K, rng)
        want = O.nf4_dequant(codes, scales, N * K, N * K if per_tensor else K).reshape(N, K)
    else:
        c = ((np.arange(N)[:, None] + np.arange(K)[None, :]) % 256).astype(np.uint8)
        c[(c & 0x7F) == 0x7F] = 0  # the NaN codes
        codes = c
        vals = torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy()
        want = (vals * (scales[0] if per_tensor else scales[:, None])).astype(np.float32)
    if op_dtype == torch.bfloat16:
        want = O.round_bf16(want)
    dy = torch.eye(N, dtype=op_dtype, device=gpu_device)
    sc = torch.from_numpy(scales).to(gpu_device).reshape(-1, 1)
    dx = P.dgrad(dy, torch.from_numpy(codes).to(gpu_device), sc, fmt=fmt, out_features=N, in_features=K,
                 out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dx.cpu().numpy(), want)


@pytest.mark.parametrize("fmt", ["nf4", "fp8"])
@pytest.mark.parametrize("op_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K,per_tensor", [(300, 200, 388, False), (64, 129, 256, True), (1000, 640, 1152, False),
                                              (7, 64, 4, False)])
def test_lowbit_dgrad_matches_oracle(gpu_device, fmt, op_dtype, M, N, K, per_tensor):
    """dX = dY @ deq(W) over the persistent quantizer's own codes, against
    float64 over the oracle's dequantized weight (rounded to bf16 for a bf16
    layer): ragged N (the contraction) and K (not a multiple of 64)."""
    from lowbit import persistent as P

    gran = "per_tensor" if per_tensor else "per_channel"
    w = seeded((N, K), seed=20262611 + K, std=0.05, outliers=0.01).to(gpu_device, op_dtype)
    dy = seeded((M, N), seed=20262612 + M, std=1e-2).to(gpu_device, op_dtype)
    if fmt == "nf4":
        codes, scale = P.quantize_nf4_persistent(w, granularity=gran)
        wd = O.nf4_dequant(codes.cpu().numpy(), scale.cpu().numpy().reshape(-1), N * K,
                           N * K if per_tensor else K).reshape(N, K)
    else:
        codes, scale = P.quantize_fp8_persistent(w, granularity=gran)
        wd = codes.float().cpu().numpy() * scale.float().cpu().numpy().reshape(-1, 1 if not per_tensor else 1)
        wd = wd.astype(np.float32)
    if op_dtype == torch.bfloat16:
        wd = O.round_bf16(wd)
    dx = P.dgrad(dy, codes, scale, fmt=fmt, out_features=N, in_features=K, out_dtype=torch.float32)
    ref = to_np32(dy).astype(np.float64) @ wd.astype(np.float64)
    err = O.rel_frobenius(dx.cpu().numpy(), ref)
    assert err <= (1e-5 if op_dtype == torch.bfloat16 else 1e-5), err


@pytest.mark.parametrize("fmt", ["nf4", "fp8"])
def test_lowbit_dgrad_split_tail_matches_unsplit(gpu_device, fmt):
    """272 tiles leave 16 past the last whole wave: with the workspace they
    run as K ranges whose fp32 partials are summed in range order; the result
    equals the unsplit call's within fp32 reassociation, and repeats are
    bit-identical (the workspace resets itself)."""
    from lowbit import _lib, ops, persistent as P

    M, N, K = 4352, 2304, 4096
    w = seeded((N, K), seed=20262621, std=0.05).to(gpu_device)
    dy = seeded((M, N), seed=20262622, std=1e-2).to(gpu_device)
    if fmt == "nf4":
        codes, scale = P.quantize_nf4_persistent(w, granularity="per_channel")
    else:
        codes, scale = P.quantize_fp8_persistent(w, granularity="per_channel")
    assert int(_lib.lib().ntlb_gemm_dq_workspace_bytes(_lib.BF16, M, K, N)) > 0
    split1 = P.dgrad(dy, codes, scale, fmt=fmt, out_features=N, in_features=K, out_dtype=torch.float32)
    split2 = P.dgrad(dy, codes, scale, fmt=fmt, out_features=N, in_features=K, out_dtype=torch.float32)
    whole = torch.empty_like(split1)
    sc = scale.reshape(-1).float().contiguous()
    _lib.call("ntlb_gemm_lowbit_dgrad_ws", 0 if fmt == "nf4" else 2, _lib.BF16, dy.data_ptr(), dy.stride(0), M, N,
              codes.contiguous().view(torch.uint8).data_ptr(), sc.data_ptr(), K, K, whole.data_ptr(), _lib.F32,
              whole.stride(0), None, 0, ops._stream())
    torch.cuda.synchronize()
    assert torch.equal(split1, split2)
    assert O.rel_frobenius(split1.cpu().numpy(), whole.cpu().numpy().astype(np.float64)) <= 1e-6


def _persistent_oracle(fmt: str, codes: torch.Tensor, scale: torch.Tensor, N: int, K: int, per_tensor: bool):
    """fp32 values of a persistent weight from its codes (the oracle's NF4
    dequantization, or e4m3 value times scale)"""
    if fmt == "nf4":
        return O.nf4_dequant(codes.cpu().numpy(), scale.float().cpu().numpy().reshape(-1), N * K,
                             N * K if per_tensor else K).reshape(N, K)
    vals = codes.cpu().view(torch.float8_e4m3fn).float().numpy() if codes.dtype == torch.uint8 else \
        codes.float().cpu().numpy()
    return (vals * scale.float().cpu().numpy().reshape(-1, 1)).astype(np.float32)


@pytest.mark.parametrize("fmt", ["nf4", "fp8"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K,per_tensor", [(300, 200, 388, False), (64, 129, 256, True), (5, 64, 100, False),
                                              (1000, 640, 1152, False)])
def test_persistent_forward_fp32_and_ragged_k_match_oracle(gpu_device, fmt, dtype, M, N, K, per_tensor):
    """Y = x @ deq(W)^T + b through linear_nf4 / linear_fp8p where the fused
    kernel does not apply (fp32 activations, or K not a multiple of 64): the
    dequantized-operand GEMM decodes the codes (masked past K), against
    float64 over the oracle's values (bf16-rounded for a bf16 layer)."""
    from lowbit import persistent as P

    gran = "per_tensor" if per_tensor else "per_channel"
    w = seeded((N, K), seed=20262631 + K, std=0.05, outliers=0.01).to(gpu_device, dtype)
    x = seeded((M, K), seed=20262632 + M).to(gpu_device, dtype)
    b = seeded((N,), seed=20262633, std=0.5).to(gpu_device, dtype)
    if fmt == "nf4":
        codes, scale = P.quantize_nf4_persistent(w, granularity=gran)
        y = P.linear_nf4(x, codes, scale, out_features=N, block=N * K if per_tensor else K, bias=b,
                         out_dtype=torch.float32)
    else:
        codes, scale = P.quantize_fp8_persistent(w, granularity=gran)
        y = P.linear_fp8p(x, codes, scale, bias=b, out_dtype=torch.float32)
    wd = _persistent_oracle(fmt, codes, scale, N, K, per_tensor)
    if dtype == torch.bfloat16:
        wd = O.round_bf16(wd)
    ref = O.gemm_ref(to_np32(x), wd, to_np32(b))
    err = O.rel_frobenius(y.cpu().numpy(), ref)
    assert err <= 1e-5, err


@pytest.mark.parametrize("fmt", ["nf4", "fp8"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_persistent_forward_ragged_k_decodes_every_code_exactly(gpu_device, fmt, dtype):
    """x = I with K = 100 returns deq(W)^T exactly: every NF4 code (or every
    finite e4m3 code) times its row scale, with the codes of the next row
    (which follow each row's 100 in memory) masked out of the contraction."""
    from lowbit import persistent as P

    N, K = 80, 100
    rng = np.random.default_rng(20262641)
    scales = np.exp(rng.uniform(np.log(1e-20), np.log(1e20), N)).astype(np.float32)
    if fmt == "nf4":
        idx = np.stack([np.resize(rng.permutation(16), K) for _ in range(N)]).astype(np.uint8)
        flat = idx.reshape(-1)
        codes = torch.from_numpy((flat[0::2] | (flat[1::2] << 4)).astype(np.uint8))
    else:
        c = ((np.arange(N)[:, None] * 7 + np.arange(K)[None, :]) % 256).astype(np.uint8)
        c[(c & 0x7F) == 0x7F] = 0
        codes = torch.from_numpy(c).view(torch.float8_e4m3fn)
    sc = torch.from_numpy(scales).reshape(N, 1)
    want = _persistent_oracle(fmt, codes if fmt == "nf4" else codes.view(torch.uint8), sc, N, K, False)
    if dtype == torch.bfloat16:
        want = O.round_bf16(want)
    x = torch.eye(K, dtype=dtype, device=gpu_device)
    if fmt == "nf4":
        y = P.linear_nf4(x, codes.to(gpu_device), sc.to(gpu_device), out_features=N, block=K,
                         out_dtype=torch.float32)
    else:
        y = P.linear_fp8p(x, codes.to(gpu_device), sc.to(gpu_device), out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy().T, want)
