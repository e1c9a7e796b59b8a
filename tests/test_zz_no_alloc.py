"""GPU test of ntlb_quant_grouped_noalloc, the grouped quantizer (tensor and
channel granularities, te_backend.py:163-185) that keeps its amax
accumulator in a library-held device array instead of a caller workspace.
Its outputs must equal, bit for bit, those of the workspace entry points
(ntlb_amax_grouped + ntlb_quant_grouped) on the same inputs, on consecutive
calls whose second one is smaller (a stale amax left by the first call would
change the second call's scales)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _noalloc(x: torch.Tensor, gr: int, gc: int, *, fmt: str, rounding: str = "nearest", seed: int = 0,
             offset: int = 0):
    from lowbit import _lib, ops

    R, K = x.shape
    ldc = ops.cdiv(K, 16) * 16
    ngr, ngc = ops.cdiv(R, gr), ops.cdiv(K, gc)
    codes = torch.zeros((R, ldc), dtype=torch.uint8, device=x.device)
    scales = torch.empty((ngr, ngc), dtype=torch.float32, device=x.device)
    dq = torch.empty((R, K), dtype=x.dtype, device=x.device)
    nan = torch.zeros(R, dtype=torch.int32, device=x.device)
    _lib.call("ntlb_quant_grouped_noalloc", x.data_ptr(), ops._dtype_code(x.dtype), R, K, x.stride(0), gr, gc,
              ops.grid_code(fmt), 127, ops.rounding_code(rounding), _lib.SCALE_AFTER_DIVIDE, seed, offset,
              codes.data_ptr(), ldc, scales.data_ptr(), dq.data_ptr(), ops._dtype_code(dq.dtype), dq.stride(0),
              nan.data_ptr(), ops._stream())
    return codes, scales, dq, nan


def _workspace(x: torch.Tensor, gr: int, gc: int, *, fmt: str, rounding: str = "nearest", seed: int = 0,
               offset: int = 0):
    from lowbit import ops

    R, K = x.shape
    return ops.quant_grouped(x, gr, gc, fmt=fmt, rounding=rounding, seed=seed, offset=offset,
                             ldc=ops.cdiv(K, 16) * 16, want_dq=True, dq_dtype=x.dtype, want_nan_rows=True)


def _input(shape, seed, std, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * std
    return x.to(torch.bfloat16).to(dev)


def _same(a, b, what):
    for name, u, v in zip(("codes", "scales", "dq", "nan_rows"), a, b):
        uu, vv = u.cpu(), v.cpu()
        if uu.dtype in (torch.bfloat16, torch.float32):
            uu, vv = uu.view(torch.int16 if uu.dtype == torch.bfloat16 else torch.int32), \
                vv.view(torch.int16 if vv.dtype == torch.bfloat16 else torch.int32)
        assert torch.equal(uu, vv), f"{what}: {name} differs"


@pytest.mark.parametrize("fmt", ["int_grid", "e4m3"])
def test_noalloc_matches_workspace_entry_points_on_two_calls(gpu_device, fmt):
    big = _input((300, 5000), 20262101, 4.0, gpu_device)
    big[7, 11] = float("nan")
    big[9, 4000] = float("inf")
    small = _input((128, 1000), 20262102, 0.01, gpu_device)  # amaxes far below the first call's
    cases = [(big, 300, 1, "channel along the last axis, 5000 groups"),
             (small, 128, 1, "second, smaller call, 1000 groups"),
             (small, 1, 1000, "per row, 128 groups"),
             (small, 128, 1000, "tensor, 1 group")]
    for x, gr, gc, what in cases:
        got = _noalloc(x, gr, gc, fmt=fmt)
        torch.cuda.synchronize()
        want = _workspace(x, gr, gc, fmt=fmt)
        _same(got, want, what)


def test_noalloc_stochastic_rounding_matches(gpu_device):
    x = _input((257, 3000), 20262103, 1.0, gpu_device)
    for gr, gc in ((257, 1), (1, 3000)):
        got = _noalloc(x, gr, gc, fmt="e4m3", rounding="stochastic", seed=11, offset=(1 << 33) + 5)
        want = _workspace(x, gr, gc, fmt="e4m3", rounding="stochastic", seed=11, offset=(1 << 33) + 5)
        _same(got, want, f"stochastic rounding, groups {gr}x{gc}")


def test_noalloc_rejects_more_groups_than_it_holds(gpu_device):
    from lowbit import _lib, ops

    x = _input((70000, 2), 20262104, 1.0, gpu_device)
    codes = torch.zeros((70000, 16), dtype=torch.uint8, device=gpu_device)
    scales = torch.empty(70000, dtype=torch.float32, device=gpu_device)
    with pytest.raises(ValueError, match="65536"):
        _lib.call("ntlb_quant_grouped_noalloc", x.data_ptr(), ops._dtype_code(x.dtype), 70000, 2, 2, 1, 2,
                  _lib.GRID_INT, 127, 0, 0, 0, 0, codes.data_ptr(), 16, scales.data_ptr(), None, 0, 0, None,
                  ops._stream())
