"""The C-ABI library loads on the CPU host, exports every symbol include/ntlowbit.h
declares, and rejects bad arguments before touching the GPU."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import PKG_PARENT, ROOT

HEADER = os.path.join(ROOT, "include", "ntlowbit.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = re.findall(r"^(?:int64_t|int|const char\*)\s+(ntlb_\w+)\s*\(([^;]*)\);", text, flags=re.M)
    out = {}
    for name, args in decls:
        args = " ".join(args.split())
        n = 0 if args in ("", "void") else args.count(",") + 1
        out[name] = n
    return out


def test_header_declares_entry_points():
    d = _declared()
    assert "ntlb_gemm_blockscaled" in d and "ntlb_quant_tile_1x128" in d
    assert len(d) >= 8


def test_library_exports_every_declared_symbol():
    from lowbit import _lib

    L = _lib.lib()
    for name in _declared():
        assert hasattr(L, name), name


def test_python_binding_matches_header_arity():
    from lowbit import _lib

    d = _declared()
    assert set(d) == set(_lib.SIGNATURES), set(d) ^ set(_lib.SIGNATURES)
    for name, n in d.items():
        assert len(_lib.SIGNATURES[name]) == n, name


def test_abi_version_and_validation_without_gpu():
    from lowbit import _lib

    L = _lib.lib()
    assert L.ntlb_abi_version() == _lib.ABI_VERSION
    # Kp not a multiple of 128: rejected before any launch
    rc = L.ntlb_gemm_blockscaled(1, 16, 128, 16, 1, 0, 0, 16, 128, 16, 1, 0, 7, 4, 4, 100, None, 0, 16, 1, 4, None,
                                 None, None)
    assert rc == _lib.NTLB_EINVAL
    assert b"multiple of 128" in L.ntlb_last_error()
    # bad grid enum on the tile quantizer
    rc = L.ntlb_quant_tile_1x128(16, 1, 4, 128, 128, 5, 127, 0, 0, 0, 0, 16, 128, 16, 1, 1, None, 0, 0, None, None)
    assert rc == _lib.NTLB_EINVAL and b"grid" in L.ntlb_last_error()


def test_product_package_never_touches_the_oracle():
    pkg = os.path.join(PKG_PARENT, "lowbit")
    for fn in os.listdir(pkg):
        if fn.endswith(".py"):
            src = open(os.path.join(pkg, fn)).read()
            assert "oracle" not in src.replace("oracle-free", ""), fn


def test_ops_reject_cpu_tensors():
    import torch

    from lowbit import ops

    with pytest.raises(RuntimeError, match="ROCm device"):
        ops.quant_tile_1x128(torch.zeros(2, 128))
