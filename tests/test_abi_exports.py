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


def test_ep_entry_points_validate_without_gpu():
    """The expert-parallel entry points reject bad shapes, enums and
    workspaces with NTLB_EINVAL and a message, before any launch; the record
    size follows the documented layout."""
    from lowbit import _lib

    L = _lib.lib()
    E = _lib.NTLB_EINVAL
    P = 4096  # a 16-byte aligned stand-in address: every call below returns before using it
    # record bytes: 128*ceil(H/128) codes, 4*ceil(H/128) scale bytes rounded to 16, 32 metadata bytes
    assert L.ntlb_ep_record_bytes(7168) == 7168 + 224 + 32
    assert L.ntlb_ep_record_bytes(200) == 256 + 16 + 32
    assert L.ntlb_ep_record_bytes(0) == 0
    # partition: n < 0, no buckets, too many buckets, bad key dtype / stride, short workspace
    part = L.ntlb_ep_partition
    assert part(P, 0, 4, -1, 1, 4, P, P, P, P, P, 64, None) == E
    assert part(P, 0, 4, 10, 1, 0, P, P, P, P, P, 64, None) == E
    assert part(P, 0, 4, 10, 1, 5000, P, P, P, P, P, 1 << 20, None) == E
    assert part(P, 2, 4, 10, 1, 4, P, P, P, P, P, 64, None) == E
    assert part(P, 0, 6, 10, 1, 4, P, P, P, P, P, 64, None) == E and b"key_stride" in L.ntlb_last_error()
    assert part(P, 0, 4, 1000, 1, 4, P, P, P, P, P, 8, None) == E and b"workspace" in L.ntlb_last_error()
    # unpack: ldc below the padded width; source ranks with offsets not ending at n; too many ranks
    offs = (ctypes.c_int64 * 3)(0, 2, 5)
    unpack = L.ntlb_ep_unpack_records
    assert unpack(P, 6, 200, P, 6, None, 0, P, 200, P, 1, 6, None, None, None, None, None, None) == E
    assert unpack(P, 6, 256, P, 6, ctypes.addressof(offs), 2, P, 256, P, 1, 6, None, None, None, P, None,
                  None) == E and b"recv_offsets" in L.ntlb_last_error()
    many = (ctypes.c_int64 * 258)(*([0] * 257 + [6]))
    assert unpack(P, 6, 256, P, 6, ctypes.addressof(many), 257, P, 256, P, 1, 6, None, None, None, P, None,
                  None) == E
    # combine: K above 32, H not a multiple of 8, unknown grid
    BF16 = 1  # NTLB_BF16 of include/ntlowbit.h
    comb = L.ntlb_ep_combine
    assert comb(P, 4, 256, P, 1, P, BF16, 2, 33, 1, P, BF16, 256, P, None) == E
    assert comb(P, 4, 250, P, 1, P, BF16, 2, 2, 1, P, BF16, 256, P, None) == E
    assert comb(P, 4, 256, P, 1, P, BF16, 2, 2, 7, P, BF16, 256, P, None) == E
    # return pack: a scale group that splits a 128-column tile
    ret = L.ntlb_ep_pack_return  # x bf16 (1), grid e4m3 (1), qmax 127, rounding nearest (0), rule 1
    assert ret(P, 1, 4, 256, 256, P, P, P, None, None, P, 100, 1, 127, 0, 1, 0, 0, P, None) == E
    assert b"scale group" in L.ntlb_last_error()
    # the split-K workspace size: zero for a K that is not whole 128-blocks
    assert L.ntlb_gemm_workspace_bytes(512, 1024, 1000) == 0
