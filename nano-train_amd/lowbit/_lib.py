"""ctypes binding of libntlowbit.so (the gfx950 kernels' C-ABI, include/ntlowbit.h).

The library is built in-tree by ``nano-train_amd/build.py``.  There is no
fallback: if the shared object is missing or does not export the ABI this
package expects, ``lib()`` raises, and so does every op that needs it.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# NTLB_LIB_PATH points at another build of the same ABI (a tuned or debug build)
LIB_PATH = os.environ.get("NTLB_LIB_PATH") or os.path.join(_HERE, "libntlowbit.so")
ABI_VERSION = 1

NTLB_OK = 0
NTLB_EINVAL = -1
NTLB_ELAUNCH = -2
NTLB_EUNSUPPORTED = -3

F32, BF16, F16 = 0, 1, 2
GRID_INT, GRID_E4M3 = 0, 1
ROUND_NEAREST, ROUND_STOCHASTIC = 0, 1
SCALE_AFTER_DIVIDE, SCALE_BEFORE_DIVIDE = 0, 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_I32 = ctypes.c_int
_F32 = ctypes.c_float

# name -> argtypes, in the order of include/ntlowbit.h
SIGNATURES = {
    "ntlb_abi_version": [],
    "ntlb_last_error": [],
    "ntlb_quant_tile_1x128": [_P, _I32, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _U64, _U64, _P, _I64, _P, _I64,
                              _I64, _P, _I32, _I64, _P, _P],
    "ntlb_quant_block_128x128": [_P, _I32, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _U64, _U64, _P, _I64, _P, _I64,
                                 _P, _I64, _I64, _P, _I32, _I64, _P, _P],
    "ntlb_amax_grouped": [_P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _P],
    "ntlb_quant_grouped": [_P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _I32, _I32, _I32, _I32, _U64, _U64, _P, _I64,
                           _P, _P, _I32, _I64, _P, _P],
    "ntlb_quant_grouped_noalloc": [_P, _I32, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _U64, _U64, _P,
                                   _I64, _P, _P, _I32, _I64, _P, _P],
    "ntlb_quant_tile_128x1_t": [_P, _I32, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _U64, _U64, _P, _I64, _P, _I64,
                                _I64, _P, _I32, _I64, _P, _P],
    "ntlb_quant_dual_1x128_128x1": [_P, _I32, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _U64, _U64, _U64, _P, _I64,
                                    _P, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _P, _P],
    "ntlb_dequant": [_I32, _P, _I64, _P, _I64, _I64, _I32, _I32, _I64, _I64, _P, _I32, _I64, _P],
    "ntlb_gemm_blockscaled": [_I32, _P, _I64, _P, _I64, _I64, _I32, _P, _I64, _P, _I64, _I64, _I32, _I64, _I64,
                              _I64, _P, _I32, _P, _I32, _I64, _P, _P, _P],
    "ntlb_gemm_blockscaled_ws": [_I32, _P, _I64, _P, _I64, _I64, _I32, _P, _I64, _P, _I64, _I64, _I32, _I64,
                                 _I64, _I64, _P, _I32, _P, _I32, _I64, _P, _P, _P, _I64, _P],
    "ntlb_gemm_grouped_blockscaled": [_I32, _P, _I64, _P, _I64, _I64, _I32, _P, _I64, _I64, _P, _I64, _I64, _I32,
                                      _I64, _P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _P, _P, _P],
    "ntlb_gemm_swiglu_quant": [_I32, _P, _I64, _P, _I64, _I64, _I32, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64,
                               _P, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _P, _I32, _I32, _I32, _U64, _U64, _P],
    "ntlb_gemm_grouped_swiglu_quant": [_I32, _P, _I64, _P, _I64, _I64, _I32, _P, _I64, _I64, _P, _I64, _I64, _I64,
                                       _P, _I32, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _P,
                                       _I32, _I32, _I32, _U64, _U64, _P],
    "ntlb_nf4_quant": [_P, _I32, _I64, _I64, _P, _P, _P, _P],
    "ntlb_nf4_dequant": [_P, _P, _I64, _I64, _P, _I32, _P],
    "ntlb_mxfp4_quant": [_P, _I32, _I64, _P, _P, _P],
    "ntlb_mxfp4_dequant": [_P, _P, _I64, _P, _I32, _P],
    "ntlb_fp8_persistent_quant": [_P, _I32, _I64, _I64, _P, _P, _P, _P],
    "ntlb_fp8_persistent_dequant": [_P, _P, _I64, _I64, _P, _I32, _P],
    "ntlb_adamw_step_refresh": [_P, _P, _I32, _P, _P, _P, _I32, _I64, _F32, _F32, _F32, _F32, _F32, _F32, _F32,
                                _F32, _I32, _I64, _P, _P, _P],
    "ntlb_gemm_nf4": [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _I32, _I64, _P],
    "ntlb_gemm_mxfp4": [_P, _I64, _P, _P, _I64, _I64, _I64, _P, _I32, _I64, _P],
    "ntlb_gemm_fp8p": [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _I32, _I64, _P],
    "ntlb_gemm_lowbit_workspace_bytes": [_I64, _I64, _I64],
    "ntlb_gemm_lowbit_ws": [_I32, _P, _I64, _P, _P, _I64, _P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _P, _I64, _P],
    "ntlb_gemm_lowbit_dq_forward_ws": [_I32, _I32, _P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _I32, _P, _I32,
                                       _I64, _P, _I64, _P],
    "ntlb_gemm_lowbit_dgrad_ws": [_I32, _I32, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _I32, _I64, _P, _I64,
                                  _P],
    "ntlb_gemm_workspace_bytes": [_I64, _I64, _I64],
    "ntlb_gemm_dq_forward": [_I32, _I32, _P, _I64, _P, _I64, _I64, _I32, _P, _I64, _P, _I64, _I64, _I32, _I64, _I64,
                             _I64, _P, _I32, _P, _I32, _I64, _P],
    "ntlb_gemm_ste_dgrad": [_I32, _P, _I64, _I64, _I64, _I32, _P, _I64, _P, _I64, _I64, _I32, _I64, _P, _I32, _I64, _P],
    "ntlb_gemm_ste_dgrad_ws": [_I32, _P, _I64, _I64, _I64, _I32, _P, _I64, _P, _I64, _I64, _I32, _I64, _P, _I32, _I64,
                               _P, _I64, _P],
    "ntlb_gemm_dq_workspace_bytes": [_I32, _I64, _I64, _I64],
    "ntlb_gemm_ste_wgrad": [_I32, _P, _I64, _I64, _I64, _I32, _P, _I64, _P, _I64, _I64, _I32, _I64, _P, _I32, _I64, _P],
    "ntlb_gemm_ste_wgrad_db": [_I32, _P, _I64, _I64, _I64, _I32, _P, _I64, _P, _I64, _I64, _I32, _I64, _P, _I32, _I64,
                               _P, _I32, _P],
    "ntlb_gemm_dense": [_I32, _P, _I64, _I32, _P, _I64, _I32, _I64, _I64, _I64, _P, _I32, _P, _I32, _I64, _P],
    "ntlb_gemm_dense_tn": [_I32, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I32, _I64, _P],
    "ntlb_colsum": [_P, _I32, _I64, _I64, _I64, _P, _I64, _P, _I32, _P],
    "ntlb_colsum_workspace_bytes": [_I64, _I64],
    "ntlb_ste_value": [_I32, _P, _P, _P, _I64, _P],
    "ntlb_ep_record_bytes": [_I64],
    "ntlb_quant_tile_1x128_fanout": [_P, _I32, _I64, _I64, _I64, _P, _I64, _I64, _I32, _I32, _I32, _I32, _U64, _U64,
                                     _P, _I64, _P, _I64, _I64, _P, _P],
    "ntlb_moe_combine_rows": [_P, _I64, _I64, _P, _P, _I32, _P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _P],
    "ntlb_ep_partition": [_P, _I32, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _I64, _P],
    "ntlb_ep_pack_records": [_P, _I32, _I64, _I64, _I64, _P, _P, _I32, _P, _I32, _I64, _I64, _I32, _I32, _I32,
                             _I32, _U64, _U64, _P, _P],
    "ntlb_ep_pack_records_grouped": [_P, _I32, _I64, _I64, _I64, _P, _P, _I32, _P, _I32, _I64, _I64, _P, _I64, _I32,
                                     _I32, _I32, _I32, _U64, _U64, _P, _P],
    "ntlb_ep_pack_return": [_P, _I32, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _U64,
                            _U64, _P, _P],
    "ntlb_ep_combine": [_P, _I64, _I64, _P, _I32, _P, _I32, _I64, _I64, _I32, _P, _I32, _I64, _P, _P],
    "ntlb_comm_quant_dequant": [_P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _I32, _I32, _I32, _I32, _U64, _U64, _P,
                                _I64, _P],
    "ntlb_gemm_grouped_ste_dgrad": [_I32, _P, _I64, _I64, _I64, _P, _I32, _I32, _P, _I64, _I64, _P, _I64, _I64, _I32,
                                    _I64, _I64, _P, _I32, _I64, _P],
    "ntlb_gemm_grouped_ste_dgrad_gate_up": [_I32, _P, _I64, _I64, _I64, _P, _I32, _I32, _P, _I64, _I64, _P, _I64,
                                            _I64, _I64, _I64, _P, _I64, _P],
    "ntlb_gemm_grouped_ste_wgrad": [_I32, _P, _I64, _I64, _I64, _P, _I32, _I32, _P, _I64, _P, _I64, _I64, _I32, _I64,
                                    _P, _I32, _I64, _I64, _P],
    "ntlb_gemm_grouped_dgrad_dense": [_I32, _P, _I64, _I64, _I64, _P, _I32, _P, _I64, _I64, _I64, _P, _I32, _I64, _P],
    "ntlb_gemm_grouped_dgrad_dense_gate_up": [_I32, _P, _I64, _I64, _I64, _P, _I32, _P, _I64, _I64, _I64, _P, _I64,
                                              _P],
    "ntlb_gemm_grouped_wgrad_dense": [_I32, _P, _I64, _I64, _I64, _P, _I32, _P, _I64, _I64, _P, _I32, _I64, _I64, _P],
    "ntlb_gemm_grouped_swiglu_quant_gu": [_I32, _P, _I64, _P, _I64, _I64, _I32, _P, _I64, _I64, _P, _I64, _I64, _I64,
                                          _P, _I32, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _P,
                                          _I32, _I32, _I32, _U64, _U64, _P, _I64, _P],
    "ntlb_moe_capacity_keep": [_P, _P, _I32, _I64, _I64, _P, _I32, _I64, _P, _P, _P, _P, _P],
    "ntlb_moe_combine_backward": [_P, _I64, _P, _I64, _I32, _P, _P, _I32, _I64, _I64, _I64, _P, _I64, _P, _P],
    "ntlb_moe_token_grad": [_P, _I64, _I32, _P, _P, _I32, _I64, _I64, _I64, _P, _I64, _P],
    "ntlb_swiglu_backward": [_P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P],
    "ntlb_ep_unpack_records": [_P, _I64, _I64, _P, _I64, _P, _I32, _P, _I64, _P, _I64, _I64, _P, _P, _P, _P, _P, _P],
    "ntlb_ep_value_record_bytes": [_I64, _I32],
    "ntlb_ep_pack_values": [_P, _I32, _I64, _I64, _I64, _P, _P, _I32, _P, _I32, _I64, _I64, _P, _I64, _I32, _I32,
                            _I32, _I32, _U64, _U64, _P, _P],
    "ntlb_ep_pack_return_values": [_P, _I32, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32,
                                   _U64, _U64, _P, _P],
    "ntlb_ep_unpack_values": [_P, _I64, _I64, _I32, _P, _I64, _P, _I32, _P, _I64, _P, _P, _P, _P, _P],
    "ntlb_ep_combine_values": [_P, _I64, _I64, _I32, _P, _I32, _P, _I32, _I64, _I64, _P, _I32, _I64, _P, _P],
}

# entry points that return a value instead of a status
RESTYPES = {"ntlb_gemm_workspace_bytes": _I64, "ntlb_ep_record_bytes": _I64, "ntlb_colsum_workspace_bytes": _I64,
            "ntlb_ep_value_record_bytes": _I64,
            "ntlb_gemm_lowbit_workspace_bytes": _I64, "ntlb_gemm_dq_workspace_bytes": _I64}

_lib = None
_lock = threading.Lock()


class LowBitKernelError(RuntimeError):
    """A C-ABI entry point returned a failure status."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libntlowbit.so not found at {LIB_PATH}; build it with "
                "`python nano-train_amd/build.py` (there is no CPU fallback)"
            )
        L = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        L.ntlb_last_error.restype = ctypes.c_char_p
        v = L.ntlb_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"libntlowbit ABI version {v} != expected {ABI_VERSION}")
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and raise on a non-zero status."""
    fn = getattr(lib(), name)
    rc = fn(*args)
    if rc != NTLB_OK:
        msg = lib().ntlb_last_error().decode(errors="replace")
        exc = ValueError if rc == NTLB_EINVAL else LowBitKernelError
        raise exc(f"{name} failed ({rc}): {msg}")
