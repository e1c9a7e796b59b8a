"""Low-bit-capable Linear layers on the MI355X kernels.

Mirrors the Linear family of nano-train's src/layers.py (Linear :465-632,
ColumnParallelLinear :1235-1360, RowParallelLinear :1363-1496) and the
_LowBitPrecisionLinearMixin (:216-458): the same constructor arguments, the
same `_persistent_*` state_dict buffers with the same dtypes, the same
forward order (persistent-weight straight-through estimator -> low-bit
backend -> per-module compute dtype -> F.linear), the same error messages,
and tolerance of legacy checkpoints that lack the persistent buffers.

Persistent NF4/FP8 weights are refreshed and dequantized by the HIP kernels of
lowbit.persistent.  When a module stores NF4 or FP8 weights, has no low-bit
compute backend, and activation and master weight share a dtype (bf16 or
fp32), the forward decodes the weight inside the GEMM instead of
materializing it; its
backward is the reference's straight-through rule (dX = dY . W_deq with the
weight decoded inside the GEMM, dW = dY^T . X).

One GPU: the tensor-parallel classes accept tp_size == 1 only.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from . import persistent as P
from .contracts import LowBitKernelSpec
from .precision import dtype_alias_to_torch

_PERSISTENT_SUFFIXES = ("_persistent_fp8_weight", "_persistent_fp4_codes", "_persistent_scale", "_persistent_numel")


class _FusedPersistentLinear(torch.autograd.Function):
    """Forward: dequant-fused GEMM over the persistent NF4 or FP8 weight, with
    the bias added in fp32 before the output rounding (F.linear(x, w_q, b),
    layers.py:595-632).  Backward: straight-through to the master weight
    (layers.py:409-436) on the library's GEMMs: dX = dY . w_q with w_q decoded
    inside the GEMM (no dequantized copy), dW = dY^T . X, db = the column sum
    of dY."""

    @staticmethod
    def forward(ctx, x, weight, bias, codes, scale, block, fmt):
        N, K = weight.shape
        if fmt == "nf4":
            y = P.linear_nf4(x, codes, scale, out_features=N, block=block, bias=bias)
        else:
            y = P.linear_fp8p(x, codes, scale, bias=bias)
        ctx.save_for_backward(x, codes, scale)
        ctx.meta = (N, K, block, weight.dtype, fmt, None if bias is None else bias.dtype)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, codes, scale = ctx.saved_tensors
        N, K, block, wdt, fmt, bdt = ctx.meta
        dx = dw = db = None
        dy2 = dy.reshape(-1, N)
        if dy2.stride(-1) != 1:
            dy2 = dy2.contiguous()
        if ctx.needs_input_grad[0]:
            # the weight is decoded inside the GEMM: no dequantized copy of W
            dx = P.dgrad(dy2, codes, scale, fmt=fmt, out_features=N, in_features=K,
                         out_dtype=x.dtype).reshape(x.shape)
        if ctx.needs_input_grad[1]:
            dw = ops.gemm_dense_tn(dy2, x.reshape(-1, K).to(dy2.dtype), out_dtype=wdt)
        if ctx.needs_input_grad[2]:
            db = ops.colsum(dy2, out_dtype=bdt)
        return dx, dw, db, None, None, None, None


class LowBitLinearMixin:
    """Per-module low-bit compute and persistent-parameter hooks (layers.py:216-458)."""

    def _init_lowbit_precision_state(self, *, module_path: str, module_type: str, precision_resolver,
                                     lowbit_capable_type: str, kernel_spec: LowBitKernelSpec) -> None:
        self._module_precision_state = precision_resolver.resolve_module_init_state(
            module_path=module_path, module_type=module_type, lowbit_capable_type=lowbit_capable_type,
            kernel_spec=kernel_spec)
        dev = self.weight.device
        self.register_buffer("_persistent_fp8_weight", torch.empty(0, device=dev), persistent=True)
        self.register_buffer("_persistent_fp4_codes", torch.empty(0, dtype=torch.uint8, device=dev), persistent=True)
        self.register_buffer("_persistent_scale", torch.empty(0, device=dev), persistent=True)
        self.register_buffer("_persistent_numel", torch.zeros((), dtype=torch.int64, device=dev), persistent=True)
        # host copy of _persistent_numel, kept in step with the buffer, so the
        # forward's "is the persistent copy current" test reads no device memory
        # (no device-to-host copy and stream sync per call; the forward can be
        # captured in a HIP graph)
        self._persistent_numel_host = 0
        bind = getattr(self._module_precision_state.lowbit_backend, "bind_parameters", None)
        if callable(bind):
            bind(self.weight, self.bias)

    # --- assignment views ---------------------------------------------------
    @property
    def module_precision_assignment(self):
        return self._module_precision_state.assignment

    @property
    def module_path(self) -> str:
        return str(self._module_precision_state.assignment.module_name)

    @property
    def master_ownership_mode(self) -> str:
        return str(getattr(self._module_precision_state, "master_ownership_mode", "module"))

    def _persistent_mode(self) -> str:
        return str(getattr(self.module_precision_assignment, "persistent_lowbit_mode", "off"))

    def _persistent_granularity(self) -> str:
        return str(getattr(self.module_precision_assignment, "persistent_scale_granularity", "per_channel"))

    def _compute_lowbit_mode(self) -> Optional[str]:
        mode = getattr(self.module_precision_assignment, "compute_lowbit_mode", None)
        return str(mode) if mode is not None and str(mode) in ("fp8", "fp4") else None

    def _compute_dtype_override(self) -> Optional[torch.dtype]:
        alias = getattr(self.module_precision_assignment, "compute_dtype_override", None)
        return None if alias is None else dtype_alias_to_torch(str(alias))

    # --- master weight binding (layers.py:269-278) ----------------------------
    def bind_optimizer_master_weight(self, master_weight: nn.Parameter) -> None:
        if not isinstance(master_weight, nn.Parameter):
            raise TypeError("master_weight must be nn.Parameter")
        if master_weight.shape != self.weight.shape:
            raise ValueError("optimizer master weight shape mismatch: "
                             f"expected={tuple(self.weight.shape)} got={tuple(master_weight.shape)}")
        with torch.no_grad():
            master_weight.copy_(self.weight.detach().to(device=master_weight.device))
        self.weight = master_weight

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs) -> None:
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,  # type: ignore
                                      unexpected_keys, error_msgs)
        self._persistent_numel_host = int(self._persistent_numel.item())  # once per load, not per forward
        optional = {prefix + s for s in _PERSISTENT_SUFFIXES}
        missing_keys[:] = [k for k in missing_keys if k not in optional]

    # --- persistent buffers (layers.py:347-407) -------------------------------
    def _clear_persistent_lowbit_buffers(self) -> None:
        dev = self.weight.device
        self._persistent_fp8_weight = torch.empty(0, device=dev)
        self._persistent_fp4_codes = torch.empty(0, dtype=torch.uint8, device=dev)
        self._persistent_scale = torch.empty(0, device=dev)
        self._persistent_numel = torch.zeros((), dtype=torch.int64, device=dev)
        self._persistent_numel_host = 0

    @torch.no_grad()
    def refresh_persistent_lowbit_params(self) -> None:
        mode = self._persistent_mode()
        if mode == "off":
            self._clear_persistent_lowbit_buffers()
            return
        granularity = self._persistent_granularity()
        if granularity not in ("per_tensor", "per_channel"):
            raise ValueError(f"Unsupported persistent_scale_granularity={granularity!r} for low-bit persistent params")
        dev = self.weight.device
        numel = torch.tensor(int(self.weight.numel()), dtype=torch.int64, device=dev)
        if mode == "fp8":
            values, scale = P.quantize_fp8_persistent(self.weight.detach(), granularity=granularity)
            self._persistent_fp8_weight = values
            self._persistent_fp4_codes = torch.empty(0, dtype=torch.uint8, device=dev)
            self._persistent_scale = scale
            self._persistent_numel = numel
            self._persistent_numel_host = int(self.weight.numel())
            return
        if mode == "fp4":
            fmt = str(getattr(self.module_precision_assignment, "fp4_persistent_format", "nf4"))
            if fmt != "nf4":
                raise ValueError("Only nf4 is supported for FP4 persistent params")
            packed, scale = P.quantize_nf4_persistent(self.weight.detach(), granularity=granularity)
            self._persistent_fp4_codes = packed
            self._persistent_fp8_weight = torch.empty(0, device=dev)
            self._persistent_scale = scale
            self._persistent_numel = numel
            self._persistent_numel_host = int(self.weight.numel())
            return
        raise ValueError(f"Unsupported persistent low-bit mode: {mode}")

    def _set_persistent_buffers(self, mode: str, codes: torch.Tensor, scales: torch.Tensor) -> None:
        """Install codes and scales computed elsewhere (the fused optimizer step)
        in the buffers and shapes refresh_persistent_lowbit_params writes."""
        dev = self.weight.device
        _, shape = P._block_and_scale_shape(self.weight, self._persistent_granularity())
        self._persistent_scale = scales.reshape(shape)
        self._persistent_numel = torch.tensor(int(self.weight.numel()), dtype=torch.int64, device=dev)
        self._persistent_numel_host = int(self.weight.numel())
        if mode == "fp8":
            self._persistent_fp8_weight = codes.view(torch.float8_e4m3fn).reshape(self.weight.shape)
            self._persistent_fp4_codes = torch.empty(0, dtype=torch.uint8, device=dev)
        else:
            self._persistent_fp4_codes = codes
            self._persistent_fp8_weight = torch.empty(0, device=dev)

    def _persistent_weight_ste(self) -> torch.Tensor:
        """Weight used in forward, with a straight-through bridge to the master (layers.py:409-436)."""
        mode = self._persistent_mode()
        if mode == "off":
            return self.weight
        if mode == "fp8":
            if self._persistent_fp8_weight.numel() != self.weight.numel():
                self.refresh_persistent_lowbit_params()
            deq = P.dequantize_fp8_persistent(self._persistent_fp8_weight, self._persistent_scale,
                                              target_dtype=self.weight.dtype)
        elif mode == "fp4":
            if self._persistent_numel_host != int(self.weight.numel()):
                self.refresh_persistent_lowbit_params()
            deq = P.dequantize_nf4_persistent(self._persistent_fp4_codes, self._persistent_scale,
                                              num_values=int(self.weight.numel()), target_shape=self.weight.shape,
                                              target_dtype=self.weight.dtype)
        else:
            raise ValueError(f"Unsupported persistent low-bit mode: {mode}")
        return self.weight + (deq - self.weight).detach()

    def _fused_persistent_forward(self, x: torch.Tensor, bias: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        """NF4 or FP8 persistent weight, no low-bit backend, activation, weight
        and bias of one dtype, bf16 or fp32, K % 4 == 0: the weight is decoded
        inside the GEMM (the dequant-fused kernel for bf16 with K % 64 == 0,
        else the dequantized-operand GEMM) instead of materialized."""
        mode = self._persistent_mode()
        dt = self.weight.dtype
        if (mode not in ("fp4", "fp8") or self._compute_lowbit_mode() is not None
                or self._compute_dtype_override() is not None or dt not in (torch.bfloat16, torch.float32)
                or x.dtype != dt or x.device.type != "cuda" or self.weight.dim() != 2
                or self.weight.shape[1] % 4 or (bias is not None and bias.dtype != dt)):
            return None
        N, K = self.weight.shape
        if mode == "fp4":
            if self._persistent_numel_host != int(self.weight.numel()):
                self.refresh_persistent_lowbit_params()
            scale = self._persistent_scale
            block = (N * K) if scale.numel() <= 1 else K
            return _FusedPersistentLinear.apply(x, self.weight, bias, self._persistent_fp4_codes, scale.float(), block,
                                                "nf4")
        if self._persistent_fp8_weight.numel() != self.weight.numel():
            self.refresh_persistent_lowbit_params()
        scale = self._persistent_scale
        return _FusedPersistentLinear.apply(x, self.weight, bias, self._persistent_fp8_weight, scale.float(),
                                            0 if scale.numel() <= 1 else K, "fp8")

    def _dispatch_lowbit_linear(self, *, x: torch.Tensor, weight: torch.Tensor,
                                bias: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        mode = self._compute_lowbit_mode()
        if mode is None:
            return None
        backend = self._module_precision_state.lowbit_backend
        if backend is None:
            name = self._module_precision_state.assignment.module_name
            raise RuntimeError(f"Module {self.__class__.__name__} ({name}) requested compute mode {mode} "
                               "without a bound low-bit backend")
        return backend.linear(x, weight, bias)

    def _linear_with_dtype_override(self, *, x, weight, bias) -> Optional[torch.Tensor]:
        dt = self._compute_dtype_override()
        if dt is None:
            return None
        return F.linear(x.to(dt), weight.to(dt), None if bias is None else bias.to(dt))

    def _lowbit_forward(self, x: torch.Tensor, bias: Optional[torch.Tensor]) -> torch.Tensor:
        fused = self._fused_persistent_forward(x, bias)
        if fused is not None:
            return fused
        weight = self._persistent_weight_ste()
        out = self._dispatch_lowbit_linear(x=x, weight=weight, bias=bias)
        if out is not None:
            return out
        out = self._linear_with_dtype_override(x=x, weight=weight, bias=bias)
        if out is not None:
            return out
        return F.linear(x, weight, bias)


class Linear(LowBitLinearMixin, nn.Module):
    """y = x W^T + b with the low-bit hooks (layers.py:465-632)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, *, param_dtype: torch.dtype,
                 param_device: Optional[torch.device], module_path: str, precision_resolver) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.empty(out_features, in_features, dtype=param_dtype, device=param_device))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, dtype=param_dtype, device=param_device))
        else:
            self.register_parameter("bias", None)
        nn.init.normal_(self.weight, std=0.02)
        if self.bias is not None:
            nn.init.zeros_(self.bias)
        self._init_lowbit_precision_state(
            module_path=module_path, module_type=type(self).__name__, precision_resolver=precision_resolver,
            lowbit_capable_type="linear",
            kernel_spec=LowBitKernelSpec(module_type="linear", in_features=in_features, out_features=out_features,
                                         has_bias=self.bias is not None))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._lowbit_forward(x, self.bias)


def _check_tp(tp_size: int) -> None:
    if tp_size != 1:
        raise NotImplementedError("this MI355X build runs on one GPU: tensor-parallel layers need tp_size == 1")


class ColumnParallelLinear(LowBitLinearMixin, nn.Module):
    """Output-sharded linear (layers.py:1235-1360); one GPU, so one shard."""

    def __init__(self, in_features: int, out_features: int, tp_rank: int, tp_size: int, bias: bool = True,
                 tp_group=None, *, param_dtype: torch.dtype, param_device: Optional[torch.device], module_path: str,
                 precision_resolver) -> None:
        super().__init__()
        _check_tp(tp_size)
        if out_features % tp_size:
            raise ValueError(f"out_features {out_features} must be divisible by tp_size {tp_size}")
        self.in_features, self.out_features = in_features, out_features
        self.tp_rank, self.tp_size, self.tp_group = tp_rank, tp_size, tp_group
        self.shard_size = out_features // tp_size
        self.weight = nn.Parameter(torch.empty(self.shard_size, in_features, dtype=param_dtype, device=param_device))
        if bias:
            self.bias = nn.Parameter(torch.empty(self.shard_size, dtype=param_dtype, device=param_device))
        else:
            self.register_parameter("bias", None)
        nn.init.normal_(self.weight, std=0.02)
        if self.bias is not None:
            nn.init.zeros_(self.bias)
        self._init_lowbit_precision_state(
            module_path=module_path, module_type=type(self).__name__, precision_resolver=precision_resolver,
            lowbit_capable_type="column_parallel_linear",
            kernel_spec=LowBitKernelSpec(module_type="column_parallel_linear", in_features=in_features,
                                         out_features=self.shard_size, has_bias=self.bias is not None))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._lowbit_forward(x, self.bias)


class RowParallelLinear(LowBitLinearMixin, nn.Module):
    """Input-sharded linear (layers.py:1363-1496): the backend sees bias=None and
    the bias is added after the (here trivial) reduction."""

    def __init__(self, in_features: int, out_features: int, tp_rank: int, tp_size: int, bias: bool = True,
                 tp_group=None, *, param_dtype: torch.dtype, param_device: Optional[torch.device], module_path: str,
                 precision_resolver) -> None:
        super().__init__()
        _check_tp(tp_size)
        if in_features % tp_size:
            raise ValueError(f"in_features {in_features} must be divisible by tp_size {tp_size}")
        self.in_features, self.out_features = in_features, out_features
        self.tp_rank, self.tp_size, self.tp_group = tp_rank, tp_size, tp_group
        self.shard_size = in_features // tp_size
        self.weight = nn.Parameter(torch.empty(out_features, self.shard_size, dtype=param_dtype, device=param_device))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, dtype=param_dtype, device=param_device))
        else:
            self.register_parameter("bias", None)
        nn.init.normal_(self.weight, std=0.02)
        if self.bias is not None:
            nn.init.zeros_(self.bias)
        self._init_lowbit_precision_state(
            module_path=module_path, module_type=type(self).__name__, precision_resolver=precision_resolver,
            lowbit_capable_type="row_parallel_linear",
            kernel_spec=LowBitKernelSpec(module_type="row_parallel_linear", in_features=self.shard_size,
                                         out_features=out_features, has_bias=self.bias is not None))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = self._lowbit_forward(x, None)
        if self.bias is not None:
            out = out + self.bias
        return out
