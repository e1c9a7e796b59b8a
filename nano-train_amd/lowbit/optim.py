"""AdamW on the device with the persistent low-bit refresh fused in.

nano-train steps its parameters with PrecisionAdamW
(src/runtime/optimizer_runtime.py:15-116) and then re-quantizes every
persistent low-bit weight with refresh_persistent_lowbit_params
(src/layers.py:353-407, called through mixed_precision.py:624-632).  Here one
kernel does both for a parameter: the AdamW update of the fp32 master,
exp_avg and exp_avg_sq, the parameter copy in its own dtype, and the NF4 or
persistent-FP8 codes and scales of that copy, when the weight's scale blocks
hold at most 2048 elements (a power of two).  Other weights get the update
kernel and then their module's own refresh.

The update is the reference's sequence of torch ops as they execute on the
GPU, operation for operation (add with alpha and addcdiv as one FMA each,
addcmul as an FMA over the rounded product, division by a scalar as a
multiplication by its float reciprocal), with the Python-double scalars cast
to float32 as torch casts them; the tests hold the two bit-identical.
"""

from __future__ import annotations

from typing import Dict, Iterable, Optional

import numpy as np
import torch

from . import ops
from ._lib import call

REFRESH_CODE = {None: 0, "nf4": 1, "fp8": 2}
FUSED_MAX_BLOCK = 2048


def adamw_scalars(*, lr: float, betas, eps: float, weight_decay: float, step: int) -> Dict[str, np.float32]:
    """The float32 scalars of one reference step (optimizer_runtime.py:93-109).

    bias corrections, step size and decay are Python doubles in the reference;
    torch casts each scalar argument to the tensor's float32."""
    beta1, beta2 = float(betas[0]), float(betas[1])
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    return {
        "beta1": np.float32(beta1),
        "one_minus_beta1": np.float32(1.0 - beta1),
        "beta2": np.float32(beta2),
        "one_minus_beta2": np.float32(1.0 - beta2),
        # tensor.div_(scalar) multiplies by the scalar's reciprocal, taken in
        # double and cast to float32
        "inv_bc2_sqrt": np.float32(1.0 / (bc2 ** 0.5)),
        "eps": np.float32(eps),
        "decay": np.float32(1.0 - lr * weight_decay),
        "neg_step_size": np.float32(-(lr / bc1)),
    }


def adamw_step_refresh(
    main_param: torch.Tensor,
    grad: torch.Tensor,
    exp_avg: torch.Tensor,
    exp_avg_sq: torch.Tensor,
    *,
    lr: float,
    betas,
    eps: float,
    weight_decay: float,
    step: int,
    param: Optional[torch.Tensor] = None,
    refresh: Optional[str] = None,
    block: int = 0,
    codes: Optional[torch.Tensor] = None,
    scales: Optional[torch.Tensor] = None,
) -> None:
    """One AdamW step in place on fp32 main_param / exp_avg / exp_avg_sq.

    param (optional) receives main_param in its own dtype.  refresh 'nf4' or
    'fp8' also writes the codes (packed NF4 nibbles, or e4m3 bytes) and scales
    of param's value for scale blocks of `block` elements."""
    for t, name in ((main_param, "main_param"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 tensor")
    if grad.shape != main_param.shape or exp_avg.shape != main_param.shape or exp_avg_sq.shape != main_param.shape:
        raise ValueError("grad and optimizer state must match the parameter's shape")
    if refresh not in REFRESH_CODE:
        raise ValueError(f"refresh must be None, 'nf4' or 'fp8', got {refresh!r}")
    ops._require_device(main_param, grad, exp_avg, exp_avg_sq, param, codes, scales)
    grad = grad.contiguous()
    if param is not None and (param.shape != main_param.shape or not param.is_contiguous()):
        raise ValueError("param must be contiguous with the master's shape")
    sc = adamw_scalars(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, step=step)
    call(
        "ntlb_adamw_step_refresh", main_param.data_ptr(), grad.data_ptr(), ops._dtype_code(grad.dtype),
        exp_avg.data_ptr(), exp_avg_sq.data_ptr(), ops._ptr(param),
        ops._dtype_code(param.dtype) if param is not None else 0, main_param.numel(), sc["beta1"],
        sc["one_minus_beta1"], sc["beta2"], sc["one_minus_beta2"], sc["inv_bc2_sqrt"], sc["eps"], sc["decay"],
        sc["neg_step_size"], REFRESH_CODE[refresh], block, ops._ptr(codes), ops._ptr(scales), ops._stream(),
    )


def _fused_block(module) -> Optional[int]:
    """The scale block of a persistent low-bit module when the fused refresh takes it
    (layers.py:86-101 groups: a weight row for per_channel, everything for per_tensor)."""
    w = module.weight
    gran = module._persistent_granularity()
    block = w.numel() // w.shape[0] if (gran == "per_channel" and w.dim() > 1) else w.numel()
    if 8 <= block <= FUSED_MAX_BLOCK and block & (block - 1) == 0:
        return block
    return None


class PrecisionAdamW:
    """Device mirror of PrecisionAdamW (optimizer_runtime.py:15-116).

    Same constructor and step(); the state dtypes must be fp32 (the reference
    defaults), which the fused kernel keeps.  attach_lowbit_refresh(model)
    makes step() also refresh the persistent low-bit buffers of the model's
    modules, in the same pass where their scale blocks allow."""

    def __init__(self, params: Iterable[torch.nn.Parameter], *, lr: float, weight_decay: float, betas, eps: float,
                 main_params_dtype: str = "fp32", main_grads_dtype: str = "fp32", exp_avg_dtype: str = "fp32",
                 exp_avg_sq_dtype: str = "fp32") -> None:
        for name, value in (("main_params_dtype", main_params_dtype), ("main_grads_dtype", main_grads_dtype),
                            ("exp_avg_dtype", exp_avg_dtype), ("exp_avg_sq_dtype", exp_avg_sq_dtype)):
            if str(value) not in ("fp32", "float32"):
                raise ValueError(f"{name}={value!r}: the device AdamW keeps fp32 optimizer state")
        self._params = [p for p in params if p.requires_grad]
        self.param_groups = [{"params": self._params, "lr": float(lr), "weight_decay": float(weight_decay),
                              "betas": tuple(betas), "eps": float(eps)}]
        self.state: Dict[torch.nn.Parameter, dict] = {}
        self._global_step = 0
        self._refresh_modules: Dict[int, torch.nn.Module] = {}
        for p in self._params:
            main = p.detach().to(dtype=torch.float32).clone().contiguous()
            self.state[p] = {"step": 0, "main_param": main, "exp_avg": torch.zeros_like(main),
                             "exp_avg_sq": torch.zeros_like(main)}

    def attach_lowbit_refresh(self, model: torch.nn.Module) -> int:
        """Refresh the persistent low-bit buffers of model's modules in step()."""
        tracked = {id(p) for p in self._params}
        n = 0
        for module in model.modules():
            if not callable(getattr(module, "refresh_persistent_lowbit_params", None)):
                continue
            weight = getattr(module, "weight", None)
            if weight is None or id(weight) not in tracked or module._persistent_mode() == "off":
                continue
            self._refresh_modules[id(weight)] = module
            n += 1
        return n

    def zero_grad(self, set_to_none: bool = True) -> None:
        for p in self._params:
            if p.grad is None:
                continue
            if set_to_none:
                p.grad = None
            else:
                p.grad.zero_()

    @torch.no_grad()
    def step(self) -> bool:
        group = self.param_groups[0]
        self._global_step += 1
        for p in self._params:
            if p.grad is None:
                continue
            st = self.state[p]
            st["step"] = int(st["step"]) + 1
            module = self._refresh_modules.get(id(p))
            kw = dict(lr=group["lr"], betas=group["betas"], eps=group["eps"], weight_decay=group["weight_decay"],
                      step=st["step"])
            target = p.data if p.data.is_contiguous() else None
            mode = module._persistent_mode() if module is not None else "off"
            block = _fused_block(module) if module is not None else None
            if module is not None and block is not None and target is not None:
                refresh = "fp8" if mode == "fp8" else "nf4"
                n = p.numel()
                nb = ops.cdiv(n, block)
                if refresh == "nf4":
                    codes = torch.empty((n + 1) // 2, dtype=torch.uint8, device=p.device)
                else:
                    codes = torch.empty(n, dtype=torch.uint8, device=p.device)
                scales = torch.empty(nb, dtype=torch.float32, device=p.device)
                adamw_step_refresh(st["main_param"], p.grad, st["exp_avg"], st["exp_avg_sq"], param=target,
                                   refresh=refresh, block=block, codes=codes, scales=scales, **kw)
                module._set_persistent_buffers(refresh, codes, scales)
            else:
                adamw_step_refresh(st["main_param"], p.grad, st["exp_avg"], st["exp_avg_sq"], param=target, **kw)
                if target is None:
                    p.data.copy_(st["main_param"].to(dtype=p.dtype))
                if module is not None:
                    module.refresh_persistent_lowbit_params()
        return True
