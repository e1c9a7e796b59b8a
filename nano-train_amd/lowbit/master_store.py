"""Optimizer-owned master weights for persistent low-bit modules.

The --lowbit-master-ownership optimizer mode of nano-train
(src/runtime/master_store.py:28-119): every module that stores its weight in a
persistent low-bit format gets a full-precision nn.Parameter clone held in a
LowBitMasterStore attached to the model, and the module's `weight` is rebound
to it.  No kernels are involved; the low-bit codes are refreshed from these
masters by refresh_persistent_lowbit_params().
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch.nn as nn

from .layers import ColumnParallelLinear
from .layers import RowParallelLinear


@dataclass(frozen=True)
class MasterBindingMetadata:
    module_path: str
    parameter_name: str
    shard_domain: str
    shape: tuple


class LowBitMasterStore(nn.Module):
    """Registry of optimizer-owned master parameters."""

    def __init__(self) -> None:
        super().__init__()
        self.masters = nn.ParameterDict()
        self.metadata: dict = {}

    def add_master(self, *, key: str, param: nn.Parameter, metadata: MasterBindingMetadata) -> nn.Parameter:
        self.masters[key] = param
        self.metadata[key] = metadata
        return self.masters[key]


def _shard_domain(module: nn.Module, path: str) -> str:
    if isinstance(module, (ColumnParallelLinear, RowParallelLinear)) and module.tp_size > 1:
        return "tensor_model_parallel"
    return "expert_model_parallel" if ".experts." in path else "data_parallel"


def materialize_optimizer_owned_masters(model: nn.Module, *, precision_config) -> Optional[LowBitMasterStore]:
    if precision_config.lowbit_master_ownership != "optimizer":
        return None
    store = LowBitMasterStore()
    bound = 0
    for _, module in model.named_modules():
        assignment = getattr(module, "module_precision_assignment", None)
        bind = getattr(module, "bind_optimizer_master_weight", None)
        weight = getattr(module, "weight", None)
        if assignment is None or not callable(bind) or not isinstance(weight, nn.Parameter):
            continue
        if getattr(assignment, "persistent_lowbit_mode", "off") == "off":
            continue
        path = str(getattr(module, "module_path", getattr(assignment, "module_name", "")))
        if not path:
            continue
        master = store.add_master(
            key=path.replace(".", "__") + "__weight",
            param=nn.Parameter(weight.detach().clone()),
            metadata=MasterBindingMetadata(path, "weight", _shard_domain(module, path), tuple(weight.shape)),
        )
        bind(master)
        bound += 1
    if bound == 0:
        return None
    model.add_module("_lowbit_master_store", store)
    return store


def get_lowbit_master_store(model: nn.Module) -> Optional[LowBitMasterStore]:
    store = getattr(model, "_lowbit_master_store", None)
    return store if isinstance(store, LowBitMasterStore) else None
