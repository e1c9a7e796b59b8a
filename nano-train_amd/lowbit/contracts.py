"""Value types of the low-bit path, mirroring nano-train's src/runtime/contracts.py.

Only the types the hot path reads are restated here, with the same names,
fields and defaults, so code written against the reference's contracts
(``LowBitKernelSpec``, ``DeepSeekV3PrecisionRecipe``, the per-module
assignment and init state) works unchanged.  ``LowBitBackendName`` gains the
``"hip"`` choice, the MI355X backend of this package.
"""

from __future__ import annotations

from dataclasses import dataclass
from dataclasses import field
from typing import Literal
from typing import Optional

PrecisionMode = Literal["fp32", "bf16", "fp16", "fp8", "fp4"]
PrecisionDType = Literal["fp32", "bf16", "fp16"]
LowBitBackendName = Literal["transformer_engine", "emulated", "hip"]
FP8Format = Literal["e4m3", "hybrid"]
FP8AmaxComputeAlgo = Literal["most_recent", "max"]
ModulePatternType = Literal["regex", "glob"]
LowBitComputeMode = Literal["fp8", "fp4"]
PersistentLowBitMode = Literal["off", "fp8", "fp4"]
PersistentScaleGranularity = Literal["per_tensor", "per_channel"]
FP4PersistentFormat = Literal["nf4"]
LowBitCapableModuleType = Literal["linear", "column_parallel_linear", "row_parallel_linear"]
MasterOwnershipMode = Literal["module", "optimizer"]
QuantGranularity = Literal["tensor", "channel", "tile_1x128", "block_128x128"]
RoundingMode = Literal["nearest", "stochastic"]
PrecisionRecipeName = Literal["default", "deepseek_v3"]
# MI355X backend only: how codes are represented on the wire and in the GEMM
LowBitCodeFormat = Literal["int_grid", "e4m3"]
LowBitBackwardRecipe = Literal["ste", "fp8"]
LowBitForwardMode = Literal["blockscaled", "reference"]


@dataclass(frozen=True)
class DeepSeekV3PrecisionRecipe:
    """DeepSeek-V3 style FP8 training recipe (contracts.py:42-52)."""

    activation_quant_granularity: QuantGranularity = "tile_1x128"
    weight_quant_granularity: QuantGranularity = "block_128x128"
    rounding_mode: RoundingMode = "stochastic"
    comm_quant_enabled: bool = True
    comm_quant_granularity: QuantGranularity = "block_128x128"
    high_precision_module_patterns: tuple[str, ...] = ()
    high_precision_grad_patterns: tuple[str, ...] = ()


@dataclass(frozen=True)
class LowBitKernelSpec:
    """Kernel metadata needed by low-bit backends (contracts.py:55-65)."""

    module_type: LowBitCapableModuleType
    in_features: int
    out_features: int
    has_bias: bool
    activation_quant_granularity: QuantGranularity = "tensor"
    weight_quant_granularity: QuantGranularity = "tensor"
    rounding_mode: RoundingMode = "nearest"


@dataclass
class ModulePrecisionPolicy:
    """Module-pattern policy (contracts.py:68-81)."""

    pattern_type: ModulePatternType = "regex"
    compute_lowbit_mode: Optional[LowBitComputeMode] = None
    compute_lowbit_include: tuple[str, ...] = ()
    compute_lowbit_exclude: tuple[str, ...] = ()
    persistent_lowbit_mode: PersistentLowBitMode = "off"
    persistent_lowbit_include: tuple[str, ...] = ()
    persistent_lowbit_exclude: tuple[str, ...] = ()
    persistent_scale_granularity: PersistentScaleGranularity = "per_channel"
    fp4_persistent_format: FP4PersistentFormat = "nf4"
    module_compute_dtype_rules: tuple[str, ...] = ()


@dataclass
class ModulePrecisionAssignment:
    """Resolved assignment for one module (contracts.py:84-94)."""

    module_name: str
    module_type: str
    compute_lowbit_mode: Optional[LowBitComputeMode]
    persistent_lowbit_mode: PersistentLowBitMode
    persistent_scale_granularity: PersistentScaleGranularity
    fp4_persistent_format: FP4PersistentFormat
    compute_dtype_override: Optional[PrecisionDType] = None


@dataclass(frozen=True)
class ModulePrecisionInitState:
    """Constructor-time state of one module (contracts.py:106-113)."""

    assignment: ModulePrecisionAssignment
    lowbit_backend: Optional[object] = None
    lowbit_capable_type: Optional[LowBitCapableModuleType] = None
    master_ownership_mode: MasterOwnershipMode = "module"


@dataclass(frozen=True)
class ModulePrecisionSummary:
    parameterized_module_count: int = 0
    lowbit_capable_module_count: int = 0
    compute_lowbit_module_count: int = 0
    persistent_lowbit_module_count: int = 0
    high_precision_exception_module_count: int = 0


@dataclass
class PrecisionConfig:
    """Resolved precision settings (contracts.py:150-183) plus the MI355X backend knobs."""

    mode: PrecisionMode = "fp32"
    params_dtype: PrecisionDType = "fp32"
    main_params_dtype: PrecisionDType = "fp32"
    main_grads_dtype: PrecisionDType = "fp32"
    exp_avg_dtype: PrecisionDType = "fp32"
    exp_avg_sq_dtype: PrecisionDType = "fp32"
    activation_dtype: PrecisionDType = "fp32"
    fp8_backend: LowBitBackendName = "transformer_engine"
    fp8_format: FP8Format = "e4m3"
    fp8_amax_history_len: int = 16
    fp8_amax_compute_algo: FP8AmaxComputeAlgo = "most_recent"
    fp4_backend: Literal["emulated", "hip"] = "emulated"
    module_precision_policy: Optional[ModulePrecisionPolicy] = None
    fp8_param: bool = False
    fp4_param: bool = False
    fp4_param_format: FP4PersistentFormat = "nf4"
    persistent_scale_granularity: PersistentScaleGranularity = "per_channel"
    lowbit_master_ownership: MasterOwnershipMode = "optimizer"
    precision_recipe_name: PrecisionRecipeName = "default"
    deepseek_v3_recipe: Optional[DeepSeekV3PrecisionRecipe] = None
    loss_scale_init: float = 65536.0
    loss_scale_growth_factor: float = 2.0
    loss_scale_backoff_factor: float = 0.5
    loss_scale_growth_interval: int = 2000
    loss_scale_min: float = 1.0
    loss_scale_max: float = 16777216.0
    # MI355X backend: code format and backward recipe (no reference counterpart)
    lowbit_code_format: LowBitCodeFormat = "int_grid"
    lowbit_backward: LowBitBackwardRecipe = "ste"
    lowbit_forward: LowBitForwardMode = "blockscaled"
    lowbit_seed: Optional[int] = None
    extra: dict = field(default_factory=dict)
