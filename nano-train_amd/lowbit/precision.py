"""Precision flags, config resolution and the per-module resolver for the MI355X backend.

This restates the precision-policy surface of nano-train (src/runtime/
precision_args.py:13-228 and src/runtime/mixed_precision.py:222-762) so that
the same command lines select the same modules and recipes; the one addition
is the backend name "hip" for --fp8-backend / --fp4-backend, which builds
lowbit.backend.HipLowBitBackend, plus four knobs the MI355X backend reads:

  --lowbit-code-format {int_grid,e4m3}  int_grid reproduces the emulated
                                        backend's integer grid (qmax = 127 / 7);
                                        e4m3 is the DeepSeek-V3 amax/448 format
  --lowbit-backward {ste,fp8}           ste = the reference's straight-through
                                        backward; fp8 = quantized dgrad/wgrad
  --lowbit-forward {blockscaled,reference}
                                        blockscaled = codes on fp8/int8 MFMA with
                                        the scales applied per 128-K block;
                                        reference = the reference's operands,
                                        bf16(q*s), on bf16 MFMA
  --lowbit-seed INT                     seed of the stochastic-rounding stream

The loss-scaling controller and the Transformer Engine backend of the
reference are not part of this path and are not restated.
"""

from __future__ import annotations

import argparse
import fnmatch
import re
from dataclasses import replace
from typing import Iterable, Optional

import torch

from .contracts import (
    DeepSeekV3PrecisionRecipe,
    LowBitKernelSpec,
    ModulePrecisionAssignment,
    ModulePrecisionInitState,
    ModulePrecisionPolicy,
    ModulePrecisionSummary,
    PrecisionConfig,
)

LOWBIT_CAPABLE_TYPES = frozenset({"linear", "column_parallel_linear", "row_parallel_linear"})
_DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def dtype_alias_to_torch(alias: str) -> torch.dtype:
    try:
        return _DTYPES[alias]
    except KeyError as exc:
        raise ValueError(f"Unsupported precision dtype alias: {alias}") from exc


# ----------------------------------------------------------------------------
# flags (precision_args.py:13-220)
# ----------------------------------------------------------------------------

def add_mixed_precision_args(parser: argparse.ArgumentParser) -> None:
    """Register the shared precision and low-bit policy flags."""
    dtypes = ["fp32", "bf16", "fp16"]
    a = parser.add_argument
    a("--precision-recipe", type=str, default="default", choices=["default", "deepseek_v3"],
      help="Precision policy preset; deepseek_v3 turns on the DeepSeek-V3 FP8 defaults")
    for flag, what in (("--bf16", "BF16"), ("--fp16", "FP16"), ("--fp8", "FP8"), ("--fp4", "FP4")):
        a(flag, action="store_true", help=f"{what} mixed precision")
    a("--fp8-backend", type=str, default="transformer_engine", choices=["transformer_engine", "emulated", "hip"],
      help="FP8 backend; hip = the MI355X kernels of this package")
    a("--fp8-format", type=str, default="e4m3", choices=["e4m3", "hybrid"])
    a("--fp8-amax-history-len", type=int, default=16)
    a("--fp8-amax-compute-algo", type=str, default="most_recent", choices=["most_recent", "max"])
    a("--fp4-backend", type=str, default="emulated", choices=["emulated", "hip"])
    for name in ("params", "main-params", "main-grads", "exp-avg", "exp-avg-sq"):
        a(f"--{name}-dtype", type=str, default=None, choices=dtypes)
    a("--loss-scale-init", type=float, default=65536.0)
    a("--loss-scale-growth-factor", type=float, default=2.0)
    a("--loss-scale-backoff-factor", type=float, default=0.5)
    a("--loss-scale-growth-interval", type=int, default=2000)
    a("--loss-scale-min", type=float, default=1.0)
    a("--loss-scale-max", type=float, default=16777216.0)
    a("--fp8-param", action="store_true", help="persistent FP8 parameter storage")
    a("--fp4-param", action="store_true", help="persistent FP4 (NF4) parameter storage")
    a("--fp4-param-format", type=str, default="nf4", choices=["nf4"])
    a("--persistent-scale-granularity", type=str, default="per_channel", choices=["per_tensor", "per_channel"])
    a("--module-pattern-type", type=str, default="regex", choices=["regex", "glob"])
    a("--compute-lowbit-mode", type=str, default=None, choices=["fp8", "fp4"])
    a("--compute-lowbit-include", action="append", default=None)
    a("--compute-lowbit-exclude", action="append", default=None)
    a("--persistent-lowbit-mode", type=str, default="off", choices=["off", "fp8", "fp4"])
    a("--persistent-lowbit-include", action="append", default=None)
    a("--persistent-lowbit-exclude", action="append", default=None)
    a("--module-compute-dtype-rule", action="append", default=None,
      help="'<pattern>=<fp32|bf16|fp16>' compute dtype override, repeatable")
    a("--lowbit-master-ownership", type=str, default="optimizer", choices=["module", "optimizer"])
    a("--fp8-rounding", type=str, default=None, choices=["nearest", "stochastic"])
    a("--fp8-activation-granularity", type=str, default=None, choices=["tile_1x128", "tensor", "channel"])
    a("--fp8-weight-granularity", type=str, default=None, choices=["block_128x128", "tensor", "channel"])
    a("--fp8-comm-quant", action=argparse.BooleanOptionalAction, default=None)
    a("--fp8-comm-granularity", type=str, default=None, choices=["block_128x128", "tensor", "channel"])
    # MI355X backend knobs
    a("--lowbit-code-format", type=str, default="int_grid", choices=["int_grid", "e4m3"])
    a("--lowbit-backward", type=str, default="ste", choices=["ste", "fp8"])
    a("--lowbit-forward", type=str, default="blockscaled", choices=["blockscaled", "reference"])
    a("--lowbit-seed", type=int, default=None)


def normalize_and_resolve_precision(args: argparse.Namespace, device: torch.device) -> PrecisionConfig:
    return resolve_precision_config(args, device)


# ----------------------------------------------------------------------------
# value normalization
# ----------------------------------------------------------------------------

def _patterns(value) -> tuple[str, ...]:
    if value is None:
        return ()
    items = [value] if isinstance(value, str) else (list(value) if isinstance(value, Iterable) else [value])
    return tuple(t for t in (str(v).strip() for v in items) if t)


def _choice(raw, allowed, message: str, *, default=None, empty_as=None):
    value = default if raw is None else str(raw)
    if empty_as is not None and value in ("", "none", "off"):
        return empty_as
    if value not in allowed:
        raise ValueError(message)
    return value


def _granularity(raw, flag: str) -> str:
    return _choice(raw, ("tensor", "channel", "tile_1x128", "block_128x128"),
                   f"{flag} must be one of tensor, channel, tile_1x128, block_128x128")


def _mode_from_flags(args) -> Optional[str]:
    chosen = [m for m in ("bf16", "fp16", "fp8", "fp4") if bool(getattr(args, m, False))]
    if len(chosen) > 1:
        raise ValueError("At most one of --bf16/--fp16/--fp8/--fp4 may be set")
    return chosen[0] if chosen else None


def _cuda_bf16(device: torch.device) -> bool:
    return device.type == "cuda" and torch.cuda.is_bf16_supported()


def _default_mode(device: torch.device) -> str:
    return "bf16" if _cuda_bf16(device) else "fp32"


def _default_dtype_for_mode(mode: str, device: torch.device) -> str:
    # mixed_precision.py:86-110: activations and parameters follow the mode;
    # low-bit modes use bf16 on a bf16-capable GPU, fp16 on other GPUs, fp32 on CPU
    if mode in ("bf16", "fp16"):
        return mode
    if mode in ("fp8", "fp4"):
        if _cuda_bf16(device):
            return "bf16"
        return "fp16" if device.type == "cuda" else "fp32"
    return "fp32"


# ----------------------------------------------------------------------------
# DeepSeek-V3 recipe (mixed_precision.py:222-291)
# ----------------------------------------------------------------------------

def default_deepseek_v3_recipe() -> DeepSeekV3PrecisionRecipe:
    return DeepSeekV3PrecisionRecipe(
        activation_quant_granularity="tile_1x128",
        weight_quant_granularity="block_128x128",
        rounding_mode="stochastic",
        comm_quant_enabled=True,
        comm_quant_granularity="block_128x128",
        # embeddings, the LM head, norms and routers stay in high precision
        high_precision_module_patterns=(
            r"(^|\\.)token_embeddings$",
            r"(^|\\.)position_embeddings$",
            r"(^|\\.)lm_head$",
            r"(^|\\.)final_norm$",
            r"(^|\\.).*norm$",
            r"(^|\\.).*router(\\.|$)",
        ),
        high_precision_grad_patterns=(r"(^|\\.)lm_head(\\.|$)", r"(^|\\.).*router(\\.|$)"),
    )


def recipe_from_args(args) -> DeepSeekV3PrecisionRecipe:
    """Recipe defaults, each overridable by its --fp8-* flag."""
    base = default_deepseek_v3_recipe()
    overrides = {}
    if getattr(args, "fp8_activation_granularity", None) is not None:
        overrides["activation_quant_granularity"] = _granularity(args.fp8_activation_granularity,
                                                                 "--fp8-activation-granularity")
    if getattr(args, "fp8_weight_granularity", None) is not None:
        overrides["weight_quant_granularity"] = _granularity(args.fp8_weight_granularity,
                                                             "--fp8-weight-granularity")
    if getattr(args, "fp8_rounding", None) is not None:
        overrides["rounding_mode"] = _choice(args.fp8_rounding, ("nearest", "stochastic"),
                                             "--fp8-rounding must be nearest or stochastic")
    if getattr(args, "fp8_comm_quant", None) is not None:
        overrides["comm_quant_enabled"] = bool(args.fp8_comm_quant)
    if getattr(args, "fp8_comm_granularity", None) is not None:
        overrides["comm_quant_granularity"] = _granularity(args.fp8_comm_granularity, "--fp8-comm-granularity")
    return replace(base, **overrides)


# ----------------------------------------------------------------------------
# module policy (mixed_precision.py:310-364)
# ----------------------------------------------------------------------------

def resolve_module_precision_policy(args, config: PrecisionConfig) -> ModulePrecisionPolicy:
    pattern_type = _choice(getattr(args, "module_pattern_type", "regex") or "regex", ("regex", "glob"),
                           "--module-pattern-type must be regex or glob")
    explicit = _choice(getattr(args, "compute_lowbit_mode", None), ("fp8", "fp4"),
                       "--compute-lowbit-mode must be fp8 or fp4", empty_as=None) \
        if getattr(args, "compute_lowbit_mode", None) not in (None, "", "none", "off") else None
    compute_mode = explicit if explicit is not None else (config.mode if config.mode in ("fp8", "fp4") else None)

    fp8_param = bool(getattr(args, "fp8_param", False))
    fp4_param = bool(getattr(args, "fp4_param", False))
    if fp8_param and fp4_param:
        raise ValueError("At most one of --fp8-param/--fp4-param may be set")
    raw_persistent = getattr(args, "persistent_lowbit_mode", None)
    flag_mode = "off" if raw_persistent in (None, "", "none") else _choice(
        raw_persistent, ("off", "fp8", "fp4"), "--persistent-lowbit-mode must be off, fp8, or fp4")
    if flag_mode == "off":
        persistent = "fp8" if fp8_param else ("fp4" if fp4_param else "off")
    else:
        if fp8_param and flag_mode != "fp8":
            raise ValueError("--fp8-param conflicts with --persistent-lowbit-mode")
        if fp4_param and flag_mode != "fp4":
            raise ValueError("--fp4-param conflicts with --persistent-lowbit-mode")
        persistent = flag_mode
    granularity = _choice(getattr(args, "persistent_scale_granularity", "per_channel") or "per_channel",
                          ("per_tensor", "per_channel"),
                          "--persistent-scale-granularity must be per_tensor or per_channel")
    fp4_format = _choice(getattr(args, "fp4_param_format", "nf4") or "nf4", ("nf4",),
                         "--fp4-param-format currently supports only nf4")
    return ModulePrecisionPolicy(
        pattern_type=pattern_type,
        compute_lowbit_mode=compute_mode,
        compute_lowbit_include=_patterns(getattr(args, "compute_lowbit_include", None)),
        compute_lowbit_exclude=_patterns(getattr(args, "compute_lowbit_exclude", None)),
        persistent_lowbit_mode=persistent,
        persistent_lowbit_include=_patterns(getattr(args, "persistent_lowbit_include", None)),
        persistent_lowbit_exclude=_patterns(getattr(args, "persistent_lowbit_exclude", None)),
        persistent_scale_granularity=granularity,
        fp4_persistent_format=fp4_format,
        module_compute_dtype_rules=_patterns(getattr(args, "module_compute_dtype_rule", None)),
    )


def _required_lowbit_modes(config: PrecisionConfig) -> set:
    modes = {config.mode} if config.mode in ("fp8", "fp4") else set()
    pol = config.module_precision_policy
    if pol is not None and pol.compute_lowbit_mode is not None:
        modes.add(pol.compute_lowbit_mode)
    return modes


# ----------------------------------------------------------------------------
# config (mixed_precision.py:635-762)
# ----------------------------------------------------------------------------

def resolve_precision_config(args, device: torch.device) -> PrecisionConfig:
    recipe_name = _choice(getattr(args, "precision_recipe", "default") or "default", ("default", "deepseek_v3"),
                          "--precision-recipe must be default or deepseek_v3")
    explicit = _mode_from_flags(args)
    if recipe_name == "deepseek_v3":
        if explicit not in (None, "fp8"):
            raise ValueError("--precision-recipe deepseek_v3 requires --fp8 (or no explicit mode)")
        mode = "fp8"
    else:
        mode = explicit or _default_mode(device)
    if mode == "bf16":
        if device.type != "cuda":
            raise ValueError("--bf16 requires CUDA")
        if not torch.cuda.is_bf16_supported():
            raise ValueError("--bf16 requires torch.cuda.is_bf16_supported()")
    if mode == "fp16" and device.type != "cuda":
        raise ValueError("--fp16 requires CUDA")

    fp8_backend = str(getattr(args, "fp8_backend", "transformer_engine"))
    fp8_format = str(getattr(args, "fp8_format", "e4m3"))
    history = int(getattr(args, "fp8_amax_history_len", 16))
    algo = str(getattr(args, "fp8_amax_compute_algo", "most_recent"))
    fp4_backend = str(getattr(args, "fp4_backend", "emulated"))
    ownership = str(getattr(args, "lowbit_master_ownership", "optimizer"))
    if mode == "fp8" and fp8_backend not in ("transformer_engine", "emulated", "hip"):
        raise ValueError("--fp8-backend must be transformer_engine, emulated or hip")
    if mode == "fp8" and fp8_format not in ("e4m3", "hybrid"):
        raise ValueError("--fp8-format must be e4m3 or hybrid")
    if mode == "fp8" and algo not in ("most_recent", "max"):
        raise ValueError("--fp8-amax-compute-algo must be most_recent or max")
    if mode == "fp8" and history < 1:
        raise ValueError("--fp8-amax-history-len must be >= 1")
    if mode == "fp4" and fp4_backend not in ("emulated", "hip"):
        raise ValueError("--fp4-backend must be emulated or hip")
    if ownership not in ("module", "optimizer"):
        raise ValueError("--lowbit-master-ownership must be module or optimizer")

    def _dtype(name: str, default: str) -> str:
        raw = getattr(args, name, None)
        value = default if raw is None else str(raw)
        if value not in _DTYPES:
            raise ValueError(f"--{name.replace('_', '-')} must be fp32, bf16, or fp16")
        return value

    growth_interval = int(getattr(args, "loss_scale_growth_interval", 2000))
    if growth_interval < 1:
        raise ValueError("--loss-scale-growth-interval must be >= 1")
    code_format = str(getattr(args, "lowbit_code_format", "int_grid") or "int_grid")
    if code_format not in ("int_grid", "e4m3"):
        raise ValueError("--lowbit-code-format must be int_grid or e4m3")
    backward = str(getattr(args, "lowbit_backward", "ste") or "ste")
    if backward not in ("ste", "fp8"):
        raise ValueError("--lowbit-backward must be ste or fp8")
    forward = str(getattr(args, "lowbit_forward", "blockscaled") or "blockscaled")
    if forward not in ("blockscaled", "reference"):
        raise ValueError("--lowbit-forward must be blockscaled or reference")

    config = PrecisionConfig(
        mode=mode,
        params_dtype=_dtype("params_dtype", _default_dtype_for_mode(mode, device)),
        main_params_dtype=_dtype("main_params_dtype", "fp32"),
        main_grads_dtype=_dtype("main_grads_dtype", "fp32"),
        exp_avg_dtype=_dtype("exp_avg_dtype", "fp32"),
        exp_avg_sq_dtype=_dtype("exp_avg_sq_dtype", "fp32"),
        activation_dtype=_default_dtype_for_mode(mode, device),
        fp8_backend=fp8_backend,
        fp8_format=fp8_format,
        fp8_amax_history_len=history,
        fp8_amax_compute_algo=algo,
        fp4_backend=fp4_backend,
        fp8_param=bool(getattr(args, "fp8_param", False)),
        fp4_param=bool(getattr(args, "fp4_param", False)),
        fp4_param_format=_choice(getattr(args, "fp4_param_format", "nf4") or "nf4", ("nf4",),
                                 "--fp4-param-format currently supports only nf4"),
        persistent_scale_granularity=_choice(
            getattr(args, "persistent_scale_granularity", "per_channel") or "per_channel",
            ("per_tensor", "per_channel"), "--persistent-scale-granularity must be per_tensor or per_channel"),
        lowbit_master_ownership=ownership,
        precision_recipe_name=recipe_name,
        deepseek_v3_recipe=recipe_from_args(args) if recipe_name == "deepseek_v3" else None,
        loss_scale_init=float(getattr(args, "loss_scale_init", 65536.0)),
        loss_scale_growth_factor=float(getattr(args, "loss_scale_growth_factor", 2.0)),
        loss_scale_backoff_factor=float(getattr(args, "loss_scale_backoff_factor", 0.5)),
        loss_scale_growth_interval=growth_interval,
        loss_scale_min=float(getattr(args, "loss_scale_min", 1.0)),
        loss_scale_max=float(getattr(args, "loss_scale_max", 16777216.0)),
        lowbit_code_format=code_format,
        lowbit_backward=backward,
        lowbit_forward=forward,
        lowbit_seed=getattr(args, "lowbit_seed", None),
    )
    if config.loss_scale_init <= 0:
        raise ValueError("--loss-scale-init must be > 0")
    if config.loss_scale_growth_factor <= 1.0:
        raise ValueError("--loss-scale-growth-factor must be > 1")
    if not 0.0 < config.loss_scale_backoff_factor < 1.0:
        raise ValueError("--loss-scale-backoff-factor must be in (0, 1)")
    if config.loss_scale_min <= 0.0:
        raise ValueError("--loss-scale-min must be > 0")
    if config.loss_scale_max < config.loss_scale_min:
        raise ValueError("--loss-scale-max must be >= --loss-scale-min")
    config.module_precision_policy = resolve_module_precision_policy(args, config)
    # availability probe: every backend this run needs must be constructible
    for needed in _required_lowbit_modes(config):
        build_lowbit_backend_for_mode(config, mode=needed, kernel_spec=None)
    return config


# ----------------------------------------------------------------------------
# backend factory (te_backend.py:393-416)
# ----------------------------------------------------------------------------

def build_lowbit_backend_for_mode(config: PrecisionConfig, *, mode: str, kernel_spec: Optional[LowBitKernelSpec]):
    """Build the low-bit backend for one mode.  Only "hip" lives in this package;
    "emulated" and "transformer_engine" are the reference's own backends."""
    if mode == "fp8":
        name = config.fp8_backend
    elif mode == "fp4":
        name = config.fp4_backend
    else:
        return None
    if name == "hip":
        from .backend import build_hip_backend

        return build_hip_backend(config, mode=mode, kernel_spec=kernel_spec)
    flag = "--fp8-backend" if mode == "fp8" else "--fp4-backend"
    raise ValueError(f"Unsupported {mode} backend: {name} ({flag} hip selects the MI355X kernels; "
                     "emulated and transformer_engine are provided by nano-train itself)")


# ----------------------------------------------------------------------------
# per-module resolver (mixed_precision.py:378-621)
# ----------------------------------------------------------------------------

def _matches(name: str, pattern: str, pattern_type: str) -> bool:
    return re.search(pattern, name) is not None if pattern_type == "regex" else fnmatch.fnmatch(name, pattern)


def _dtype_rules(raw) -> tuple:
    rules = []
    for rule in _patterns(raw):
        if "=" not in rule:
            raise ValueError("--module-compute-dtype-rule must use '<pattern>=<fp32|bf16|fp16>' format")
        pattern, dt = (p.strip() for p in rule.split("=", 1))
        if not pattern:
            raise ValueError("--module-compute-dtype-rule pattern cannot be empty")
        if dt not in _DTYPES:
            raise ValueError("--module-compute-dtype-rule dtype must be one of fp32, bf16, fp16")
        rules.append((pattern, dt))
    return tuple(rules)


class ModulePrecisionResolverImpl:
    """Constructor-time precision state for every parameterized module."""

    def __init__(self, config: PrecisionConfig) -> None:
        self._config = replace(config)
        self._policy = config.module_precision_policy or ModulePrecisionPolicy()
        self._rules = _dtype_rules(self._policy.module_compute_dtype_rules)
        self._seen: set = set()
        self._compute_hits: set = set()
        self._persistent_hits: set = set()
        self._hp_hits: set = set()
        self._rule_hits: set = set()
        self._counts = dict(param=0, capable=0, compute=0, persistent=0, hp=0)

    def _selected(self, path: str, include, exclude, default_all: bool):
        include_hit = any(_matches(path, p, self._policy.pattern_type) for p in include) if include else False
        chosen = include_hit if include else default_all
        if chosen and any(_matches(path, p, self._policy.pattern_type) for p in exclude):
            chosen = False
        return chosen, include_hit

    def resolve_module_init_state(self, *, module_path: str, module_type: str, lowbit_capable_type=None,
                                  kernel_spec: Optional[LowBitKernelSpec] = None) -> ModulePrecisionInitState:
        if not module_path:
            raise ValueError("module_path must be non-empty for precision resolution")
        if module_path in self._seen:
            raise ValueError(f"Duplicate module_path for precision resolution: {module_path}")
        self._seen.add(module_path)
        self._counts["param"] += 1
        pol = self._policy
        capable = lowbit_capable_type in LOWBIT_CAPABLE_TYPES
        self._counts["capable"] += int(capable)

        compute_sel, hit = self._selected(module_path, pol.compute_lowbit_include, pol.compute_lowbit_exclude,
                                          pol.compute_lowbit_mode is not None and capable)
        if hit:
            self._compute_hits.add(module_path)
        persist_sel, hit = self._selected(module_path, pol.persistent_lowbit_include, pol.persistent_lowbit_exclude,
                                          pol.persistent_lowbit_mode != "off" and capable)
        if hit:
            self._persistent_hits.add(module_path)
        if compute_sel and not capable and pol.compute_lowbit_mode is not None:
            raise ValueError("compute_lowbit patterns matched modules without low-bit support: "
                             f"{module_path} ({module_type})")
        if persist_sel and not capable and pol.persistent_lowbit_mode != "off":
            raise ValueError("persistent_lowbit patterns matched modules without low-bit support: "
                             f"{module_path} ({module_type})")
        compute_mode = pol.compute_lowbit_mode if (capable and compute_sel) else None
        persistent_mode = pol.persistent_lowbit_mode if (capable and persist_sel) else "off"

        recipe = self._config.deepseek_v3_recipe
        if recipe is not None and any(re.search(p, module_path) for p in recipe.high_precision_module_patterns):
            self._hp_hits.add(module_path)
            self._counts["hp"] += 1
            compute_mode, persistent_mode = None, "off"

        override = None
        for pattern, dt in self._rules:
            if _matches(module_path, pattern, pol.pattern_type):
                override = dt
                self._rule_hits.add((pattern, dt))
        if compute_mode is not None and override is not None:
            raise ValueError("module matched both low-bit compute and compute-dtype override: "
                             f"{module_path}. Adjust --compute-lowbit-* or --module-compute-dtype-rule.")
        self._counts["compute"] += int(compute_mode is not None)
        self._counts["persistent"] += int(persistent_mode != "off")

        assignment = ModulePrecisionAssignment(
            module_name=module_path, module_type=module_type, compute_lowbit_mode=compute_mode,
            persistent_lowbit_mode=persistent_mode, persistent_scale_granularity=pol.persistent_scale_granularity,
            fp4_persistent_format=pol.fp4_persistent_format, compute_dtype_override=override)
        backend = None
        if compute_mode is not None:
            spec = kernel_spec
            if spec is not None and recipe is not None:
                # the recipe sets granularity and rounding of every low-bit module
                spec = replace(spec, activation_quant_granularity=recipe.activation_quant_granularity,
                               weight_quant_granularity=recipe.weight_quant_granularity,
                               rounding_mode=recipe.rounding_mode)
            backend = build_lowbit_backend_for_mode(self._config, mode=compute_mode, kernel_spec=spec)
            if backend is None:
                raise RuntimeError(f"No backend available for compute mode {compute_mode} at module {module_path}")
        return ModulePrecisionInitState(assignment=assignment, lowbit_backend=backend,
                                        lowbit_capable_type=lowbit_capable_type,
                                        master_ownership_mode=self._config.lowbit_master_ownership)

    def finalize(self) -> ModulePrecisionSummary:
        pol = self._policy
        if pol.compute_lowbit_include and not self._compute_hits:
            raise ValueError("compute_lowbit include patterns matched zero modules")
        if pol.persistent_lowbit_include and not self._persistent_hits:
            raise ValueError("persistent_lowbit include patterns matched zero modules")
        unmatched = [f"{p}={d}" for p, d in self._rules if (p, d) not in self._rule_hits]
        if unmatched:
            raise ValueError(f"module compute dtype rules matched zero modules: {unmatched[:3]}")
        if self._config.mode in ("fp8", "fp4") and self._counts["compute"] == 0:
            raise RuntimeError(
                f"Low-bit mode '{self._config.mode}' is active but zero modules were assigned for low-bit "
                "compute. Check --compute-lowbit-include/--compute-lowbit-exclude or verify the model uses "
                "low-bit-capable layers.")
        recipe = self._config.deepseek_v3_recipe
        if recipe is not None and recipe.high_precision_module_patterns and not self._hp_hits:
            raise ValueError("DeepSeek-V3 high_precision_module_patterns matched zero modules")
        c = self._counts
        return ModulePrecisionSummary(c["param"], c["capable"], c["compute"], c["persistent"], c["hp"])

    def deepseek_v3_recipe(self) -> Optional[DeepSeekV3PrecisionRecipe]:
        return self._config.deepseek_v3_recipe


def build_module_precision_resolver(config: PrecisionConfig) -> ModulePrecisionResolverImpl:
    return ModulePrecisionResolverImpl(config)


def finalize_module_precision_resolver(resolver) -> ModulePrecisionSummary:
    return resolver.finalize()


def refresh_persistent_lowbit_params(model: torch.nn.Module) -> int:
    """Call refresh_persistent_lowbit_params() on every module that has it."""
    count = 0
    for module in model.modules():
        fn = getattr(module, "refresh_persistent_lowbit_params", None)
        if callable(fn):
            fn()
            count += 1
    return count
