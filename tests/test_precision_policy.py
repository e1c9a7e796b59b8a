"""CPU tests of the flag surface, recipe propagation and per-module resolution,
mirroring nano-train's tests/test_fp8_granularity_semantics.py:76-98,
test_deepseek_v3_precision_recipe.py, test_module_precision_policy_resolution.py,
test_lowbit_linear_backends.py:123-159, test_persistent_lowbit_checkpoint_compat.py
and test_master_store_binding.py.  Nothing here launches a kernel."""

from __future__ import annotations

import argparse

import pytest
import torch

from _args import precision_args


def _resolver(**kw):
    from lowbit.precision import build_module_precision_resolver, resolve_precision_config

    config = resolve_precision_config(precision_args(**kw), torch.device("cpu"))
    return config, build_module_precision_resolver(config)


def _linear(resolver, path="decoder.blocks.0.mlp.fc1", i=257, o=129, bias=True):
    from lowbit.layers import Linear

    return Linear(i, o, bias, param_dtype=torch.float32, param_device=None, module_path=path,
                  precision_resolver=resolver)


def test_flags_accept_hip_and_keep_reference_defaults():
    ns = precision_args()
    assert ns.fp8_backend == "transformer_engine" and ns.fp4_backend == "emulated"
    assert ns.precision_recipe == "default" and ns.lowbit_master_ownership == "optimizer"
    assert ns.lowbit_code_format == "int_grid" and ns.lowbit_backward == "ste"
    from lowbit.precision import add_mixed_precision_args

    p = argparse.ArgumentParser()
    add_mixed_precision_args(p)
    assert p.parse_args(["--fp8", "--fp8-backend", "hip"]).fp8_backend == "hip"
    with pytest.raises(SystemExit):
        p.parse_args(["--fp8-backend", "bogus"])


def test_invalid_backend_message_names_the_flag():
    from lowbit.precision import resolve_precision_config

    with pytest.raises(ValueError, match="fp8-backend"):
        resolve_precision_config(precision_args(fp8=True, fp8_backend="bogus"), torch.device("cpu"))
    # the reference's own backends are not part of this package
    with pytest.raises(ValueError, match="fp8-backend"):
        resolve_precision_config(precision_args(fp8=True, fp8_backend="emulated"), torch.device("cpu"))


def test_deepseek_recipe_propagates_tile_block_stochastic_to_backend():
    _, res = _resolver(precision_recipe="deepseek_v3", fp8=True, fp8_backend="hip")
    layer = _linear(res)
    backend = layer._module_precision_state.lowbit_backend
    assert backend is not None and backend.name == "hip"
    assert backend._activation_granularity == "tile_1x128"
    assert backend._weight_granularity == "block_128x128"
    assert backend._rounding_mode == "stochastic"


def test_recipe_overrides_propagate_to_backend():
    _, res = _resolver(precision_recipe="deepseek_v3", fp8=True, fp8_backend="hip",
                       fp8_activation_granularity="tensor", fp8_weight_granularity="channel",
                       fp8_rounding="nearest")
    b = _linear(res)._module_precision_state.lowbit_backend
    assert (b._activation_granularity, b._weight_granularity, b._rounding_mode) == ("tensor", "channel", "nearest")


def test_default_fp8_is_per_tensor_nearest():
    _, res = _resolver(fp8=True, fp8_backend="hip")
    b = _linear(res)._module_precision_state.lowbit_backend
    assert (b._activation_granularity, b._weight_granularity, b._rounding_mode) == ("tensor", "tensor", "nearest")
    assert b.bits == 8 and b.code_format == "int_grid"


def test_fp4_mode_uses_qmax_7_and_code_format_flag():
    _, res = _resolver(fp4=True, fp4_backend="hip")
    assert _linear(res)._module_precision_state.lowbit_backend.bits == 4
    _, res = _resolver(fp8=True, fp8_backend="hip", lowbit_code_format="e4m3", lowbit_backward="fp8")
    b = _linear(res)._module_precision_state.lowbit_backend
    assert b.code_format == "e4m3" and b.backward_recipe == "fp8"


def test_comm_quant_recipe_defaults_and_overrides():
    """test_moe_fp8_comm_quant.py:79-88: the deepseek_v3 recipe enables the MoE
    payload quantization at block_128x128 with stochastic rounding, and
    --fp8-comm-quant False turns it off; --fp8-comm-granularity replaces the
    granularity (mixed_precision.py recipe overrides)."""
    config, _ = _resolver(precision_recipe="deepseek_v3", fp8_backend="hip")
    r = config.deepseek_v3_recipe
    assert r.comm_quant_enabled is True
    assert r.comm_quant_granularity == "block_128x128"
    assert r.rounding_mode == "stochastic"
    config, _ = _resolver(precision_recipe="deepseek_v3", fp8_backend="hip", fp8_comm_quant=False)
    assert config.deepseek_v3_recipe.comm_quant_enabled is False
    config, _ = _resolver(precision_recipe="deepseek_v3", fp8_backend="hip", fp8_comm_granularity="tensor")
    assert config.deepseek_v3_recipe.comm_quant_granularity == "tensor"
    with pytest.raises(ValueError):
        _resolver(precision_recipe="deepseek_v3", fp8_backend="hip", fp8_comm_granularity="rows")


def test_recipe_requires_fp8_and_high_precision_exceptions():
    from lowbit.precision import resolve_precision_config

    with pytest.raises(ValueError, match="deepseek_v3 requires --fp8"):
        resolve_precision_config(precision_args(precision_recipe="deepseek_v3", bf16=True), torch.device("cpu"))
    config, res = _resolver(precision_recipe="deepseek_v3", fp8_backend="hip")
    assert config.mode == "fp8" and config.deepseek_v3_recipe.comm_quant_enabled
    router = _linear(res, path="decoder.blocks.0.mlp.router")
    assert router._module_precision_state.lowbit_backend is None
    assert router.module_precision_assignment.compute_lowbit_mode is None


def test_include_exclude_and_finalize_errors():
    from lowbit.precision import finalize_module_precision_resolver

    _, res = _resolver(fp8=True, fp8_backend="hip", compute_lowbit_include=[r"mlp"],
                       compute_lowbit_exclude=[r"fc2$"])
    a = _linear(res, path="blk.mlp.fc1")
    b = _linear(res, path="blk.mlp.fc2")
    c = _linear(res, path="blk.attn.qkv")
    assert a._module_precision_state.lowbit_backend is not None
    assert b._module_precision_state.lowbit_backend is None
    assert c._module_precision_state.lowbit_backend is None
    summary = finalize_module_precision_resolver(res)
    assert summary.compute_lowbit_module_count == 1 and summary.parameterized_module_count == 3
    with pytest.raises(ValueError, match="Duplicate module_path"):
        _linear(res, path="blk.mlp.fc1")
    _, res2 = _resolver(fp8=True, fp8_backend="hip", compute_lowbit_include=["nomatch"])
    _linear(res2, path="x.fc")
    with pytest.raises(ValueError, match="matched zero modules"):
        finalize_module_precision_resolver(res2)


def test_compute_dtype_rule_conflicts_with_lowbit():
    with pytest.raises(ValueError, match="both low-bit compute and compute-dtype override"):
        _, res = _resolver(fp8=True, fp8_backend="hip", module_compute_dtype_rule=["fc1=bf16"])
        _linear(res, path="blk.fc1")


def test_unassigned_modules_bypass_the_backend_on_cpu():
    _, res = _resolver(bf16=False)
    layer = _linear(res, path="m.fc", i=8, o=4)
    assert layer._module_precision_state.lowbit_backend is None
    x = torch.randn(3, 8)
    torch.testing.assert_close(layer(x), torch.nn.functional.linear(x, layer.weight, layer.bias))


def test_hip_backend_has_no_cpu_path():
    _, res = _resolver(fp8=True, fp8_backend="hip")
    layer = _linear(res, i=128, o=128)
    with pytest.raises(RuntimeError, match="ROCm device"):
        layer(torch.randn(2, 128))


def test_persistent_buffers_and_legacy_checkpoint_load():
    _, res = _resolver(fp8=True, fp8_backend="hip", fp4_param=True)
    layer = _linear(res, i=64, o=32)
    sd = layer.state_dict()
    for k in ("_persistent_fp8_weight", "_persistent_fp4_codes", "_persistent_scale", "_persistent_numel"):
        assert k in sd
    assert sd["_persistent_fp4_codes"].dtype == torch.uint8 and sd["_persistent_numel"].dtype == torch.int64
    legacy = {"weight": torch.randn(32, 64), "bias": torch.zeros(32)}
    _, res2 = _resolver(fp8=True, fp8_backend="hip", fp4_param=True)
    fresh = _linear(res2, i=64, o=32)
    missing, unexpected = fresh.load_state_dict(legacy, strict=True), None
    assert torch.equal(fresh.weight, legacy["weight"])


def test_master_store_binding():
    from lowbit.master_store import get_lowbit_master_store, materialize_optimizer_owned_masters

    config, res = _resolver(fp8=True, fp8_backend="hip", fp8_param=True)
    model = torch.nn.Sequential()
    model.add_module("fc", _linear(res, path="blocks.0.experts.3.up", i=16, o=8))
    before = model.fc.weight.detach().clone()
    store = materialize_optimizer_owned_masters(model, precision_config=config)
    assert store is not None and get_lowbit_master_store(model) is store
    key = "blocks__0__experts__3__up__weight"
    assert model.fc.weight is store.masters[key]
    assert torch.equal(model.fc.weight.detach(), before)
    assert store.metadata[key].shard_domain == "expert_model_parallel"
    config2, res2 = _resolver(fp8=True, fp8_backend="hip", fp8_param=True, lowbit_master_ownership="module")
    assert materialize_optimizer_owned_masters(torch.nn.Sequential(), precision_config=config2) is None


def test_tensor_parallel_layers_need_one_shard():
    from lowbit.layers import ColumnParallelLinear, RowParallelLinear

    _, res = _resolver(fp8=True, fp8_backend="hip")
    col = ColumnParallelLinear(32, 16, 0, 1, param_dtype=torch.float32, param_device=None, module_path="c",
                               precision_resolver=res)
    row = RowParallelLinear(16, 32, 0, 1, param_dtype=torch.float32, param_device=None, module_path="r",
                            precision_resolver=res)
    assert col._module_precision_state.lowbit_backend is not None
    assert row._module_precision_state.assignment.module_type == "RowParallelLinear"
    with pytest.raises(NotImplementedError, match="tp_size == 1"):
        ColumnParallelLinear(32, 16, 0, 2, param_dtype=torch.float32, param_device=None, module_path="c2",
                             precision_resolver=res)
