"""Host-side API contracts (CPU): recipe registry, module replacement, module base classes,
cache geometry and validation, run modes, coverage report, op argument checks."""
import inspect

import pytest
import torch
from torch import nn

import tt_symbiote_amd as ts
from oracle.bailing_moe_v2 import (BailingMoeV2Attention, BailingMoeV2Config,
                                   BailingMoeV2DecoderLayer, BailingMoeV2ForCausalLM,
                                   BailingMoeV2SparseMoeBlock)
from tt_symbiote_amd import hip_ops
from tt_symbiote_amd.core.module import StatefulHIPModule, StatelessHIPModule, HIPModule
from tt_symbiote_amd.registry import TT_MODEL_REGISTRY, register_recipe


def _tiny_model(layers=2):
    cfg = BailingMoeV2Config(hidden_size=256, num_attention_heads=2, num_key_value_heads=1,
                             head_dim=128, num_experts=64, num_experts_per_tok=4,
                             moe_intermediate_size=64, n_group=8, topk_group=4,
                             num_hidden_layers=layers, first_k_dense_replace=1,
                             intermediate_size=128, vocab_size=100)
    return BailingMoeV2ForCausalLM(cfg)


def test_recipe_registered_and_hooks():
    recipe = TT_MODEL_REGISTRY["BailingMoeV2ForCausalLM"]
    assert callable(recipe.build_module_dict)
    assert callable(recipe.post_register)
    sig = inspect.signature(recipe.make_kv_cache)
    assert "model" in sig.parameters and "device" in sig.parameters
    assert any(p.kind == p.VAR_KEYWORD for p in sig.parameters.values())


def test_build_module_dict_is_flat_class_map():
    model = _tiny_model()
    mapping = TT_MODEL_REGISTRY["BailingMoeV2ForCausalLM"].build_module_dict(model)
    assert isinstance(mapping, dict)
    assert mapping[BailingMoeV2DecoderLayer] is ts.HIPBailingMoEDecoderLayer
    assert mapping[BailingMoeV2Attention] is ts.HIPBailingMoEAttention
    assert mapping[BailingMoeV2SparseMoeBlock] is ts.HIPBailingMoE
    assert mapping[type(model.model)] is ts.HIPBailingMoeV2Model
    for k, v in mapping.items():
        assert isinstance(k, type) and isinstance(v, type)


def test_apply_recipe_swaps_layers_and_keeps_fallback():
    model = _tiny_model(layers=2)
    swapped = ts.apply_recipe(model, kv_cache_kwargs={"block_size": 32, "max_num_blocks": 8})
    # the trunk is swapped as a whole (its from_torch converts the layers); the lm_head by
    # post_register
    assert set(swapped) == {"model"}
    assert isinstance(model.model, ts.HIPBailingMoeV2Model)
    assert isinstance(model.lm_head, ts.HIPLMHead) and model.lm_head.vocab_size == 100
    assert type(model.model.torch_layer).__name__ == "BailingMoeV2Model"
    l0, l1 = model.model.layers[0], model.model.layers[1]
    assert isinstance(l0, ts.HIPBailingMoEDecoderLayer) and l0.is_dense_layer
    assert isinstance(l1.mlp, ts.HIPBailingMoE) and not l1.is_dense_layer
    assert isinstance(l1.attention, ts.HIPBailingMoEAttention)
    assert type(l1.torch_layer).__name__ == "BailingMoeV2DecoderLayer"
    assert l1.attention.module_name == "model.layers.1.attention"
    assert model._tt_kv_cache_kwargs == {"block_size": 32, "max_num_blocks": 8}
    names = [n for n, _ in model.named_modules()]
    assert "model.layers.1.mlp" in names


def test_register_modules_exclude_and_containers():
    model = _tiny_model(layers=2)
    mapping = {BailingMoeV2SparseMoeBlock: ts.HIPBailingMoE}
    swapped = ts.register_modules(model, mapping, exclude_replacement={"model.layers.1.mlp"})
    assert swapped == {}
    holder = nn.Module()
    holder.blocks = {"a": _tiny_model(2).model.layers[1].mlp}
    swapped = ts.register_modules(holder, mapping)
    assert isinstance(holder.blocks["a"], ts.HIPBailingMoE)
    with pytest.raises(TypeError):
        ts.register_modules(model, mapping, exclude_replacement=["x"])


def test_module_base_contracts():
    with pytest.raises(TypeError):
        class Direct(HIPModule):  # noqa: F841
            pass
    with pytest.raises(TypeError):
        class NoReset(StatefulHIPModule):  # noqa: F841
            def forward(self):
                return 0

    class Ok(StatelessHIPModule):
        def forward(self, x):
            return x + 1

    m = Ok()
    with pytest.raises(RuntimeError, match="device is not set"):
        m(1)


def test_run_mode_selection(monkeypatch):
    from tt_symbiote_amd.core.run_config import get_run_implementation, NormalRun

    monkeypatch.delenv("SYMBIOTE_RUN_MODE", raising=False)
    monkeypatch.delenv("TT_SYMBIOTE_RUN_MODE", raising=False)
    assert get_run_implementation() is NormalRun
    monkeypatch.setenv("TT_SYMBIOTE_RUN_MODE", "CPU")
    with pytest.raises(ValueError):
        get_run_implementation()


def test_duplicate_recipe_warns():
    with pytest.warns(UserWarning):
        @register_recipe(hf_class_name="BailingMoeV2ForCausalLM")
        class Dup:
            def build_module_dict(self, model):
                return {}
    # restore the real recipe
    from tt_symbiote_amd import recipe_bailing_moe_v2 as r
    TT_MODEL_REGISTRY["BailingMoeV2ForCausalLM"] = r.BailingMoEV2Recipe()


def test_paged_config_geometry():
    cfg = ts.PagedAttentionConfig(block_size=32, max_num_blocks=128, batch_size=4)
    assert cfg.max_seq_length == 4096
    assert cfg.blocks_per_sequence == 32
    cache = ts.HIPPagedAttentionKVCache(2, 4, 128, cfg)
    assert cache.page_table.shape == (4, 32)
    assert torch.equal(cache.page_table.flatten(), torch.arange(128, dtype=torch.int32))
    assert cache.get_seq_length(0) == 0
    with pytest.raises(RuntimeError, match="not on device"):
        cache.set_vllm_page_table(torch.zeros(4, 32, dtype=torch.int32))
    cache.update_seq_length(0, 5)
    cache.update_seq_length(0, 1)
    assert cache.get_seq_length(0) == 6 and cache._seen_tokens == 6
    cache.reset()
    assert cache.get_seq_length(0) == 0
    with pytest.raises(NotImplementedError):
        ts.HIPPagedAttentionKVCache(1, 4, 64, cfg)


def test_coverage_report_shape():
    model = _tiny_model(1)
    rep = ts.compatibility.report(model)
    assert set(rep) >= {"model_class", "modules_swapped", "runtime_observed", "regressions",
                        "summary"}


def test_ops_reject_cpu_tensors():
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        hip_ops.rmsnorm(x, torch.ones(64, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(ValueError, match="GPU tensor"):
        hip_ops.moe_route_permute(torch.zeros(2, 64), torch.zeros(64), n_group=8, topk_group=4,
                                  top_k=4, routed_scale=1.0)


def test_router_weight_splits_exactly_into_three_bf16_planes():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(256, 2048, generator=g) * 0.02
    w[0, :8] = torch.tensor([1.0, -3.75, 1e-3, 123.456, -1e-6, 0.0, 2.0 ** -60, 7.1e4])
    planes = hip_ops.split_router_weight(w)
    assert planes.shape == (3, 256, 2048) and planes.dtype == torch.bfloat16
    back = (planes[0].float() + planes[1].float()) + planes[2].float()
    assert torch.equal(back, w)
    # the planes are the mantissa bytes from the top: |hi| >= 128|mid| >= 128^2|lo| per value
    hi, mid, lo = (p.float().abs() for p in planes)
    assert bool((hi >= 128 * mid).all()) and bool((mid >= 128 * lo).all())
    # a weight with a single significant byte is all hi
    assert torch.equal(hip_ops.split_router_weight(torch.full((2, 64), 0.5))[1:].float(),
                       torch.zeros(2, 2, 64))
