"""``AutoModelForCausalLM`` (CPU): HF loading of a saved BailingMoeV2 checkpoint followed by the
recipe, as the reference's auto factory (models/auto/auto_factory.py:38-121)."""
import pytest
import torch

import tt_symbiote_amd as ts
from hf_bailing import tiny_hf_model


def test_from_pretrained_applies_the_recipe(tmp_path):
    saved = tiny_hf_model(seed=4)
    saved.save_pretrained(tmp_path)
    kv = {"block_size": 16, "max_num_blocks": 128, "batch_size": 2}
    model = ts.AutoModelForCausalLM.from_pretrained(str(tmp_path), kv_cache_kwargs=kv)
    assert type(model).__name__ == "BailingMoeV2ForCausalLM"
    assert isinstance(model.model, ts.HIPBailingMoeV2Model)
    assert isinstance(model.lm_head, ts.HIPLMHead)
    assert [type(layer).__name__ for layer in model.model.layers] == \
        ["HIPBailingMoEDecoderLayer"] * 3
    assert model.model.layers[0].is_dense_layer and not model.model.layers[1].is_dense_layer
    assert model._tt_kv_cache_kwargs == kv and model._tt_symbiote_has_recipe
    # the swapped modules hold the checkpoint's weights (not a fresh init)
    assert torch.equal(model.model._host["embed"], saved.model.word_embeddings.weight)
    assert torch.equal(model.lm_head._host["w"], saved.lm_head.weight)
    att = model.model.layers[2].attention
    assert torch.equal(att._host["qkv_w"],
                       saved.model.layers[2].attention.query_key_value.weight)


def test_from_config_without_a_recipe_returns_the_hf_model():
    from transformers.models.glm4_moe.configuration_glm4_moe import Glm4MoeConfig

    cfg = Glm4MoeConfig(vocab_size=50, hidden_size=32, intermediate_size=48,
                        num_hidden_layers=1, num_attention_heads=2, num_key_value_heads=1,
                        head_dim=16, moe_intermediate_size=8, n_routed_experts=4,
                        num_experts_per_tok=2, first_k_dense_replace=1)
    with pytest.warns(UserWarning, match="no registered recipe"):
        model = ts.AutoModelForCausalLM.from_config(cfg, kv_cache_kwargs={"block_size": 32})
    assert type(model).__name__ == "Glm4MoeForCausalLM"
    assert isinstance(model.model, torch.nn.Module)
    assert model._tt_kv_cache_kwargs == {"block_size": 32}
    assert not getattr(model, "_tt_symbiote_has_recipe", False)
