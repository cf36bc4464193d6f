"""An HF-loadable ``BailingMoeV2ForCausalLM`` for the tests (test infrastructure).

The real class is Hub remote code (``inclusionAI/Ling-mini-2.0``, trust_remote_code), absent
offline. This wraps the oracle's modules (same attribute names as the remote code) in
transformers' ``PreTrainedModel`` / ``GenerationMixin`` and registers them with the Auto classes
under ``model_type = "bailing_moe_v2"``, so ``save_pretrained`` / ``from_pretrained`` and HF
``generate`` run as they would on the real checkpoint. The forward mirrors the remote code's
``BailingMoeV2ForCausalLM.forward``: trunk, then ``lm_head`` on the last hidden state.
"""
from __future__ import annotations

import torch
from torch import nn
from transformers import (AutoConfig, AutoModelForCausalLM, GenerationMixin, PretrainedConfig,
                          PreTrainedModel)
from transformers.modeling_outputs import CausalLMOutputWithPast

from oracle.bailing_moe_v2 import BailingMoeV2Config, BailingMoeV2Model, init_weights_


class BailingMoeV2HFConfig(PretrainedConfig):
    model_type = "bailing_moe_v2"

    def __init__(self, **kwargs):
        fields = vars(BailingMoeV2Config())
        for key, default in fields.items():
            setattr(self, key, kwargs.pop(key, default))
        kwargs.setdefault("tie_word_embeddings", False)
        super().__init__(**kwargs)


class BailingMoeV2ForCausalLM(PreTrainedModel, GenerationMixin):
    config_class = BailingMoeV2HFConfig
    base_model_prefix = "model"

    def __init__(self, config: BailingMoeV2HFConfig):
        super().__init__(config)
        self.model = BailingMoeV2Model(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self.post_init()

    def _init_weights(self, module):
        return None  # weights come from init_weights_ (seeded) or the checkpoint

    @property
    def device(self) -> torch.device:
        # after the recipe the trunk is a HIP module (no nn.Parameters left to ask)
        trunk = self._modules.get("model")
        dev = getattr(trunk, "device", None)
        if isinstance(dev, torch.device):
            return dev
        return super().device

    def forward(self, input_ids=None, attention_mask=None, position_ids=None,
                past_key_values=None, cache_position=None, use_cache=None, logits_to_keep=0,
                **kwargs):
        out = self.model(input_ids=input_ids, position_ids=position_ids,
                         past_key_values=past_key_values, cache_position=cache_position)
        h = getattr(out, "last_hidden_state", None)
        if h is None:
            h = out[0] if isinstance(out, tuple) else out
        if logits_to_keep:
            h = h[:, -logits_to_keep:]
        logits = self.lm_head(h).float()
        return CausalLMOutputWithPast(logits=logits, past_key_values=past_key_values)


AutoConfig.register("bailing_moe_v2", BailingMoeV2HFConfig, exist_ok=True)
AutoModelForCausalLM.register(BailingMoeV2HFConfig, BailingMoeV2ForCausalLM, exist_ok=True)


def tiny_hf_model(seed: int = 0, **overrides) -> BailingMoeV2ForCausalLM:
    """A 3-layer model (dense layer 0, MoE layers 1-2) with Ling's attention geometry per head,
    bf16-representable weights and an lm_head scaled x8 (greedy choices away from near ties)."""
    kw = dict(hidden_size=512, num_attention_heads=4, num_key_value_heads=2, head_dim=128,
              num_experts=64, num_experts_per_tok=4, moe_intermediate_size=128, n_group=8,
              topk_group=4, num_hidden_layers=3, first_k_dense_replace=1, intermediate_size=384,
              vocab_size=1000, partial_rotary_factor=0.5, rope_theta=1e6,
              max_position_embeddings=4096)
    kw.update(overrides)
    model = BailingMoeV2ForCausalLM(BailingMoeV2HFConfig(**kw)).eval()
    init_weights_(model, torch.Generator().manual_seed(seed))
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(p.bfloat16().float())
        model.lm_head.weight.mul_(8.0)
    return model
