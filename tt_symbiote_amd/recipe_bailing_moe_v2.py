"""Module-replacement recipe for ``BailingMoeV2ForCausalLM`` (Ling-mini-2.0).

Reference: ``BailingMoEV2Recipe`` (modeling_bailing_moe_v2.py:708-736), registered under the
same HF class name. ``build_module_dict`` returns one flat ``{torch_class: hip_class}`` dict
covering the classes of the hot path found in the loaded model: the decoder layer (whose
``from_torch`` converts its attention and MoE children), and -- for models or sub-trees used
without the layer wrapper -- the attention and sparse-MoE classes themselves. The HF classes
are remote code, so they are matched by class name on the model instance.
``make_kv_cache(model, device, batch_size=1, **kwargs)`` allocates the paged cache
(``block_size`` default 64, ``max_num_blocks`` default 32, as the reference).

As the reference's ``{type(model.model): TTNNBailingMoeV2Model, ...}`` (modeling_bailing_moe_v2.py
:715-719), the HF trunk (``BailingMoeV2Model``) is swapped for :class:`HIPBailingMoeV2Model`
(embedding, decoder layers, final norm), and ``post_register`` swaps ``model.lm_head`` for
:class:`HIPLMHead` (the reference maps ``nn.Linear`` to a TTNN linear), so
:func:`tt_symbiote_amd.generate.greedy_generate` runs the whole model on the device.
"""
from __future__ import annotations

from .modules.attention import HIPBailingMoEAttention
from .modules.decoder_layer import HIPBailingMoEDecoderLayer
from .modules.kv_cache import HIPPagedAttentionKVCache, PagedAttentionConfig
from .modules.model import HIPBailingMoeV2Model, HIPLMHead
from .modules.moe import HIPBailingMoE
from .registry import register_recipe

_LAYER_CLASSES = {"BailingMoeV2DecoderLayer"}
_ATTENTION_CLASSES = {"BailingMoeV2Attention", "BailingMoeV2SdpaAttention",
                      "BailingMoeV2FlashAttention2"}
_MOE_CLASSES = {"BailingMoeV2SparseMoeBlock"}
_MODEL_CLASSES = {"BailingMoeV2Model"}


@register_recipe(hf_class_name="BailingMoeV2ForCausalLM")
class BailingMoEV2Recipe:
    # design-time coverage lists (modeling_bailing_moe_v2.py:656-705), for this hot path
    tt_implemented = ["BailingMoeV2Model", "BailingMoeV2DecoderLayer",
                      "BailingMoeV2SdpaAttention", "BailingMoeV2Attention",
                      "BailingMoeV2SparseMoeBlock", "BailingMoeV2Gate", "BailingMoeV2MLP",
                      "BailingMoeV2RMSNorm", "Linear"]
    cpu_fallback: list = []
    host_glue = ["BailingMoeV2PreTrainedModel", "BailingMoeV2ForCausalLM",
                 "BailingMoeV2RotaryEmbedding"]
    out_of_scope = ["BailingMoeV2FlashAttention2", "BailingMoeV2MTPLayer"]

    def build_module_dict(self, model):
        mapping = {}
        modules = model.modules() if hasattr(model, "modules") else []
        for m in modules:
            name = type(m).__name__
            if name in _MODEL_CLASSES:
                mapping[type(m)] = HIPBailingMoeV2Model
            elif name in _LAYER_CLASSES:
                mapping[type(m)] = HIPBailingMoEDecoderLayer
            elif name in _ATTENTION_CLASSES:
                mapping[type(m)] = HIPBailingMoEAttention
            elif name in _MOE_CLASSES:
                mapping[type(m)] = HIPBailingMoE
        return mapping

    def post_register(self, model):
        children = getattr(model, "_modules", {})
        head = children.get("lm_head")
        if head is not None and type(head).__name__ == "Linear":
            new = HIPLMHead.from_torch(head)
            new._unique_name = "lm_head"
            children["lm_head"] = new      # spliced in as register_modules does
        return None

    def make_kv_cache(self, model, device, batch_size: int = 1, **kwargs):
        """The paged cache (reference: modeling_bailing_moe_v2.py:724-736). ``dtype``
        (``torch.bfloat16`` by default, or ``torch.float8_e4m3fn`` for the fp8 cache) is this
        build's addition."""
        import torch

        config = PagedAttentionConfig(
            block_size=kwargs.get("block_size", 64),
            max_num_blocks=kwargs.get("max_num_blocks", 32),
            batch_size=batch_size)
        cfg = model.config
        head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        return HIPPagedAttentionKVCache(
            num_layers=cfg.num_hidden_layers, num_kv_heads=cfg.num_key_value_heads,
            head_dim=head_dim, config=config, device=None,
            dtype=kwargs.get("dtype", torch.bfloat16)).to_device(device)
