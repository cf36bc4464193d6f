"""MI355X-native BailingMoeV2 (Ling-mini-2.0) decode hot path behind the tt_symbiote
module-replacement API.

    import tt_symbiote_amd as ts
    model = ts.AutoModelForCausalLM.from_pretrained(path, trust_remote_code=True,
                                                    kv_cache_kwargs={"max_num_blocks": 512})
    # (or ts.apply_recipe(model) on an already-loaded HF model)
    ts.set_device(model, "cuda:0")      # bind to the GPU, move weights, allocate the paged cache
    out = model.generate(input_ids, max_new_tokens=64, past_key_values=model._tt_kv_cache)

The compute runs in hand-written gfx950 HIP kernels behind a C ABI
(``include/symbiote_mi355x.h``, ``lib/libsymbiote_mi355x.so``); importing this package does
not touch the GPU or load the library.
"""
from . import recipe_bailing_moe_v2  # noqa: F401  -- registers the recipe
from .auto import AutoModelForCausalLM
from .core.module import (HIPModule, StatefulHIPModule, StatefulTTNNModule, StatelessHIPModule,
                          StatelessTTNNModule, TTNNModule)
from .modules import (HIPBailingMoE, HIPBailingMoEAttention, HIPBailingMoEDecoderLayer,
                      HIPBailingMoeV2MLP, HIPBailingMoeV2Model, HIPLMHead,
                      HIPPagedAttentionKVCache, PagedAttentionConfig)
from .registry import TT_MODEL_REGISTRY, register_recipe
from .utils import compatibility
from .utils.device_management import set_device
from .utils.module_replacement import register_modules


def apply_recipe(model, kv_cache_kwargs=None, exclude_replacement=None):
    """Swap the hot-path modules of an already-loaded HF model using its registered recipe
    (the replacement steps of the reference's ``from_pretrained``, auto_factory.py:105-121).
    Returns ``{module_name: hip module}``."""
    recipe = TT_MODEL_REGISTRY.get(type(model).__name__)
    if recipe is None:
        raise KeyError(f"no recipe registered for {type(model).__name__}")
    swapped = register_modules(model, recipe.build_module_dict(model),
                               exclude_replacement=exclude_replacement)
    recipe.post_register(model)
    model._tt_kv_cache_kwargs = dict(kv_cache_kwargs or {})
    return swapped


__all__ = ["AutoModelForCausalLM", "apply_recipe", "set_device", "register_modules", "register_recipe",
           "TT_MODEL_REGISTRY", "compatibility", "HIPModule", "StatelessHIPModule",
           "StatefulHIPModule", "TTNNModule", "StatelessTTNNModule", "StatefulTTNNModule",
           "HIPBailingMoE", "HIPBailingMoEAttention", "HIPBailingMoEDecoderLayer",
           "HIPBailingMoeV2MLP", "HIPBailingMoeV2Model", "HIPLMHead",
           "HIPPagedAttentionKVCache", "PagedAttentionConfig"]
