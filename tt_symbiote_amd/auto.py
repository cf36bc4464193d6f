"""``AutoModelForCausalLM``: HF loading followed by the registered recipe.

Reference: ``_BaseAutoModelClass.from_pretrained`` (models/auto/auto_factory.py:38-121) and the
user path of examples/e2e/run_ling_mini_2_0.py:57-86:

    model = tt_symbiote_amd.AutoModelForCausalLM.from_pretrained(
        path, trust_remote_code=True, kv_cache_kwargs={"max_num_blocks": 512})
    tt_symbiote_amd.set_device(model, "cuda:0")          # binds and allocates model._tt_kv_cache
    out = model.generate(**inputs, max_new_tokens=64, past_key_values=model._tt_kv_cache)

``kv_cache_kwargs`` is popped before the call reaches transformers and kept on the model as
``_tt_kv_cache_kwargs`` for the recipe's ``make_kv_cache`` (``set_device`` reads it). When no
recipe is registered for the loaded class, the HF model is returned unchanged with a warning.
"""
from __future__ import annotations

import warnings
from typing import Any

from .registry import TT_MODEL_REGISTRY
from .utils.module_replacement import register_modules

__all__ = ["AutoModelForCausalLM"]


class AutoModelForCausalLM:
    """Thin wrapper over ``transformers.AutoModelForCausalLM`` that applies the recipe."""

    @staticmethod
    def _hf_auto_class():
        from transformers import AutoModelForCausalLM as HFAuto

        return HFAuto

    @classmethod
    def _finish(cls, model: Any, kv_cache_kwargs) -> Any:
        model._tt_kv_cache_kwargs = dict(kv_cache_kwargs) if kv_cache_kwargs else {}
        name = type(model).__name__
        recipe = TT_MODEL_REGISTRY.get(name)
        if recipe is None:
            warnings.warn(f"{name} has no registered recipe: the HF model is returned unchanged "
                          "and set_device will bind no HIP module", stacklevel=3)
            return model
        register_modules(model, recipe.build_module_dict(model))
        recipe.post_register(model)
        model._tt_symbiote_has_recipe = True
        return model

    @classmethod
    def from_pretrained(cls, pretrained_name_or_path: Any, *args: Any, **kwargs: Any) -> Any:
        kv_cache_kwargs = kwargs.pop("kv_cache_kwargs", None)
        model = cls._hf_auto_class().from_pretrained(pretrained_name_or_path, *args, **kwargs)
        return cls._finish(model, kv_cache_kwargs)

    @classmethod
    def from_config(cls, config: Any, *args: Any, **kwargs: Any) -> Any:
        """As :meth:`from_pretrained`, for a randomly initialised model of ``config``."""
        kv_cache_kwargs = kwargs.pop("kv_cache_kwargs", None)
        model = cls._hf_auto_class().from_config(config, *args, **kwargs)
        return cls._finish(model, kv_cache_kwargs)
