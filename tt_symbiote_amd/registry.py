"""Recipe registry (reference: models/auto/auto_mappings.py:26-105).

A recipe turns a loaded HF model into a ``{torch_class: hip_class}`` replacement dict
(``build_module_dict``), may patch the model after replacement (``post_register``), and may
allocate model-owned device state once a device is bound (``make_kv_cache``, called by
``set_device``). Recipes register under the HF model class name.
"""
from __future__ import annotations

import warnings
from typing import Any, Callable, Dict, Protocol, runtime_checkable

__all__ = ["Recipe", "TT_MODEL_REGISTRY", "register_recipe"]


@runtime_checkable
class Recipe(Protocol):
    def build_module_dict(self, model: Any) -> Dict[type, type]:  # pragma: no cover
        ...

    def post_register(self, model: Any) -> None:  # pragma: no cover
        ...


TT_MODEL_REGISTRY: Dict[str, Any] = {}


def register_recipe(hf_class_name: str) -> Callable[[type], type]:
    """Class decorator: instantiate the recipe and register it under ``hf_class_name``."""
    if not isinstance(hf_class_name, str) or not hf_class_name:
        raise ValueError(f"hf_class_name must name an HF model class, got {hf_class_name!r}")

    def decorator(cls):
        inst = cls()
        if not hasattr(inst, "build_module_dict"):
            raise TypeError(f"{cls.__name__} cannot be a recipe: it defines no "
                            "build_module_dict(model) returning the module replacements")
        if not hasattr(inst, "post_register"):
            inst.post_register = lambda model: None
        if not hasattr(inst, "make_kv_cache"):
            inst.make_kv_cache = lambda model, device, **kwargs: None
        if hf_class_name in TT_MODEL_REGISTRY:
            warnings.warn(f"{cls.__name__} replaces the recipe already registered for "
                          f"{hf_class_name!r}", stacklevel=2)
        TT_MODEL_REGISTRY[hf_class_name] = inst
        return cls

    return decorator
