"""Class-keyed replacement of ``nn.Module`` children by HIP modules.

Same contract as the reference's ``register_modules`` (utils/module_replacement.py:148-167):
for every sub-module whose class is a key of ``old_class_to_new_class_dict`` the value's
``from_torch`` builds the replacement, which is spliced into the tree in place (children in
``_modules`` and modules held in public dict / list / tuple attributes). A swapped module is not
descended into -- its ``from_torch`` owns its subtree. ``exclude_replacement`` holds qualified
module names to leave alone. Returns ``{module_name: new module}`` for this call's swaps.
"""
from __future__ import annotations

from typing import Dict, Optional, Set

from torch import nn

from ..core.module import HIPModule


def _make(old, mapping, names, model_config, exclude):
    cls = mapping.get(old.__class__)
    if cls is None:
        return None
    name = names.get(old)
    if name is not None and name in exclude:
        return None
    new = cls.from_torch(old)
    if isinstance(new, HIPModule):
        if name is not None:
            new._unique_name = name
            new.override_children_module_names()
        new.set_model_config(model_config)
    return new


def _walk(obj, mapping, model_config, names, exclude, result):
    def swap_in_container(container, keys):
        for k in keys:
            v = container[k]
            if isinstance(v, nn.Module) and v.__class__ in mapping:
                new = _make(v, mapping, names, model_config, exclude)
                if new is not None:
                    container[k] = new
                    if isinstance(new, HIPModule):
                        result[new.module_name] = new
                    continue
            if isinstance(v, (nn.Module, HIPModule)):
                _walk(v, mapping, model_config, names, exclude, result)

    if isinstance(obj, nn.Module):
        swap_in_container(obj._modules, [k for k, v in obj._modules.items() if v is not None])
    if isinstance(obj, (nn.Module, HIPModule)):
        for attr in list(vars(obj)):
            if attr.startswith("_") or attr == "torch_layer":
                continue
            value = getattr(obj, attr, None)
            if isinstance(value, dict):
                swap_in_container(value, list(value))
            elif isinstance(value, list):
                swap_in_container(value, list(range(len(value))))
            elif isinstance(value, tuple):
                lst = list(value)
                swap_in_container(lst, list(range(len(lst))))
                if any(a is not b for a, b in zip(lst, value)):
                    setattr(obj, attr, type(value)(lst) if type(value) is tuple else tuple(lst))
            elif isinstance(obj, HIPModule) and isinstance(value, (nn.Module, HIPModule)):
                if isinstance(value, nn.Module) and value.__class__ in mapping:
                    new = _make(value, mapping, names, model_config, exclude)
                    if new is not None:
                        setattr(obj, attr, new)
                        if isinstance(new, HIPModule):
                            result[new.module_name] = new
                        continue
                _walk(value, mapping, model_config, names, exclude, result)


def register_modules(model, old_class_to_new_class_dict, model_config=None,
                     exclude_replacement: Optional[Set[str]] = None) -> Dict[str, HIPModule]:
    """Replace sub-modules of ``model`` whose class is a key of the mapping."""
    if exclude_replacement is None:
        exclude_replacement = set()
    if not isinstance(exclude_replacement, set) or not all(
            isinstance(k, str) for k in exclude_replacement):
        raise TypeError("exclude_replacement must be a set of module-name strings")
    names = {m: n for n, m in model.named_modules()} if isinstance(model, nn.Module) else {}
    result: Dict[str, HIPModule] = {}
    _walk(model, dict(old_class_to_new_class_dict), model_config, names, exclude_replacement,
          result)
    return result
