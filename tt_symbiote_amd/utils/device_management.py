"""``set_device(model, device)``: bind every HIP module of a model to one GPU.

Mirrors the reference's contract (utils/device_management.py:157-470): a strict two-argument
call that walks the model (``_modules`` children and public dict/list/tuple attributes), binds
each HIP module to the device, runs ``preprocess_weights`` / ``move_weights_to_device`` on each,
then asks the model's registered recipe for its KV cache (``make_kv_cache(model, device,
**model._tt_kv_cache_kwargs)``) and attaches it as ``model._tt_kv_cache``, and finally records
the swapped classes for ``compatibility.report``.

Differences, by design: the device is a torch device (``"cuda:0"``, ``torch.device`` or an
index) on an MI355X (gfx950); an unsupported device raises instead of silently swapping the
module back to its torch layer; weight-move failures raise instead of warning.
"""
from __future__ import annotations

from typing import Any

import torch
from torch import nn

from ..core.module import HIPModule
from . import compatibility

SUPPORTED_ARCHS = ("gfx950",)


def _resolve_device(device) -> torch.device:
    if isinstance(device, int):
        device = torch.device("cuda", device)
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(f"set_device: expected a GPU device, got {device}")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    return device


def device_arch(device: torch.device) -> str:
    props = torch.cuda.get_device_properties(device)
    return getattr(props, "gcnArchName", "").split(":")[0]


def check_device_supported(device: torch.device) -> None:
    if not torch.cuda.is_available():
        raise RuntimeError("set_device: no GPU is visible to this process")
    arch = device_arch(device)
    if arch not in SUPPORTED_ARCHS:
        raise RuntimeError(
            f"set_device: {device} is {arch or 'an unknown arch'}; the kernels are built for "
            f"{', '.join(SUPPORTED_ARCHS)} only")


def _hip_modules(obj, seen=None):
    """Yield every HIPModule reachable from ``obj`` (pre-order, each once)."""
    if seen is None:
        seen = set()
    if id(obj) in seen:
        return
    seen.add(id(obj))
    if isinstance(obj, HIPModule):
        yield obj
    if isinstance(obj, nn.Module):
        children = list(obj._modules.values())
    elif isinstance(obj, HIPModule):
        children = []
    else:
        return
    for attr in list(vars(obj)):
        if attr.startswith("_") or attr == "torch_layer":
            continue
        value = vars(obj)[attr]
        if isinstance(value, (nn.Module, HIPModule)):
            children.append(value)
        elif isinstance(value, dict):
            children.extend(v for v in value.values() if isinstance(v, (nn.Module, HIPModule)))
        elif isinstance(value, (list, tuple)):
            children.extend(v for v in value if isinstance(v, (nn.Module, HIPModule)))
    for child in children:
        if child is not None:
            yield from _hip_modules(child, seen)


def set_device(obj: Any, device) -> None:
    """Bind every HIP module in ``obj`` to ``device`` and prepare its device state."""
    dev = _resolve_device(device)
    check_device_supported(dev)
    compatibility.reset_swapped_registry()
    modules = list(_hip_modules(obj))
    for m in modules:
        m.to_device(dev)
    with torch.cuda.device(dev):
        for m in modules:
            m.preprocess_weights()
            m.move_weights_to_device()

    from ..registry import TT_MODEL_REGISTRY

    recipe = TT_MODEL_REGISTRY.get(type(obj).__name__)
    if recipe is not None and hasattr(recipe, "make_kv_cache"):
        kv_kwargs = getattr(obj, "_tt_kv_cache_kwargs", None) or {}
        kv = recipe.make_kv_cache(obj, dev, **kv_kwargs)
        if kv is not None:
            obj._tt_kv_cache = kv
    try:
        obj._tt_symbiote_device_set = True
    except Exception:
        pass
    for m in modules:
        layer = m._fallback_torch_layer
        if layer is not None:
            compatibility.record_swapped_class(m.module_name, type(layer).__name__)
