"""Module base classes of the HIP-backed replacements.

Mirrors the lifecycle of the reference's ``TTNNModule`` (core/module.py:62-324):
``from_torch`` keeps the HF layer as ``_fallback_torch_layer``; ``preprocess_weights`` (host,
once) and ``move_weights_to_device`` (once, after ``to_device``) recurse into child modules;
``__call__`` dispatches through the run mode's ``module_run``; modules are plain Python objects
spliced into the HF ``nn.Module`` tree by :func:`tt_symbiote_amd.register_modules`.

As in the reference, a module class must declare its trace-state contract by extending
:class:`StatelessHIPModule` or :class:`StatefulHIPModule` (core/module.py:327-372); a stateful
module (one whose forward mutates persistent state such as the paged KV cache) must implement
``reset_trace_state``. Here the "trace" is a HIP graph capture of the decode step.
"""
from __future__ import annotations

from typing import Optional

import torch


def _set_names_recursively(module, prefix: str) -> None:
    for name, child in module.named_children():
        full = f"{prefix}.{name}" if prefix else name
        if isinstance(child, HIPModule):
            child._unique_name = full
            child.override_children_module_names()
        elif isinstance(child, torch.nn.Module):
            for sub_name, sub in child.named_modules(prefix=full):
                if isinstance(sub, HIPModule):
                    sub._unique_name = sub_name


class HIPModule:
    """Base class of the HIP-backed modules. Not directly subclassable (see module docstring)."""

    def __init_subclass__(cls, **kwargs):
        super().__init_subclass__(**kwargs)
        if HIPModule in cls.__bases__ and not cls.__dict__.get("_allow_direct_subclass", False):
            raise TypeError(
                f"{cls.__qualname__}: pick a graph-capture contract by deriving from "
                "StatelessHIPModule (the forward leaves no state behind) or StatefulHIPModule "
                "(the forward writes persistent state, e.g. KV slots, and must define "
                "reset_trace_state), not from HIPModule itself")

    def __init__(self):
        self._device: Optional[torch.device] = None
        self._preprocessed_weight = False
        self._weights_on_device = False
        self._fallback_torch_layer = None
        self._unique_name: Optional[str] = None
        self._model_config = {}
        self.training = False

    # ---- dispatch ----
    def call(self, *args, **kwargs):
        from .run_config import get_run_implementation

        return get_run_implementation().module_run(self, *args, **kwargs)

    def __call__(self, *args, **kwargs):
        return self.call(*args, **kwargs)

    def forward(self, *args, **kwargs):
        raise NotImplementedError("forward must be implemented by subclasses")

    # ---- weights ----
    def preprocess_weights(self):
        if self._preprocessed_weight:
            return
        self._preprocessed_weight = True
        self.preprocess_weights_impl()

    def move_weights_to_device(self):
        if not self._preprocessed_weight:
            raise RuntimeError(f"{self.module_name}: preprocess_weights() must run first")
        if self.device is None:
            raise RuntimeError(f"{self.module_name}: device not set; call set_device(model, device)")
        if self._weights_on_device:
            return
        self._weights_on_device = True
        self.move_weights_to_device_impl()

    def deallocate_weights(self):
        self.deallocate_weights_impl()
        self._weights_on_device = False

    def preprocess_weights_impl(self):
        for child in self.__dict__.values():
            if isinstance(child, HIPModule):
                child.preprocess_weights()
        return self

    def move_weights_to_device_impl(self):
        for child in self.__dict__.values():
            if isinstance(child, HIPModule):
                if child.device is None:
                    child.to_device(self.device)
                child.move_weights_to_device()
        return self

    def deallocate_weights_impl(self):
        for child in self.__dict__.values():
            if isinstance(child, HIPModule):
                child.deallocate_weights()
        return self

    # ---- device / config ----
    def to_device(self, device):
        self._device = torch.device(device) if device is not None else None
        return self

    @property
    def device(self) -> Optional[torch.device]:
        return self._device

    def set_model_config(self, model_config):
        self._model_config = model_config if model_config is not None else {}

    @property
    def model_config(self):
        return self._model_config

    @classmethod
    def from_torch(cls, torch_layer, *args, **kwargs):
        new = cls(*args, **kwargs)
        new._fallback_torch_layer = torch_layer
        return new

    @property
    def torch_layer(self):
        return self._fallback_torch_layer

    def train(self, mode: bool = True):
        self.training = mode
        if self._fallback_torch_layer is not None:
            self._fallback_torch_layer.train(mode)
        return self

    def eval(self):
        return self.train(False)

    # ---- naming / traversal (nn.Module-compatible subset) ----
    @property
    def module_name(self) -> str:
        if self._unique_name is None:
            self._unique_name = f"{self.__class__.__name__}_{id(self)}"
        return self._unique_name

    def override_children_module_names(self):
        _set_names_recursively(self, self.module_name)

    def named_children(self):
        for name, child in self.__dict__.items():
            if name in ("_fallback_torch_layer", "torch_layer"):
                continue
            if isinstance(child, (torch.nn.Module, HIPModule)):
                yield name, child
            elif isinstance(child, dict):
                for k, v in child.items():
                    if isinstance(v, (torch.nn.Module, HIPModule)):
                        yield f"{name}[{k}]", v
            elif isinstance(child, (list, tuple)):
                # list members are named like nn.ModuleList children: "layers.0", "layers.1", ...
                for i, v in enumerate(child):
                    if isinstance(v, (torch.nn.Module, HIPModule)):
                        yield f"{name}.{i}", v

    def children(self):
        for _, c in self.named_children():
            yield c

    def named_modules(self, memo=None, prefix="", remove_duplicate=True):
        if memo is None:
            memo = set()
        if remove_duplicate:
            if self in memo:
                return
            memo.add(self)
        yield prefix, self
        for name, child in self.named_children():
            child_prefix = prefix + ("." if prefix else "") + name
            yield from child.named_modules(memo, child_prefix, remove_duplicate)

    def modules(self):
        for _, m in self.named_modules():
            yield m

    def parameters(self, recurse: bool = True):
        return iter(())

    def _apply(self, fn, recurse=True):
        return self

    def __repr__(self):
        lines = []
        for key, value in self.named_children():
            mod = repr(value).replace("\n", "\n  ")
            lines.append(f"({key}): {mod}")
        s = f"{self.__class__.__name__}(module_name={self.module_name}"
        if lines:
            s += "\n  " + "\n  ".join(lines) + "\n"
        return s + ")"

    # ---- graph-capture hooks ----
    def reset_trace_state(self):
        """Called before a forward that will be captured; restores per-call state."""


class StatelessHIPModule(HIPModule):
    """Forward mutates no persistent state; reset_trace_state is a no-op."""

    _allow_direct_subclass = True

    def reset_trace_state(self):
        return None


class StatefulHIPModule(HIPModule):
    """Forward mutates persistent state (e.g. writes the paged KV cache); subclasses must
    implement their own reset_trace_state (checked at class creation)."""

    _allow_direct_subclass = True

    def __init_subclass__(cls, **kwargs):
        super().__init_subclass__(**kwargs)
        for klass in cls.__mro__:
            if klass is StatefulHIPModule:
                raise TypeError(
                    f"{cls.__qualname__} writes persistent state (StatefulHIPModule) and so "
                    "must define reset_trace_state() for graph capture")
            if "reset_trace_state" in vars(klass):
                break


# Names of the reference's base classes, for code written against them.
TTNNModule = HIPModule
StatelessTTNNModule = StatelessHIPModule
StatefulTTNNModule = StatefulHIPModule
