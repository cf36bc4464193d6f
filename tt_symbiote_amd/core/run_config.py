"""Run-mode dispatch of the HIP modules.

Mirrors the reference's ``NormalRun.module_run`` (core/run_config.py:595-647): check that a
device is bound, run lazy weight preparation, time the forward, and record the outcome in the
coverage ledger (utils/compatibility.py). One deliberate difference: the reference catches any
exception from the device forward and re-runs the torch layer (run_config.py:629-643). Here an
exception is recorded and re-raised -- the HIP path never falls back to a CPU or torch
implementation, so a result always comes from the kernels or not at all.

The mode is selected with ``SYMBIOTE_RUN_MODE`` (or the reference's ``TT_SYMBIOTE_RUN_MODE``);
only ``NORMAL`` exists.
"""
from __future__ import annotations

import os
import threading
import time
from collections import defaultdict
from typing import Dict, List


class DispatchManager:
    """Per-module host wall-time ledger (reference: run_config.py:247-352)."""

    _lock = threading.Lock()
    timings: Dict[str, List[float]] = defaultdict(list)
    current_module_name = None

    @classmethod
    def record_timing(cls, module_name: str, phase: str, seconds: float) -> None:
        with cls._lock:
            cls.timings[f"{module_name}:{phase}"].append(seconds)

    @classmethod
    def set_current_module_name(cls, name):
        cls.current_module_name = name

    @classmethod
    def clear_timings(cls) -> None:
        with cls._lock:
            cls.timings.clear()

    @classmethod
    def summary(cls) -> Dict[str, dict]:
        with cls._lock:
            return {k: {"calls": len(v), "total_s": sum(v), "mean_s": sum(v) / len(v)}
                    for k, v in cls.timings.items() if v}

    @classmethod
    def save_stats_to_file(cls, path: str) -> None:
        import csv

        with open(path, "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(["key", "calls", "total_s", "mean_s"])
            for k, v in sorted(cls.summary().items()):
                w.writerow([k, v["calls"], v["total_s"], v["mean_s"]])


class NormalRun:
    """Run the HIP forward; errors propagate (no fallback)."""

    record_timings = False

    def __new__(cls, *args, **kwargs):
        raise TypeError("This class cannot be instantiated")

    @staticmethod
    def module_run(self, *args, **kwargs):
        from ..utils import compatibility

        if self.device is None:
            raise RuntimeError(
                f"{self.module_name}: device is not set. Call "
                "`tt_symbiote_amd.set_device(model, device)` before invoking the model.")
        self.preprocess_weights()
        self.move_weights_to_device()
        DispatchManager.set_current_module_name(self.module_name)
        t0 = time.perf_counter() if NormalRun.record_timings else 0.0
        try:
            result = self.forward(*args, **kwargs)
        except Exception:
            compatibility.record_runtime_failure(self.module_name, _source_class_name(self))
            raise
        finally:
            DispatchManager.set_current_module_name(None)
        if NormalRun.record_timings:
            DispatchManager.record_timing(self.module_name, "forward", time.perf_counter() - t0)
        compatibility.record_runtime_success(self.module_name, _source_class_name(self))
        return result


def _source_class_name(module) -> str:
    layer = getattr(module, "_fallback_torch_layer", None)
    return type(layer).__name__ if layer is not None else type(module).__name__


_RUN_MODE_REGISTRY = {"NORMAL": NormalRun}


def get_run_implementation():
    mode = os.environ.get("SYMBIOTE_RUN_MODE") or os.environ.get("TT_SYMBIOTE_RUN_MODE") or "NORMAL"
    if mode not in _RUN_MODE_REGISTRY:
        raise ValueError(f"Invalid run mode {mode!r}; valid modes: {sorted(_RUN_MODE_REGISTRY)}")
    return _RUN_MODE_REGISTRY[mode]
