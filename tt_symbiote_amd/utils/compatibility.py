"""Runtime coverage ledger: which HF classes were swapped, ran on the GPU, or failed.

Mirrors the observable shape of the reference's ``compatibility.report`` (utils/compatibility.py
:187-270): ``set_device`` records the swapped modules; every successful HIP forward bumps a
per-module success counter; a HIP forward that raised is recorded as a failure (the reference
records a torch fallback there; this library has none). ``regressions`` lists the failing HF
classes the recipe does not declare as expected CPU classes.
"""
from __future__ import annotations

import threading
from collections import Counter
from typing import Any, Dict

_LOCK = threading.Lock()
_FAILURES: Dict[str, str] = {}
_SUCCESS: Dict[str, str] = {}
_SUCCESS_CALLS: Counter = Counter()
_SWAPPED: Dict[str, str] = {}


def record_runtime_failure(module_name: str, class_name: str) -> None:
    with _LOCK:
        _FAILURES[module_name] = class_name


def record_runtime_success(module_name: str, class_name: str) -> None:
    with _LOCK:
        _SUCCESS[module_name] = class_name
        _SUCCESS_CALLS[module_name] += 1


def record_swapped_class(module_name: str, class_name: str) -> None:
    with _LOCK:
        _SWAPPED[module_name] = class_name


def reset_swapped_registry() -> None:
    with _LOCK:
        _SWAPPED.clear()


def reset_runtime_observations() -> None:
    with _LOCK:
        _FAILURES.clear()
        _SUCCESS.clear()
        _SUCCESS_CALLS.clear()


def report(model: Any) -> Dict[str, Any]:
    from ..registry import TT_MODEL_REGISTRY

    recipe = TT_MODEL_REGISTRY.get(type(model).__name__)
    expected_cpu = set(getattr(recipe, "cpu_fallback", []) or [])
    with _LOCK:
        swapped = dict(_SWAPPED)
        successes = dict(_SUCCESS)
        calls = dict(_SUCCESS_CALLS)
        failures = dict(_FAILURES)
    swapped_by_class = Counter(swapped.values())
    success_by_class: Counter = Counter()
    for name, cls in successes.items():
        success_by_class[cls] += calls.get(name, 0)
    failures_by_class = Counter(failures.values())
    regressions = sorted(c for c in failures_by_class if c not in expected_cpu)
    return {
        "model_class": type(model).__name__,
        "modules_swapped": {"by_class": dict(swapped_by_class), "by_module": swapped},
        "runtime_observed": {
            "successes_by_class": dict(success_by_class),
            "failures_by_class": dict(failures_by_class),
            "failures_by_module": failures,
        },
        "regressions": regressions,
        "summary": {
            "modules_swapped_count": sum(swapped_by_class.values()),
            "runtime_successes": sum(success_by_class.values()),
            "runtime_failures": sum(failures_by_class.values()),
            "regression_count": len(regressions),
        },
    }
