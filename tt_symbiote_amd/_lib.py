"""ctypes binding of ``libsymbiote_mi355x.so`` (the C ABI declared in
``include/symbiote_mi355x.h``).

The library is loaded lazily, always after ``torch`` so that the HIP runtime already in the
process (torch's ``libamdhip64.so.7``) is the one the kernels bind to. There is no fallback: a
missing library raises :class:`HipExtensionMissing`, and a non-zero status from any entry point
raises :class:`SymbioteKernelError` with the library's message.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  -- must be imported before the HIP library is loaded

from .build import LIB_PATH

_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_size = ctypes.c_size_t
_c_ll = ctypes.c_longlong
_vp = ctypes.c_void_p

# name -> (restype, argtypes)
_SIGNATURES = {
    "sym_last_error": (ctypes.c_char_p, []),
    "sym_abi_version": (_c_int, []),
    "sym_rmsnorm_bf16": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_float, _vp, _vp, _vp]),
    "sym_rmsnorm_f32": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_float, _vp, _vp, _vp]),
    "sym_attn_decode_prologue": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int,
         _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp],
    ),
    "sym_paged_kv_write": (
        _c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp]
    ),
    "sym_paged_kv_fill": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp],
    ),
    "sym_paged_gqa_decode_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "sym_paged_gqa_decode": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_float, _vp, _c_size, _vp, _vp],
    ),
    "sym_paged_gqa_decode_noalloc": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_float, _vp, _vp],
    ),
    "sym_attn_decode_step": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float,
         _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float, _vp, _c_size, _vp,
         _vp],
    ),
    "sym_paged_kv_fill_fp8": (
        _c_int,
        [_vp, _vp, _c_ll, _c_ll, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp,
         _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp],
    ),
    "sym_paged_gqa_decode_fp8": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_float, _vp, _c_size, _vp, _vp],
    ),
    "sym_attn_decode_step_fp8": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float,
         _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float, _vp,
         _c_size, _vp, _vp],
    ),
    "sym_embedding_bf16": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "sym_lm_head_greedy_workspace_bytes": (_c_size, [_c_int, _c_int]),
    "sym_lm_head_greedy": (
        _c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp, _c_size, _vp, _vp]
    ),
    "sym_greedy_advance": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _c_int, _vp]),
    "sym_linear_bf16": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_int, _vp]),
    "sym_rmsnorm_linear_bf16": (
        _c_int, [_vp, _vp, _c_float, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_int, _vp]
    ),
    "sym_linear_residual_bf16": (
        _c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp]
    ),
    "sym_moe_router_logits_norm": (
        _c_int, [_vp, _vp, _c_int, _vp, _c_float, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp]
    ),
    "sym_moe_router_logits": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "sym_moe_router_logits_split": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "sym_moe_route_workspace_bytes": (_c_size, [_c_int, _c_int]),
    "sym_moe_route_permute": (
        _c_int,
        [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int, _vp,
         _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _vp],
    ),
    "sym_moe_grouped_swiglu": (
        _c_int,
        [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp],
    ),
    "sym_moe_gate_up": (
        _c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp]
    ),
    "sym_moe_down": (
        _c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp]
    ),
    "sym_moe_gate_up_fp8": (
        _c_int,
        [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp],
    ),
    "sym_moe_down_fp8": (
        _c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp]
    ),
    "sym_moe_unpermute_combine": (
        _c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp]
    ),
    "sym_hbm_read_probe": (_c_int, [_vp, _c_size, _vp, _vp]),
    "sym_attn_prefill_prologue": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float,
         _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp],
    ),
    "sym_prefill_attention": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _vp, _vp],
    ),
    "sym_gemm_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_int, _vp]),
    "sym_gemm_bf16_res_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "sym_moe_tiled_workspace_bytes": (_c_size, []),
    "sym_moe_gate_up_tiled": (
        _c_int,
        [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp,
         _c_size, _vp],
    ),
    "sym_moe_down_tiled": (
        _c_int,
        [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _c_int, _vp,
         _c_size, _vp],
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


class HipExtensionMissing(RuntimeError):
    """The compiled gfx950 library is not present; the HIP path cannot run."""


class SymbioteKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, func: str, code: int, message: str):
        super().__init__(f"{func} failed with status {code}: {message}")
        self.func = func
        self.code = code


_lock = threading.Lock()
_lib = None


def library_path() -> str:
    """The library this process loads: the in-tree build."""
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the kernel library."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not os.path.exists(path):
                raise HipExtensionMissing(
                    f"{path} is missing: build it with `python -m tt_symbiote_amd.build` "
                    "(or __graft_entry__.build()) before running the HIP path"
                )
            lib = ctypes.CDLL(path)
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke an int-returning entry point and raise on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.sym_last_error()
        raise SymbioteKernelError(name, rc, msg.decode() if msg else "")


def query(name: str, *args) -> int:
    """Invoke a size query (returns size_t)."""
    return int(getattr(load(), name)(*args))
