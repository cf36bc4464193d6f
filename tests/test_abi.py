"""The C-ABI library (CPU side): it loads, exports every entry point the header declares, and
rejects bad arguments with a status code before launching anything."""
import ctypes
import os
import re

import pytest

from tt_symbiote_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "symbiote_mi355x.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(sym_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert set(_declared()) == set(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.sym_abi_version() == 2


def test_workspace_queries():
    q = _lib.query
    assert q("sym_paged_gqa_decode_workspace_bytes", 32, 16, 128, 4128) >= 32 * 16 * 17 * 130 * 4
    assert q("sym_paged_gqa_decode_workspace_bytes", 0, 16, 128, 100) == 0
    # the permute keeps its state in LDS up to 2048 tokens, then per-(256-token chunk, expert)
    # counts
    assert q("sym_moe_route_workspace_bytes", 32, 256) == 0
    assert q("sym_moe_route_workspace_bytes", 2048, 256) == 0
    assert q("sym_moe_route_workspace_bytes", 2049, 256) == 9 * 256 * 4
    assert q("sym_moe_route_workspace_bytes", 9942, 512) == 39 * 512 * 4


def _call(name, *args):
    lib = _lib.load()
    rc = getattr(lib, name)(*args)
    return rc, lib.sym_last_error().decode()


FAKE = ctypes.c_void_p(16)  # never dereferenced: validation fails first


def test_decode_rejects_unsupported_head_dim():
    rc, msg = _call("sym_paged_gqa_decode", FAKE, FAKE, FAKE, FAKE, FAKE, 2, 8, 2, 64, 16, 4,
                    8, 64, 1.0, FAKE, 1 << 20, FAKE, None)
    assert rc == 2 and "head_dim" in msg


def test_decode_rejects_group_size_and_workspace():
    rc, _ = _call("sym_paged_gqa_decode", FAKE, FAKE, FAKE, FAKE, FAKE, 2, 12, 4, 128, 16, 4, 8,
                  64, 1.0, FAKE, 1 << 20, FAKE, None)
    assert rc == 2
    rc, msg = _call("sym_paged_gqa_decode", FAKE, FAKE, FAKE, FAKE, FAKE, 2, 8, 2, 128, 16, 4,
                    8, 64, 1.0, FAKE, 16, FAKE, None)
    assert rc == 3 and "workspace" in msg
    rc, _ = _call("sym_paged_gqa_decode", FAKE, FAKE, FAKE, FAKE, FAKE, 2, 8, 2, 128, 16, 4, 8,
                  65, 1.0, FAKE, 1 << 20, FAKE, None)
    assert rc == 1  # max_context beyond the page table


def test_route_rejects_bad_configs():
    args = lambda T, E, ng, tg, k: (FAKE, 1, FAKE, T, E, ng, tg, k, 1.0, 1, 1, FAKE, FAKE, FAKE,
                                    FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, None)
    assert _call("sym_moe_route_permute", *args(4, 96, 8, 4, 8))[0] == 2      # E not supported
    assert _call("sym_moe_route_permute", *args(4, 256, 7, 4, 8))[0] == 1     # n_group
    assert _call("sym_moe_route_permute", *args(4, 256, 8, 9, 8))[0] == 1     # topk_group
    assert _call("sym_moe_route_permute", *args(4, 256, 8, 4, 33))[0] == 1    # top_k
    assert _call("sym_moe_route_permute", *args(4, 64, 64, 4, 2))[0] == 2     # group of 1
    assert _call("sym_moe_route_permute", *args(4, 64, 8, 1, 9))[0] == 1      # k > kept experts
    bad_parts = list(args(4, 256, 8, 4, 8))
    bad_parts[1] = 0
    assert _call("sym_moe_route_permute", *bad_parts)[0] == 1
    assert _call("sym_moe_route_permute", *args(0, 256, 8, 4, 8))[0] == 0     # empty batch
    small_ws = list(args(5000, 256, 8, 4, 8))
    small_ws[-2] = 100
    rc, msg = _call("sym_moe_route_permute", *small_ws)
    assert rc == 3 and "workspace" in msg


def test_gemm_and_norm_reject_bad_shapes():
    rc, _ = _call("sym_moe_grouped_swiglu", FAKE, 4, 2000, 512, FAKE, FAKE, FAKE, FAKE, FAKE,
                  257, FAKE, FAKE, FAKE, FAKE, None)
    assert rc == 2
    rc, _ = _call("sym_moe_grouped_swiglu", None, 4, 2048, 512, FAKE, FAKE, FAKE, FAKE, FAKE,
                  257, FAKE, FAKE, FAKE, FAKE, None)
    assert rc == 1
    rc, _ = _call("sym_rmsnorm_bf16", FAKE, None, FAKE, 4, 100, 1e-6, FAKE, None, None)
    assert rc == 2
    rc, _ = _call("sym_rmsnorm_bf16", FAKE, FAKE, FAKE, 4, 128, 1e-6, FAKE, None, None)
    assert rc == 1  # residual without residual_out
    rc, _ = _call("sym_paged_kv_fill", FAKE, FAKE, FAKE, FAKE, FAKE, 0, 60, 10, 2, 128, 16, 4,
                  8, None)
    assert rc == 1  # positions beyond the page table


def test_gemm_with_bf16_residual_rejects_bad_arguments():
    # a, w, bias, residual, M, N, K, out, stream
    rc, msg = _call("sym_gemm_bf16_res_bf16", FAKE, FAKE, None, None, 64, 2048, 2048, FAKE, None)
    assert rc == 1 and "residual" in msg
    rc, _ = _call("sym_gemm_bf16_res_bf16", FAKE, FAKE, None, FAKE, 64, 2040, 2048, FAKE, None)
    assert rc == 2  # N not a multiple of 16
    rc, _ = _call("sym_gemm_bf16_res_bf16", FAKE, FAKE, None, FAKE, 64, 2048, 2000, FAKE, None)
    assert rc == 2  # K not a multiple of 64
    rc, msg = _call("sym_gemm_bf16_res_bf16", FAKE, FAKE, None, ctypes.c_void_p(18), 64, 2048,
                    2048, FAKE, None)
    assert rc == 1 and "aligned" in msg
    rc, _ = _call("sym_gemm_bf16_res_bf16", FAKE, FAKE, None, None, 0, 2048, 2048, FAKE, None)
    assert rc == 0  # nothing to do


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(_lib.HipExtensionMissing):
        _lib.load()


def test_linear_and_router_reject_bad_shapes():
    assert _call("sym_linear_bf16", FAKE, FAKE, None, 4, 100, 2048, FAKE, 0, None)[0] == 2
    assert _call("sym_linear_bf16", FAKE, FAKE, None, 4, 128, 100, FAKE, 0, None)[0] == 2
    assert _call("sym_linear_bf16", None, FAKE, None, 4, 128, 128, FAKE, 0, None)[0] == 1
    assert _call("sym_linear_bf16", FAKE, FAKE, None, 0, 128, 128, FAKE, 0, None)[0] == 0
    assert _call("sym_moe_router_logits", FAKE, FAKE, 4, 2000, 256, FAKE, None)[0] == 2
    assert _call("sym_moe_router_logits", FAKE, FAKE, 4, 2048, 250, FAKE, None)[0] == 2
    assert _call("sym_moe_router_logits", FAKE, None, 4, 2048, 256, FAKE, None)[0] == 1
    assert _call("sym_moe_router_logits_split", FAKE, FAKE, 4, 2000, 256, FAKE, None)[0] == 2
    assert _call("sym_moe_router_logits_split", FAKE, FAKE, 4, 2048, 250, FAKE, None)[0] == 2
    assert _call("sym_moe_router_logits_split", FAKE, None, 4, 2048, 256, FAKE, None)[0] == 1
    assert _call("sym_moe_router_logits_split", FAKE, FAKE, 0, 2048, 256, FAKE, None)[0] == 0


def _prototype_arg_counts():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    counts = {}
    for m in re.finditer(r"\b(sym_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text):
        args = m.group(2).strip()
        counts[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return counts


def test_binding_argument_counts_match_header():
    counts = _prototype_arg_counts()
    assert set(counts) == set(_declared())
    for name, n in counts.items():
        assert len(_lib._SIGNATURES[name][1]) == n, name


def test_fp8_entry_points_reject_bad_shapes():
    # fp8 GEMMs: H must be a multiple of 512, I of 128
    args = lambda H, I: (FAKE, 4, H, I, FAKE, FAKE, FAKE, FAKE, FAKE, 65, FAKE, FAKE, FAKE, None)
    assert _call("sym_moe_gate_up_fp8", *args(256, 512))[0] == 2
    assert _call("sym_moe_gate_up_fp8", *args(2048, 64))[0] == 2
    assert _call("sym_moe_gate_up_fp8", *args(2048, 512)[:1], 0, *args(2048, 512)[2:])[0] == 0
    dargs = lambda H, I: (FAKE, 4, H, I, FAKE, FAKE, FAKE, FAKE, 65, FAKE, FAKE, FAKE, None)
    assert _call("sym_moe_down_fp8", *dargs(2048, 192))[0] == 2
    # fp8 cache: the block size must divide 256; strides must be multiples of 8
    fill = lambda bs, ts, hs, rows=2, seq_rows=None: (
        FAKE, FAKE, ts, hs, FAKE, None, seq_rows, 2, 10, 4, 128, FAKE, FAKE, FAKE, FAKE, FAKE,
        rows, 8, bs, 64, None)
    rc, msg = _call("sym_paged_kv_fill_fp8", *fill(48, 512, 128))
    assert rc == 2 and "block_size" in msg
    assert _call("sym_paged_kv_fill_fp8", *fill(32, 500, 128))[0] == 1
    # two sequences need two page-table rows unless each names its own row
    rc, msg = _call("sym_paged_kv_fill_fp8", *fill(32, 512, 128, rows=1))
    assert rc == 1 and "rows" in msg
    rc, msg = _call("sym_paged_gqa_decode_fp8", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 16, 4,
                    128, 48, 8, 64, 300, 1.0, FAKE, 1 << 20, FAKE, None)
    assert rc == 2 and "block_size" in msg
    rc, _ = _call("sym_paged_gqa_decode_fp8", FAKE, FAKE, FAKE, None, FAKE, FAKE, FAKE, 2, 16, 4,
                  128, 32, 8, 64, 256, 1.0, FAKE, 1 << 20, FAKE, None)
    assert rc == 1   # one scale array missing
