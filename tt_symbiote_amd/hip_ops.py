"""torch-facing wrappers of the C-ABI kernels.

Every wrapper checks device, dtype, contiguity and shapes on the host before it launches
anything, passes raw pointers plus ``torch.cuda.current_stream()``, and raises on a non-zero
status. Outputs are allocated with torch (caching allocator) unless the caller passes them in.
There is no CPU path here: CPU tensors are rejected.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib

HEAD_DIM = 128


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class KernelTimer:
    """Brackets chosen entry points with HIP events on the launching stream.

    Install with :func:`set_kernel_timer`; each wrapped call records a start/end event pair on
    ``torch.cuda.current_stream()`` (the stream the kernel is launched on). After a
    synchronisation, :meth:`mean_ms` gives the average duration per call."""

    def __init__(self, names):
        self.names = set(names)
        self.events = {n: [] for n in self.names}

    def wrap(self, name, fn):
        if name not in self.names:
            return fn()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        out = fn()
        end.record()
        self.events[name].append((start, end))
        return out

    def mean_ms(self, name) -> float:
        ev = self.events[name]
        return sum(s.elapsed_time(e) for s, e in ev) / len(ev) if ev else float("nan")

    def count(self, name) -> int:
        return len(self.events[name])


_timer = None


def set_kernel_timer(timer) -> None:
    global _timer
    _timer = timer


def _timed(name, fn):
    return fn() if _timer is None else _timer.wrap(name, fn)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _check(t: torch.Tensor, name: str, dtype: torch.dtype, device: torch.device = None,
           align: int = 16) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be a GPU tensor (got device {t.device})")
    if device is not None and t.device != device:
        raise ValueError(f"{name}: on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if t.data_ptr() % align:
        # the kernels use 16-byte vector loads (``align`` 4: an array read one int at a time)
        raise ValueError(f"{name}: data pointer must be {align}-byte aligned")


def _check_shape(t: torch.Tensor, name: str, shape: tuple) -> None:
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")


# -------------------------------------------------------------------------------------------
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
            residual_out: Optional[torch.Tensor] = None):
    """RMSNorm over the last dim (bf16 out) of x in bf16 or fp32. With ``residual`` (bf16):
    returns (normed, x + residual) with the sum in fp32 (the layer's residual stream)."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"x: dtype {x.dtype} (bf16 or fp32)")
    _check(x, "x", x.dtype)
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    _check(weight, "weight", torch.bfloat16, x.device)
    _check_shape(weight, "weight", (cols,))
    if out is None:
        out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16, x.device)
    _check_shape(out, "out", tuple(x.shape))
    if residual is not None:
        _check(residual, "residual", torch.bfloat16, x.device)
        _check_shape(residual, "residual", tuple(x.shape))
        if residual_out is None:
            residual_out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
        _check(residual_out, "residual_out", torch.float32, x.device)
        _check_shape(residual_out, "residual_out", tuple(x.shape))
    _lib.call("sym_rmsnorm_f32" if x.dtype == torch.float32 else "sym_rmsnorm_bf16", _ptr(x),
              _ptr(residual), _ptr(weight), rows, cols, float(eps), _ptr(out),
              _ptr(residual_out), _stream())
    return (out, residual_out) if residual is not None else out


def linear(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None,
           out_dtype: torch.dtype = torch.bfloat16, out: Optional[torch.Tensor] = None):
    """x [M, K] bf16 . w [N, K]^T (+ bias [N]) -> [M, N] in ``out_dtype`` (bf16 or fp32)."""
    _check(x, "x", torch.bfloat16)
    if x.dim() != 2:
        raise ValueError(f"x must be [M, K], got {tuple(x.shape)}")
    M, K = x.shape
    _check(w, "w", torch.bfloat16, x.device)
    if w.dim() != 2 or w.shape[1] != K:
        raise ValueError(f"w must be [N, {K}], got {tuple(w.shape)}")
    N = w.shape[0]
    if bias is not None:
        _check(bias, "bias", torch.bfloat16, x.device)
        _check_shape(bias, "bias", (N,))
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype {out_dtype} (bf16 or fp32)")
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype, device=x.device)
    _check(out, "out", out_dtype, x.device)
    _check_shape(out, "out", (M, N))
    _timed("linear", lambda: _lib.call(
        "sym_linear_bf16", _ptr(x), _ptr(w), _ptr(bias), M, N, K, _ptr(out),
        1 if out_dtype == torch.float32 else 0, _stream()))
    return out


def gemm(a: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None,
         residual: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.bfloat16,
         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """a [M, K] . w [N, K]^T (+ bias) (+ residual) with the tiled MFMA kernel (prefill-size M).
    The residual is fp32, or bf16 with an fp32 output (added in fp32 in the epilogue)."""
    _check(a, "a", torch.bfloat16)
    if a.dim() != 2:
        raise ValueError(f"a must be [M, K], got {tuple(a.shape)}")
    M, K = a.shape
    _check(w, "w", torch.bfloat16, a.device)
    if w.dim() != 2 or w.shape[1] != K:
        raise ValueError(f"w must be [N, {K}], got {tuple(w.shape)}")
    N = w.shape[0]
    if bias is not None:
        _check(bias, "bias", torch.bfloat16, a.device)
        _check_shape(bias, "bias", (N,))
    res16 = residual is not None and residual.dtype == torch.bfloat16
    if residual is not None:
        _check(residual, "residual", torch.bfloat16 if res16 else torch.float32, a.device)
        _check_shape(residual, "residual", (M, N))
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype {out_dtype} (bf16 or fp32)")
    if res16 and out_dtype != torch.float32:
        raise TypeError("a bf16 residual needs out_dtype=torch.float32")
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype, device=a.device)
    _check(out, "out", out_dtype, a.device)
    _check_shape(out, "out", (M, N))
    if res16:
        _timed("gemm", lambda: _lib.call(
            "sym_gemm_bf16_res_bf16", _ptr(a), _ptr(w), _ptr(bias), _ptr(residual), M, N, K,
            _ptr(out), _stream()))
    else:
        _timed("gemm", lambda: _lib.call(
            "sym_gemm_bf16", _ptr(a), _ptr(w), _ptr(bias), _ptr(residual), M, N, K, _ptr(out),
            1 if out_dtype == torch.float32 else 0, _stream()))
    return out


def rmsnorm_linear(x: torch.Tensor, gamma: torch.Tensor, eps: float, w: torch.Tensor,
                   bias: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.bfloat16,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(RMSNorm(x) * gamma) [M, K] . w [N, K]^T (+ bias) in one kernel."""
    _check(x, "x", torch.bfloat16)
    if x.dim() != 2:
        raise ValueError(f"x must be [M, K], got {tuple(x.shape)}")
    M, K = x.shape
    _check(gamma, "gamma", torch.bfloat16, x.device)
    _check_shape(gamma, "gamma", (K,))
    _check(w, "w", torch.bfloat16, x.device)
    if w.dim() != 2 or w.shape[1] != K:
        raise ValueError(f"w must be [N, {K}], got {tuple(w.shape)}")
    N = w.shape[0]
    if bias is not None:
        _check(bias, "bias", torch.bfloat16, x.device)
        _check_shape(bias, "bias", (N,))
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype {out_dtype} (bf16 or fp32)")
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype, device=x.device)
    _check(out, "out", out_dtype, x.device)
    _check_shape(out, "out", (M, N))
    _timed("linear", lambda: _lib.call(
        "sym_rmsnorm_linear_bf16", _ptr(x), _ptr(gamma), float(eps), _ptr(w), _ptr(bias), M, N,
        K, _ptr(out), 1 if out_dtype == torch.float32 else 0, _stream()))
    return out


def linear_residual(x: torch.Tensor, w: torch.Tensor, residual: torch.Tensor,
                    bias: Optional[torch.Tensor] = None):
    """(x . w^T + bias + residual) in fp32 [M, N], and the per-16-column sums of squares of its
    rows [N/16, M] (the statistics of the RMSNorm that follows)."""
    _check(x, "x", torch.bfloat16)
    if x.dim() != 2:
        raise ValueError(f"x must be [M, K], got {tuple(x.shape)}")
    M, K = x.shape
    _check(w, "w", torch.bfloat16, x.device)
    if w.dim() != 2 or w.shape[1] != K:
        raise ValueError(f"w must be [N, {K}], got {tuple(w.shape)}")
    N = w.shape[0]
    _check(residual, "residual", torch.bfloat16, x.device)
    _check_shape(residual, "residual", (M, N))
    if bias is not None:
        _check(bias, "bias", torch.bfloat16, x.device)
        _check_shape(bias, "bias", (N,))
    if N % 16:
        raise ValueError(f"N={N} must be a multiple of 16")
    out = torch.empty(M, N, dtype=torch.float32, device=x.device)
    parts = torch.empty(N // 16, M, dtype=torch.float32, device=x.device)
    _timed("linear", lambda: _lib.call(
        "sym_linear_residual_bf16", _ptr(x), _ptr(w), _ptr(bias), _ptr(residual), M, N, K,
        _ptr(out), _ptr(parts), _stream()))
    return out, parts


# -------------------------------------------------------------------------------------------
@dataclass
class PagedLayout:
    """Geometry of one layer's paged KV pools and the page table."""

    num_blocks: int
    num_kv_heads: int
    block_size: int
    head_dim: int
    max_blocks_per_seq: int


def _check_pools(k_pool, v_pool, block_tables, batch: int, k_scale=None,
                 v_scale=None) -> PagedLayout:
    """bf16 pools, or fp8 e4m3fn pools with their [num_blocks, Hkv] fp32 scales."""
    fp8 = k_pool.dtype == torch.float8_e4m3fn if isinstance(k_pool, torch.Tensor) else False
    dt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    _check(k_pool, "k_pool", dt)
    _check(v_pool, "v_pool", dt, k_pool.device)
    if fp8:
        if k_scale is None or v_scale is None:
            raise ValueError("an fp8 KV cache needs k_scale and v_scale [num_blocks, Hkv]")
        for t, n in ((k_scale, "k_scale"), (v_scale, "v_scale")):
            _check(t, n, torch.float32, k_pool.device)
            _check_shape(t, n, tuple(k_pool.shape[:2]))
        bs = k_pool.shape[2] if k_pool.dim() == 4 else 0
        if bs < 8 or 256 % bs:
            raise ValueError(f"fp8 KV cache: block_size {bs} must be a multiple of 8 dividing 256")
        # the fp8 V pool is dim-major inside each (block, head): [num_blocks, Hkv, D, block_size]
        if k_pool.dim() != 4 or v_pool.dim() != 4 or \
                tuple(v_pool.shape) != (k_pool.shape[0], k_pool.shape[1], k_pool.shape[3], bs):
            raise ValueError(f"fp8 pools must be K [num_blocks, Hkv, block_size, D] and V "
                             f"[num_blocks, Hkv, D, block_size], got {tuple(k_pool.shape)} / "
                             f"{tuple(v_pool.shape)}")
    elif k_scale is not None or v_scale is not None:
        raise ValueError("k_scale / v_scale given for a bf16 KV cache")
    if not fp8 and (k_pool.dim() != 4 or k_pool.shape != v_pool.shape):
        raise ValueError(f"k_pool/v_pool must be [num_blocks, Hkv, block_size, D] and equal, got "
                         f"{tuple(k_pool.shape)} / {tuple(v_pool.shape)}")
    nb, hkv, bs, d = k_pool.shape
    if d != HEAD_DIM:
        raise ValueError(f"head_dim {d} unsupported (kernels implement {HEAD_DIM})")
    _check(block_tables, "block_tables", torch.int32, k_pool.device)
    if block_tables.dim() != 2 or block_tables.shape[0] < batch:
        raise ValueError(f"block_tables must be [>= {batch}, max_blocks_per_seq], got "
                         f"{tuple(block_tables.shape)}")
    return PagedLayout(nb, hkv, bs, d, block_tables.shape[1])



def fp8_v_rows(v_pool: torch.Tensor) -> torch.Tensor:
    """The fp8 V pool [num_blocks, Hkv, D, block_size] (dim-major inside each (block, head)) seen
    as token rows [num_blocks, Hkv, block_size, D] (a transposed view)."""
    return v_pool.transpose(-1, -2)


def fp8_v_pool(rows: torch.Tensor) -> torch.Tensor:
    """Token rows [num_blocks, Hkv, block_size, D] of fp8 V codes in the V pool's layout
    [num_blocks, Hkv, D, block_size] (a contiguous copy)."""
    return rows.transpose(-1, -2).contiguous()

def attn_decode_prologue(qkv: torch.Tensor, positions: torch.Tensor, k_pool: torch.Tensor,
                         v_pool: torch.Tensor, block_tables: torch.Tensor, *, num_heads: int,
                         num_kv_heads: int, rotary_dim: int, rope_cs: Optional[torch.Tensor],
                         q_norm_w: Optional[torch.Tensor], k_norm_w: Optional[torch.Tensor],
                         eps: float, q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """QK-norm + partial RoPE on q/k of ``qkv`` [B, (Hq+2Hkv)*D]; writes k/v into the pools at
    ``positions``; returns q [B, Hq, D]."""
    _check(qkv, "qkv", torch.bfloat16)
    B = qkv.shape[0]
    _check_shape(qkv, "qkv", (B, (num_heads + 2 * num_kv_heads) * HEAD_DIM))
    _check(positions, "positions", torch.int32, qkv.device)
    _check_shape(positions, "positions", (B,))
    lay = _check_pools(k_pool, v_pool, block_tables, B)
    if lay.num_kv_heads != num_kv_heads:
        raise ValueError(f"pool has {lay.num_kv_heads} kv heads, module {num_kv_heads}")
    use_norm = q_norm_w is not None
    if use_norm:
        for t, n in ((q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w")):
            _check(t, n, torch.bfloat16, qkv.device)
            _check_shape(t, n, (HEAD_DIM,))
    max_pos = 0
    if rotary_dim:
        _check(rope_cs, "rope_cs", torch.float32, qkv.device)
        if rope_cs.dim() != 2 or rope_cs.shape[1] != rotary_dim:
            raise ValueError(f"rope_cs must be [max_pos, {rotary_dim}], got {tuple(rope_cs.shape)}")
        max_pos = rope_cs.shape[0]
    if q_out is None:
        q_out = torch.empty(B, num_heads, HEAD_DIM, dtype=torch.bfloat16, device=qkv.device)
    _check(q_out, "q_out", torch.bfloat16, qkv.device)
    _check_shape(q_out, "q_out", (B, num_heads, HEAD_DIM))
    _lib.call("sym_attn_decode_prologue", _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w),
              _ptr(rope_cs), max_pos, _ptr(positions), B, num_heads, num_kv_heads, HEAD_DIM,
              rotary_dim, float(eps), 1 if use_norm else 0, _ptr(q_out), _ptr(k_pool),
              _ptr(v_pool), _ptr(block_tables), lay.max_blocks_per_seq, lay.block_size,
              lay.num_blocks, _stream())
    return q_out


def attn_decode_step(qkv: torch.Tensor, positions: torch.Tensor, k_pool: torch.Tensor,
                     v_pool: torch.Tensor, block_tables: torch.Tensor, scale: float, *,
                     num_heads: int, num_kv_heads: int, rotary_dim: int,
                     rope_cs: Optional[torch.Tensor], q_norm_w: Optional[torch.Tensor],
                     k_norm_w: Optional[torch.Tensor], eps: float,
                     max_context: Optional[int] = None, workspace: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None, k_scale: Optional[torch.Tensor] = None,
                     v_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The fused decode step: :func:`attn_decode_prologue` (QK-norm, RoPE, k/v written into the
    pools at ``positions``) and :func:`paged_gqa_decode` in one pass; returns the attention
    output [B, Hq, D]. fp8 pools take their per-(block, head) scales."""
    _check(qkv, "qkv", torch.bfloat16)
    B = qkv.shape[0]
    _check_shape(qkv, "qkv", (B, (num_heads + 2 * num_kv_heads) * HEAD_DIM))
    _check(positions, "positions", torch.int32, qkv.device)
    _check_shape(positions, "positions", (B,))
    lay = _check_pools(k_pool, v_pool, block_tables, B, k_scale, v_scale)
    if lay.num_kv_heads != num_kv_heads:
        raise ValueError(f"pool has {lay.num_kv_heads} kv heads, module {num_kv_heads}")
    use_norm = q_norm_w is not None
    if use_norm:
        for t, n in ((q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w")):
            _check(t, n, torch.bfloat16, qkv.device)
            _check_shape(t, n, (HEAD_DIM,))
    max_pos = 0
    if rotary_dim:
        _check(rope_cs, "rope_cs", torch.float32, qkv.device)
        if rope_cs.dim() != 2 or rope_cs.shape[1] != rotary_dim:
            raise ValueError(f"rope_cs must be [max_pos, {rotary_dim}], got {tuple(rope_cs.shape)}")
        max_pos = rope_cs.shape[0]
    cap = lay.max_blocks_per_seq * lay.block_size
    if max_context is None:
        max_context = cap
    if not 0 < max_context <= cap:
        raise ValueError(f"max_context {max_context} outside (0, {cap}]")
    need = paged_decode_workspace_bytes(B, num_heads, max_context)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=qkv.device)
    _check(workspace, "workspace", torch.uint8, qkv.device)
    if out is None:
        out = torch.empty(B, num_heads, HEAD_DIM, dtype=torch.bfloat16, device=qkv.device)
    _check(out, "out", torch.bfloat16, qkv.device)
    _check_shape(out, "out", (B, num_heads, HEAD_DIM))
    if k_scale is not None:
        _timed("paged_gqa_decode", lambda: _lib.call(
            "sym_attn_decode_step_fp8", _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w),
            _ptr(rope_cs), max_pos, _ptr(positions), B, num_heads, num_kv_heads, HEAD_DIM,
            rotary_dim, float(eps), 1 if use_norm else 0, _ptr(k_pool), _ptr(v_pool),
            _ptr(k_scale), _ptr(v_scale), _ptr(block_tables), lay.max_blocks_per_seq,
            lay.block_size, lay.num_blocks, int(max_context), float(scale), _ptr(workspace),
            workspace.numel(), _ptr(out), _stream()))
        return out
    _timed("paged_gqa_decode", lambda: _lib.call(
        "sym_attn_decode_step", _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(rope_cs),
        max_pos, _ptr(positions), B, num_heads, num_kv_heads, HEAD_DIM, rotary_dim, float(eps),
        1 if use_norm else 0, _ptr(k_pool), _ptr(v_pool), _ptr(block_tables),
        lay.max_blocks_per_seq, lay.block_size, lay.num_blocks, int(max_context), float(scale),
        _ptr(workspace), workspace.numel(), _ptr(out), _stream()))
    return out


def attn_prefill_prologue(qkv: torch.Tensor, positions: torch.Tensor, seq_ids: torch.Tensor,
                          k_pool: torch.Tensor, v_pool: torch.Tensor, block_tables: torch.Tensor,
                          *, num_heads: int, num_kv_heads: int, rotary_dim: int,
                          rope_cs: Optional[torch.Tensor], q_norm_w: Optional[torch.Tensor],
                          k_norm_w: Optional[torch.Tensor], eps: float):
    """QK-norm + partial RoPE of T packed tokens (token t at positions[t] of page-table row
    seq_ids[t]); k/v written into bf16 pools (not when the pools are fp8: those are filled from
    the returned k, v by :func:`paged_kv_fill_fp8`); returns q [T, Hq, D], k, v [T, Hkv, D]."""
    _check(qkv, "qkv", torch.bfloat16)
    T = qkv.shape[0]
    _check_shape(qkv, "qkv", (T, (num_heads + 2 * num_kv_heads) * HEAD_DIM))
    for t, n in ((positions, "positions"), (seq_ids, "seq_ids")):
        _check(t, n, torch.int32, qkv.device)
        _check_shape(t, n, (T,))
    write_pools = k_pool.dtype == torch.bfloat16
    if write_pools:
        lay = _check_pools(k_pool, v_pool, block_tables, 1)
    else:
        if k_pool.dtype != torch.float8_e4m3fn or v_pool.dtype != torch.float8_e4m3fn:
            raise TypeError(f"pools must be bf16 or float8_e4m3fn, got {k_pool.dtype}")
        _check(block_tables, "block_tables", torch.int32, qkv.device)
        nb, hkv, bs, _ = k_pool.shape
        lay = PagedLayout(nb, hkv, bs, HEAD_DIM, block_tables.shape[1])
    if lay.num_kv_heads != num_kv_heads:
        raise ValueError(f"pool has {lay.num_kv_heads} kv heads, module {num_kv_heads}")
    use_norm = q_norm_w is not None
    if use_norm:
        for t, n in ((q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w")):
            _check(t, n, torch.bfloat16, qkv.device)
            _check_shape(t, n, (HEAD_DIM,))
    max_pos = 0
    if rotary_dim:
        _check(rope_cs, "rope_cs", torch.float32, qkv.device)
        if rope_cs.dim() != 2 or rope_cs.shape[1] != rotary_dim:
            raise ValueError(f"rope_cs must be [max_pos, {rotary_dim}], got {tuple(rope_cs.shape)}")
        max_pos = rope_cs.shape[0]
    bf = dict(dtype=torch.bfloat16, device=qkv.device)
    q = torch.empty(T, num_heads, HEAD_DIM, **bf)
    k = torch.empty(T, num_kv_heads, HEAD_DIM, **bf)
    v = torch.empty(T, num_kv_heads, HEAD_DIM, **bf)
    _lib.call("sym_attn_prefill_prologue", _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w),
              _ptr(rope_cs), max_pos, _ptr(positions), _ptr(seq_ids), T, num_heads,
              num_kv_heads, HEAD_DIM, rotary_dim, float(eps), 1 if use_norm else 0, _ptr(q),
              _ptr(k), _ptr(v), _ptr(k_pool) if write_pools else None,
              _ptr(v_pool) if write_pools else None, _ptr(block_tables),
              lay.max_blocks_per_seq, lay.block_size, lay.num_blocks, _stream())
    return q, k, v


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      cu_seqlens: torch.Tensor, max_seqlen: int, scale: float,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal GQA attention of packed sequences (rows cu_seqlens[s] .. cu_seqlens[s+1]-1):
    q [T, Hq, D], k, v [T, Hkv, D] -> [T, Hq, D] (bf16)."""
    _check(q, "q", torch.bfloat16)
    if q.dim() != 3 or q.shape[2] != HEAD_DIM:
        raise ValueError(f"q must be [T, Hq, {HEAD_DIM}], got {tuple(q.shape)}")
    T, Hq, _ = q.shape
    _check(k, "k", torch.bfloat16, q.device)
    _check(v, "v", torch.bfloat16, q.device)
    if k.dim() != 3 or k.shape[0] != T or k.shape[2] != HEAD_DIM or v.shape != k.shape:
        raise ValueError(f"k/v must be [{T}, Hkv, {HEAD_DIM}], got {tuple(k.shape)}")
    Hkv = k.shape[1]
    _check(cu_seqlens, "cu_seqlens", torch.int32, q.device)
    if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 1:
        raise ValueError("cu_seqlens must be [n_seqs + 1]")
    if out is None:
        out = torch.empty_like(q)
    _check(out, "out", torch.bfloat16, q.device)
    _check_shape(out, "out", tuple(q.shape))
    _timed("prefill_attention", lambda: _lib.call(
        "sym_prefill_attention", _ptr(q), _ptr(k), _ptr(v), _ptr(cu_seqlens),
        cu_seqlens.numel() - 1, int(max_seqlen), Hq, Hkv, HEAD_DIM, float(scale), _ptr(out),
        _stream()))
    return out


def paged_kv_write(k_new: torch.Tensor, v_new: torch.Tensor, k_pool: torch.Tensor,
                   v_pool: torch.Tensor, block_tables: torch.Tensor,
                   positions: torch.Tensor) -> None:
    """Write one token per sequence: k_new/v_new [B, Hkv, D] at slot positions[b]."""
    _check(k_new, "k_new", torch.bfloat16)
    _check(v_new, "v_new", torch.bfloat16, k_new.device)
    B = k_new.shape[0]
    lay = _check_pools(k_pool, v_pool, block_tables, B)
    _check_shape(k_new, "k_new", (B, lay.num_kv_heads, HEAD_DIM))
    _check_shape(v_new, "v_new", (B, lay.num_kv_heads, HEAD_DIM))
    _check(positions, "positions", torch.int32, k_new.device)
    _check_shape(positions, "positions", (B,))
    _lib.call("sym_paged_kv_write", _ptr(k_new), _ptr(v_new), _ptr(k_pool), _ptr(v_pool),
              _ptr(block_tables), _ptr(positions), B, lay.num_kv_heads, HEAD_DIM, lay.block_size,
              lay.max_blocks_per_seq, lay.num_blocks, _stream())


def paged_kv_fill(k: torch.Tensor, v: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                  block_tables: torch.Tensor, batch_idx: int, start_pos: int = 0) -> None:
    """Write a prompt's K/V [Hkv, S, D] for sequence ``batch_idx`` from ``start_pos``."""
    _check(k, "k", torch.bfloat16)
    _check(v, "v", torch.bfloat16, k.device)
    lay = _check_pools(k_pool, v_pool, block_tables, batch_idx + 1)
    if k.dim() != 3 or k.shape[0] != lay.num_kv_heads or k.shape[2] != HEAD_DIM:
        raise ValueError(f"k must be [Hkv={lay.num_kv_heads}, S, {HEAD_DIM}], got {tuple(k.shape)}")
    _check_shape(v, "v", tuple(k.shape))
    _lib.call("sym_paged_kv_fill", _ptr(k), _ptr(v), _ptr(k_pool), _ptr(v_pool),
              _ptr(block_tables), int(batch_idx), int(start_pos), k.shape[1], lay.num_kv_heads,
              HEAD_DIM, lay.block_size, lay.max_blocks_per_seq, lay.num_blocks, _stream())


def paged_decode_workspace_bytes(batch: int, num_heads: int, max_context: int) -> int:
    return _lib.query("sym_paged_gqa_decode_workspace_bytes", batch, num_heads, HEAD_DIM,
                      max_context)



def paged_gqa_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                     block_tables: torch.Tensor, positions: torch.Tensor, scale: float,
                     max_context: Optional[int] = None, workspace: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None, k_scale: Optional[torch.Tensor] = None,
                     v_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode attention of q [B, Hq, D] over slots 0..positions[b] of each sequence (bf16
    pools, or fp8 pools with their scales)."""
    _check(q, "q", torch.bfloat16)
    if q.dim() != 3 or q.shape[2] != HEAD_DIM:
        raise ValueError(f"q must be [B, Hq, {HEAD_DIM}], got {tuple(q.shape)}")
    B, Hq, _ = q.shape
    lay = _check_pools(k_pool, v_pool, block_tables, B, k_scale, v_scale)
    _check(positions, "positions", torch.int32, q.device)
    _check_shape(positions, "positions", (B,))
    cap = lay.max_blocks_per_seq * lay.block_size
    if max_context is None:
        max_context = cap
    if not 0 < max_context <= cap:
        raise ValueError(f"max_context {max_context} outside (0, {cap}]")
    need = paged_decode_workspace_bytes(B, Hq, max_context)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _check(workspace, "workspace", torch.uint8, q.device)
    if out is None:
        out = torch.empty_like(q)
    _check(out, "out", torch.bfloat16, q.device)
    _check_shape(out, "out", tuple(q.shape))
    if k_scale is not None:
        _timed("paged_gqa_decode", lambda: _lib.call(
            "sym_paged_gqa_decode_fp8", _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(k_scale),
            _ptr(v_scale), _ptr(block_tables), _ptr(positions), B, Hq, lay.num_kv_heads,
            HEAD_DIM, lay.block_size, lay.max_blocks_per_seq, lay.num_blocks, int(max_context),
            float(scale), _ptr(workspace), workspace.numel(), _ptr(out), _stream()))
        return out
    _timed("paged_gqa_decode", lambda: _lib.call(
        "sym_paged_gqa_decode", _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_tables),
        _ptr(positions), B, Hq, lay.num_kv_heads, HEAD_DIM, lay.block_size,
        lay.max_blocks_per_seq, lay.num_blocks, int(max_context), float(scale),
        _ptr(workspace), workspace.numel(), _ptr(out), _stream()))
    return out


def paged_gqa_decode_noalloc(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                             block_tables: torch.Tensor, positions: torch.Tensor, scale: float,
                             out: torch.Tensor, max_context: Optional[int] = None) -> torch.Tensor:
    """:func:`paged_gqa_decode` (bf16 pools) through the allocation-free entry point: the split
    partials live in the library's fixed per-GPU scratch array, and ``out`` [B, Hq, D] bf16 is
    the caller's, so the call allocates no device memory. Calls that overlap in time on one GPU
    race on that array."""
    _check(q, "q", torch.bfloat16)
    if q.dim() != 3 or q.shape[2] != HEAD_DIM:
        raise ValueError(f"q must be [B, Hq, {HEAD_DIM}], got {tuple(q.shape)}")
    B, Hq, _ = q.shape
    lay = _check_pools(k_pool, v_pool, block_tables, B)
    _check(positions, "positions", torch.int32, q.device)
    _check_shape(positions, "positions", (B,))
    cap = lay.max_blocks_per_seq * lay.block_size
    if max_context is None:
        max_context = cap
    if not 0 < max_context <= cap:
        raise ValueError(f"max_context {max_context} outside (0, {cap}]")
    _check(out, "out", torch.bfloat16, q.device)
    _check_shape(out, "out", tuple(q.shape))
    _timed("paged_gqa_decode", lambda: _lib.call(
        "sym_paged_gqa_decode_noalloc", _ptr(q), _ptr(k_pool), _ptr(v_pool),
        _ptr(block_tables), _ptr(positions), B, Hq, lay.num_kv_heads, HEAD_DIM, lay.block_size,
        lay.max_blocks_per_seq, lay.num_blocks, int(max_context), float(scale), _ptr(out),
        _stream()))
    return out


def paged_kv_fill_fp8(k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
                      max_seqlen: int, k_pool: torch.Tensor, v_pool: torch.Tensor,
                      k_scale: torch.Tensor, v_scale: torch.Tensor, block_tables: torch.Tensor,
                      start_pos: Optional[torch.Tensor] = None, layout: str = "thd",
                      seq_rows: Optional[torch.Tensor] = None) -> None:
    """Append tokens to an fp8 KV cache (per-(block, head) power-of-two scales, requantising a
    block's earlier tokens when its scale grows). Sequence s = tokens cu_seqlens[s] ..
    cu_seqlens[s+1]-1 at positions start_pos[s] + i (0 when start_pos is None) in page-table row
    seq_rows[s] (s when seq_rows is None). ``layout``: "thd" for k, v [T, Hkv, D]; "htd" for
    k, v [Hkv, T, D]."""
    _check(k, "k", torch.bfloat16)
    _check(v, "v", torch.bfloat16, k.device)
    _check_shape(v, "v", tuple(k.shape))
    _check(cu_seqlens, "cu_seqlens", torch.int32, k.device)
    n = cu_seqlens.numel() - 1
    if n < 0 or cu_seqlens.dim() != 1:
        raise ValueError("cu_seqlens must be [n_seqs + 1]")
    lay = _check_pools(k_pool, v_pool, block_tables, 1 if seq_rows is not None else n,
                       k_scale, v_scale)
    if k_pool.dtype != torch.float8_e4m3fn:
        raise TypeError("paged_kv_fill_fp8 needs float8_e4m3fn pools")
    if k.dim() != 3 or k.shape[2] != HEAD_DIM:
        raise ValueError(f"k must be 3-D with head_dim {HEAD_DIM}, got {tuple(k.shape)}")
    if layout == "thd":
        T, hkv, _ = k.shape
        strides = (hkv * HEAD_DIM, HEAD_DIM)
    elif layout == "htd":
        hkv, T, _ = k.shape
        strides = (HEAD_DIM, T * HEAD_DIM)
    else:
        raise ValueError(f"layout {layout!r}")
    if hkv != lay.num_kv_heads:
        raise ValueError(f"k has {hkv} kv heads, the pool {lay.num_kv_heads}")
    for t, name in ((start_pos, "start_pos"), (seq_rows, "seq_rows")):
        if t is not None:
            _check(t, name, torch.int32, k.device, align=4)
            _check_shape(t, name, (n,))
    _lib.call("sym_paged_kv_fill_fp8", _ptr(k), _ptr(v), strides[0], strides[1],
              _ptr(cu_seqlens), _ptr(start_pos), _ptr(seq_rows), n, int(max_seqlen),
              lay.num_kv_heads, HEAD_DIM, _ptr(k_pool), _ptr(v_pool), _ptr(k_scale),
              _ptr(v_scale), _ptr(block_tables), block_tables.shape[0], lay.max_blocks_per_seq,
              lay.block_size, lay.num_blocks, _stream())


# -------------------------------------------------------------------------------------------
def embedding(ids: torch.Tensor, table: torch.Tensor,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[t] = table[ids[t]] for ids [T] int32 and a [V, H] bf16 table (ids outside [0, V)
    give zero rows)."""
    _check(table, "table", torch.bfloat16)
    if table.dim() != 2:
        raise ValueError(f"table must be [V, H], got {tuple(table.shape)}")
    V, H = table.shape
    _check(ids, "ids", torch.int32, table.device)
    T = ids.numel()
    if out is None:
        out = torch.empty(T, H, dtype=torch.bfloat16, device=table.device)
    _check(out, "out", torch.bfloat16, table.device)
    _check_shape(out, "out", (T, H))
    _lib.call("sym_embedding_bf16", _ptr(ids), _ptr(table), T, H, V, _ptr(out), _stream())
    return out


def lm_head_greedy(x: torch.Tensor, w: torch.Tensor, ids: Optional[torch.Tensor] = None,
                   workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """ids[b] = argmax_v x[b] . w[v] (x [B, H] bf16, w [V, H] bf16, fp32 logits; ties go to the
    lowest index) -> [B] int32."""
    _check(x, "x", torch.bfloat16)
    _check(w, "w", torch.bfloat16, x.device)
    B, H = x.shape
    V = w.shape[0]
    _check_shape(w, "w", (V, H))
    if ids is None:
        ids = torch.empty(B, dtype=torch.int32, device=x.device)
    _check(ids, "ids", torch.int32, x.device)
    _check_shape(ids, "ids", (B,))
    need = _lib.query("sym_lm_head_greedy_workspace_bytes", B, V)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _check(workspace, "workspace", torch.uint8, x.device)
    _timed("lm_head", lambda: _lib.call(
        "sym_lm_head_greedy", _ptr(x), _ptr(w), B, H, V, _ptr(workspace), workspace.numel(),
        _ptr(ids), _stream()))
    return ids


def lm_head_greedy_workspace_bytes(batch: int, vocab: int) -> int:
    return _lib.query("sym_lm_head_greedy_workspace_bytes", batch, vocab)


def greedy_advance(ids: torch.Tensor, positions: torch.Tensor,
                   history: Optional[torch.Tensor] = None,
                   hist_base: Optional[torch.Tensor] = None) -> None:
    """positions += 1; history[b, positions[b] - hist_base[b]] = ids[b] (inside the row)."""
    _check(ids, "ids", torch.int32)
    B = ids.numel()
    _check(positions, "positions", torch.int32, ids.device)
    _check_shape(positions, "positions", (B,))
    cols = 0
    if history is not None:
        _check(history, "history", torch.int32, ids.device)
        if history.dim() != 2 or history.shape[0] != B:
            raise ValueError(f"history must be [{B}, n], got {tuple(history.shape)}")
        cols = history.shape[1]
        _check(hist_base, "hist_base", torch.int32, ids.device)
        _check_shape(hist_base, "hist_base", (B,))
    _lib.call("sym_greedy_advance", _ptr(ids), B, _ptr(positions), _ptr(history),
              _ptr(hist_base), cols, _stream())


# -------------------------------------------------------------------------------------------
@dataclass
class RouteResult:
    """Outputs of :func:`moe_route_permute` (all on the device)."""

    topk_idx: torch.Tensor       # [T, K] int32
    topk_w: torch.Tensor         # [T, K] fp32
    expert_counts: torch.Tensor  # [E] int32
    expert_offsets: torch.Tensor  # [E+1] int32
    sorted_tokens: torch.Tensor  # [T*K (+T)] int32
    inv_perm: torch.Tensor       # [T, K] int32
    seg_expert: torch.Tensor     # [E+1] int32
    seg_offset: torch.Tensor     # [E+1] int32
    seg_count: torch.Tensor      # [E+1] int32
    n_segments: torch.Tensor     # [1] int32
    with_shared: bool

    @property
    def rows(self) -> int:
        return self.sorted_tokens.numel()


LOGIT_PARTS = 4


def moe_router_logits(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """fp32 router logits of x [T, H] (bf16) against w [E, H] (fp32), returned as the four
    partial sums [4, T, E] over quarters of H (their left-to-right sum is the logits)."""
    _check(x, "x", torch.bfloat16)
    if x.dim() != 2:
        raise ValueError(f"x must be [T, H], got {tuple(x.shape)}")
    T, H = x.shape
    _check(w, "w", torch.float32, x.device)
    if w.dim() != 2 or w.shape[1] != H:
        raise ValueError(f"w must be [E, {H}], got {tuple(w.shape)}")
    E = w.shape[0]
    parts = torch.empty(LOGIT_PARTS, T, E, dtype=torch.float32, device=x.device)
    _timed("moe_router_logits", lambda: _lib.call(
        "sym_moe_router_logits", _ptr(x), _ptr(w), T, H, E, _ptr(parts), _stream()))
    return parts


ROUTER_SPLIT_MIN_TOKENS = 1536  # from this many tokens the router logits run on bf16 MFMA tiles
# (measured: 26 against 33 us at 1024 tokens, 48 against 34 us at 2048)


def split_router_weight(w: torch.Tensor) -> torch.Tensor:
    """The fp32 gate weight [E, H] as three bf16 planes [3, E, H] with w = hi + mid + lo exactly
    (hi = w with its low 16 bits cleared, mid likewise of w - hi, lo = w - hi - mid: 8 mantissa
    bits each). Raises if a value does not split exactly (e.g. a subnormal remainder)."""
    w = w.detach().to(torch.float32).contiguous()
    mask = torch.tensor(-65536, dtype=torch.int32, device=w.device)
    hi = (w.view(torch.int32) & mask).view(torch.float32)
    r1 = w - hi
    mid = (r1.view(torch.int32) & mask).view(torch.float32)
    lo = r1 - mid
    planes = torch.stack([hi, mid, lo]).to(torch.bfloat16).contiguous()
    back = (planes[0].float() + planes[1].float()) + planes[2].float()
    if not torch.equal(back.view(torch.int32), w.view(torch.int32)):
        raise ValueError("router weight does not split exactly into three bf16 planes")
    return planes


def moe_router_logits_split(x: torch.Tensor, w_planes: torch.Tensor) -> torch.Tensor:
    """fp32 router logits of x [T, H] (bf16) against the split gate weight w_planes [3, E, H]
    (:func:`split_router_weight`), on bf16 MFMA tiles; returned as the three partial logits
    [3, T, E] (hi, mid, lo planes), summed left to right by :func:`moe_route_permute`."""
    _check(x, "x", torch.bfloat16)
    if x.dim() != 2:
        raise ValueError(f"x must be [T, H], got {tuple(x.shape)}")
    T, H = x.shape
    _check(w_planes, "w_planes", torch.bfloat16, x.device)
    if w_planes.dim() != 3 or w_planes.shape[0] != 3 or w_planes.shape[2] != H:
        raise ValueError(f"w_planes must be [3, E, {H}], got {tuple(w_planes.shape)}")
    E = w_planes.shape[1]
    parts = torch.empty(3, T, E, dtype=torch.float32, device=x.device)
    _timed("moe_router_logits", lambda: _lib.call(
        "sym_moe_router_logits_split", _ptr(x), _ptr(w_planes), T, H, E, _ptr(parts),
        _stream()))
    return parts


def moe_router_logits_norm(h: torch.Tensor, ss_parts: torch.Tensor, gamma: torch.Tensor,
                           eps: float, w: torch.Tensor, xn_out: Optional[torch.Tensor] = None):
    """Router logits (four partial sums [4, T, E]) of xn = bf16(RMSNorm(h) * gamma), with h the
    fp32 residual stream [T, H] and ss_parts [n, T] the partial sums of squares of its rows;
    also returns xn (bf16 [T, H]) for the expert GEMMs."""
    _check(h, "h", torch.float32)
    if h.dim() != 2:
        raise ValueError(f"h must be [T, H], got {tuple(h.shape)}")
    T, H = h.shape
    _check(ss_parts, "ss_parts", torch.float32, h.device)
    if ss_parts.dim() != 2 or ss_parts.shape[1] != T:
        raise ValueError(f"ss_parts must be [n, {T}], got {tuple(ss_parts.shape)}")
    _check(gamma, "gamma", torch.bfloat16, h.device)
    _check_shape(gamma, "gamma", (H,))
    _check(w, "w", torch.float32, h.device)
    if w.dim() != 2 or w.shape[1] != H:
        raise ValueError(f"w must be [E, {H}], got {tuple(w.shape)}")
    E = w.shape[0]
    parts = torch.empty(LOGIT_PARTS, T, E, dtype=torch.float32, device=h.device)
    if xn_out is None:
        xn_out = torch.empty(T, H, dtype=torch.bfloat16, device=h.device)
    _check(xn_out, "xn_out", torch.bfloat16, h.device)
    _check_shape(xn_out, "xn_out", (T, H))
    _timed("moe_router_logits", lambda: _lib.call(
        "sym_moe_router_logits_norm", _ptr(h), _ptr(ss_parts), ss_parts.shape[0], _ptr(gamma),
        float(eps), _ptr(w), T, H, E, _ptr(parts), _ptr(xn_out), _stream()))
    return parts, xn_out


def moe_route_permute(logits: torch.Tensor, bias: torch.Tensor, *, n_group: int,
                      topk_group: int, top_k: int, routed_scale: float,
                      renormalize: bool = True, with_shared: bool = True) -> RouteResult:
    """Fused sigmoid/bias/group-limited top-k router + expert-sorted permute. ``logits`` is
    [T, E], or [P, T, E] partial sums added left to right (as from :func:`moe_router_logits`)."""
    _check(logits, "logits", torch.float32)
    if logits.dim() == 2:
        n_parts = 1
        T, E = logits.shape
    elif logits.dim() == 3:
        n_parts, T, E = logits.shape
    else:
        raise ValueError(f"logits must be [T, E] or [P, T, E], got {tuple(logits.shape)}")
    dev = logits.device
    _check(bias, "bias", torch.float32, dev)
    _check_shape(bias, "bias", (E,))
    i32 = dict(dtype=torch.int32, device=dev)
    rows = T * top_k + (T if with_shared else 0)
    res = RouteResult(
        topk_idx=torch.empty(T, top_k, **i32),
        topk_w=torch.empty(T, top_k, dtype=torch.float32, device=dev),
        expert_counts=torch.empty(E, **i32),
        expert_offsets=torch.empty(E + 1, **i32),
        sorted_tokens=torch.empty(rows, **i32),
        inv_perm=torch.empty(T, top_k, **i32),
        seg_expert=torch.empty(E + 1, **i32),
        seg_offset=torch.empty(E + 1, **i32),
        seg_count=torch.empty(E + 1, **i32),
        n_segments=torch.empty(1, **i32),
        with_shared=bool(with_shared),
    )
    if T == 0:
        return res
    ws_bytes = _lib.query("sym_moe_route_workspace_bytes", T, E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    _timed("moe_route_permute", lambda: _lib.call(
              "sym_moe_route_permute", _ptr(logits), n_parts, _ptr(bias), T, E, int(n_group),
              int(topk_group), int(top_k), float(routed_scale), 1 if renormalize else 0,
              1 if with_shared else 0, _ptr(res.topk_idx), _ptr(res.topk_w),
              _ptr(res.expert_counts), _ptr(res.expert_offsets), _ptr(res.sorted_tokens),
              _ptr(res.inv_perm), _ptr(res.seg_expert), _ptr(res.seg_offset),
              _ptr(res.seg_count), _ptr(res.n_segments), _ptr(ws) if ws is not None else None,
              ws_bytes, _stream()))
    return res


TILED_MIN_TOKENS = 128  # from this many tokens the expert GEMMs use the tiled (MFMA-bound) kernels


def moe_tiled_workspace(device=None) -> torch.Tensor:
    """A zeroed tile-counter workspace for the tiled grouped expert GEMMs
    (``sym_moe_tiled_workspace_bytes()`` bytes). Every launch leaves it zeroed, so it can be
    reused by any number of launches ordered on one stream."""
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    return torch.zeros(_lib.query("sym_moe_tiled_workspace_bytes"), dtype=torch.uint8, device=dev)


FP8_BLOCK = 128


@dataclass
class BlockFp8:
    """A weight stored as OCP fp8 e4m3fn with one fp32 scale per 128 x 128 block of its last two
    dims: w[..., n, k] = float(q[..., n, k]) * scale[..., n // 128, k // 128]."""
    q: torch.Tensor      # [..., N, K] torch.float8_e4m3fn
    scale: torch.Tensor  # [..., N / 128, K / 128] float32

    @property
    def shape(self):
        return self.q.shape

    def check(self, name: str, device=None):
        _check(self.q, name + ".q", torch.float8_e4m3fn, device)
        _check(self.scale, name + ".scale", torch.float32, device)
        *lead, n, k = self.q.shape
        if n % FP8_BLOCK or k % FP8_BLOCK:
            raise ValueError(f"{name}: dims {n} x {k} must be multiples of {FP8_BLOCK}")
        _check_shape(self.scale, name + ".scale", (*lead, n // FP8_BLOCK, k // FP8_BLOCK))

    def numel_bytes(self) -> int:
        return self.q.numel() + 4 * self.scale.numel()


def quantize_block_fp8(w: torch.Tensor) -> BlockFp8:
    """Weight intake for the fp8 format: per 128 x 128 block, scale = amax / 448 (1 for an
    all-zero block) and q = e4m3fn(w / scale) (round to nearest even, clamped to +-448). Runs
    once when weights are prepared, on whatever device w is on."""
    *lead, n, k = w.shape
    if n % FP8_BLOCK or k % FP8_BLOCK:
        raise ValueError(f"dims {n} x {k} must be multiples of {FP8_BLOCK}")
    wb = w.float().reshape(*lead, n // FP8_BLOCK, FP8_BLOCK, k // FP8_BLOCK, FP8_BLOCK)
    amax = wb.abs().amax(dim=(-3, -1))
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (wb / scale[..., :, None, :, None]).clamp(-448.0, 448.0)
    q = q.reshape(*lead, n, k).to(torch.float8_e4m3fn)
    return BlockFp8(q.contiguous(), scale.contiguous())


def moe_grouped_swiglu(x: torch.Tensor, route: RouteResult, w_gate_up,
                       w_down, h: Optional[torch.Tensor] = None,
                       y: Optional[torch.Tensor] = None, kernel: str = "auto",
                       y_dtype: torch.dtype = torch.float32,
                       workspace: Optional[torch.Tensor] = None):
    """h = silu(x Wg^T) * (x Wu^T), y = h Wd^T per segment; returns (h [rows, I], y [rows, H]).
    The weights are bf16 tensors, or BlockFp8 (fp8 e4m3fn + 128 x 128 block scales, dequantized
    in the kernel). ``kernel``: "stream" (weight-streaming kernels for decode-size segments),
    "tiled" (256 x 256 / 128 x 256 MFMA tiles for prefill-size segments, bf16 only) or "auto"
    (tiled from TILED_MIN_TOKENS tokens with bf16 weights). ``y_dtype``: fp32, or bf16 with the tiled kernels
    (half the bytes of y written and read back by the combine). ``workspace``: the tiled
    kernels' tile counters (:func:`moe_tiled_workspace`, zeroed, left zeroed by every launch);
    a fresh one per call when None. Calls that may overlap on different streams need different
    workspaces."""
    _check(x, "x", torch.bfloat16)
    if x.dim() != 2:
        raise ValueError(f"x must be [T, H], got {tuple(x.shape)}")
    T, H = x.shape
    dev = x.device
    fp8 = isinstance(w_gate_up, BlockFp8)
    if fp8 != isinstance(w_down, BlockFp8):
        raise ValueError("w_gate_up and w_down must both be bf16 or both BlockFp8")
    if fp8:
        w_gate_up.check("w_gate_up", dev)
        w_down.check("w_down", dev)
        s_gate_up, s_down = w_gate_up.scale, w_down.scale
        w_gate_up, w_down = w_gate_up.q, w_down.q
    else:
        _check(w_gate_up, "w_gate_up", torch.bfloat16, dev)
        _check(w_down, "w_down", torch.bfloat16, dev)
    if w_gate_up.dim() != 3 or w_gate_up.shape[2] != H or w_gate_up.shape[1] % 2:
        raise ValueError(f"w_gate_up must be [S, 2I, {H}], got {tuple(w_gate_up.shape)}")
    S, I2, _ = w_gate_up.shape
    I = I2 // 2
    _check_shape(w_down, "w_down", (S, H, I))
    max_segments = route.seg_expert.numel()
    E = route.expert_counts.numel()
    if S < E + (1 if route.with_shared else 0):
        raise ValueError(f"weight stack has {S} slots; routing needs {E} experts"
                         f"{' + shared' if route.with_shared else ''}")
    if route.topk_idx.shape[0] != T:
        raise ValueError(f"routing covers {route.topk_idx.shape[0]} tokens, x has {T}")
    rows = route.rows
    if h is None:
        h = torch.empty(rows, I, dtype=torch.bfloat16, device=dev)
    if kernel not in ("auto", "stream", "tiled"):
        raise ValueError(f"kernel {kernel!r}")
    tiled = not fp8 and (kernel == "tiled" or (kernel == "auto" and T >= TILED_MIN_TOKENS))
    if y_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"y_dtype {y_dtype} (fp32 or bf16)")
    if y_dtype == torch.bfloat16 and not tiled:
        raise ValueError("a bf16 y needs the tiled kernels")
    if y is None:
        y = torch.empty(rows, H, dtype=y_dtype, device=dev)
    _check(h, "h", torch.bfloat16, dev)
    _check_shape(h, "h", (rows, I))
    _check(y, "y", y_dtype, dev)
    _check_shape(y, "y", (rows, H))
    stream = _stream()
    if fp8:
        if kernel == "tiled":
            raise NotImplementedError("fp8 expert weights: only the streaming kernels")
        _timed("moe_gate_up", lambda: _lib.call(
            "sym_moe_gate_up_fp8", _ptr(x), T, H, I, _ptr(route.sorted_tokens),
            _ptr(route.seg_expert), _ptr(route.seg_offset), _ptr(route.seg_count),
            _ptr(route.n_segments), max_segments, _ptr(w_gate_up), _ptr(s_gate_up), _ptr(h),
            stream))
        _timed("moe_down", lambda: _lib.call(
            "sym_moe_down_fp8", _ptr(h), T, H, I, _ptr(route.seg_expert), _ptr(route.seg_offset),
            _ptr(route.seg_count), _ptr(route.n_segments), max_segments, _ptr(w_down),
            _ptr(s_down), _ptr(y), stream))
        return h, y
    if tiled:
        if workspace is None:
            workspace = moe_tiled_workspace(dev)
        _check(workspace, "workspace", torch.uint8, dev)
        ws, ws_bytes = _ptr(workspace), workspace.numel()
        _timed("moe_gate_up", lambda: _lib.call(
            "sym_moe_gate_up_tiled", _ptr(x), T, H, I, rows, _ptr(route.sorted_tokens),
            _ptr(route.seg_expert), _ptr(route.seg_offset), _ptr(route.seg_count),
            _ptr(route.n_segments), max_segments, _ptr(w_gate_up), _ptr(h), ws, ws_bytes,
            stream))
        _timed("moe_down", lambda: _lib.call(
            "sym_moe_down_tiled", _ptr(h), T, H, I, rows, _ptr(route.seg_expert),
            _ptr(route.seg_offset), _ptr(route.seg_count), _ptr(route.n_segments), max_segments,
            _ptr(w_down), _ptr(y), 1 if y.dtype == torch.bfloat16 else 0, ws, ws_bytes, stream))
        return h, y
    _timed("moe_gate_up", lambda: _lib.call(
        "sym_moe_gate_up", _ptr(x), T, H, I, _ptr(route.sorted_tokens), _ptr(route.seg_expert),
        _ptr(route.seg_offset), _ptr(route.seg_count), _ptr(route.n_segments), max_segments,
        _ptr(w_gate_up), _ptr(h), stream))
    _timed("moe_down", lambda: _lib.call(
        "sym_moe_down", _ptr(h), T, H, I, _ptr(route.seg_expert), _ptr(route.seg_offset),
        _ptr(route.seg_count), _ptr(route.n_segments), max_segments, _ptr(w_down), _ptr(y),
        stream))
    return h, y


def moe_unpermute_combine(y: torch.Tensor, route: RouteResult,
                          residual: Optional[torch.Tensor] = None,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[t] = sum_k w[t,k] y[inv[t,k]] (+ shared row) (+ residual[t], fp32), bf16 [T, H];
    y is fp32 or bf16."""
    if y.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"y: dtype {y.dtype} (fp32 or bf16)")
    _check(y, "y", y.dtype)
    T, K = route.topk_idx.shape
    H = y.shape[1]
    dev = y.device
    _check_shape(y, "y", (route.rows, H))
    if residual is not None:
        _check(residual, "residual", torch.float32, dev)
        _check_shape(residual, "residual", (T, H))
    if out is None:
        out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    _check(out, "out", torch.bfloat16, dev)
    _check_shape(out, "out", (T, H))
    shared_row0 = T * K if route.with_shared else -1
    _lib.call("sym_moe_unpermute_combine", _ptr(y), 1 if y.dtype == torch.bfloat16 else 0,
              _ptr(route.inv_perm), _ptr(route.topk_w), T,
              K, H, shared_row0, _ptr(residual), _ptr(out), _stream())
    return out


def hbm_read_bandwidth(nbytes: int = 1 << 30, reps: int = 10,
                       device: Optional[torch.device] = None) -> float:
    """Streaming-read bandwidth in GB/s of ``sym_hbm_read_probe`` over ``nbytes`` of HBM (HIP
    events around ``reps`` launches on the current stream, after one untimed launch)."""
    dev = device or torch.device("cuda", torch.cuda.current_device())
    nbytes -= nbytes % 16
    buf = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    run = lambda: _lib.call("sym_hbm_read_probe", _ptr(buf), nbytes, _ptr(sink), _stream())
    run()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    secs = e0.elapsed_time(e1) * 1e-3 / reps
    del buf
    return nbytes / secs / 1e9
