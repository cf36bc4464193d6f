"""HIP-backed BailingMoeV2 attention (decode over the paged KV cache).

Replaces ``TTNNBailingMoEAttention`` (ttnn_attention.py:1889-2517). ``from_torch`` reads the
same HF fields (ttnn_attention.py:1954-2042): ``config.num_attention_heads`` /
``num_key_value_heads`` / ``head_dim`` / ``partial_rotary_factor`` / ``use_qk_norm`` /
``rope_theta`` (default 600000 as the reference, ttnn_attention.py:2088) /
``max_position_embeddings``, ``query_key_value.weight|bias``, ``dense.weight|bias``,
``query_layernorm`` / ``key_layernorm``, ``layer_idx``. The Q/K rows keep HF's split-half RoPE
layout (no Meta-interleave permutation: that layout exists for TT's rotary kernel).

``forward`` routes by sequence length, as the reference (ttnn_attention.py:2480-2517):

Decode step (``seq_len == 1``; ttnn_attention.py:2308-2466):
  qkv  = x W_qkv^T (+b)                          skinny-GEMM kernel
  o    = fused decode step (split-K + merge)     QK RMSNorm, partial RoPE, paged KV write and
                                                  paged GQA decode in one pass
  out  = o W_dense^T (+b)                         skinny-GEMM kernel
Positions are per-sequence device int32 (``cache_position`` / ``position_ids`` per row); when
absent, the cache's host counter is used for every row, as in the reference
(ttnn_attention.py:2285-2287).

Prefill (``seq_len > 1``; ttnn_attention.py:2153-2230): batch row b is a prompt at positions
0 .. S-1 written into page-table row b (the reference fills batch row 0 only, 2205-2210); tiled
QKV GEMM, prefill prologue (QK-norm, RoPE, paged KV write of every token), causal varlen flash
attention, tiled dense GEMM.

The cache's host counters advance with each write (decode by 1, prefill by S) unless the caller
tracks them itself (``update_seq_length``), as the reference's paged_update_on_device /
paged_fill_on_device do (ttnn_attention.py:224-233, 259-269).
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from .. import hip_ops
from ..core.module import StatefulHIPModule
from .kv_cache import HIPPagedAttentionKVCache

_ROPE_TABLES: Dict[Tuple, torch.Tensor] = {}


def rope_table(head_dim: int, rotary_dim: int, theta: float, max_pos: int,
               device: torch.device) -> torch.Tensor:
    """[max_pos, rotary_dim] fp32 = [cos(pos*f_i) | sin(pos*f_i)], f_i = theta^-(2i/rotary_dim)
    (the HF default RoPE, hf_compat.py:83-97), shared by every layer with the same geometry."""
    key = (head_dim, rotary_dim, float(theta), int(max_pos), str(device))
    tab = _ROPE_TABLES.get(key)
    if tab is None:
        inv_freq = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.int64).float()
                                    / rotary_dim))
        pos = torch.arange(max_pos, dtype=torch.float32)
        freqs = pos[:, None] * inv_freq[None, :]
        tab = torch.cat([freqs.cos(), freqs.sin()], dim=1).contiguous().to(device)
        _ROPE_TABLES[key] = tab
    return tab


class HIPBailingMoEAttention(StatefulHIPModule):
    def __init__(self):
        super().__init__()
        self.num_heads = None
        self.num_kv_heads = None
        self.head_dim = None
        self.hidden_size = None
        self.layer_idx = 0
        self.use_qk_norm = False
        self.rotary_dim = 0
        self.rope_theta = 600000.0
        self.max_position_embeddings = 8192
        self.norm_eps = 1e-6
        self.scaling = None
        self._host = {}
        self._dev = {}

    @classmethod
    def from_torch(cls, torch_attn):
        cfg = torch_attn.config
        heads = cfg.num_attention_heads
        head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // heads
        qkv = torch_attn.query_key_value
        use_qk_norm = bool(getattr(cfg, "use_qk_norm", False))
        eps = getattr(cfg, "rms_norm_eps", 1e-6)
        if use_qk_norm:
            eps = getattr(torch_attn.query_layernorm, "variance_epsilon", eps)
        new = cls.from_weights(
            num_heads=heads, num_kv_heads=cfg.num_key_value_heads, head_dim=head_dim,
            hidden_size=cfg.hidden_size, layer_idx=getattr(torch_attn, "layer_idx", 0),
            qkv_weight=qkv.weight, qkv_bias=qkv.bias, dense_weight=torch_attn.dense.weight,
            dense_bias=torch_attn.dense.bias,
            q_norm_weight=torch_attn.query_layernorm.weight if use_qk_norm else None,
            k_norm_weight=torch_attn.key_layernorm.weight if use_qk_norm else None,
            partial_rotary_factor=getattr(cfg, "partial_rotary_factor", 1.0),
            rope_theta=getattr(cfg, "rope_theta", 600000.0),
            max_position_embeddings=getattr(cfg, "max_position_embeddings", 8192), norm_eps=eps)
        new._fallback_torch_layer = torch_attn
        return new

    @classmethod
    def from_weights(cls, *, num_heads, num_kv_heads, head_dim, hidden_size, qkv_weight,
                     dense_weight, qkv_bias=None, dense_bias=None, q_norm_weight=None,
                     k_norm_weight=None, partial_rotary_factor=1.0, rope_theta=600000.0,
                     max_position_embeddings=8192, norm_eps=1e-6, layer_idx=0):
        if head_dim != hip_ops.HEAD_DIM:
            raise NotImplementedError(f"head_dim {head_dim} (kernels implement {hip_ops.HEAD_DIM})")
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads {num_heads} not a multiple of num_kv_heads {num_kv_heads}")
        if (q_norm_weight is None) != (k_norm_weight is None):
            raise ValueError("q_norm_weight and k_norm_weight must be given together")
        new = cls()
        new.num_heads = num_heads
        new.num_kv_heads = num_kv_heads
        new.head_dim = head_dim
        new.hidden_size = hidden_size
        new.layer_idx = int(layer_idx)
        new.use_qk_norm = q_norm_weight is not None
        new.rotary_dim = int(head_dim * partial_rotary_factor)
        new.rope_theta = float(rope_theta)
        new.max_position_embeddings = int(max_position_embeddings)
        new.norm_eps = float(norm_eps)
        new.scaling = head_dim ** -0.5
        rows = (num_heads + 2 * num_kv_heads) * head_dim
        if tuple(qkv_weight.shape) != (rows, hidden_size):
            raise ValueError(f"qkv weight {tuple(qkv_weight.shape)}, expected {(rows, hidden_size)}")
        if tuple(dense_weight.shape) != (hidden_size, num_heads * head_dim):
            raise ValueError(f"dense weight {tuple(dense_weight.shape)}")
        new._host = dict(qkv_w=qkv_weight, qkv_b=qkv_bias, dense_w=dense_weight,
                         dense_b=dense_bias, q_norm=q_norm_weight, k_norm=k_norm_weight)
        return new

    def preprocess_weights_impl(self):
        bf = torch.bfloat16
        self._host = {k: (None if v is None else v.detach().to(bf).contiguous())
                      for k, v in self._host.items()}
        return super().preprocess_weights_impl()

    def move_weights_to_device_impl(self):
        dev = self.device
        self._dev = {k: (None if v is None else v.to(dev)) for k, v in self._host.items()}
        self._dev["rope"] = (rope_table(self.head_dim, self.rotary_dim, self.rope_theta,
                                        self.max_position_embeddings, dev)
                             if self.rotary_dim else None)
        self._host = {}
        return super().move_weights_to_device_impl()

    def deallocate_weights_impl(self):
        self._dev = {}
        return super().deallocate_weights_impl()

    def reset_trace_state(self):
        # The KV write position comes from the device positions tensor of each call, so a
        # captured decode step writes exactly one slot per replay; no host state to roll back.
        return None

    # ------------------------------------------------------------------
    def _positions(self, cache: HIPPagedAttentionKVCache, cache_position, position_ids,
                   batch: int) -> torch.Tensor:
        pos = cache_position if cache_position is not None else position_ids
        if pos is None:
            pos = torch.full((batch,), cache.get_seq_length(self.layer_idx), dtype=torch.int32)
        if not isinstance(pos, torch.Tensor):
            pos = torch.as_tensor(pos)
        pos = pos.reshape(-1)
        if pos.numel() != batch:
            if pos.numel() == 1:
                pos = pos.expand(batch)
            else:
                pos = pos.reshape(batch, -1)[:, -1]
        if pos.dtype != torch.int32 or pos.device != self.device:
            pos = pos.to(device=self.device, dtype=torch.int32)
        return pos.contiguous()

    @staticmethod
    def _cache_of(past_key_values, past_key_value) -> HIPPagedAttentionKVCache:
        cache = past_key_values if past_key_values is not None else past_key_value
        if not isinstance(cache, HIPPagedAttentionKVCache):
            raise NotImplementedError(
                "HIPBailingMoEAttention needs the paged KV cache (model._tt_kv_cache) as "
                "past_key_values")
        return cache

    def qkv_projection(self, x: torch.Tensor, norm_weight: Optional[torch.Tensor] = None,
                       norm_eps: float = 1e-6) -> torch.Tensor:
        """qkv [B, (Hq+2Hkv)*D] of x [B, H] (bf16); with ``norm_weight`` the preceding RMSNorm
        (the decoder layer's input_layernorm) runs inside the projection kernel."""
        d = self._dev
        if norm_weight is None:
            return hip_ops.linear(x, d["qkv_w"], d["qkv_b"])
        return hip_ops.rmsnorm_linear(x, norm_weight, norm_eps, d["qkv_w"], d["qkv_b"])

    def decode_from_qkv(self, qkv: torch.Tensor, cache: HIPPagedAttentionKVCache,
                        cache_position=None, position_ids=None) -> torch.Tensor:
        """QK-norm, RoPE, KV write and paged decode of one token per sequence: the attention
        output [B, Hq*D] (bf16) before the dense projection."""
        d = self._dev
        B = qkv.shape[0]
        pos = self._positions(cache, cache_position, position_ids, B)
        o = hip_ops.attn_decode_step(
            qkv, pos, cache.key_cache(self.layer_idx), cache.value_cache(self.layer_idx),
            cache.page_table_device, self.scaling, num_heads=self.num_heads,
            num_kv_heads=self.num_kv_heads, rotary_dim=self.rotary_dim, rope_cs=d["rope"],
            q_norm_w=d["q_norm"], k_norm_w=d["k_norm"], eps=self.norm_eps,
            max_context=cache.max_context, workspace=cache.decode_workspace(B, self.num_heads),
            k_scale=cache.key_scale(self.layer_idx), v_scale=cache.value_scale(self.layer_idx))
        cache.advance(self.layer_idx, 1)
        return o.view(B, self.num_heads * self.head_dim)

    def dense_residual(self, o: torch.Tensor, residual: torch.Tensor):
        """h = residual + o W_dense^T (+b) in fp32 [B, H], and the per-16-column sums of squares
        of h's rows (the statistics of the post-attention RMSNorm)."""
        d = self._dev
        return hip_ops.linear_residual(o, d["dense_w"], residual, d["dense_b"])

    def prefill_varlen(self, x: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                       positions: torch.Tensor, seq_ids: torch.Tensor,
                       cache: HIPPagedAttentionKVCache,
                       out_dtype: torch.dtype = torch.bfloat16,
                       residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Prefill of packed sequences: x [T, H] (bf16, already normalised by the layer), token
        t of sequence seq_ids[t] at positions[t] (0 .. L-1; page-table row seq_ids[t]). Writes
        the sequences' K/V into the paged cache and returns the attention output after the
        dense projection, [T, H] in ``out_dtype`` (bf16, or fp32 for a caller that adds the
        residual in fp32). With ``residual`` (bf16 [T, H]) the output is fp32 and already holds
        it, added in fp32 in the projection's epilogue. The host counters are not advanced here
        (the forward methods do).
        With an fp8 cache the K/V are appended per block after the prologue, at the page-table
        row and start position of each sequence's first token."""
        d = self._dev
        T = x.shape[0]
        qkv = hip_ops.gemm(x, d["qkv_w"], d["qkv_b"])
        q, k, v = hip_ops.attn_prefill_prologue(
            qkv, positions, seq_ids, cache.key_cache(self.layer_idx),
            cache.value_cache(self.layer_idx), cache.page_table_device,
            num_heads=self.num_heads, num_kv_heads=self.num_kv_heads,
            rotary_dim=self.rotary_dim, rope_cs=d["rope"], q_norm_w=d["q_norm"],
            k_norm_w=d["k_norm"], eps=self.norm_eps)
        if cache.is_fp8 and T > 0:
            first = cu_seqlens[:-1].long().clamp(max=T - 1)
            hip_ops.paged_kv_fill_fp8(
                k, v, cu_seqlens, max_seqlen, cache.key_cache(self.layer_idx),
                cache.value_cache(self.layer_idx), cache.key_scale(self.layer_idx),
                cache.value_scale(self.layer_idx), cache.page_table_device,
                start_pos=positions[first].contiguous(), seq_rows=seq_ids[first].contiguous())
        o = hip_ops.prefill_attention(q, k, v, cu_seqlens, max_seqlen, self.scaling)
        if residual is not None:
            return hip_ops.gemm(o.view(-1, self.num_heads * self.head_dim), d["dense_w"],
                                d["dense_b"], residual=residual, out_dtype=torch.float32)
        return hip_ops.gemm(o.view(-1, self.num_heads * self.head_dim), d["dense_w"],
                            d["dense_b"], out_dtype=out_dtype)

    def prefill_rows(self, x: torch.Tensor, cache: HIPPagedAttentionKVCache,
                     cache_position=None, position_ids=None) -> torch.Tensor:
        """Prefill of B equal-length prompts x [B, S, H] (bf16): row b at positions 0 .. S-1 of
        page-table row b. Returns [B, S, H] bf16 and advances the counters by S."""
        B, S, H = x.shape
        if B > cache.page_table.shape[0]:
            raise ValueError(f"{B} prompts for a page table of {cache.page_table.shape[0]} rows")
        pos = cache_position if cache_position is not None else position_ids
        if prefill_continues(cache, self.layer_idx, pos):
            raise NotImplementedError(
                "prefill starting at a cached position (a prompt continuing earlier tokens); "
                "as the reference's prefill, prompts start at position 0")
        positions, seq_ids, cu = equal_length_packing(B, S, x.device)
        out = self.prefill_varlen(x.reshape(B * S, H).contiguous(), cu, S, positions, seq_ids,
                                  cache)
        cache.advance(self.layer_idx, S)
        return out.view(B, S, H)

    def forward(self, hidden_states: torch.Tensor, position_embeddings=None,
                attention_mask=None, past_key_values=None, past_key_value=None,
                cache_position=None, position_ids=None, **kwargs):
        cache = self._cache_of(past_key_values, past_key_value)
        B, S, H = hidden_states.shape
        x = hidden_states
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        if S != 1:
            return self.prefill_rows(x, cache, cache_position, position_ids), None, cache
        d = self._dev
        qkv = self.qkv_projection(x.reshape(B, H).contiguous())
        o = self.decode_from_qkv(qkv, cache, cache_position, position_ids)
        out = hip_ops.linear(o, d["dense_w"], d["dense_b"])
        return out.view(B, 1, H), None, cache


def prefill_continues(cache: HIPPagedAttentionKVCache, layer_idx: int, pos) -> bool:
    """True when a prefill would continue a cached sequence instead of starting at position 0:
    the layer's host counter is past 0 (checked without a device sync, whatever device the
    positions are on), or host-side positions start past 0."""
    if cache.get_seq_length(layer_idx) != 0:
        return True
    return (isinstance(pos, torch.Tensor) and pos.device.type == "cpu" and pos.numel() > 0
            and int(pos.reshape(-1)[0]) != 0)


def equal_length_packing(B: int, S: int, device):
    """(positions [B*S], seq_ids [B*S], cu_seqlens [B+1]) int32 on ``device`` for B prompts of S
    tokens packed row after row (prompt b = page-table row b, positions 0 .. S-1), built on the
    device without a host round trip."""
    i32 = dict(dtype=torch.int32, device=device)
    positions = torch.arange(S, **i32).repeat(B)
    seq_ids = torch.arange(B, **i32).repeat_interleave(S)
    cu = torch.arange(0, B * S + 1, S, **i32)
    return positions, seq_ids, cu


def varlen_packing(cu_seqlens: torch.Tensor, T: int):
    """(positions [T], seq_ids [T]) int32 of packed sequences (sequence s = rows cu_seqlens[s]
    .. cu_seqlens[s+1]-1 at positions 0 .. L-1, page-table row s), on cu_seqlens' device
    without a host round trip."""
    cu = cu_seqlens.to(torch.int32).contiguous()
    t = torch.arange(T, dtype=torch.int32, device=cu.device)
    seq_ids = torch.searchsorted(cu[1:].contiguous(), t, right=True).to(torch.int32)
    positions = (t - cu[seq_ids.long()]).to(torch.int32)
    return positions.contiguous(), seq_ids.contiguous()
