"""HIP-backed BailingMoeV2 attention (decode over the paged KV cache).

Replaces ``TTNNBailingMoEAttention`` (ttnn_attention.py:1889-2517). ``from_torch`` reads the
same HF fields (ttnn_attention.py:1954-2042): ``config.num_attention_heads`` /
``num_key_value_heads`` / ``head_dim`` / ``partial_rotary_factor`` / ``use_qk_norm`` /
``rope_theta`` (default 600000 as the reference, ttnn_attention.py:2088) /
``max_position_embeddings``, ``query_key_value.weight|bias``, ``dense.weight|bias``,
``query_layernorm`` / ``key_layernorm``, ``layer_idx``. The Q/K rows keep HF's split-half RoPE
layout (no Meta-interleave permutation: that layout exists for TT's rotary kernel).

Decode step (``seq_len == 1`` with a paged cache; ttnn_attention.py:2308-2466):
  qkv  = x W_qkv^T (+b)                          skinny-GEMM kernel
  o    = fused decode step (split-K + merge)     QK RMSNorm, partial RoPE, paged KV write and
                                                  paged GQA decode in one pass
  out  = o W_dense^T (+b)                         skinny-GEMM kernel
Positions are per-sequence device int32 (``cache_position`` / ``position_ids`` per row); when
absent, the cache's host counter is used for every row, as in the reference.
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
        return o.view(B, self.num_heads * self.head_dim)

    def dense_residual(self, o: torch.Tensor, residual: torch.Tensor):
        """h = residual + o W_dense^T (+b) in fp32 [B, H], and the per-16-column sums of squares
        of h's rows (the statistics of the post-attention RMSNorm)."""
        d = self._dev
        return hip_ops.linear_residual(o, d["dense_w"], residual, d["dense_b"])

    def prefill_varlen(self, x: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                       positions: torch.Tensor, seq_ids: torch.Tensor,
                       cache: HIPPagedAttentionKVCache) -> torch.Tensor:
        """Prefill of packed sequences: x [T, H] (bf16, already normalised by the layer), token
        t of sequence seq_ids[t] at positions[t] (0 .. L-1). Writes the sequences' K/V into the
        paged cache (page-table row = sequence) and returns the attention output after the
        dense projection, [T, H] bf16. With an fp8 cache the sequences start at position 0 and
        sequence s uses page-table row s (the K/V are appended per block after the prologue)."""
        d = self._dev
        qkv = hip_ops.gemm(x, d["qkv_w"], d["qkv_b"])
        q, k, v = hip_ops.attn_prefill_prologue(
            qkv, positions, seq_ids, cache.key_cache(self.layer_idx),
            cache.value_cache(self.layer_idx), cache.page_table_device,
            num_heads=self.num_heads, num_kv_heads=self.num_kv_heads,
            rotary_dim=self.rotary_dim, rope_cs=d["rope"], q_norm_w=d["q_norm"],
            k_norm_w=d["k_norm"], eps=self.norm_eps)
        if cache.is_fp8:
            hip_ops.paged_kv_fill_fp8(
                k, v, cu_seqlens, max_seqlen, cache.key_cache(self.layer_idx),
                cache.value_cache(self.layer_idx), cache.key_scale(self.layer_idx),
                cache.value_scale(self.layer_idx), cache.page_table_device)
        o = hip_ops.prefill_attention(q, k, v, cu_seqlens, max_seqlen, self.scaling)
        return hip_ops.gemm(o.view(-1, self.num_heads * self.head_dim), d["dense_w"],
                            d["dense_b"])

    def forward(self, hidden_states: torch.Tensor, position_embeddings=None,
                attention_mask=None, past_key_values=None, past_key_value=None,
                cache_position=None, position_ids=None, **kwargs):
        cache = self._cache_of(past_key_values, past_key_value)
        B, S, H = hidden_states.shape
        if S != 1:
            raise NotImplementedError("prefill (seq_len > 1) is not implemented on the HIP path")
        d = self._dev
        x = hidden_states.reshape(B, H)
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        qkv = self.qkv_projection(x.contiguous())
        o = self.decode_from_qkv(qkv, cache, cache_position, position_ids)
        out = hip_ops.linear(o, d["dense_w"], d["dense_b"])
        return out.view(B, 1, H), None, cache
