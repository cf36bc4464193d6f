"""HIP-backed BailingMoeV2 decoder layer (the caller of the attention and MoE modules).

Replaces ``TTNNBailingMoEDecoderLayer`` (modeling_bailing_moe_v2.py:345-483): ``from_torch``
wraps ``input_layernorm`` / ``post_attention_layernorm``, converts ``attention`` and picks the
MoE block or the dense MLP by ``first_k_dense_replace`` (modeling_bailing_moe_v2.py:374-401).
Forward keeps the reference's residual structure
  h1  = x + attention(rmsnorm(x))
  out = h1 + mlp(rmsnorm(h1))
with the norms and residual adds fused into the kernels (MoE layers): the QKV projection applies
the input RMSNorm, the dense projection adds x and emits h1 = x + attn in fp32 with its rows'
sums of squares (the residual stream inside the layer is never rounded), the router-logits
kernel applies the post-attention RMSNorm, and the MoE
combine kernel adds h1 into its output, which is rounded to bf16 once.
"""
from __future__ import annotations

import torch

from .. import hip_ops
from ..core.module import StatefulHIPModule
from .attention import HIPBailingMoEAttention, equal_length_packing, prefill_continues, \
    varlen_packing
from .moe import HIPBailingMoE, HIPBailingMoeV2MLP


def _is_sparse_moe(mlp) -> bool:
    return hasattr(mlp, "experts") and hasattr(mlp, "gate")


class HIPBailingMoEDecoderLayer(StatefulHIPModule):
    def __init__(self):
        super().__init__()
        self.attention = None
        self.mlp = None
        self.is_dense_layer = False
        self.hidden_size = None
        self.eps = 1e-6
        self._host = {}
        self._dev = {}

    @classmethod
    def from_torch(cls, torch_layer):
        new = cls()
        new._fallback_torch_layer = torch_layer
        ln1, ln2 = torch_layer.input_layernorm, torch_layer.post_attention_layernorm
        new.hidden_size = ln1.weight.shape[0]
        new.eps = float(getattr(ln1, "variance_epsilon", getattr(ln1, "eps", 1e-6)))
        new._host = dict(ln1=ln1.weight, ln2=ln2.weight)
        attn = torch_layer.attention
        new.attention = (attn if isinstance(attn, HIPBailingMoEAttention)
                         else HIPBailingMoEAttention.from_torch(attn))
        mlp = torch_layer.mlp
        if isinstance(mlp, (HIPBailingMoE, HIPBailingMoeV2MLP)):
            new.mlp = mlp
        elif _is_sparse_moe(mlp):
            new.mlp = HIPBailingMoE.from_torch(mlp)
        else:
            new.mlp = HIPBailingMoeV2MLP.from_torch(mlp)
        new.is_dense_layer = isinstance(new.mlp, HIPBailingMoeV2MLP)
        return new

    @classmethod
    def from_modules(cls, attention: HIPBailingMoEAttention, mlp, input_layernorm_weight,
                     post_attention_layernorm_weight, eps: float = 1e-6):
        new = cls()
        new.attention = attention
        new.mlp = mlp
        new.is_dense_layer = isinstance(mlp, HIPBailingMoeV2MLP)
        new.hidden_size = input_layernorm_weight.shape[0]
        new.eps = float(eps)
        new._host = dict(ln1=input_layernorm_weight, ln2=post_attention_layernorm_weight)
        return new

    def preprocess_weights_impl(self):
        self._host = {k: v.detach().to(torch.bfloat16).contiguous() for k, v in self._host.items()}
        return super().preprocess_weights_impl()

    def move_weights_to_device_impl(self):
        self._dev = {k: v.to(self.device) for k, v in self._host.items()}
        self._host = {}
        return super().move_weights_to_device_impl()

    def prefill_varlen(self, x: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                       cache, positions: torch.Tensor = None,
                       seq_ids: torch.Tensor = None) -> torch.Tensor:
        """Prefill of packed sequences x [T, H] (bf16), sequence s = rows cu_seqlens[s] ..
        cu_seqlens[s+1]-1 at positions 0 .. L-1 (page-table row s of the cache, unless
        ``positions`` / ``seq_ids`` say otherwise per token). Returns the layer output [T, H]
        (bf16); the sequences' K/V are written into the paged cache. The host counters are not
        advanced here (:meth:`forward` does)."""
        x = x.to(torch.bfloat16).contiguous()
        T, H = x.shape
        if positions is None or seq_ids is None:
            positions, seq_ids = varlen_packing(cu_seqlens.to(x.device), T)
        positions = positions.to(device=x.device, dtype=torch.int32).contiguous()
        seq_ids = seq_ids.to(device=x.device, dtype=torch.int32).contiguous()
        xn = hip_ops.rmsnorm(x, self._dev["ln1"], self.eps)
        # the residual joins the dense projection's fp32 accumulator in its epilogue (one
        # rounding less than a bf16 output, and no separate pass over the fp32 rows)
        h1 = self.attention.prefill_varlen(xn, cu_seqlens, max_seqlen, positions, seq_ids,
                                           cache, residual=x)
        xn2 = hip_ops.rmsnorm(h1, self._dev["ln2"], self.eps)
        return self.mlp(xn2, residual=h1)

    def reset_trace_state(self):
        # The only persistent mutation of a decode step is the KV-slot write of the child
        # attention, which handles its own state; this layer keeps none between calls.
        return None

    def forward(self, hidden_states, attention_mask=None, position_ids=None,
                past_key_value=None, output_attentions=False, output_router_logits=False,
                use_cache=False, position_embeddings=None, cache_position=None,
                past_key_values=None, **kwargs):
        cache = past_key_values if past_key_values is not None else past_key_value
        x = hidden_states
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        attn = self.attention
        if x.dim() == 2:
            x = x.unsqueeze(1)
        x = x.contiguous()
        B, S, H = x.shape
        if S != 1:
            # equal-length prompts, positions 0 .. S-1 of page-table rows 0 .. B-1
            kv = attn._cache_of(cache, None)
            pos = cache_position if cache_position is not None else position_ids
            if prefill_continues(kv, attn.layer_idx, pos):
                raise NotImplementedError(
                    "prefill starting at a cached position (a prompt continuing earlier "
                    "tokens); as the reference's prefill, prompts start at position 0")
            positions, seq_ids, cu = equal_length_packing(B, S, x.device)
            out = self.prefill_varlen(x.view(B * S, H), cu, S, kv, positions=positions,
                                      seq_ids=seq_ids)
            kv.advance(attn.layer_idx, S)
            outputs = (out.view(B, S, H),)
            if output_attentions:
                outputs += (None,)
            if use_cache:
                outputs += (cache,)
            if output_router_logits:
                outputs += (None,)
            return outputs
        if self.is_dense_layer:
            # the attention half as in the MoE layers (input RMSNorm inside the QKV projection,
            # the residual added in fp32 inside the dense projection); the post-attention
            # RMSNorm then reads the fp32 residual stream
            x2 = x.view(B, H)
            qkv = attn.qkv_projection(x2, self._dev["ln1"], self.eps)
            o = attn.decode_from_qkv(qkv, attn._cache_of(cache, None), cache_position,
                                     position_ids)
            h1, _ = attn.dense_residual(o, x2)
            xn2 = hip_ops.rmsnorm(h1, self._dev["ln2"], self.eps)
            out = self.mlp(xn2, residual=h1).view(B, S, H)
        else:
            # input RMSNorm inside the QKV projection; residual add and the post-attention
            # RMSNorm's statistics inside the dense projection; that RMSNorm itself inside the
            # router-logits kernel
            x2 = x.view(B, H)
            qkv = attn.qkv_projection(x2, self._dev["ln1"], self.eps)
            o = attn.decode_from_qkv(qkv, attn._cache_of(cache, None), cache_position,
                                     position_ids)
            h1, ss = attn.dense_residual(o, x2)
            out = self.mlp.forward_from_residual(h1, ss, self._dev["ln2"], self.eps)
            out = out.view(B, S, H)
        outputs = (out,)
        if output_attentions:
            outputs += (None,)
        if use_cache:
            outputs += (cache,)
        if output_router_logits:
            outputs += (None,)
        return outputs
