"""CPU restatement of the BailingMoeV2 (Ling-mini-2.0) modules -- the parity oracle.

TEST INFRASTRUCTURE ONLY. The HF ``BailingMoeV2*`` classes the reference swaps are Hub remote
code (``inclusionAI/Ling-mini-2.0``, trust_remote_code) that is neither in the reference tree nor
in the installed transformers, so this file restates them from the reference's own code:

* class and attribute names are the ones the reference reads (``query_key_value``, ``dense``,
  ``query_layernorm``, ``key_layernorm``, ``gate.weight``, ``gate.expert_bias``, ``experts[i]
  .gate_proj/up_proj/down_proj``, ``shared_experts``, ``input_layernorm``,
  ``post_attention_layernorm``; ttnn_attention.py:1954-2042, ttnn_moe.py:1497-1647,
  modeling_bailing_moe_v2.py:374-401), so recipes keyed on them swap these modules;
* RMSNorm: DeepseekV2RMSNorm (ttnn_normalization.py:54-68);
* RoPE: default inv_freq over rotary_dim = head_dim * partial_rotary_factor
  (hf_compat.py:83-97) and the split-half partial rotary of TorchRotaryPositionEmbedding
  (ttnn_rope.py:23-62);
* attention order qkv -> split -> qk-norm -> rope -> cache write -> SDPA -> dense
  (ttnn_attention.py:2153-2230, 2308-2466), scale head_dim^-0.5 (ttnn_attention.py:1973);
* router: Glm4MoeRouteTokenToExperts (ttnn_moe.py:413-436) on fp32 logits, norm_topk_prob True
  (ttnn_moe.py:1532), via :func:`oracle.route.route_torch`;
* experts: Glm4MoeNaiveMoe (ttnn_moe.py:313-352) loop with index_add; shared expert added on the
  MoE input (ttnn_moe.py:1487-1490);
* decoder layer residual structure (modeling_bailing_moe_v2.py:417-483).

Choices the reference cannot pin (stated, see also the fixture metadata): router logits in fp32;
dropped groups masked with 0.0 (the torch form, ttnn_moe.py:429); ``+1e-20`` in the normaliser;
ties to the lower index.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

from .paged_kv import PagedKVCacheRef
from .route import route_torch


class BailingMoeV2Config:
    """The configuration fields the hot path reads (Ling-mini-2.0 values as defaults,
    tests/experimental/bailing_moe_v2/shapes.json)."""

    model_type = "bailing_moe_v2"

    def __init__(self, hidden_size=2048, intermediate_size=5120, moe_intermediate_size=512,
                 num_attention_heads=16, num_key_value_heads=4, head_dim=128, num_experts=256,
                 num_experts_per_tok=8, num_shared_experts=1, n_group=8, topk_group=4,
                 routed_scaling_factor=2.5, norm_topk_prob=True, first_k_dense_replace=1,
                 num_hidden_layers=20, rms_norm_eps=1e-6, rope_theta=1e6,
                 partial_rotary_factor=0.5, use_qk_norm=True, use_qkv_bias=False, use_bias=False,
                 vocab_size=157184, max_position_embeddings=32768, hidden_act="silu",
                 initializer_range=0.02, num_nextn_predict_layers=0, **kwargs):
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.moe_intermediate_size = moe_intermediate_size
        self.num_attention_heads = num_attention_heads
        self.num_key_value_heads = num_key_value_heads
        self.head_dim = head_dim
        self.num_experts = num_experts
        self.num_experts_per_tok = num_experts_per_tok
        self.num_shared_experts = num_shared_experts
        self.n_group = n_group
        self.topk_group = topk_group
        self.routed_scaling_factor = routed_scaling_factor
        self.norm_topk_prob = norm_topk_prob
        self.first_k_dense_replace = first_k_dense_replace
        self.num_hidden_layers = num_hidden_layers
        self.rms_norm_eps = rms_norm_eps
        self.rope_theta = rope_theta
        self.partial_rotary_factor = partial_rotary_factor
        self.use_qk_norm = use_qk_norm
        self.use_qkv_bias = use_qkv_bias
        self.use_bias = use_bias
        self.vocab_size = vocab_size
        self.max_position_embeddings = max_position_embeddings
        self.hidden_act = hidden_act
        self.initializer_range = initializer_range
        self.num_nextn_predict_layers = num_nextn_predict_layers
        for k, v in kwargs.items():
            setattr(self, k, v)


class BailingMoeV2RMSNorm(nn.Module):
    def __init__(self, hidden_size, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, hidden_states):
        input_dtype = hidden_states.dtype
        hidden_states = hidden_states.to(torch.float32)
        variance = hidden_states.pow(2).mean(-1, keepdim=True)
        hidden_states = hidden_states * torch.rsqrt(variance + self.variance_epsilon)
        return self.weight * hidden_states.to(input_dtype)


def rope_inv_freq(head_dim: int, partial_rotary_factor: float, theta: float) -> torch.Tensor:
    dim = int(head_dim * partial_rotary_factor)
    return 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.int64).float() / dim))


class BailingMoeV2RotaryEmbedding(nn.Module):
    def __init__(self, config: BailingMoeV2Config):
        super().__init__()
        self.register_buffer(
            "inv_freq",
            rope_inv_freq(config.head_dim, getattr(config, "partial_rotary_factor", 1.0),
                          getattr(config, "rope_theta", 600000.0)),
            persistent=False)

    @torch.no_grad()
    def forward(self, x, position_ids):
        pos = position_ids.to(torch.float32)                       # [B, S]
        freqs = pos[..., None] * self.inv_freq.float()[None, None]  # [B, S, rd/2]
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


def rotate_half(x):
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_partial_rotary(q, k, cos, sin, unsqueeze_dim=1):
    """q, k [B, H, S, D]; cos, sin [B, S, rotary_dim]; rotary on the first rotary_dim dims."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    rd = cos.shape[-1]
    q_rot, q_pass = q[..., :rd], q[..., rd:]
    k_rot, k_pass = k[..., :rd], k[..., rd:]
    q_embed = (q_rot * cos) + (rotate_half(q_rot) * sin)
    k_embed = (k_rot * cos) + (rotate_half(k_rot) * sin)
    return torch.cat([q_embed, q_pass], dim=-1), torch.cat([k_embed, k_pass], dim=-1)


class BailingMoeV2MLP(nn.Module):
    def __init__(self, config: BailingMoeV2Config, intermediate_size: int):
        super().__init__()
        self.config = config
        self.hidden_size = config.hidden_size
        self.intermediate_size = intermediate_size
        self.gate_proj = nn.Linear(self.hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(self.hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, self.hidden_size, bias=False)
        self.act_fn = nn.SiLU()

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


class BailingMoeV2Gate(nn.Module):
    def __init__(self, config: BailingMoeV2Config):
        super().__init__()
        self.config = config
        self.top_k = config.num_experts_per_tok
        self.num_experts = config.num_experts
        self.n_group = config.n_group
        self.topk_group = config.topk_group
        self.routed_scaling_factor = config.routed_scaling_factor
        self.weight = nn.Parameter(torch.empty(self.num_experts, config.hidden_size))
        self.register_buffer("expert_bias", torch.zeros(self.num_experts, dtype=torch.float32))

    def forward(self, hidden_states):
        x = hidden_states.reshape(-1, hidden_states.shape[-1])
        logits = F.linear(x.float(), self.weight.float())
        topk_idx, topk_weight = route_torch(
            logits, self.expert_bias.float(), n_group=self.n_group, topk_group=self.topk_group,
            top_k=self.top_k, routed_scale=self.routed_scaling_factor, renormalize=True)
        override = getattr(self, "route_override", None)
        if override is not None:
            # test hook: evaluate the block with a given expert choice per token (weights from
            # this gate's own sigmoid scores)
            topk_idx = override.to(torch.int64).reshape(topk_idx.shape)
            w = torch.sigmoid(logits).gather(1, topk_idx)
            topk_weight = w / (w.sum(-1, keepdim=True) + 1e-20) * self.routed_scaling_factor
        self.last_routing = (logits.detach(), topk_idx, topk_weight.detach())
        return topk_idx, topk_weight, logits


class BailingMoeV2SparseMoeBlock(nn.Module):
    def __init__(self, config: BailingMoeV2Config):
        super().__init__()
        self.config = config
        self.num_experts_per_tok = config.num_experts_per_tok
        self.experts = nn.ModuleList(
            [BailingMoeV2MLP(config, config.moe_intermediate_size) for _ in range(config.num_experts)])
        self.gate = BailingMoeV2Gate(config)
        self.shared_experts = None
        if config.num_shared_experts:
            self.shared_experts = BailingMoeV2MLP(
                config, config.moe_intermediate_size * config.num_shared_experts)

    def forward(self, hidden_states):
        identity = hidden_states
        shape = hidden_states.shape
        topk_idx, topk_weight, router_logits = self.gate(hidden_states)
        x = hidden_states.reshape(-1, shape[-1])
        y = torch.zeros_like(x)
        for e in torch.unique(topk_idx).tolist():
            tok, kpos = torch.where(topk_idx == e)
            out = self.experts[e](x[tok]) * topk_weight[tok, kpos, None]
            y.index_add_(0, tok, out.to(y.dtype))
        y = y.view(shape)
        if self.shared_experts is not None:
            y = y + self.shared_experts(identity)
        return y, router_logits


class BailingMoeV2Attention(nn.Module):
    def __init__(self, config: BailingMoeV2Config, layer_idx: int = 0):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.num_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.hidden_size = config.hidden_size
        self.query_key_value = nn.Linear(
            self.hidden_size, (self.num_heads + 2 * self.num_key_value_heads) * self.head_dim,
            bias=config.use_qkv_bias)
        self.dense = nn.Linear(self.num_heads * self.head_dim, self.hidden_size, bias=config.use_bias)
        if config.use_qk_norm:
            self.query_layernorm = BailingMoeV2RMSNorm(self.head_dim, eps=config.rms_norm_eps)
            self.key_layernorm = BailingMoeV2RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.rotary_emb = BailingMoeV2RotaryEmbedding(config)
        self.scaling = self.head_dim ** -0.5

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                past_key_value=None, past_key_values=None, cache_position=None,
                position_ids=None, **kwargs):
        cache = past_key_values if past_key_values is not None else past_key_value
        B, S, _ = hidden_states.shape
        Hq, Hkv, D = self.num_heads, self.num_key_value_heads, self.head_dim
        qkv = self.query_key_value(hidden_states).view(B, S, Hq + 2 * Hkv, D)
        q = qkv[:, :, :Hq].transpose(1, 2)
        k = qkv[:, :, Hq:Hq + Hkv].transpose(1, 2)
        v = qkv[:, :, Hq + Hkv:].transpose(1, 2)
        if self.config.use_qk_norm:
            q = self.query_layernorm(q)
            k = self.key_layernorm(k)
        pos = cache_position if cache_position is not None else position_ids
        if pos is None:
            pos = torch.arange(S).expand(B, S)
        pos = torch.as_tensor(pos).to(torch.int64)
        if pos.dim() == 1:
            pos = pos.view(B, S) if pos.numel() == B * S else pos.view(1, S).expand(B, S)
        if position_embeddings is None:
            position_embeddings = self.rotary_emb(v, pos)
        cos, sin = position_embeddings
        q, k = apply_partial_rotary(q, k, cos, sin)

        out = torch.empty(B, Hq, S, D, dtype=q.dtype)
        group = Hq // Hkv
        if isinstance(cache, PagedKVCacheRef):
            for s in range(S):
                cache.write(self.layer_idx, pos[:, s], k[:, :, s], v[:, :, s])
            for b in range(B):
                n = int(pos[b].max()) + 1
                kb, vb = cache.gather(self.layer_idx, b, n)
                kb = kb.to(q.dtype).repeat_interleave(group, dim=0)
                vb = vb.to(q.dtype).repeat_interleave(group, dim=0)
                mask = torch.arange(n)[None, :] <= pos[b][:, None]   # [S, n]
                out[b] = F.scaled_dot_product_attention(
                    q[b:b + 1], kb[None], vb[None], attn_mask=mask[None, None],
                    scale=self.scaling)[0]
        else:
            kk = k.repeat_interleave(group, dim=1)
            vv = v.repeat_interleave(group, dim=1)
            out = F.scaled_dot_product_attention(q, kk, vv, is_causal=S > 1, scale=self.scaling)
        out = out.transpose(1, 2).reshape(B, S, Hq * D)
        return self.dense(out), None, cache


class BailingMoeV2DecoderLayer(nn.Module):
    def __init__(self, config: BailingMoeV2Config, layer_idx: int):
        super().__init__()
        self.hidden_size = config.hidden_size
        self.attention = BailingMoeV2Attention(config, layer_idx)
        dense = config.num_experts is None or layer_idx < config.first_k_dense_replace
        self.mlp = (BailingMoeV2MLP(config, config.intermediate_size) if dense
                    else BailingMoeV2SparseMoeBlock(config))
        self.input_layernorm = BailingMoeV2RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = BailingMoeV2RMSNorm(config.hidden_size,
                                                            eps=config.rms_norm_eps)

    def forward(self, hidden_states, attention_mask=None, position_ids=None, past_key_value=None,
                output_attentions=False, output_router_logits=False, use_cache=False,
                position_embeddings=None, cache_position=None, **kwargs):
        residual = hidden_states
        hidden_states = self.input_layernorm(hidden_states)
        hidden_states, _, present = self.attention(
            hidden_states=hidden_states, position_embeddings=position_embeddings,
            attention_mask=attention_mask, past_key_value=past_key_value,
            cache_position=cache_position, position_ids=position_ids)
        hidden_states = residual + hidden_states
        residual = hidden_states
        hidden_states = self.post_attention_layernorm(hidden_states)
        hidden_states = self.mlp(hidden_states)
        if isinstance(hidden_states, tuple):
            hidden_states = hidden_states[0]
        hidden_states = residual + hidden_states
        return (hidden_states,)


class BailingMoeV2Model(nn.Module):
    def __init__(self, config: BailingMoeV2Config):
        super().__init__()
        self.config = config
        self.word_embeddings = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(
            [BailingMoeV2DecoderLayer(config, i) for i in range(config.num_hidden_layers)])
        self.norm = BailingMoeV2RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.rotary_emb = BailingMoeV2RotaryEmbedding(config)

    def forward(self, input_ids=None, inputs_embeds=None, position_ids=None,
                past_key_values=None, cache_position=None, **kwargs):
        h = inputs_embeds if inputs_embeds is not None else self.word_embeddings(input_ids)
        for layer in self.layers:
            h = layer(h, position_ids=position_ids, past_key_value=past_key_values,
                      cache_position=cache_position)[0]
        return self.norm(h)


class BailingMoeV2ForCausalLM(nn.Module):
    def __init__(self, config: BailingMoeV2Config):
        super().__init__()
        self.config = config
        self.model = BailingMoeV2Model(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)

    def forward(self, input_ids=None, **kwargs):
        return self.lm_head(self.model(input_ids=input_ids, **kwargs))


def init_weights_(module: nn.Module, generator: torch.Generator, std: float = 0.02,
                  bias_std: float = 0.01) -> nn.Module:
    """Seeded random init: Linear/Embedding weights ~ N(0, std); RMSNorm weights 1 + N(0, std);
    gate.weight ~ N(0, std), gate.expert_bias ~ N(0, bias_std)."""
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.endswith("layernorm.weight") or name.endswith("norm.weight"):
                p.copy_(1.0 + std * torch.randn(p.shape, generator=generator))
            elif p.dim() >= 2:
                p.copy_(std * torch.randn(p.shape, generator=generator))
            else:
                p.zero_()
        for name, b in module.named_buffers():
            if name.endswith("expert_bias"):
                b.copy_(bias_std * torch.randn(b.shape, generator=generator))
    return module


def config_from_shape(shape, **overrides) -> BailingMoeV2Config:
    """Config of a one-layer MoE model with the geometry of a LayerShape-like object."""
    kw = dict(hidden_size=shape.hidden_size, num_attention_heads=shape.num_heads,
              num_key_value_heads=shape.num_kv_heads, head_dim=shape.head_dim,
              num_experts=shape.num_experts, num_experts_per_tok=shape.top_k,
              moe_intermediate_size=shape.moe_intermediate_size,
              num_shared_experts=shape.num_shared_experts, n_group=shape.n_group,
              topk_group=shape.topk_group, routed_scaling_factor=shape.routed_scaling_factor,
              rope_theta=shape.rope_theta, partial_rotary_factor=shape.partial_rotary_factor,
              rms_norm_eps=shape.rms_norm_eps, use_qk_norm=shape.use_qk_norm,
              max_position_embeddings=shape.max_position_embeddings, num_hidden_layers=1,
              first_k_dense_replace=0)
    kw.update(overrides)
    return BailingMoeV2Config(**kw)


def decoder_layer_from_weights(w: dict, shape, layer_idx: int = 0,
                               dtype: torch.dtype = torch.float32) -> BailingMoeV2DecoderLayer:
    """Oracle decoder layer holding the weights of a synthetic-layer dict (keys: ln1, ln2,
    qkv_w, dense_w, q_norm, k_norm, gate_w, expert_bias, gate_up [E,2I,H], down [E,H,I],
    shared_gate_up, shared_down), cast to ``dtype`` (the router bias stays fp32)."""
    cfg = config_from_shape(shape)
    with torch.device("meta"):
        layer = BailingMoeV2DecoderLayer(cfg, layer_idx)
    layer = layer.to_empty(device="cpu").to(dtype)
    I = shape.moe_intermediate_size

    def cp(dst, src):
        dst.data.copy_(src.detach().to("cpu", dtype))

    with torch.no_grad():
        cp(layer.input_layernorm.weight, w["ln1"])
        cp(layer.post_attention_layernorm.weight, w["ln2"])
        att = layer.attention
        cp(att.query_key_value.weight, w["qkv_w"])
        cp(att.dense.weight, w["dense_w"])
        if shape.use_qk_norm:
            cp(att.query_layernorm.weight, w["q_norm"])
            cp(att.key_layernorm.weight, w["k_norm"])
        att.rotary_emb.inv_freq = rope_inv_freq(shape.head_dim, shape.partial_rotary_factor,
                                                shape.rope_theta)
        moe = layer.mlp
        cp(moe.gate.weight, w["gate_w"])
        moe.gate.expert_bias = w["expert_bias"].detach().to("cpu", torch.float32).clone()
        gu = w["gate_up"].detach().to("cpu")
        dn = w["down"].detach().to("cpu")
        for e, ex in enumerate(moe.experts):
            cp(ex.gate_proj.weight, gu[e, :I])
            cp(ex.up_proj.weight, gu[e, I:])
            cp(ex.down_proj.weight, dn[e])
        if moe.shared_experts is not None:
            sgu = w["shared_gate_up"].detach().to("cpu")
            Is = sgu.shape[0] // 2
            cp(moe.shared_experts.gate_proj.weight, sgu[:Is])
            cp(moe.shared_experts.up_proj.weight, sgu[Is:])
            cp(moe.shared_experts.down_proj.weight, w["shared_down"])
    return layer.eval()


def dense_decoder_layer_from_weights(w: dict, shape, intermediate_size: int,
                                     dtype: torch.dtype = torch.float32) -> BailingMoeV2DecoderLayer:
    """Oracle decoder layer with the dense SwiGLU MLP (layer_idx < first_k_dense_replace,
    modeling_bailing_moe_v2.py:388-399) from a weights dict with the attention and norm keys of
    :func:`decoder_layer_from_weights` plus mlp_gate / mlp_up [I, H] and mlp_down [H, I]."""
    cfg = config_from_shape(shape, first_k_dense_replace=1, intermediate_size=intermediate_size)
    with torch.device("meta"):
        layer = BailingMoeV2DecoderLayer(cfg, 0)
    layer = layer.to_empty(device="cpu").to(dtype)
    assert isinstance(layer.mlp, BailingMoeV2MLP)

    def cp(dst, src):
        dst.data.copy_(src.detach().to("cpu", dtype))

    with torch.no_grad():
        cp(layer.input_layernorm.weight, w["ln1"])
        cp(layer.post_attention_layernorm.weight, w["ln2"])
        att = layer.attention
        cp(att.query_key_value.weight, w["qkv_w"])
        cp(att.dense.weight, w["dense_w"])
        if shape.use_qk_norm:
            cp(att.query_layernorm.weight, w["q_norm"])
            cp(att.key_layernorm.weight, w["k_norm"])
        att.rotary_emb.inv_freq = rope_inv_freq(shape.head_dim, shape.partial_rotary_factor,
                                                shape.rope_theta)
        cp(layer.mlp.gate_proj.weight, w["mlp_gate"])
        cp(layer.mlp.up_proj.weight, w["mlp_up"])
        cp(layer.mlp.down_proj.weight, w["mlp_down"])
    return layer.eval()
