"""Seeded synthetic workloads of the BailingMoeV2 decode path (no checkpoints or datasets).

``LayerShape`` holds the Ling-mini-2.0 layer geometry (tests/experimental/bailing_moe_v2/
shapes.json: hidden 2048, 16 query / 4 kv heads of 128, 256 experts top-8 with moe intermediate
512, 1 shared expert, 8 groups keep 4, routed scale 2.5, RMSNorm eps 1e-6; RoPE theta 1e6 and a
partial rotary factor of 0.5).

``layer_weights`` draws a random-init layer: every matrix N(0, 0.02) rounded to bf16, RMSNorm
weights 1 + N(0, 0.02), router expert bias N(0, 0.01) in fp32. ``paged_context`` builds a ragged
paged KV cache: per-sequence cached lengths, blocks of ``block_size`` tokens placed through a
shuffled pool ``slack`` times larger than needed, K/V ~ N(0, 1) in bf16.

Both the benchmark and the tests draw their inputs here, so the same seed gives the same layer.
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass
from typing import Dict, Optional

import torch


@dataclass(frozen=True)
class LayerShape:
    hidden_size: int = 2048
    num_heads: int = 16
    num_kv_heads: int = 4
    head_dim: int = 128
    num_experts: int = 256
    top_k: int = 8
    moe_intermediate_size: int = 512
    num_shared_experts: int = 1
    n_group: int = 8
    topk_group: int = 4
    routed_scaling_factor: float = 2.5
    rope_theta: float = 1e6
    partial_rotary_factor: float = 0.5
    rms_norm_eps: float = 1e-6
    use_qk_norm: bool = True
    max_position_embeddings: int = 16384

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    def expert_bytes(self) -> int:
        """bf16 bytes of one expert's three matrices."""
        return 3 * self.moe_intermediate_size * self.hidden_size * 2

    def attention_weight_bytes(self) -> int:
        qkv = (self.num_heads + 2 * self.num_kv_heads) * self.head_dim * self.hidden_size
        dense = self.hidden_size * self.num_heads * self.head_dim
        return 2 * (qkv + dense)


LING_MINI_2 = LayerShape()


def _randn(g: torch.Generator, shape, device, scale: float = 1.0) -> torch.Tensor:
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32) * scale


def layer_weights(shape: LayerShape = LING_MINI_2, seed: int = 0, device="cpu",
                  std: float = 0.02, bias_std: float = 0.01) -> Dict[str, torch.Tensor]:
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    H, Hq, Hkv, D = shape.hidden_size, shape.num_heads, shape.num_kv_heads, shape.head_dim
    E, I = shape.num_experts, shape.moe_intermediate_size
    bf = torch.bfloat16
    w = {
        "ln1": (1.0 + _randn(g, (H,), dev, std)).to(bf),
        "ln2": (1.0 + _randn(g, (H,), dev, std)).to(bf),
        "qkv_w": _randn(g, ((Hq + 2 * Hkv) * D, H), dev, std).to(bf),
        "dense_w": _randn(g, (H, Hq * D), dev, std).to(bf),
        "q_norm": (1.0 + _randn(g, (D,), dev, std)).to(bf),
        "k_norm": (1.0 + _randn(g, (D,), dev, std)).to(bf),
        "gate_w": _randn(g, (E, H), dev, std).to(bf),
        "expert_bias": _randn(g, (E,), dev, bias_std),
    }
    gate_up = torch.empty(E, 2 * I, H, dtype=bf, device=dev)
    down = torch.empty(E, H, I, dtype=bf, device=dev)
    chunk = 16
    for e0 in range(0, E, chunk):
        e1 = min(E, e0 + chunk)
        gate_up[e0:e1] = _randn(g, (e1 - e0, 2 * I, H), dev, std).to(bf)
        down[e0:e1] = _randn(g, (e1 - e0, H, I), dev, std).to(bf)
    w["gate_up"] = gate_up
    w["down"] = down
    Is = I * shape.num_shared_experts
    if shape.num_shared_experts:
        w["shared_gate_up"] = _randn(g, (2 * Is, H), dev, std).to(bf)
        w["shared_down"] = _randn(g, (H, Is), dev, std).to(bf)
    return w


@dataclass
class PagedContext:
    k_pool: torch.Tensor       # [num_blocks, Hkv, block_size, D] bf16
    v_pool: torch.Tensor
    page_table: torch.Tensor   # [B, max_blocks_per_seq] int32
    positions: torch.Tensor    # [B] int32: slot of the new token = cached tokens
    context_lens: torch.Tensor  # [B] int64 cached tokens before the step

    @property
    def block_size(self) -> int:
        return self.k_pool.shape[2]

    def kv_bytes_read(self) -> int:
        """bf16 K+V bytes a decode step reads: (ctx+1) slots per sequence."""
        hkv, d = self.k_pool.shape[1], self.k_pool.shape[3]
        return int((self.context_lens + 1).sum()) * hkv * d * 2 * 2


def paged_context(batch: int, ctx_lo: int, ctx_hi: int, *, block_size: int = 32,
                  num_kv_heads: int = 4, head_dim: int = 128, seed: int = 0,
                  slack: float = 1.25, pool_blocks: Optional[int] = None,
                  device="cpu", kv_device=None) -> PagedContext:
    """Cached lengths uniform in [ctx_lo, ctx_hi]; each sequence gets ceil((ctx+1)/block_size)
    blocks (room for the new token) drawn without replacement from a shuffled pool of
    ceil(slack * total) blocks (or ``pool_blocks``)."""
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (batch,), generator=g)
    nblk = [(int(c) + 1 + block_size - 1) // block_size for c in ctx]
    total = sum(nblk)
    nb = pool_blocks if pool_blocks is not None else int(math.ceil(slack * total))
    if nb < total:
        raise ValueError(f"pool of {nb} blocks cannot hold {total}")
    perm = torch.randperm(nb, generator=g)
    mbps = max(nblk)
    table = torch.zeros(batch, mbps, dtype=torch.int32)
    off = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    kv_dev = torch.device(kv_device if kv_device is not None else device)
    gk = torch.Generator(device=kv_dev).manual_seed(seed + 1)
    shape = (nb, num_kv_heads, block_size, head_dim)
    k_pool = torch.randn(shape, generator=gk, device=kv_dev).to(torch.bfloat16)
    v_pool = torch.randn(shape, generator=gk, device=kv_dev).to(torch.bfloat16)
    dev = torch.device(device)
    return PagedContext(k_pool=k_pool.to(dev), v_pool=v_pool.to(dev), page_table=table.to(dev),
                        positions=ctx.to(torch.int32).to(dev), context_lens=ctx)


def fp8_kv_pools(pool: torch.Tensor):
    """Synthetic contents of an fp8 KV cache from a bf16 pool [nb, Hkv, bs, D]: per (block,
    head) the power-of-two scale at or above amax / 448 and the e4m3fn bytes of pool / scale
    (what appending the block's tokens to an empty block produces), as token rows [nb, Hkv, bs,
    D] (``hip_ops.fp8_v_pool`` gives a V pool's layout). Setup only."""
    amax = pool.float().abs().amax(dim=(2, 3))
    scale = torch.where(amax > 0, torch.exp2(torch.ceil(torch.log2(amax / 448.0))),
                        torch.zeros_like(amax))
    safe = torch.where(scale > 0, scale, torch.ones_like(scale))
    q = (pool.float() / safe[..., None, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale.contiguous()


def decode_layer_config(name: str) -> dict:
    """The decode workloads of the Ling-mini-2.0 layer: 'single' (one sequence of 512 cached
    tokens, 16+1 blocks of 32 placed by a random permutation of a 64-block pool) and 'batch32'
    (32 sequences, cached lengths uniform in [128, 4096], block size 32, pool 1.25x)."""
    if name == "single":
        return dict(batch=1, ctx_lo=512, ctx_hi=512, block_size=32, pool_blocks=64)
    if name == "batch32":
        return dict(batch=32, ctx_lo=128, ctx_hi=4096, block_size=32, slack=1.25)
    raise KeyError(name)


def prefill_layer_config() -> dict:
    """The prefill workload: 8 prompts of lengths uniform in [256, 2048] packed varlen, block size
    32, pool 1.25x shuffled; routing skewed so expert load follows a Zipf law (s = 1.1)."""
    return dict(n_seqs=8, len_lo=256, len_hi=2048, block_size=32, slack=1.25, zipf_s=1.1)


def zipf_expert_bias(num_experts: int, s: float, seed: int, strength: float = 0.1) -> torch.Tensor:
    """Router expert-bias offsets that make expert selection Zipf-skewed: expert of popularity
    rank r (a seeded permutation) gets strength * log(r^-s); the bias only moves selection, not
    the routing weights."""
    g = torch.Generator().manual_seed(seed)
    rank = torch.empty(num_experts)
    rank[torch.randperm(num_experts, generator=g)] = torch.arange(1, num_experts + 1).float()
    return strength * torch.log(rank.pow(-s))


@dataclass
class PrefillBatch:
    """Packed prompts: x [T, H] bf16, cu_seqlens [n+1] int32, page table [n, blocks] int32 over a
    zero pool of num_blocks blocks."""

    x: torch.Tensor
    cu_seqlens: torch.Tensor
    lens: list
    page_table: torch.Tensor
    num_blocks: int

    @property
    def tokens(self) -> int:
        return int(sum(self.lens))


def prefill_batch(n_seqs: int, len_lo: int, len_hi: int, hidden: int, *, block_size: int = 32,
                  slack: float = 1.25, seed: int = 0, device="cpu") -> PrefillBatch:
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(len_lo, len_hi + 1, (n_seqs,), generator=g).tolist()
    nblk = [(L + block_size - 1) // block_size for L in lens]
    nb = int(math.ceil(slack * sum(nblk)))
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    pt = torch.zeros(n_seqs, max(nblk), dtype=torch.int32)
    o = 0
    for i, n in enumerate(nblk):
        pt[i, :n] = perm[o:o + n]
        o += n
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32)
    x = torch.randn(sum(lens), hidden, generator=g).to(torch.bfloat16)
    dev = torch.device(device)
    return PrefillBatch(x.to(dev), cu.to(dev), lens, pt.to(dev), nb)


def build_decoder_layer(w: Dict[str, torch.Tensor], shape: LayerShape = LING_MINI_2,
                        layer_idx: int = 0, weight_format: str = "bf16"):
    """HIP decoder layer (attention + MoE) from a :func:`layer_weights` dict (not yet bound
    to a device); ``weight_format`` "fp8_e4m3" stores the experts block-scaled in fp8."""
    from .modules.attention import HIPBailingMoEAttention
    from .modules.decoder_layer import HIPBailingMoEDecoderLayer
    from .modules.moe import HIPBailingMoE

    attn = HIPBailingMoEAttention.from_weights(
        num_heads=shape.num_heads, num_kv_heads=shape.num_kv_heads, head_dim=shape.head_dim,
        hidden_size=shape.hidden_size, qkv_weight=w["qkv_w"], dense_weight=w["dense_w"],
        q_norm_weight=w["q_norm"] if shape.use_qk_norm else None,
        k_norm_weight=w["k_norm"] if shape.use_qk_norm else None,
        partial_rotary_factor=shape.partial_rotary_factor, rope_theta=shape.rope_theta,
        max_position_embeddings=shape.max_position_embeddings, norm_eps=shape.rms_norm_eps,
        layer_idx=layer_idx)
    moe = HIPBailingMoE.from_weights(
        gate_weight=w["gate_w"], expert_bias=w["expert_bias"], w_gate_up=w["gate_up"],
        w_down=w["down"], shared_gate_up=w.get("shared_gate_up"),
        shared_down=w.get("shared_down"), top_k=shape.top_k, n_group=shape.n_group,
        topk_group=shape.topk_group, routed_scaling_factor=shape.routed_scaling_factor,
        weight_format=weight_format)
    return HIPBailingMoEDecoderLayer.from_modules(attn, moe, w["ln1"], w["ln2"],
                                                  eps=shape.rms_norm_eps)


def dense_layer_weights(shape: LayerShape = LING_MINI_2, intermediate_size: int = 5120,
                        seed: int = 0, device="cpu", std: float = 0.02) -> Dict[str, torch.Tensor]:
    """Random-init weights of a decoder layer with the dense SwiGLU MLP (the layers before
    first_k_dense_replace): the attention and norm entries of :func:`layer_weights` plus
    ``mlp_gate`` / ``mlp_up`` [intermediate, H] and ``mlp_down`` [H, intermediate], bf16."""
    w = layer_weights(dataclasses.replace(shape, num_experts=8, moe_intermediate_size=128,
                                          num_shared_experts=0), seed=seed, device=device,
                      std=std)
    for k in ("gate_w", "expert_bias", "gate_up", "down"):
        del w[k]
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed + 1000)
    H = shape.hidden_size
    w["mlp_gate"] = _randn(g, (intermediate_size, H), dev, std).to(torch.bfloat16)
    w["mlp_up"] = _randn(g, (intermediate_size, H), dev, std).to(torch.bfloat16)
    w["mlp_down"] = _randn(g, (H, intermediate_size), dev, std).to(torch.bfloat16)
    return w


def build_dense_decoder_layer(shape: LayerShape = LING_MINI_2, intermediate_size: int = 5120,
                              seed: int = 0, device="cpu", layer_idx: int = 0,
                              std: float = 0.02):
    """HIP decoder layer with the dense SwiGLU MLP (the layers before first_k_dense_replace),
    weights from :func:`dense_layer_weights`."""
    from .modules.attention import HIPBailingMoEAttention
    from .modules.decoder_layer import HIPBailingMoEDecoderLayer
    from .modules.moe import HIPBailingMoeV2MLP

    w = dense_layer_weights(shape, intermediate_size, seed=seed, device=device, std=std)
    H = shape.hidden_size
    gate, up, down = w["mlp_gate"], w["mlp_up"], w["mlp_down"]
    attn = HIPBailingMoEAttention.from_weights(
        num_heads=shape.num_heads, num_kv_heads=shape.num_kv_heads, head_dim=shape.head_dim,
        hidden_size=H, qkv_weight=w["qkv_w"], dense_weight=w["dense_w"],
        q_norm_weight=w["q_norm"] if shape.use_qk_norm else None,
        k_norm_weight=w["k_norm"] if shape.use_qk_norm else None,
        partial_rotary_factor=shape.partial_rotary_factor, rope_theta=shape.rope_theta,
        max_position_embeddings=shape.max_position_embeddings, norm_eps=shape.rms_norm_eps,
        layer_idx=layer_idx)
    mlp = HIPBailingMoeV2MLP.from_weights(gate, up, down)
    return HIPBailingMoEDecoderLayer.from_modules(attn, mlp, w["ln1"], w["ln2"],
                                                  eps=shape.rms_norm_eps)


def model_config(num_layers: int = 20, vocab_size: int = 157184,
                 first_k_dense_replace: int = 1, dense_intermediate_size: int = 5120) -> dict:
    """The whole-model greedy workload: Ling-mini-2.0 shape (20 layers, layer 0 dense with
    intermediate 5120, 19 MoE layers), vocab 157184, batch 64 prompts of 2048 random ids, 128
    greedy tokens, paged KV with block size 32 and 8192 blocks."""
    return dict(num_layers=num_layers, vocab_size=vocab_size,
                first_k_dense_replace=first_k_dense_replace,
                dense_intermediate_size=dense_intermediate_size, batch=64, prompt_len=2048,
                new_tokens=128, block_size=32, max_num_blocks=8192)
