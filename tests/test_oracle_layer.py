"""Pins of the attention, MoE, RMSNorm and RoPE oracles (CPU).

  * paged decode reference (gather + torch SDPA) vs an explicit float64 loop reading each slot's
    physical block by hand; invariance under a relabelling of physical blocks; cache
    write/gather round trip;
  * MoE block vs transformers' DeepseekV3MoE (same routing algorithm + SwiGLU experts + shared
    expert) loaded with the same weights;
  * RMSNorm vs transformers' DeepseekV3RMSNorm; full-rotary RoPE vs transformers'
    apply_rotary_pos_emb; partial RoPE: pass-through dims untouched, position 0 is the
    identity, each rotated pair keeps its norm, rotations compose (pos a then b = a + b).
"""
import math

import pytest
import torch

from oracle.bailing_moe_v2 import (BailingMoeV2Config, BailingMoeV2RMSNorm,
                                   BailingMoeV2RotaryEmbedding, BailingMoeV2SparseMoeBlock,
                                   apply_partial_rotary, init_weights_)
from oracle.paged_kv import PagedKVCacheRef, gather_sequence, paged_decode_naive, \
    paged_decode_ref


def _ctx(B=3, Hkv=2, bs=8, D=16, lens=(5, 17, 30), nb=20, seed=0):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(nb, Hkv, bs, D, generator=g)
    v = torch.randn(nb, Hkv, bs, D, generator=g)
    perm = torch.randperm(nb, generator=g)
    mbps = max((n + 1 + bs - 1) // bs for n in lens)
    table = torch.zeros(B, mbps, dtype=torch.int64)
    off = 0
    for b, n in enumerate(lens):
        m = (n + 1 + bs - 1) // bs
        table[b, :m] = perm[off:off + m]
        off += m
    return k, v, table, torch.tensor(lens)


def test_paged_decode_ref_matches_naive_loop():
    k, v, table, pos = _ctx()
    q = torch.randn(3, 4, 16, generator=torch.Generator().manual_seed(1))
    ref = paged_decode_ref(q, k, v, table, pos, scale=16 ** -0.5, dtype=torch.float64)
    naive = paged_decode_naive(q, k, v, table, pos, scale=16 ** -0.5)
    torch.testing.assert_close(ref, naive, rtol=1e-10, atol=1e-10)


def test_paged_decode_invariant_to_block_relabelling():
    k, v, table, pos = _ctx()
    q = torch.randn(3, 4, 16, generator=torch.Generator().manual_seed(2))
    out = paged_decode_ref(q, k, v, table, pos, scale=0.25)
    relabel = torch.randperm(k.shape[0], generator=torch.Generator().manual_seed(3))
    k2 = torch.empty_like(k)
    v2 = torch.empty_like(v)
    k2[relabel] = k
    v2[relabel] = v
    out2 = paged_decode_ref(q, k2, v2, relabel[table], pos, scale=0.25)
    torch.testing.assert_close(out, out2, rtol=0, atol=0)


def test_cache_write_then_gather_round_trip():
    k, v, table, pos = _ctx()
    cache = PagedKVCacheRef([k.clone()], [v.clone()], table)
    kn = torch.randn(3, 2, 16)
    vn = torch.randn(3, 2, 16)
    cache.write(0, pos, kn, vn)
    for b in range(3):
        kb, vb = cache.gather(0, b, int(pos[b]) + 1)
        torch.testing.assert_close(kb[:, -1], kn[b])
        torch.testing.assert_close(vb[:, -1], vn[b])
        torch.testing.assert_close(kb[:, :-1], gather_sequence(k, table[b], int(pos[b])))


def test_moe_block_matches_transformers_deepseek_v3():
    from transformers.models.deepseek_v3.configuration_deepseek_v3 import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3MoE

    H, I, E = 64, 32, 64
    cfg = BailingMoeV2Config(hidden_size=H, moe_intermediate_size=I, num_experts=E,
                             num_experts_per_tok=6, n_group=8, topk_group=3,
                             routed_scaling_factor=2.5, num_shared_experts=1)
    ours = BailingMoeV2SparseMoeBlock(cfg)
    init_weights_(ours, torch.Generator().manual_seed(0), std=0.1, bias_std=0.05)
    dcfg = DeepseekV3Config(hidden_size=H, moe_intermediate_size=I, n_routed_experts=E,
                            num_experts_per_tok=6, n_group=8, topk_group=3,
                            routed_scaling_factor=2.5, norm_topk_prob=True, n_shared_experts=1,
                            hidden_act="silu")
    if not hasattr(dcfg, "num_local_experts"):
        dcfg.num_local_experts = E
    ref = DeepseekV3MoE(dcfg)
    with torch.no_grad():
        ref.gate.weight.copy_(ours.gate.weight)
        ref.gate.e_score_correction_bias.copy_(ours.gate.expert_bias)
        for e, ex in enumerate(ours.experts):
            ref.experts.gate_up_proj[e, :I] = ex.gate_proj.weight
            ref.experts.gate_up_proj[e, I:] = ex.up_proj.weight
            ref.experts.down_proj[e] = ex.down_proj.weight
        ref.shared_experts.gate_proj.weight.copy_(ours.shared_experts.gate_proj.weight)
        ref.shared_experts.up_proj.weight.copy_(ours.shared_experts.up_proj.weight)
        ref.shared_experts.down_proj.weight.copy_(ours.shared_experts.down_proj.weight)
    x = torch.randn(2, 40, H, generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        got, _ = ours(x)
        want = ref(x)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_rmsnorm_matches_transformers():
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3RMSNorm

    ours = BailingMoeV2RMSNorm(96, eps=1e-6)
    ref = DeepseekV3RMSNorm(96, eps=1e-6)
    with torch.no_grad():
        w = torch.randn(96)
        ours.weight.copy_(w)
        ref.weight.copy_(w)
    x = torch.randn(5, 96) * 3
    torch.testing.assert_close(ours(x), ref(x))
    # closed form: a constant row c normalises to sign(c) * weight (up to eps)
    c = torch.full((1, 96), -2.0)
    torch.testing.assert_close(ours(c), -w.view(1, -1), rtol=1e-5, atol=1e-5)


def test_full_rope_matches_transformers():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    cfg = BailingMoeV2Config(head_dim=64, partial_rotary_factor=1.0, rope_theta=10000.0)
    rot = BailingMoeV2RotaryEmbedding(cfg)
    pos = torch.tensor([[0, 3, 17], [5, 100, 2049]])
    q = torch.randn(2, 4, 3, 64)
    k = torch.randn(2, 2, 3, 64)
    cos, sin = rot(q, pos)
    got_q, got_k = apply_partial_rotary(q, k, cos, sin)
    want_q, want_k = apply_rotary_pos_emb(q, k, cos, sin)
    torch.testing.assert_close(got_q, want_q)
    torch.testing.assert_close(got_k, want_k)


@pytest.mark.parametrize("factor", [0.5, 1.0])
def test_partial_rope_properties(factor):
    D = 128
    cfg = BailingMoeV2Config(head_dim=D, partial_rotary_factor=factor, rope_theta=1e6)
    rot = BailingMoeV2RotaryEmbedding(cfg)
    rd = int(D * factor)
    assert rot.inv_freq.numel() == rd // 2
    assert math.isclose(float(rot.inv_freq[0]), 1.0)
    assert math.isclose(float(rot.inv_freq[1]), 1e6 ** (-2 / rd), rel_tol=1e-6)
    q = torch.randn(1, 3, 1, D, dtype=torch.float64)
    k = torch.randn(1, 1, 1, D, dtype=torch.float64)

    def apply(x, p):
        cos, sin = rot(x, torch.tensor([[p]]))
        return apply_partial_rotary(x, k, cos.double(), sin.double())[0]

    torch.testing.assert_close(apply(q, 0), q)                 # identity at position 0
    out = apply(q, 777)
    torch.testing.assert_close(out[..., rd:], q[..., rd:])     # pass-through dims
    h = rd // 2
    n_in = q[..., :h] ** 2 + q[..., h:rd] ** 2
    n_out = out[..., :h] ** 2 + out[..., h:rd] ** 2
    torch.testing.assert_close(n_in, n_out)                     # pairs keep their norm
    torch.testing.assert_close(apply(apply(q, 300), 477), apply(q, 777), rtol=1e-4, atol=1e-4)


def test_dense_decoder_layer_from_weights_wiring():
    """The dense-MLP oracle layer holds the dict's matrices in their places (gate, up and down
    not swapped) and computes h1 + down(silu(gate(n)) * up(n)) on n = RMSNorm(h1)."""
    import dataclasses

    from oracle.bailing_moe_v2 import dense_decoder_layer_from_weights
    from tt_symbiote_amd.workloads import LING_MINI_2, dense_layer_weights

    shape = dataclasses.replace(LING_MINI_2, hidden_size=256, num_heads=2, num_kv_heads=1)
    w = dense_layer_weights(shape, intermediate_size=384, seed=4)
    layer = dense_decoder_layer_from_weights(w, shape, 384)
    assert torch.equal(layer.mlp.gate_proj.weight, w["mlp_gate"].float())
    assert torch.equal(layer.mlp.up_proj.weight, w["mlp_up"].float())
    assert torch.equal(layer.mlp.down_proj.weight, w["mlp_down"].float())
    assert torch.equal(layer.attention.query_key_value.weight, w["qkv_w"].float())
    x = torch.randn(1, 5, 256, generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        out = layer(x)[0]
        h1 = x + layer.attention(layer.input_layernorm(x))[0]
        n = layer.post_attention_layernorm(h1)
        g = n @ w["mlp_gate"].float().T
        u = n @ w["mlp_up"].float().T
        want = h1 + (g * torch.sigmoid(g) * u) @ w["mlp_down"].float().T
    torch.testing.assert_close(out, want, rtol=1e-5, atol=1e-5)
