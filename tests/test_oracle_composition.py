"""Pins of the oracle's composition (CPU): attention, decoder layer and whole model.

The oracle restates the BailingMoeV2 modules (modeling_bailing_moe_v2.py:403-483,
ttnn_attention.py:2308-2466, ttnn_moe.py:1413-1490). transformers' Glm4Moe classes have the same
structure: fused-free q/k/v projections with per-head QK RMSNorm before a partial split-half
RoPE, GQA attention scaled by head_dim^-0.5, an output projection, pre-norm residual blocks, a
sigmoid group-limited router with a score-correction bias, SwiGLU experts plus a shared expert
on the MoE input, and an embedding -> layers -> final norm -> lm_head model. Loaded with the same
weights (the fused query_key_value rows split into q/k/v), they must agree with the oracle:

  * attention prefill (causal, no cache) and a decode step (oracle: paged cache through a
    shuffled page table; transformers: DynamicCache), partial_rotary_factor 0.5 and 1.0;
  * MoE and dense decoder layers, prefill and decode;
  * a two-layer ForCausalLM (dense layer 0, MoE layer 1): prefill logits and three greedy
    decode steps.

The router's dropped-group fill differs (0.0 in the reference's torch form, ttnn_moe.py:429;
-inf in transformers); the inputs keep every kept-group score positive, where both fills pick
the same experts, and the tests assert that precondition.

Planted mistakes in the oracle (a wrong attention scale, full instead of partial RoPE, a missing
QK-norm) must break the agreement, which shows the comparison can fail.
"""
import pytest
import torch

from oracle.bailing_moe_v2 import (BailingMoeV2Attention, BailingMoeV2Config,
                                   BailingMoeV2DecoderLayer, BailingMoeV2ForCausalLM,
                                   init_weights_)
from oracle.paged_kv import PagedKVCacheRef

glm = pytest.importorskip("transformers.models.glm4_moe.modeling_glm4_moe")
from transformers.cache_utils import DynamicCache  # noqa: E402
from transformers.models.glm4_moe.configuration_glm4_moe import Glm4MoeConfig  # noqa: E402

H, HQ, HKV, D = 64, 4, 2, 16
I_MOE, I_DENSE, E, TOPK, NGROUP, TOPKG = 24, 40, 16, 4, 4, 2
VOCAB = 97
TOL = dict(rtol=2e-5, atol=2e-5)


def _configs(factor: float, layers: int = 1, first_dense: int = 0):
    ours = BailingMoeV2Config(
        hidden_size=H, intermediate_size=I_DENSE, moe_intermediate_size=I_MOE,
        num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D, num_experts=E,
        num_experts_per_tok=TOPK, num_shared_experts=1, n_group=NGROUP, topk_group=TOPKG,
        routed_scaling_factor=2.5, first_k_dense_replace=first_dense, num_hidden_layers=layers,
        rms_norm_eps=1e-6, rope_theta=1e6, partial_rotary_factor=factor, use_qk_norm=True,
        vocab_size=VOCAB, max_position_embeddings=256)
    theirs = Glm4MoeConfig(
        vocab_size=VOCAB, hidden_size=H, intermediate_size=I_DENSE, num_hidden_layers=layers,
        num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D, hidden_act="silu",
        max_position_embeddings=256, rms_norm_eps=1e-6,
        rope_parameters={"rope_type": "default", "rope_theta": 1e6,
                         "partial_rotary_factor": factor},
        attention_bias=False, moe_intermediate_size=I_MOE, num_experts_per_tok=TOPK,
        n_shared_experts=1, n_routed_experts=E, routed_scaling_factor=2.5, n_group=NGROUP,
        topk_group=TOPKG, first_k_dense_replace=first_dense, norm_topk_prob=True,
        use_qk_norm=True, tie_word_embeddings=False)
    theirs._attn_implementation = "eager"
    return ours, theirs


def _copy_attention(src: BailingMoeV2Attention, dst) -> None:
    w = src.query_key_value.weight
    with torch.no_grad():
        dst.q_proj.weight.copy_(w[:HQ * D])
        dst.k_proj.weight.copy_(w[HQ * D:(HQ + HKV) * D])
        dst.v_proj.weight.copy_(w[(HQ + HKV) * D:])
        dst.o_proj.weight.copy_(src.dense.weight)
        dst.q_norm.weight.copy_(src.query_layernorm.weight)
        dst.k_norm.weight.copy_(src.key_layernorm.weight)


def _copy_mlp(src, dst) -> None:
    with torch.no_grad():
        dst.gate_proj.weight.copy_(src.gate_proj.weight)
        dst.up_proj.weight.copy_(src.up_proj.weight)
        dst.down_proj.weight.copy_(src.down_proj.weight)


def _copy_layer(src: BailingMoeV2DecoderLayer, dst) -> None:
    _copy_attention(src.attention, dst.self_attn)
    with torch.no_grad():
        dst.input_layernorm.weight.copy_(src.input_layernorm.weight)
        dst.post_attention_layernorm.weight.copy_(src.post_attention_layernorm.weight)
    if hasattr(src.mlp, "experts"):
        moe = src.mlp
        with torch.no_grad():
            dst.mlp.gate.weight.copy_(moe.gate.weight)
            dst.mlp.gate.e_score_correction_bias.copy_(moe.gate.expert_bias)
            for e, ex in enumerate(moe.experts):
                dst.mlp.experts.gate_up_proj[e, :I_MOE] = ex.gate_proj.weight
                dst.mlp.experts.gate_up_proj[e, I_MOE:] = ex.up_proj.weight
                dst.mlp.experts.down_proj[e] = ex.down_proj.weight
        _copy_mlp(moe.shared_experts, dst.mlp.shared_experts)
    else:
        _copy_mlp(src.mlp, dst.mlp)


def _paged_cache(n_layers: int, B: int, n_slots: int, bs: int = 8, seed: int = 5):
    """Zeroed pools behind a shuffled page table (the reversed-table idea of the reference's
    page-table test, generalised to a random permutation)."""
    nblk = (n_slots + bs - 1) // bs
    nb = B * nblk + 3
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    table = perm[:B * nblk].view(B, nblk)
    k = [torch.zeros(nb, HKV, bs, D) for _ in range(n_layers)]
    v = [torch.zeros(nb, HKV, bs, D) for _ in range(n_layers)]
    return PagedKVCacheRef(k, v, table)


def _causal_mask(S: int, past: int = 0) -> torch.Tensor:
    q = torch.arange(past, past + S)[:, None]
    kk = torch.arange(past + S)[None, :]
    m = torch.zeros(S, past + S)
    m[kk > q] = float("-inf")
    return m[None, None]


def _positions(B: int, start: int, S: int) -> torch.Tensor:
    return torch.arange(start, start + S).view(1, S).expand(B, S)


def _assert_router_fill_irrelevant(moe, x: torch.Tensor) -> None:
    """Every token has at least top_k experts with a positive biased score, so masking the
    dropped groups with 0.0 or -inf selects the same experts."""
    logits = torch.nn.functional.linear(x.reshape(-1, H).float(), moe.gate.weight.float())
    c = torch.sigmoid(logits) + moe.gate.expert_bias
    assert bool(((c > 0).sum(-1) >= TOPK).all())


@pytest.mark.parametrize("factor", [0.5, 1.0])
def test_attention_prefill_matches_glm4moe(factor):
    ours_cfg, theirs_cfg = _configs(factor)
    torch.manual_seed(0)
    ours = init_weights_(BailingMoeV2Attention(ours_cfg, 0), torch.Generator().manual_seed(1),
                         std=0.15)
    theirs = glm.Glm4MoeAttention(theirs_cfg, 0)
    _copy_attention(ours, theirs)
    rot = glm.Glm4MoeRotaryEmbedding(theirs_cfg)
    B, S = 2, 9
    x = torch.randn(B, S, H, generator=torch.Generator().manual_seed(2))
    pos = _positions(B, 0, S)
    with torch.no_grad():
        got = ours(x, position_ids=pos)[0]
        want = theirs(x, rot(x, pos), _causal_mask(S))[0]
    torch.testing.assert_close(got, want, **TOL)


@pytest.mark.parametrize("factor", [0.5, 1.0])
def test_attention_decode_over_paged_cache_matches_glm4moe(factor):
    ours_cfg, theirs_cfg = _configs(factor)
    ours = init_weights_(BailingMoeV2Attention(ours_cfg, 0), torch.Generator().manual_seed(3),
                         std=0.15)
    theirs = glm.Glm4MoeAttention(theirs_cfg, 0)
    _copy_attention(ours, theirs)
    rot = glm.Glm4MoeRotaryEmbedding(theirs_cfg)
    B, S = 3, 13
    g = torch.Generator().manual_seed(4)
    prompt = torch.randn(B, S, H, generator=g)
    paged = _paged_cache(1, B, S + 4)
    dyn = DynamicCache(config=theirs_cfg)
    with torch.no_grad():
        pos = _positions(B, 0, S)
        ours(prompt, position_ids=pos, past_key_values=paged)
        theirs(prompt, rot(prompt, pos), _causal_mask(S), past_key_values=dyn)
        for step in range(3):
            x = torch.randn(B, 1, H, generator=g)
            cpos = torch.full((B,), S + step, dtype=torch.int64)
            got = ours(x, cache_position=cpos, past_key_values=paged)[0]
            want = theirs(x, rot(x, cpos.view(B, 1)), None, past_key_values=dyn)[0]
            torch.testing.assert_close(got, want, **TOL)


@pytest.mark.parametrize("dense", [False, True], ids=["moe", "dense"])
@pytest.mark.parametrize("factor", [0.5, 1.0])
def test_decoder_layer_prefill_and_decode_match_glm4moe(factor, dense):
    ours_cfg, theirs_cfg = _configs(factor, first_dense=1 if dense else 0)
    ours = init_weights_(BailingMoeV2DecoderLayer(ours_cfg, 0), torch.Generator().manual_seed(6),
                         std=0.15, bias_std=0.05)
    theirs = glm.Glm4MoeDecoderLayer(theirs_cfg, 0)
    assert hasattr(theirs.mlp, "experts") != dense
    _copy_layer(ours, theirs)
    rot = glm.Glm4MoeRotaryEmbedding(theirs_cfg)
    B, S = 2, 11
    g = torch.Generator().manual_seed(7)
    prompt = torch.randn(B, S, H, generator=g)
    paged = _paged_cache(1, B, S + 4)
    dyn = DynamicCache(config=theirs_cfg)
    with torch.no_grad():
        if not dense:
            _assert_router_fill_irrelevant(ours.mlp, ours.post_attention_layernorm(prompt))
        pos = _positions(B, 0, S)
        got = ours(prompt, position_ids=pos, past_key_value=paged)[0]
        want = theirs(prompt, attention_mask=_causal_mask(S), position_ids=pos,
                      past_key_values=dyn, position_embeddings=rot(prompt, pos))
        torch.testing.assert_close(got, want, **TOL)
        for step in range(2):
            x = torch.randn(B, 1, H, generator=g)
            cpos = torch.full((B,), S + step, dtype=torch.int64)
            got = ours(x, cache_position=cpos, past_key_value=paged)[0]
            want = theirs(x, attention_mask=None, position_ids=cpos.view(B, 1),
                          past_key_values=dyn, position_embeddings=rot(x, cpos.view(B, 1)))
            torch.testing.assert_close(got, want, **TOL)


def _model_pair(factor: float):
    ours_cfg, theirs_cfg = _configs(factor, layers=2, first_dense=1)
    ours = init_weights_(BailingMoeV2ForCausalLM(ours_cfg), torch.Generator().manual_seed(8),
                         std=0.15, bias_std=0.05)
    theirs = glm.Glm4MoeForCausalLM(theirs_cfg).eval()
    with torch.no_grad():
        theirs.model.embed_tokens.weight.copy_(ours.model.word_embeddings.weight)
        theirs.model.norm.weight.copy_(ours.model.norm.weight)
        theirs.lm_head.weight.copy_(ours.lm_head.weight)
    for a, b in zip(ours.model.layers, theirs.model.layers):
        _copy_layer(a, b)
    return ours, theirs, theirs_cfg


@pytest.mark.parametrize("factor", [0.5, 1.0])
def test_causal_lm_prefill_and_greedy_decode_match_glm4moe(factor):
    ours, theirs, theirs_cfg = _model_pair(factor)
    B, S = 2, 10
    ids = torch.randint(0, VOCAB, (B, S), generator=torch.Generator().manual_seed(9))
    paged = _paged_cache(2, B, S + 8)
    dyn = DynamicCache(config=theirs_cfg)
    with torch.no_grad():
        got = ours(input_ids=ids, position_ids=_positions(B, 0, S), past_key_values=paged)
        want = theirs(input_ids=ids, past_key_values=dyn, use_cache=True).logits
        torch.testing.assert_close(got, want, **TOL)
        tok = got[:, -1].argmax(-1)
        for step in range(3):
            cpos = torch.full((B,), S + step, dtype=torch.int64)
            got = ours(input_ids=tok.view(B, 1), cache_position=cpos, past_key_values=paged)
            want = theirs(input_ids=tok.view(B, 1), past_key_values=dyn, use_cache=True).logits
            torch.testing.assert_close(got, want, **TOL)
            assert torch.equal(got[:, -1].argmax(-1), want[:, -1].argmax(-1))
            tok = got[:, -1].argmax(-1)


@pytest.mark.parametrize("mistake", ["scale", "full_rope", "no_qk_norm"])
def test_planted_oracle_mistakes_break_agreement(mistake, monkeypatch):
    """The comparison above is sensitive: each plausible slip in the oracle's attention makes
    it fail."""
    import oracle.bailing_moe_v2 as om

    ours_cfg, theirs_cfg = _configs(0.5)
    ours = init_weights_(BailingMoeV2Attention(ours_cfg, 0), torch.Generator().manual_seed(1),
                         std=0.15)
    theirs = glm.Glm4MoeAttention(theirs_cfg, 0)
    _copy_attention(ours, theirs)
    rot = glm.Glm4MoeRotaryEmbedding(theirs_cfg)
    if mistake == "scale":
        ours.scaling = 1.0 / D
    elif mistake == "full_rope":
        ours.rotary_emb.inv_freq = om.rope_inv_freq(D, 1.0, 1e6)
    else:
        ours.config = BailingMoeV2Config(**{**ours_cfg.__dict__, "use_qk_norm": False})
    B, S = 2, 9
    x = torch.randn(B, S, H, generator=torch.Generator().manual_seed(2))
    pos = _positions(B, 0, S)
    with torch.no_grad():
        got = ours(x, position_ids=pos)[0]
        want = theirs(x, rot(x, pos), _causal_mask(S))[0]
    assert not torch.allclose(got, want, **TOL)
