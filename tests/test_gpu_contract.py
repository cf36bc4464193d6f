"""The reference's module and cache contract on the GPU (through the C ABI).

  * attention module, prefill then decode through ``forward`` over a reversed page table, as the
    reference's page-table test (tests/experimental/glm4_moe/Tier4/test_vllm_page_table_hook.py
    :89-150): outputs against the oracle attention (fp32, same reversed table), the table
    round trip, and ``get_seq_length`` 5 after the 5-token prefill, 6 after one decode; a decode
    without ``cache_position`` goes at the counter (7th slot);
  * decoder layer: a decode without ``cache_position`` equals one at the explicit position;
  * ``AutoModelForCausalLM.from_pretrained`` + ``set_device`` + HF ``generate(...,
    past_key_values=model._tt_kv_cache)`` (examples/e2e/run_ling_mini_2_0.py:57-86): the
    tokens equal the device greedy loop's up to an LM-head near tie, and every layer's counter
    ends at prompt + new - 1;
  * prefill split into several packed groups (later groups at page-table rows > 0) equals one
    group, tokens and cache bytes, for the bf16 and the fp8 cache.
"""
import pytest
import torch

import tt_symbiote_amd as ts
from hf_bailing import tiny_hf_model
from oracle.bailing_moe_v2 import (BailingMoeV2Attention, BailingMoeV2Config,
                                   BailingMoeV2DecoderLayer, init_weights_)
from oracle.paged_kv import PagedKVCacheRef
from tt_symbiote_amd.generate import greedy_generate, model_parts

pytestmark = pytest.mark.gpu


def _bf16_exact(module):
    with torch.no_grad():
        for p in module.parameters():
            p.copy_(p.bfloat16().float())
    return module


def _assert_close(got, want, what):
    got = got.float().cpu()
    want = want.float().cpu()
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    assert err <= 2e-2 and err <= 2e-2 * max(scale, 1e-3) + 2e-3, \
        f"{what}: max err {err:.3e} (max |ref| {scale:.3e})"


def test_attention_prefill_then_decode_over_reversed_page_table(device):
    cfg = BailingMoeV2Config(hidden_size=512, num_attention_heads=8, num_key_value_heads=4,
                             head_dim=128, partial_rotary_factor=0.5, rope_theta=1e6,
                             use_qk_norm=True, max_position_embeddings=2048)
    torch_attn = _bf16_exact(init_weights_(BailingMoeV2Attention(cfg, 0),
                                           torch.Generator().manual_seed(0), std=0.05))
    hip_attn = ts.HIPBailingMoEAttention.from_torch(torch_attn)
    ts.set_device(hip_attn, device)

    paged_config = ts.PagedAttentionConfig(block_size=32, max_num_blocks=64, batch_size=1)
    cache = ts.HIPPagedAttentionKVCache(num_layers=2, num_kv_heads=4, head_dim=128,
                                        config=paged_config).to_device(device)
    bps = paged_config.blocks_per_sequence
    reversed_pt = torch.arange(bps - 1, -1, -1, dtype=torch.int32).unsqueeze(0)
    cache.set_vllm_page_table(reversed_pt)
    assert torch.equal(cache.page_table_device.cpu()[0, :bps], reversed_pt[0])
    ref_cache = PagedKVCacheRef([torch.zeros(64, 4, 32, 128)], [torch.zeros(64, 4, 32, 128)],
                                reversed_pt)
    g = torch.Generator().manual_seed(1)

    hidden = torch.randn(1, 5, 512, generator=g).bfloat16()
    out = hip_attn(hidden.to(device), position_embeddings=None, past_key_values=cache,
                   cache_position=torch.arange(5).unsqueeze(0))[0]
    with torch.no_grad():
        ref = torch_attn(hidden.float(), past_key_values=ref_cache,
                         position_ids=torch.arange(5).unsqueeze(0))[0]
    assert out.shape == (1, 5, 512)
    _assert_close(out, ref, "paged prefill")
    assert cache.get_seq_length(0) == 5
    # the prompt's K rows sit in the physical blocks the reversed table names
    _assert_close(cache.key_cache(0)[bps - 1, :, :5].cpu(), ref_cache.k_pools[0][bps - 1, :, :5],
                  "prefill K rows")

    hidden_d = torch.randn(1, 1, 512, generator=g).bfloat16()
    out_d = hip_attn(hidden_d.to(device), position_embeddings=None, past_key_values=cache,
                     cache_position=torch.arange(5, 6).unsqueeze(0))[0]
    with torch.no_grad():
        ref_d = torch_attn(hidden_d.float(), past_key_values=ref_cache,
                           cache_position=torch.tensor([5]))[0]
    _assert_close(out_d, ref_d, "paged decode")
    assert cache.get_seq_length(0) == 6

    # no cache_position: the token goes at the counter (slot 6), as the reference's decode
    hidden_e = torch.randn(1, 1, 512, generator=g).bfloat16()
    out_e = hip_attn(hidden_e.to(device), past_key_values=cache)[0]
    with torch.no_grad():
        ref_e = torch_attn(hidden_e.float(), past_key_values=ref_cache,
                           cache_position=torch.tensor([6]))[0]
    _assert_close(out_e, ref_e, "decode at the counter")
    assert cache.get_seq_length(0) == 7 and cache.get_seq_length(1) == 0


def test_decoder_layer_decode_without_cache_position_uses_the_counter(device):
    cfg = BailingMoeV2Config(hidden_size=512, num_attention_heads=4, num_key_value_heads=2,
                             head_dim=128, num_experts=64, num_experts_per_tok=4,
                             moe_intermediate_size=128, n_group=8, topk_group=4,
                             first_k_dense_replace=0, partial_rotary_factor=0.5,
                             max_position_embeddings=2048)
    torch_layer = _bf16_exact(init_weights_(BailingMoeV2DecoderLayer(cfg, 0),
                                            torch.Generator().manual_seed(2)))
    layer = ts.HIPBailingMoEDecoderLayer.from_torch(torch_layer)
    ts.set_device(layer, device)
    pc = ts.PagedAttentionConfig(block_size=16, max_num_blocks=64, batch_size=2)
    caches = [ts.HIPPagedAttentionKVCache(1, 2, 128, pc).to_device(device) for _ in range(2)]
    g = torch.Generator().manual_seed(3)
    prompt = torch.randn(2, 7, 512, generator=g).bfloat16().to(device)
    x = torch.randn(2, 1, 512, generator=g).bfloat16().to(device)
    outs = []
    for i, cache in enumerate(caches):
        layer(prompt, past_key_values=cache)
        assert cache.get_seq_length(0) == 7
        pos = torch.full((2,), 7, dtype=torch.int32) if i == 0 else None
        outs.append(layer(x, past_key_values=cache, cache_position=pos)[0])
        assert cache.get_seq_length(0) == 8
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(caches[0].key_cache(0), caches[1].key_cache(0))
    # a prompt continuing the cached sequences is refused whatever device its positions are on
    # (the host counter is checked), and nothing is written
    k_before = caches[0].key_cache(0).clone()
    for pos in (torch.arange(8, 15, device=device), torch.arange(8, 15), None):
        with pytest.raises(NotImplementedError, match="cached position"):
            layer(prompt, past_key_values=caches[0], cache_position=pos)
    assert torch.equal(caches[0].key_cache(0), k_before) and caches[0].get_seq_length(0) == 8
    # the refused calls were recorded in the process-wide coverage ledger as failures
    assert ts.compatibility.report(layer)["summary"]["runtime_failures"] >= 1
    ts.compatibility.reset_runtime_observations()
    caches[0].reset()
    layer(prompt, past_key_values=caches[0], cache_position=torch.arange(7, device=device))
    assert caches[0].get_seq_length(0) == 7


def _first_divergence(a: torch.Tensor, b: torch.Tensor):
    diff = (a != b).nonzero()
    return None if diff.numel() == 0 else tuple(int(v) for v in diff[0])


def test_auto_model_and_hf_generate_through_the_swapped_model(device, tmp_path):
    tiny_hf_model(seed=6).save_pretrained(tmp_path)
    B, S, n_new = 2, 12, 8
    kv = {"block_size": 16, "max_num_blocks": 128, "batch_size": B}
    model = ts.AutoModelForCausalLM.from_pretrained(str(tmp_path), kv_cache_kwargs=kv)
    ts.set_device(model, device)
    twin = ts.AutoModelForCausalLM.from_pretrained(str(tmp_path), kv_cache_kwargs=kv)
    ts.set_device(twin, device)
    ids = torch.randint(0, 1000, (B, S), generator=torch.Generator().manual_seed(7))
    with torch.no_grad():
        out = model.generate(ids.to(device), max_new_tokens=n_new, do_sample=False,
                             past_key_values=model._tt_kv_cache, return_dict_in_generate=True,
                             output_scores=True)
    hf_tokens = out.sequences[:, S:].cpu()
    assert hf_tokens.shape == (B, n_new)
    cache = model._tt_kv_cache
    for layer in range(3):
        assert cache.get_seq_length(layer) == S + n_new - 1
    trunk, head = model_parts(twin)
    dev_tokens = greedy_generate(trunk, head, ids, twin._tt_kv_cache, n_new).tokens.long()
    first = _first_divergence(hf_tokens, dev_tokens)
    if first is not None:
        b, j = first
        top2 = out.scores[j][b].float().topk(2).values
        margin = float(top2[0] - top2[1])
        assert margin < 1e-2 * max(float(top2[0].abs()), 1.0), \
            f"row {b} step {j}: HF generate {int(hf_tokens[b, j])}, device loop " \
            f"{int(dev_tokens[b, j])}, logit margin {margin:.3e}"


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn], ids=["bf16", "fp8"])
def test_prefill_in_several_groups_equals_one_group(device, kv_dtype):
    base = tiny_hf_model(seed=8)
    lens = [24, 17, 31, 9]
    prompts = [torch.randint(0, 1000, (L,), generator=torch.Generator().manual_seed(9 + L))
               for L in lens]
    results = []
    for prefill_tokens in (16384, 40):   # one group; then groups [0], [1], [2, 3]
        hip = tiny_hf_model(seed=8)
        hip.load_state_dict(base.state_dict())
        ts.apply_recipe(hip, kv_cache_kwargs={"block_size": 16, "max_num_blocks": 256,
                                              "batch_size": 4, "dtype": kv_dtype})
        ts.set_device(hip, device)
        trunk, head = model_parts(hip)
        cache = hip._tt_kv_cache
        assert cache.dtype == kv_dtype
        r = greedy_generate(trunk, head, prompts, cache, 6, prefill_tokens=prefill_tokens)
        pools = [cache.key_cache(i).view(torch.uint8).cpu() for i in range(3)]
        pools += [cache.value_cache(i).view(torch.uint8).cpu() for i in range(3)]
        scales = ([cache.key_scale(i).cpu() for i in range(3)] if cache.is_fp8 else [])
        results.append((r.tokens, pools, scales))
    (t1, p1, s1), (t2, p2, s2) = results
    assert torch.equal(t1, t2)
    assert all(torch.equal(a, b) for a, b in zip(p1, p2))
    assert all(torch.equal(a, b) for a, b in zip(s1, s2))


@pytest.mark.parametrize("rows", [3, 70])
@pytest.mark.parametrize("V", [1000, 1024])
def test_lm_head_logits_for_any_vocab_size(device, rows, V):
    g = torch.Generator().manual_seed(rows + V)
    w = (torch.randn(V, 512, generator=g) * 0.05).bfloat16()
    x = torch.randn(rows, 512, generator=g).bfloat16()
    head = ts.HIPLMHead.from_weight(w)
    ts.set_device(head, device)
    got = head(x.to(device)).cpu()
    want = x.float() @ w.float().T
    assert got.shape == (rows, V) and got.dtype == torch.float32
    assert bool(((got - want).abs() <= 1e-3 + 1e-3 * want.abs()).all())
