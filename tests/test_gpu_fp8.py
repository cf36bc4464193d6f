"""The fp8 formats on the GPU, through the C ABI, against the fp8 oracle (oracle/fp8.py).

  * grouped SwiGLU with 128 x 128 block-scaled e4m3fn expert weights vs fp32 torch over the
    oracle's dequantisation of the same bytes (the "dequantise, then compute" reference);
  * fp8 KV fill over ragged sequences with non-zero starts (so partly filled blocks are
    appended to, and requantised when their scale grows): pools and scales bit-exact against
    the oracle's kv_block_append;
  * fp8 paged decode vs fp32 attention over the oracle-dequantised pools;
  * the fused fp8 decode step equals the prologue + fp8 fill of the new token + plain fp8
    decode (outputs, pools and scales bit-exact);
  * the decoder layer with fp8 experts and an fp8 cache vs the oracle layer on the dequantised
    weights and pools (bf16 reference), max-abs <= 2e-2.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import tt_symbiote_amd as ts
from oracle.fp8 import decode_e4m3, dequant_blocks, kv_block_append
from oracle.paged_kv import PagedKVCacheRef, paged_decode_ref
from tt_symbiote_amd import hip_ops
from tt_symbiote_amd.workloads import paged_context

pytestmark = pytest.mark.gpu


def _close(got, want, atol, rtol):
    got = got.float().cpu()
    want = want.float().cpu()
    err = (got - want).abs()
    bound = atol + rtol * want.abs()
    assert bool((err <= bound).all()), \
        f"max err {err.max().item():.3e}, worst excess {(err - bound).max().item():.3e}"


def _deq(bf: hip_ops.BlockFp8) -> torch.Tensor:
    q = bf.q.view(torch.uint8).cpu().numpy()
    return torch.from_numpy(dequant_blocks(q, bf.scale.cpu().numpy()))


# ------------------------------------------------------------------------------ grouped GEMM
@pytest.mark.parametrize("T,E,H,I,top_k,skew", [
    (1, 64, 512, 128, 4, False),
    (32, 256, 2048, 512, 8, False),
    (128, 256, 2048, 512, 8, False),
    (90, 64, 1024, 256, 6, True),       # segments of more than 16 rows (several passes)
])
def test_grouped_swiglu_fp8(device, T, E, H, I, top_k, skew):
    g = torch.Generator().manual_seed(T + H)
    x = torch.randn(T, H, generator=g).bfloat16()
    slots = E + 1
    wgu = (torch.randn(slots, 2 * I, H, generator=g) * 0.05).bfloat16()
    wd = (torch.randn(slots, H, I, generator=g) * 0.05).bfloat16()
    wgu[3, :128, :128] = 0                                   # an all-zero block (scale 1)
    logits = torch.randn(T, E, generator=g) * 2
    if skew:
        logits[:, :4] += 6.0
    res = hip_ops.moe_route_permute(logits.to(device), torch.zeros(E, device=device),
                                    n_group=8, topk_group=4, top_k=top_k, routed_scale=2.5,
                                    with_shared=True)
    qgu = hip_ops.quantize_block_fp8(wgu.to(device))
    qd = hip_ops.quantize_block_fp8(wd.to(device))
    h, y = hip_ops.moe_grouped_swiglu(x.to(device), res, qgu, qd)
    torch.cuda.synchronize()
    wgu_f, wd_f = _deq(qgu), _deq(qd)
    st = res.sorted_tokens.cpu().long()
    ns = int(res.n_segments.item())
    hk, yk, xf = h.cpu(), y.cpu(), x.float()
    for e, o, c in zip(res.seg_expert.cpu()[:ns].tolist(), res.seg_offset.cpu()[:ns].tolist(),
                       res.seg_count.cpu()[:ns].tolist()):
        rows = slice(o, o + c)
        xe = xf[st[rows]]
        h_ref = F.silu(xe @ wgu_f[e, :I].T) * (xe @ wgu_f[e, I:].T)
        _close(hk[rows], h_ref, atol=2e-3, rtol=8e-3)
        y_ref = hk[rows].float() @ wd_f[e].T
        torch.testing.assert_close(yk[rows], y_ref, rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------------------ KV fill
def _fp8_pools(nb, Hkv, bs, device):
    """Empty fp8 pools: K [nb, Hkv, bs, 128], V dim-major [nb, Hkv, 128, bs], and scales."""
    zk = torch.zeros(nb, Hkv, bs, 128, dtype=torch.float8_e4m3fn, device=device)
    zv = torch.zeros(nb, Hkv, 128, bs, dtype=torch.float8_e4m3fn, device=device)
    s = torch.zeros(nb, Hkv, dtype=torch.float32, device=device)
    return zk, zv, s, s.clone()


def _oracle_fill(kp, vp, ks, vs, k, v, cu, starts, table, bs):
    """kv_block_append over numpy pools (codes [nb, Hkv, bs, D], scales [nb, Hkv])."""
    n = len(cu) - 1
    Hkv = kp.shape[1]
    for s in range(n):
        L = cu[s + 1] - cu[s]
        st = starts[s]
        if L <= 0 or st < 0:
            continue
        p = st
        while p < st + L:
            blk = p // bs
            p1 = min(st + L, (blk + 1) * bs)
            phys = int(table[s, blk])
            n_old = p - blk * bs
            rows = np.arange(cu[s] + (p - st), cu[s] + (p1 - st))
            for g in range(Hkv):
                for pool, sc, src in ((kp, ks, k), (vp, vs, v)):
                    codes, snew = kv_block_append(pool[phys, g], sc[phys, g], n_old,
                                                  src[rows, g])
                    pool[phys, g] = codes
                    sc[phys, g] = snew
            p = p1


def test_kv_fill_fp8_bit_exact(device):
    bs, Hkv, D = 32, 4, 128
    lens = [1, 31, 33, 100, 7, 64]
    g = torch.Generator().manual_seed(11)
    nb = 64
    perm = torch.randperm(nb, generator=g)
    table = torch.full((len(lens), 8), -1, dtype=torch.int32)
    for s in range(len(lens)):
        table[s] = perm[s * 8:(s + 1) * 8].to(torch.int32)
    kp, vp, ks, vs = _fp8_pools(nb, Hkv, bs, device)
    okp = np.zeros((nb, Hkv, bs, D), np.uint8)
    ovp, oks, ovs = okp.copy(), np.zeros((nb, Hkv), np.float32), np.zeros((nb, Hkv), np.float32)
    # first call: prompts from position 0; second call: appends from where they ended, with
    # some sequences scaled up (their last block's scale grows) and some down
    starts1 = [0] * len(lens)
    second = [5, 2, 40, 3, 1, 30]
    scale2 = [3.0, 0.3, 1.0, 8.0, 0.5, 2.0]
    for call, (Ls, starts, mult) in enumerate(((lens, starts1, [1.0] * 6),
                                                (second, lens, scale2))):
        cu = np.concatenate([[0], np.cumsum(Ls)]).astype(np.int32)
        T = int(cu[-1])
        k = torch.randn(T, Hkv, D, generator=g)
        v = torch.randn(T, Hkv, D, generator=g)
        for s in range(len(Ls)):
            k[cu[s]:cu[s + 1]] *= mult[s]
            v[cu[s]:cu[s + 1]] *= mult[s] * 0.7
        k, v = k.bfloat16(), v.bfloat16()
        hip_ops.paged_kv_fill_fp8(
            k.to(device), v.to(device), torch.from_numpy(cu).to(device), max(Ls), kp, vp, ks, vs,
            table.to(device), start_pos=torch.tensor(starts, dtype=torch.int32, device=device))
        _oracle_fill(okp, ovp, oks, ovs, k.float().numpy(), v.float().numpy(), cu, starts,
                     table.numpy(), bs)
    torch.cuda.synchronize()
    assert np.array_equal(ks.cpu().numpy(), oks)
    assert np.array_equal(vs.cpu().numpy(), ovs)
    assert np.array_equal(kp.view(torch.uint8).cpu().numpy(), okp)
    # the V pool is dim-major inside each (block, head); the oracle keeps token rows
    assert np.array_equal(hip_ops.fp8_v_rows(vp.view(torch.uint8)).cpu().numpy(), ovp)


def test_kv_fill_fp8_htd_layout_and_skips(device):
    """[Hkv, S, D] input (paged_fill_on_device's layout) equals the [S, Hkv, D] one; a negative
    start skips the sequence."""
    bs, Hkv, S = 16, 2, 45
    g = torch.Generator().manual_seed(12)
    k = torch.randn(S, Hkv, 128, generator=g).bfloat16().to(device)
    v = torch.randn(S, Hkv, 128, generator=g).bfloat16().to(device)
    table = torch.arange(8, dtype=torch.int32).reshape(2, 4).to(device)
    cu = torch.tensor([0, S], dtype=torch.int32, device=device)
    a = _fp8_pools(8, Hkv, bs, device)
    b = _fp8_pools(8, Hkv, bs, device)
    hip_ops.paged_kv_fill_fp8(k, v, cu, S, *a, table)
    hip_ops.paged_kv_fill_fp8(k.transpose(0, 1).contiguous(), v.transpose(0, 1).contiguous(),
                              cu, S, *b, table, layout="htd")
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.uint8) if x.dtype != torch.float32 else x,
                           y.view(torch.uint8) if y.dtype != torch.float32 else y)
    c = _fp8_pools(8, Hkv, bs, device)
    hip_ops.paged_kv_fill_fp8(k, v, cu, S, *c, table,
                              start_pos=torch.tensor([-1], dtype=torch.int32, device=device))
    assert not bool(c[0].view(torch.uint8).any()) and not bool(c[2].any())


# ------------------------------------------------------------------------------ decode
def _random_fp8_cache(nb, Hkv, bs, seed, device):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 256, (2, nb, Hkv, bs, 128), generator=g, dtype=torch.int32)
    codes[(codes & 0x7F) == 0x7F] = 0x10                      # no NaN codes
    codes = codes.to(torch.uint8)
    scales = 2.0 ** torch.randint(-9, -4, (2, nb, Hkv), generator=g).float()
    kp = codes[0].view(torch.float8_e4m3fn).to(device)
    vp = hip_ops.fp8_v_pool(codes[1].view(torch.float8_e4m3fn)).to(device)  # dim-major V
    return kp, vp, scales[0].to(device), scales[1].to(device), codes, scales


def _deq_pool(codes, scales):
    vals = torch.from_numpy(decode_e4m3(codes.numpy()))
    return vals * scales[..., None, None]


@pytest.mark.parametrize("B,Hq,Hkv,bs,lo,hi", [
    (1, 16, 4, 32, 512, 512),
    (16, 16, 4, 32, 128, 3000),
    (4, 8, 8, 16, 0, 40),
    (3, 16, 2, 64, 250, 600),
    (2, 32, 4, 32, 1000, 2100),
])
def test_paged_decode_fp8(device, B, Hq, Hkv, bs, lo, hi):
    ctx = paged_context(B, lo, hi, block_size=bs, num_kv_heads=Hkv, seed=B + Hq + bs)
    nb = ctx.k_pool.shape[0]
    kp, vp, ks, vs, codes, scales = _random_fp8_cache(nb, Hkv, bs, B * 3 + Hkv, device)
    q = torch.randn(B, Hq, 128, generator=torch.Generator().manual_seed(1)).bfloat16()
    scale = 128 ** -0.5
    out = hip_ops.paged_gqa_decode(q.to(device), kp, vp, ctx.page_table.to(device),
                                   ctx.positions.to(device), scale, k_scale=ks, v_scale=vs)
    ref = paged_decode_ref(q.float(), _deq_pool(codes[0], scales[0]),
                           _deq_pool(codes[1], scales[1]), ctx.page_table, ctx.positions, scale)
    _close(out, ref, atol=1e-2, rtol=1e-2)


def test_paged_decode_fp8_split_boundaries(device):
    """Contexts on either side of the 512-token split of the fp8 kernel (and of its 16-token
    tiles and 128-token waves)."""
    lens = [0, 1, 15, 16, 127, 128, 255, 256, 511, 512, 513, 1023, 1024, 1535]
    B, Hq, Hkv, bs = len(lens), 8, 2, 32
    nblk = [(L + 1 + bs - 1) // bs for L in lens]
    nb = sum(nblk) + 7
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(9))
    table = torch.zeros(B, max(nblk), dtype=torch.int32)
    o = 0
    for i, n in enumerate(nblk):
        table[i, :n] = perm[o:o + n].to(torch.int32)
        o += n
    pos = torch.tensor(lens, dtype=torch.int32)
    kp, vp, ks, vs, codes, scales = _random_fp8_cache(nb, Hkv, bs, 21, device)
    q = torch.randn(B, Hq, 128, generator=torch.Generator().manual_seed(3)).bfloat16()
    out = hip_ops.paged_gqa_decode(q.to(device), kp, vp, table.to(device), pos.to(device), 0.1,
                                   k_scale=ks, v_scale=vs)
    ref = paged_decode_ref(q.float(), _deq_pool(codes[0], scales[0]),
                           _deq_pool(codes[1], scales[1]), table, pos, 0.1)
    _close(out, ref, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("B,Hq,Hkv,rd,use_norm,lo,hi,bs,cap", [
    (8, 16, 4, 64, True, 5, 3000, 32, None),
    (5, 16, 2, 128, False, 0, 300, 16, None),
    (6, 8, 8, 64, True, 250, 600, 64, None),
    (6, 16, 4, 64, True, 100, 700, 32, 500),       # some positions beyond the attention cap
])
def test_decode_step_fp8_matches_fill_then_decode(device, B, Hq, Hkv, rd, use_norm, lo, hi, bs,
                                                   cap):
    D = 128
    ctx = paged_context(B, lo, hi, block_size=bs, num_kv_heads=Hkv, seed=B * 5 + Hkv)
    nb = ctx.k_pool.shape[0]
    pt = ctx.page_table.clone()
    pos = ctx.positions.clone()
    pos[0] = -1
    pt[1, int(pos[1]) // bs] = -1
    g = torch.Generator().manual_seed(B + rd)
    qkv = (torch.randn(B, (Hq + 2 * Hkv) * D, generator=g) * 1.5).bfloat16().to(device)
    qn = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    kn = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    inv = 1.0 / (1e6 ** (torch.arange(0, rd, 2).float() / rd))
    fr = torch.arange(4096).float()[:, None] * inv[None]
    table = torch.cat([fr.cos(), fr.sin()], 1).contiguous().to(device)
    pt_d, pos_d = pt.to(device), pos.to(device)
    kw = dict(num_heads=Hq, num_kv_heads=Hkv, rotary_dim=rd, rope_cs=table,
              q_norm_w=qn if use_norm else None, k_norm_w=kn if use_norm else None, eps=1e-6)
    max_context = cap or pt.shape[1] * bs
    kp1, vp1, ks1, vs1, _, _ = _random_fp8_cache(nb, Hkv, bs, 7, device)
    kp2, vp2, ks2, vs2 = kp1.clone(), vp1.clone(), ks1.clone(), vs1.clone()
    seq = torch.arange(B, dtype=torch.int32, device=device)
    q, k, v = hip_ops.attn_prefill_prologue(qkv, pos_d, seq, kp1, vp1, pt_d, **kw)
    cu = torch.arange(B + 1, dtype=torch.int32, device=device)
    hip_ops.paged_kv_fill_fp8(k, v, cu, 1, kp1, vp1, ks1, vs1, pt_d, start_pos=pos_d)
    ref = hip_ops.paged_gqa_decode(q, kp1, vp1, pt_d, pos_d, 0.09, max_context=max_context,
                                   k_scale=ks1, v_scale=vs1)
    out = hip_ops.attn_decode_step(qkv, pos_d, kp2, vp2, pt_d, 0.09, max_context=max_context,
                                   k_scale=ks2, v_scale=vs2, **kw)
    torch.cuda.synchronize()
    assert torch.equal(ks2, ks1) and torch.equal(vs2, vs1)
    assert torch.equal(kp2.view(torch.uint8), kp1.view(torch.uint8))
    assert torch.equal(vp2.view(torch.uint8), vp1.view(torch.uint8))
    assert torch.equal(out, ref)
    assert not bool(out[0].any())


# ------------------------------------------------------------------------------ layer
def test_decoder_layer_fp8(device):
    """Batch-32 decode step of the Ling-shaped layer with fp8 experts and an fp8 KV cache vs
    the oracle layer holding the dequantised (bf16) expert weights and pools. Bound: max-abs
    <= 2e-2 on the output; the new token's K lands in its slot within fp8 rounding."""
    from oracle.bailing_moe_v2 import decoder_layer_from_weights
    from tt_symbiote_amd.workloads import (LING_MINI_2, build_decoder_layer, decode_layer_config,
                                           fp8_kv_pools, layer_weights)
    from test_gpu_layer import TOL, _oracle_with_gpu_routing

    w = layer_weights(LING_MINI_2, seed=0)
    layer = build_decoder_layer(w, LING_MINI_2, weight_format="fp8_e4m3")
    ts.set_device(layer, device)
    layer.mlp.keep_last_route = True
    dev_w = layer.mlp._dev
    E = LING_MINI_2.num_experts
    gu = _deq(dev_w["gate_up"]).bfloat16()
    dn = _deq(dev_w["down"]).bfloat16()
    wq = dict(w, gate_up=gu[:E], down=dn[:E], shared_gate_up=gu[E], shared_down=dn[E])
    oracle = decoder_layer_from_weights(wq, LING_MINI_2, dtype=torch.float32)

    cfg = decode_layer_config("batch32")
    ctx = paged_context(cfg["batch"], cfg["ctx_lo"], cfg["ctx_hi"], block_size=cfg["block_size"],
                        num_kv_heads=4, seed=1, slack=cfg["slack"])
    nb = ctx.k_pool.shape[0]
    # K/V ~ N(0, 1) quantised per (block, head), as appending them to empty blocks would
    kp, ks = fp8_kv_pools(ctx.k_pool.to(device))
    vp, vs = fp8_kv_pools(ctx.v_pool.to(device))
    codes = torch.stack([kp.view(torch.uint8).cpu(), vp.view(torch.uint8).cpu()])
    scales = torch.stack([ks.cpu(), vs.cpu()])
    vp = hip_ops.fp8_v_pool(vp)  # the cache's V layout
    pcfg = ts.PagedAttentionConfig(block_size=cfg["block_size"], max_num_blocks=nb, batch_size=1)
    cache = ts.HIPPagedAttentionKVCache(1, 4, 128, pcfg, dtype=torch.float8_e4m3fn)
    cache.to_device(device)
    cache.key_cache(0).copy_(kp)
    cache.value_cache(0).copy_(vp)
    cache.key_scale(0).copy_(ks)
    cache.value_scale(0).copy_(vs)
    cache.set_vllm_page_table(ctx.page_table)
    x = torch.randn(cfg["batch"], 1, 2048, generator=torch.Generator().manual_seed(2)).bfloat16()
    out = layer(x.to(device), past_key_values=cache, cache_position=ctx.positions.to(device))[0]
    torch.cuda.synchronize()
    ref_cache = PagedKVCacheRef([_deq_pool(codes[0], scales[0])],
                                [_deq_pool(codes[1], scales[1])], ctx.page_table)
    ref, flips = _oracle_with_gpu_routing(
        oracle, layer.mlp,
        lambda: oracle(x.float(), past_key_value=ref_cache,
                       cache_position=ctx.positions.long())[0])
    err = (out.float().cpu() - ref).abs().max().item()
    print(f"fp8 layer: max|gpu-oracle| = {err:.3e}, routing flips on tokens {flips}")
    assert err <= TOL
    ksc = cache.key_scale(0).cpu()
    kc = cache.key_cache(0).view(torch.uint8).cpu()
    for b in range(cfg["batch"]):
        p = int(ctx.positions[b])
        phys = int(ctx.page_table[b, p // ctx.block_size])
        k_gpu = torch.from_numpy(decode_e4m3(kc[phys, :, p % ctx.block_size].numpy()))
        k_gpu = k_gpu * ksc[phys][:, None]
        k_ref = ref_cache.k_pools[0][phys, :, p % ctx.block_size]
        err_k = (k_gpu - k_ref).abs()
        assert bool((err_k <= 2.0 ** -4 * k_ref.abs() + 2.0 ** -9 * ksc[phys][:, None]
                     + 3e-2).all())
