"""The BailingMoeV2 workloads at their full sizes on the GPU (through the C ABI), against the
oracle where the oracle can run in a test's time and through size-independent properties
elsewhere.

  * fp8 decode: batch 128, cached lengths U[1024, 8192], fp8 e4m3 block-scaled experts and an
    fp8 KV cache. The whole batch runs on the GPU; 16 of its sequences are compared with the
    oracle layer on the dequantised weights and on those sequences' dequantised blocks.
  * prefill: 8 packed prompts of U[256, 2048] tokens with Zipf-skewed expert load. The shortest
    and the longest prompt against the oracle (GPU routing replayed); for every token of every
    prompt, the K and V rows the prologue wrote into the paged pool against fp32 (input RMSNorm,
    projection, QK-norm, RoPE); the permutation of all the assignments bit-exact against the C
    oracle; the expert load skewed as drawn.
  * whole model: 20 layers (dense layer 0, 19 MoE), vocab 157184, batch 64 prompts of 2048
    tokens, 128 greedy tokens: the captured decode loop gives exactly the eager loop's tokens.

Tolerances as the layer tests: max-abs 2e-2 on layer outputs; a routing difference only at a
router near tie (selection margin < 2e-3), where the oracle takes the GPU's choice.
"""
import numpy as np
import pytest
import torch

import tt_symbiote_amd as ts
from oracle.bailing_moe_v2 import decoder_layer_from_weights, rope_inv_freq, rotate_half
from oracle.fp8 import decode_e4m3, dequant_blocks
from oracle.paged_kv import PagedKVCacheRef
from oracle.route import permute_c, route_torch, selection_margins
from test_gpu_layer import FLIP_MARGIN, TOL, _oracle_with_gpu_routing
from tt_symbiote_amd import hip_ops
from tt_symbiote_amd.workloads import (LING_MINI_2, build_decoder_layer,
                                       build_dense_decoder_layer, fp8_kv_pools, layer_weights,
                                       model_config, paged_context, prefill_batch,
                                       prefill_layer_config, zipf_expert_bias)

pytestmark = pytest.mark.gpu


def _dequant_sequences(codes, scales, page_table, positions, block_size, seqs):
    """fp32 pool of the blocks of sequences ``seqs`` (codes [nb, Hkv, bs, D] e4m3 bytes,
    scales [nb, Hkv]) and the page table of those sequences over it."""
    nblk = [(int(positions[b]) + 1 + block_size - 1) // block_size for b in seqs]
    phys = torch.cat([page_table[b, :n].long() for b, n in zip(seqs, nblk)])
    vals = torch.from_numpy(decode_e4m3(codes[phys].numpy()))
    pool = vals * scales[phys][..., None, None]
    table = torch.zeros(len(seqs), max(nblk), dtype=torch.int64)
    o = 0
    for i, n in enumerate(nblk):
        table[i, :n] = torch.arange(o, o + n)
        o += n
    return pool, table


def test_fp8_decode_layer_batch128_long_contexts(device):
    shape = LING_MINI_2
    E = shape.num_experts
    w = layer_weights(shape, seed=0)
    layer = build_decoder_layer(w, shape, weight_format="fp8_e4m3")
    ts.set_device(layer, device)
    layer.mlp.keep_last_route = True
    deq = {}
    for name in ("gate_up", "down"):
        bf = layer.mlp._dev[name]
        deq[name] = torch.from_numpy(dequant_blocks(bf.q.view(torch.uint8).cpu().numpy(),
                                                    bf.scale.cpu().numpy())).bfloat16()
    wq = dict(w, gate_up=deq["gate_up"][:E], down=deq["down"][:E],
              shared_gate_up=deq["gate_up"][E], shared_down=deq["down"][E])
    oracle = decoder_layer_from_weights(wq, shape, dtype=torch.float32)
    del deq, wq

    B, bs = 128, 32
    ctx = paged_context(B, 1024, 8192, block_size=bs, num_kv_heads=4, seed=1, slack=1.25,
                        kv_device=device)
    kp, ks = fp8_kv_pools(ctx.k_pool)
    vp, vs = fp8_kv_pools(ctx.v_pool)
    nb = kp.shape[0]
    pcfg = ts.PagedAttentionConfig(block_size=bs, max_num_blocks=nb, batch_size=1)
    cache = ts.HIPPagedAttentionKVCache(1, 4, 128, pcfg, dtype=torch.float8_e4m3fn)
    cache.to_device(device)
    cache.key_cache(0).copy_(kp)
    cache.value_cache(0).copy_(hip_ops.fp8_v_pool(vp))
    cache.key_scale(0).copy_(ks)
    cache.value_scale(0).copy_(vs)
    cache.set_vllm_page_table(ctx.page_table)
    x = torch.randn(B, 1, 2048, generator=torch.Generator().manual_seed(2)).bfloat16()
    out = layer(x.to(device), past_key_values=cache,
                cache_position=ctx.positions.to(device))[0]
    torch.cuda.synchronize()
    assert int(ctx.context_lens.min()) >= 1024 and int(ctx.context_lens.max()) <= 8192

    seqs = list(range(0, B, 8))
    kpool, table = _dequant_sequences(kp.view(torch.uint8).cpu(), ks.cpu(), ctx.page_table,
                                      ctx.positions, bs, seqs)
    vpool, _ = _dequant_sequences(vp.view(torch.uint8).cpu(), vs.cpu(), ctx.page_table,
                                  ctx.positions, bs, seqs)
    del kp, vp, ctx.k_pool, ctx.v_pool
    ref_cache = PagedKVCacheRef([kpool], [vpool], table)
    pos = ctx.positions[seqs].long()
    ref, flips = _oracle_with_gpu_routing(
        oracle, layer.mlp,
        lambda: oracle(x[seqs].float(), past_key_value=ref_cache, cache_position=pos)[0],
        rows=seqs)
    err = (out[seqs].float().cpu() - ref).abs().max().item()
    print(f"fp8 batch 128: {int(ctx.context_lens.sum())} cached tokens, max|gpu-oracle| over "
          f"{len(seqs)} sequences = {err:.3e}, routing flips {flips}")
    assert err <= TOL
    assert bool(torch.isfinite(out.float()).all())


def _rope_rows(x: torch.Tensor, pos: torch.Tensor, head_dim: int, factor: float,
               theta: float) -> torch.Tensor:
    """The oracle's partial RoPE (split-half on the first head_dim * factor dims) of rows
    x [T, H, D] at positions pos [T], fp32."""
    fr = pos.float()[:, None] * rope_inv_freq(head_dim, factor, theta)[None]
    emb = torch.cat([fr, fr], -1)
    rd = emb.shape[-1]
    xr, xp = x[..., :rd], x[..., rd:]
    return torch.cat([xr * emb.cos()[:, None] + rotate_half(xr) * emb.sin()[:, None], xp], -1)


def test_prefill_layer_8_prompts_zipf(device):
    shape = LING_MINI_2
    E, H, D, Hq, Hkv = shape.num_experts, shape.hidden_size, 128, shape.num_heads, \
        shape.num_kv_heads
    wl = prefill_layer_config()
    w = layer_weights(shape, seed=0)
    w["expert_bias"] = w["expert_bias"] + zipf_expert_bias(E, wl["zipf_s"], seed=3)
    pb = prefill_batch(wl["n_seqs"], wl["len_lo"], wl["len_hi"], H, block_size=wl["block_size"],
                       slack=wl["slack"], seed=1)
    layer = build_decoder_layer(w, shape)
    ts.set_device(layer, device)
    layer.mlp.keep_last_route = True
    bs = wl["block_size"]
    cfg = ts.PagedAttentionConfig(block_size=bs, max_num_blocks=pb.num_blocks, batch_size=1)
    cache = ts.HIPPagedAttentionKVCache(1, Hkv, D, cfg)
    cache.to_device(device)
    cache.set_vllm_page_table(pb.page_table)
    out = layer.prefill_varlen(pb.x.to(device), pb.cu_seqlens.to(device), max(pb.lens), cache)
    torch.cuda.synchronize()
    out = out.float().cpu()
    T = pb.tokens
    route = layer.mlp.last_route
    gpu_idx = route.topk_idx.cpu()
    print(f"prefill: {T} tokens in prompts {pb.lens}")
    assert T > 4000 and min(pb.lens) >= 256 and max(pb.lens) <= 2048

    # the permutation of every assignment, bit-exact
    p = permute_c(gpu_idx.numpy(), E, with_shared=True)
    for key in ("expert_counts", "expert_offsets", "sorted_tokens", "inv_perm", "n_segments"):
        assert np.array_equal(getattr(route, key).cpu().numpy(), p[key]), key
    ns = int(p["n_segments"][0])
    for key in ("seg_expert", "seg_offset", "seg_count"):
        assert np.array_equal(getattr(route, key).cpu().numpy()[:ns], p[key][:ns]), key
    counts = p["expert_counts"].astype(np.float64)
    assert counts.max() / counts.mean() > 4.0   # Zipf-skewed load

    # K and V rows of every token in the pool, against fp32
    x = pb.x.float()
    xn = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + shape.rms_norm_eps) * w["ln1"].float()
    wk = w["qkv_w"].float()[Hq * D:(Hq + 2 * Hkv) * D]
    kv = (xn @ wk.T).view(T, 2 * Hkv, D)
    k, v = kv[:, :Hkv], kv[:, Hkv:]
    k = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + shape.rms_norm_eps) * \
        w["k_norm"].float()
    pos = torch.cat([torch.arange(L) for L in pb.lens])
    seq = torch.repeat_interleave(torch.arange(len(pb.lens)), torch.tensor(pb.lens))
    k = _rope_rows(k, pos, D, shape.partial_rotary_factor, shape.rope_theta)
    rows = pb.page_table[seq, pos // bs].long()
    kg = cache.key_cache(0).float().cpu()[rows, :, pos % bs]
    vg = cache.value_cache(0).float().cpu()[rows, :, pos % bs]
    k_err = (kg - k).abs() - 1e-2 * k.abs()
    v_err = (vg - v).abs() - 1e-2 * v.abs()
    assert k_err.max().item() <= 3e-2 and v_err.max().item() <= 3e-2

    # the shortest and the longest prompt against the oracle
    oracle = decoder_layer_from_weights(w, shape, dtype=torch.float32)
    gate = oracle.mlp.gate
    kw = dict(n_group=gate.n_group, topk_group=gate.topk_group, top_k=gate.top_k)
    cu = pb.cu_seqlens.tolist()
    for s in (int(np.argmin(pb.lens)), int(np.argmax(pb.lens))):
        a, b, L = cu[s], cu[s + 1], pb.lens[s]
        nblk = (L + bs - 1) // bs
        ref_cache = PagedKVCacheRef([torch.zeros(nblk, Hkv, bs, D)],
                                    [torch.zeros(nblk, Hkv, bs, D)],
                                    torch.arange(nblk)[None])
        gate.route_override = gpu_idx[a:b]
        try:
            with torch.no_grad():
                ref = oracle(x[a:b][None], past_key_value=ref_cache,
                             cache_position=torch.arange(L)[None])[0][0]
        finally:
            gate.route_override = None
        logits = gate.last_routing[0]
        own, _ = route_torch(logits, gate.expert_bias, routed_scale=1.0, **kw)
        same = (gpu_idx[a:b].long().sort(-1).values == own.sort(-1).values).all(-1)
        flips = (~same).nonzero().flatten().tolist()
        if flips:
            margins = selection_margins(logits, gate.expert_bias, **kw)
            assert all(float(margins[t]) < FLIP_MARGIN for t in flips), (s, flips)
        diff = (out[a:b] - ref).abs()
        # the 2e-2 bar on top of the bf16 output's own rounding (up to 1.6e-2 where |y| >= 4)
        err = (diff - _bf16_half_ulp(ref)).max().item()
        print(f"prompt {s} ({L} tokens): max|gpu-oracle| = {diff.max().item():.3e} "
              f"({err:.3e} beyond the output's bf16 rounding, max |y| {ref.abs().max().item():.1f}, "
              f"max|gpu-bf16(oracle)| {(out[a:b] - ref.bfloat16().float()).abs().max().item():.3e}), "
              f"routing flips {len(flips)}")
        assert err <= TOL


# The whole-model run's oracle checkpoints: sequences (one per prefill group of 8 prompts, at
# both ends of the batch), layers (the dense layer, the first and the last MoE layer) and decode
# steps (the first and the last).
TRACK_SEQS = (0, 21, 42, 63)
TRACK_LAYERS = (0, 1, 19)
TRACK_STEPS = (1, 127)


def _bf16_half_ulp(y: torch.Tensor) -> torch.Tensor:
    """Half the bf16 spacing at each value of y (the most that rounding y to bf16 moves it)."""
    _, e = torch.frexp(y.float())
    return torch.ldexp(torch.ones_like(y, dtype=torch.float32), e - 9)


class _LayerTap:
    """Records, in the eager loop, the tracked sequences' rows entering and leaving one decoder
    layer and the GPU's expert choice for them: at the prompt's last token (prefill) and at
    the tracked decode steps (the layer's n-th decode call is step n)."""

    def __init__(self, layer, seqs, steps):
        self.seqs, self.steps, self.step = seqs, steps, 0
        self.rec = {}
        mlp = layer.mlp
        moe = not layer.is_dense_layer
        if moe:
            mlp.keep_last_route = True
        fwd, pre = layer.forward, layer.prefill_varlen

        def keep(point, x, y, rows, seqs_here):
            x, y = x.reshape(-1, x.shape[-1]), y.reshape(-1, y.shape[-1])
            idx = mlp.last_route.topk_idx if moe else None
            for b, r in zip(seqs_here, rows):
                self.rec[(b, point)] = (x[r].cpu(), y[r].cpu(),
                                        None if idx is None else idx[r].cpu().long())

        def forward(hidden_states, *a, **kw):
            out = fwd(hidden_states, *a, **kw)
            self.step += 1
            if self.step in self.steps:
                keep(self.step, hidden_states, out[0], list(self.seqs), list(self.seqs))
            return out

        def prefill_varlen(x, cu_seqlens, max_seqlen, cache, positions=None, seq_ids=None):
            out = pre(x, cu_seqlens, max_seqlen, cache, positions=positions, seq_ids=seq_ids)
            sid = seq_ids.cpu()
            here = [b for b in self.seqs if bool((sid == b).any())]
            rows = [int((sid == b).nonzero().max()) for b in here]
            keep(0, x, out, rows, here)
            return out

        layer.forward, layer.prefill_varlen = forward, prefill_varlen


class _HeadTap:
    """Records every greedy call of the LM head in the eager loop: its input (the GPU's final
    normed hidden rows) and the ids it chose."""

    def __init__(self, head):
        self.calls = []
        greedy = head.greedy

        def tapped(x, ids=None):
            out = greedy(x, ids=ids)
            self.calls.append((x.reshape(-1, x.shape[-1]).clone(), out.clone()))
            return out

        head.greedy = tapped


def _routed_oracle(oracle_layer, gpu_idx, run):
    """Run the oracle MoE layer with the GPU's expert choice ``gpu_idx`` [n, K]; the oracle's
    own choice may differ only at a router near tie. Returns the output."""
    gate = oracle_layer.mlp.gate
    gate.route_override = gpu_idx
    try:
        with torch.no_grad():
            out = run()
    finally:
        gate.route_override = None
    logits = gate.last_routing[0]
    kw = dict(n_group=gate.n_group, topk_group=gate.topk_group, top_k=gate.top_k)
    own, _ = route_torch(logits, gate.expert_bias, routed_scale=1.0, **kw)
    diff = (own.sort(-1).values != gpu_idx.sort(-1).values).any(-1)
    if bool(diff.any()):
        m = selection_margins(logits, gate.expert_bias, **kw)[diff]
        assert bool((m < FLIP_MARGIN).all()), f"routing differs at margins {m.tolist()}"
    return out


def test_whole_model_generate_graph_equals_eager(device):
    """The 20-layer, vocab-157184 model at batch 64 (prompts of 2048 tokens, 128 greedy tokens):
      * the captured decode loop gives exactly the eager loop's tokens;
      * layers 0 (dense), 1 and 19 against the fp32 oracle layer for 4 sequences at the prompt's
        last token and at decode steps 1 and 127: the oracle runs the recorded input row over
        the sequence's own cache pages as the GPU wrote them, with the GPU's expert choice;
        max-abs 2e-2 on the layer output beyond the rounding of the output to bf16, and the
        new K/V slot as the oracle writes it;
      * every chosen token (64 x 128) is the argmax of exact (float64) logits of the GPU's own
        final hidden rows, or equal to the maximum within fp32 summation rounding."""
    from oracle.bailing_moe_v2 import dense_decoder_layer_from_weights
    from tt_symbiote_amd.generate import greedy_generate
    from tt_symbiote_amd.modules.model import HIPBailingMoeV2Model, HIPLMHead
    from tt_symbiote_amd.workloads import dense_layer_weights

    shape = LING_MINI_2
    mc = model_config()
    B, L, n_new, V, H = mc["batch"], mc["prompt_len"], mc["new_tokens"], mc["vocab_size"], \
        shape.hidden_size
    dense_I = mc["dense_intermediate_size"]
    layers = []
    for i in range(mc["num_layers"]):
        if i < mc["first_k_dense_replace"]:
            layer = build_dense_decoder_layer(shape, dense_I, seed=i, device=device, layer_idx=i)
        else:
            lw = layer_weights(shape, seed=i, device=device)
            layer = build_decoder_layer(lw, shape, layer_idx=i)
            del lw
        ts.set_device(layer, device)
        layers.append(layer)
    g = torch.Generator(device=device).manual_seed(100)
    embed = (torch.randn(V, H, generator=g, device=device) * 0.02).bfloat16()
    head_w = (torch.randn(V, H, generator=g, device=device) * 0.02).bfloat16()
    norm_w = (1.0 + 0.02 * torch.randn(H, generator=g, device=device)).bfloat16()
    trunk = HIPBailingMoeV2Model.from_modules(embed, layers, norm_w, shape.rms_norm_eps)
    head = HIPLMHead.from_weight(head_w)
    ts.set_device(trunk, device)
    ts.set_device(head, device)
    del embed, head_w
    cfg = ts.PagedAttentionConfig(block_size=mc["block_size"],
                                  max_num_blocks=mc["max_num_blocks"], batch_size=B)
    cache = ts.HIPPagedAttentionKVCache(mc["num_layers"], shape.num_kv_heads, shape.head_dim,
                                        cfg, device=device)
    prompts = torch.randint(0, V, (B, L), generator=torch.Generator().manual_seed(7))

    taps = {i: _LayerTap(layers[i], TRACK_SEQS, TRACK_STEPS) for i in TRACK_LAYERS}
    head_tap = _HeadTap(head)
    eager = greedy_generate(trunk, head, prompts, cache, n_new, use_graph=False)
    del head.greedy                                 # the graph run uses the plain method
    for i in TRACK_LAYERS:
        del layers[i].forward, layers[i].prefill_varlen
    # the tracked sequences' pages as the eager loop wrote them (the graph loop rewrites them
    # with the same bytes)
    bs = mc["block_size"]
    nblk = (L + n_new - 1 + bs - 1) // bs
    pages = {}
    for i in TRACK_LAYERS:
        for b in TRACK_SEQS:
            blocks = cache.page_table[b, :nblk].long().to(device)
            pages[(i, b)] = (cache.key_cache(i)[blocks].float().cpu(),
                             cache.value_cache(i)[blocks].float().cpu())
    cache.reset()
    graph = greedy_generate(trunk, head, prompts, cache, n_new, use_graph=True)
    assert eager.tokens.shape == (B, n_new)
    assert torch.equal(eager.tokens, graph.tokens)
    assert cache.get_seq_length(0) == L + n_new - 1
    # the tokens are not degenerate (a stuck loop would repeat one id)
    assert len(torch.unique(graph.tokens)) > B
    print(f"whole model: {B} x {n_new} tokens identical between the captured and the eager "
          f"loop; decode {graph.decode_s / graph.decode_steps * 1e3:.2f} ms/step", flush=True)

    # every greedy choice against exact logits of the GPU's own final hidden rows
    w64 = head.weight.double()
    n_rows = ties = 0
    min_gap = float("inf")
    for x, ids in head_tap.calls:
        logits = x.double() @ w64.T
        top2 = logits.topk(2, dim=-1)
        picked = logits.gather(1, ids.long()[:, None])[:, 0]
        gap = top2.values[:, 0] - picked
        exact = ids.long() == top2.indices[:, 0]
        assert bool(((gap <= 1e-4) | exact).all()), \
            f"LM head choice {gap.max().item():.3e} below the maximum logit"
        ties += int((~exact).sum())
        n_rows += ids.numel()
        min_gap = min(min_gap, float((top2.values[:, 0] - top2.values[:, 1]).min()))
    del w64
    assert n_rows == B * n_new
    print(f"LM head: {n_rows} choices, {n_rows - ties} the exact argmax, {ties} within fp32 "
          f"rounding of it; smallest top-2 gap {min_gap:.3e}", flush=True)

    # the tracked layers against the oracle over the GPU-written pages
    worst, scale = {}, {}
    for i in TRACK_LAYERS:
        if i < mc["first_k_dense_replace"]:
            w = dense_layer_weights(shape, dense_I, seed=i, device=device)
            oracle = dense_decoder_layer_from_weights({k: v.cpu() for k, v in w.items()},
                                                      shape, dense_I)
        else:
            w = layer_weights(shape, seed=i, device=device)
            oracle = decoder_layer_from_weights({k: v.cpu() for k, v in w.items()}, shape)
        del w
        for b in TRACK_SEQS:
            kb, vb = pages[(i, b)]
            for point in (0,) + TRACK_STEPS:
                x_in, y_gpu, idx = taps[i].rec[(b, point)]
                p = L - 1 + point                # the position of the token the layer ran
                ref_cache = PagedKVCacheRef([kb.clone()], [vb.clone()],
                                            torch.arange(nblk)[None])
                run = lambda: oracle(x_in.float().view(1, 1, H), past_key_value=ref_cache,
                                     cache_position=torch.tensor([p]))[0]
                if idx is None:
                    with torch.no_grad():
                        y_ref = run()
                else:
                    y_ref = _routed_oracle(oracle, idx[None], run)
                y_ref = y_ref.view(H)
                # the 2e-2 bar on top of the bf16 output's own rounding (half an ulp of the
                # exact value): the residual stream grows through the layers (|y| above 8 at
                # layer 19), where rounding alone exceeds 2e-2
                excess = (y_gpu.float() - y_ref).abs() - _bf16_half_ulp(y_ref)
                err = excess.max().item()
                scale[(i, point)] = max(scale.get((i, point), 0.0), y_ref.abs().max().item())
                slot = (p // bs, p % bs)
                kv_err = max((kb[slot[0], :, slot[1]] -
                              ref_cache.k_pools[0][slot[0], :, slot[1]]).abs().max().item(),
                             (vb[slot[0], :, slot[1]] -
                              ref_cache.v_pools[0][slot[0], :, slot[1]]).abs().max().item())
                worst[(i, point)] = max(worst.get((i, point), 0.0), err)
                assert err <= TOL, \
                    f"layer {i} seq {b} position {p}: max err {err:.3e} beyond bf16 rounding"
                assert kv_err <= 3e-2, f"layer {i} seq {b} position {p}: K/V slot {kv_err:.3e}"
        del oracle
    print("oracle checkpoints, max over sequences " + str(TRACK_SEQS) + " of the error beyond "
          "the output's bf16 rounding (and max |y|): " + "; ".join(
              f"layer {i} {'prefill' if pt == 0 else 'step ' + str(pt)} {e:.2e} "
              f"({scale[(i, pt)]:.1f})" for (i, pt), e in sorted(worst.items())), flush=True)
