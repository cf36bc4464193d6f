"""Decode benchmark of one Ling-mini-2.0-shaped BailingMoeV2 decoder layer on one MI355X.

Workload: one decode step of the layer (input RMSNorm, fused QKV projection, QK-norm + partial
RoPE + paged KV write, paged GQA decode attention, output projection, residual + RMSNorm,
router, top-k/permute, grouped SwiGLU experts + shared expert, combine + residual) for a batch
of 32 sequences whose cached lengths are uniform in [128, 4096], block size 32, block pool
1.25x the blocks needed, shuffled. Random-init bf16 weights (seed 0), K/V ~ N(0, 1).
A step writes the new token's K/V at each sequence's slot and reads every cached token; the
same step is repeated (same positions), so every step does identical work.

Prints one JSON line: tokens/s through the layer (batch / step time), the HBM roofline
fraction of the dominant kernel (grouped gate/up SwiGLU GEMM: bytes from the step's actual
routing / its average duration, measured with HIP events on its stream) and of the whole layer,
and the CPU oracle timed on this host's cores on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode tokens/sec @bs32 Ling-mini-2.0-shape, 1 GPU; % HBM roofline/layer"
STEPS_PER_GRAPH = 10
HBM_PEAK_GBS = 8000.0


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=5)
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches instead of replaying a captured HIP graph")
    ap.add_argument("--workload", choices=["decode", "prefill", "fp8", "generate"],
                    default="decode",
                    help="decode: the batch-32 decode step (the headline metric); prefill: 8 "
                         "packed prompts of U[256, 2048] tokens through the same layer; fp8: "
                         "the batch-128 decode step with fp8 experts and an fp8 KV cache; "
                         "generate: greedy generation with the whole 20-layer model")
    ap.add_argument("--replays-only", action="store_true",
                    help="decode workloads: stop after the timed graph replays (no per-kernel "
                         "eager pass, no bandwidth probe, no JSON), so a kernel trace ends with "
                         "the replayed steps")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain copy kernel (torch.neg, bf16) over 512 MiB three "
                         "times: the reference point that scales the FETCH_SIZE / WRITE_SIZE "
                         "counters to bytes")
    return ap.parse_args()


PMC_SUMMARY = os.path.join(ROOT, "profiles", "moe_gate_up_kernel.decode_bs32.pmc.json")
PMC_SUMMARY_FP8 = os.path.join(ROOT, "profiles", "moe_gate_up_fp8_kernel.decode_bs128.pmc.json")
CALIB_BYTES = 512 << 20


def copy_calibration() -> None:
    import torch

    n = CALIB_BYTES // 2
    src = torch.ones(n, dtype=torch.bfloat16, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    _log(f"copy calibration: 3 x torch.neg over {CALIB_BYTES >> 20} MiB read + written")


def measured_traffic(path: str = PMC_SUMMARY):
    """HBM bytes per launch of the gate/up kernel from the committed FETCH_SIZE / WRITE_SIZE
    summary of this workload (None when absent)."""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes")


def algorithmic_bytes(shape, ctx, n_routed_active: int, B: int) -> dict:
    """HBM bytes one decode step must move at minimum (bf16 weights and KV)."""
    H, I = shape.hidden_size, shape.moe_intermediate_size
    expert = 3 * I * H * 2
    gate_up_w = (n_routed_active + shape.num_shared_experts) * 2 * I * H * 2
    rows = B * shape.top_k + B * shape.num_shared_experts
    gate_up = gate_up_w + B * H * 2 + rows * I * 2          # weights + x + h
    kv_read = ctx.kv_bytes_read()
    kv_write = B * shape.num_kv_heads * shape.head_dim * 2 * 2
    layer = (shape.attention_weight_bytes() + kv_read + kv_write
             + shape.num_experts * H * 4                      # fp32 router weights
             + (n_routed_active + shape.num_shared_experts) * expert
             + 2 * H * 2 + 2 * shape.head_dim * 2            # norm weights
             + 4 * B * H * 2)                                 # activations in/out
    return dict(gate_up=gate_up, layer=layer, kv_read=kv_read,
                experts=(n_routed_active + shape.num_shared_experts) * expert)


def _cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", read from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_oracle_layer(layer, k_pool, v_pool, page_table, positions, x, steps: int, label: str):
    """Median seconds of `steps` decode steps (after 2 warm-up steps) of the oracle layer."""
    import torch

    from oracle.paged_kv import PagedKVCacheRef

    times = []
    with torch.no_grad():
        for i in range(steps + 2):
            cache = PagedKVCacheRef([k_pool], [v_pool], page_table)
            t0 = time.perf_counter()
            layer(x, past_key_value=cache, cache_position=positions)
            dt = time.perf_counter() - t0
            if i >= 2:
                times.append(dt)
            _log(f"cpu baseline {label} step {i}: {dt * 1e3:.1f} ms")
    return statistics.median(times)


def cpu_baseline(w_gpu, shape, ctx, x, steps: int, legs=True) -> dict:
    """The oracle (HF-shaped CPU module forward) on the host's cores: the reported leg is the
    same layer and batch as the GPU run in fp32; with ``legs`` the bf16 module and the
    single-sequence workload (one sequence of 512 cached tokens, 16 + 1 blocks of 32 placed by
    a random permutation of a 64-block pool) are timed too, fp32 and bf16."""
    import torch

    from oracle.bailing_moe_v2 import decoder_layer_from_weights
    from tt_symbiote_amd.workloads import decode_layer_config, paged_context

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    w = {k: v.cpu() for k, v in w_gpu.items()}
    B = x.shape[0]
    single = decode_layer_config("single")
    one = paged_context(1, single["ctx_lo"], single["ctx_hi"], block_size=single["block_size"],
                        num_kv_heads=shape.num_kv_heads, pool_blocks=single["pool_blocks"],
                        seed=11)
    x1 = torch.randn(1, 1, shape.hidden_size, generator=torch.Generator().manual_seed(12))
    cases = [("batch", ctx, x.cpu())]
    if legs:
        cases.append(("single", one, x1))
    results = []
    for dtype in ((torch.float32, torch.bfloat16) if legs else (torch.float32,)):
        layer = decoder_layer_from_weights(w, shape, dtype=dtype)
        for name, c, xc in cases:
            n = xc.shape[0]
            label = f"{name}/{str(dtype).split('.')[-1]}"
            med = _time_oracle_layer(layer, c.k_pool.to(dtype).cpu(), c.v_pool.to(dtype).cpu(),
                                     c.page_table.cpu(), c.positions.cpu().long(),
                                     xc.to(dtype), steps, label)
            # a sequence's position is its number of cached tokens
            cached = int(c.positions.cpu().long().sum())
            results.append({"workload": f"batch {n}, {cached} cached tokens",
                            "dtype": str(dtype).split(".")[-1],
                            "ms_per_step": med * 1e3, "tokens_per_s": n / med})
        del layer
    del w
    head = results[0]
    out = {"value": head["tokens_per_s"], "unit": "tokens/s", "cores": torch.get_num_threads(),
           "kind": "port",
           "sample": f"{steps} decode steps (median, after 2 warm-up) of the same layer and "
                     f"batch of {B} in fp32 on the host CPU; {head['ms_per_step']:.1f} ms/step",
           "os_cpu_count": os.cpu_count(), "cpu_model": _cpu_model()}
    if legs:
        out["legs"] = results
    return out


MFMA_BF16_PEAK_TFLOPS = 2500.0


def prefill_main(args) -> None:
    """Prefill of 8 packed prompts (lengths U[256, 2048] from the seed, Zipf-skewed expert load)
    through one layer: tokens/s, and the MFMA roofline of the dominant kernel (the tiled grouped
    gate/up GEMM)."""
    import torch

    import tt_symbiote_amd as ts
    from tt_symbiote_amd import hip_ops
    from tt_symbiote_amd.workloads import (LING_MINI_2, build_decoder_layer, layer_weights,
                                           prefill_batch, prefill_layer_config, zipf_expert_bias)

    dev = torch.device("cuda:0")
    shape = LING_MINI_2
    wl = prefill_layer_config()
    w = layer_weights(shape, seed=args.seed, device=dev)
    w["expert_bias"] = w["expert_bias"] + zipf_expert_bias(
        shape.num_experts, wl["zipf_s"], seed=args.seed + 3).to(dev)
    pb = prefill_batch(wl["n_seqs"], wl["len_lo"], wl["len_hi"], shape.hidden_size,
                       block_size=wl["block_size"], slack=wl["slack"], seed=args.seed + 1,
                       device=dev)
    layer = build_decoder_layer(w, shape)
    ts.set_device(layer, dev)
    layer.mlp.keep_last_route = True
    cfg = ts.PagedAttentionConfig(block_size=wl["block_size"], max_num_blocks=pb.num_blocks,
                                  batch_size=1)
    cache = ts.HIPPagedAttentionKVCache(1, shape.num_kv_heads, shape.head_dim, cfg)
    cache.to_device(dev)
    cache.set_vllm_page_table(pb.page_table)
    T = pb.tokens
    cu = pb.cu_seqlens
    lens_t = torch.tensor(pb.lens)
    positions = torch.cat([torch.arange(L) for L in pb.lens]).to(torch.int32).to(dev)
    seq_ids = torch.repeat_interleave(torch.arange(len(pb.lens)), lens_t).to(torch.int32).to(dev)

    def step():
        return layer.prefill_varlen(pb.x, cu, max(pb.lens), cache, positions, seq_ids)

    _log(f"prefill: {T} tokens in {len(pb.lens)} prompts {pb.lens}")
    for _ in range(max(1, args.warmup)):
        step()
    torch.cuda.synchronize()
    counts = layer.mlp.last_route.expert_counts.float()
    steps = max(1, args.steps)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    timer = hip_ops.KernelTimer(["moe_gate_up", "moe_down", "prefill_attention", "gemm"])
    hip_ops.set_kernel_timer(timer)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    hip_ops.set_kernel_timer(None)
    K, H, I = shape.top_k, shape.hidden_size, shape.moe_intermediate_size
    rows = T * K + T * shape.num_shared_experts
    gu_ms = timer.mean_ms("moe_gate_up")
    gu_tflops = 2.0 * rows * 2 * I * H / (gu_ms * 1e-3) / 1e12
    layer_flops = (2.0 * T * H * (shape.num_heads + 2 * shape.num_kv_heads) * shape.head_dim
                   + 2.0 * T * H * shape.num_heads * shape.head_dim
                   + sum(2.0 * L * L * shape.num_heads * shape.head_dim for L in pb.lens)
                   + 2.0 * T * H * shape.num_experts
                   + 2.0 * rows * 3 * I * H)
    _log(f"prefill step {ms:.2f} ms | gate_up {gu_ms * 1e3:.0f} us ({gu_tflops:.0f} TFLOP/s) | "
         f"down {timer.mean_ms('moe_down') * 1e3:.0f} us | attention "
         f"{timer.mean_ms('prefill_attention') * 1e3:.0f} us | projections "
         f"{timer.mean_ms('gemm') * 1e3:.0f} us each | expert load max/mean "
         f"{counts.max().item() / counts.mean().item():.1f}")
    print(json.dumps({
        "metric": "prefill tokens/sec, 8 packed prompts U[256,2048], Ling-mini-2.0-shape layer, "
                  "1 GPU",
        "value": T / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init bf16 weights (seed 0), Zipf-skewed expert bias (s=1.1)",
        "config": {"workload": "BailingMoeV2 decoder layer prefill, 8 packed prompts "
                               "U[256,2048], block size 32", "tokens": T, "lens": pb.lens,
                   "expert_load_max_over_mean": counts.max().item() / counts.mean().item()},
        "roofline": {"bound": "mfma", "kernel": "gemm_tile_kernel<GateUp> (grouped gate/up)",
                     "achieved": gu_tflops, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": gu_tflops / MFMA_BF16_PEAK_TFLOPS, "traffic": None,
                     "flops_per_launch": 2.0 * rows * 2 * I * H,
                     "avg_launch_us": gu_ms * 1e3},
        "layer_tflops": layer_flops / (ms * 1e-3) / 1e12,
        "cpu_baseline": None,
    }), flush=True)


def fp8_workload_config() -> dict:
    """The quantised decode workload: batch 128, cached lengths uniform in [1024, 8192], block
    size 32, pool 1.25x shuffled; fp8 e4m3fn experts with 128 x 128 block scales and an fp8 KV
    cache with per-(block, head) scales."""
    return dict(batch=128, ctx_lo=1024, ctx_hi=8192, block_size=32, slack=1.25)


def fp8_algorithmic_bytes(shape, ctx, n_routed_active: int, B: int) -> dict:
    """HBM bytes one fp8 decode step must move: e4m3fn expert weights + their fp32 block
    scales, e4m3fn K/V + one fp32 scale per (block, head) read, bf16 attention weights."""
    H, I, D, hkv = shape.hidden_size, shape.moe_intermediate_size, shape.head_dim, \
        shape.num_kv_heads
    n_exp = n_routed_active + shape.num_shared_experts
    expert = 3 * I * H + 3 * I * H // (128 * 128) * 4
    rows = B * shape.top_k + B * shape.num_shared_experts
    gate_up = n_exp * (2 * I * H + 2 * I * H // (128 * 128) * 4) + B * H * 2 + rows * I * 2
    tokens = int((ctx.context_lens + 1).sum())
    blocks = int(((ctx.context_lens + 1 + ctx.block_size - 1) // ctx.block_size).sum())
    kv_read = tokens * hkv * D * 2 + blocks * hkv * 2 * 4
    kv_write = B * hkv * D * 2
    layer = (shape.attention_weight_bytes() + kv_read + kv_write
             + shape.num_experts * H * 4 + n_exp * expert
             + 2 * H * 2 + 2 * D * 2 + 4 * B * H * 2)
    return dict(gate_up=gate_up, layer=layer, kv_read=kv_read, experts=n_exp * expert)


def generate_main(args) -> None:
    """Greedy generation with the whole Ling-mini-2.0-shaped model: 20 layers (layer 0 dense,
    intermediate 5120; 19 MoE layers), vocab 157184, batch 64 prompts of 2048 random ids, 128
    new tokens, paged KV (block 32, 8192 blocks). value = decode tokens/s (64 x 127 / the time
    of the 127 captured decode steps after the first token)."""
    import torch

    from tt_symbiote_amd import hip_ops
    from tt_symbiote_amd.generate import greedy_generate
    from tt_symbiote_amd.modules.kv_cache import HIPPagedAttentionKVCache, PagedAttentionConfig
    from tt_symbiote_amd.modules.model import HIPBailingMoeV2Model, HIPLMHead
    from tt_symbiote_amd.utils.device_management import set_device
    from tt_symbiote_amd.workloads import (LING_MINI_2, build_decoder_layer,
                                           build_dense_decoder_layer, layer_weights,
                                           model_config)

    dev = torch.device("cuda:0")
    shape = LING_MINI_2
    mc = model_config()
    B, L, n_new = mc["batch"], mc["prompt_len"], mc["new_tokens"]
    V, H = mc["vocab_size"], shape.hidden_size
    _log(f"building {mc['num_layers']} layers on the GPU ...")
    layers = []
    for i in range(mc["num_layers"]):
        if i < mc["first_k_dense_replace"]:
            layers.append(build_dense_decoder_layer(
                shape, mc["dense_intermediate_size"], seed=args.seed + i, device=dev,
                layer_idx=i))
        else:
            w = layer_weights(shape, seed=args.seed + i, device=dev)
            layers.append(build_decoder_layer(w, shape, layer_idx=i))
            del w
        set_device(layers[-1], dev)
        if not layers[-1].is_dense_layer:
            layers[-1].mlp.keep_last_route = True
    g = torch.Generator(device=dev).manual_seed(args.seed + 100)
    embed = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    head_w = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    norm_w = (1.0 + 0.02 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
    trunk = HIPBailingMoeV2Model.from_modules(embed, layers, norm_w, shape.rms_norm_eps)
    head = HIPLMHead.from_weight(head_w)
    set_device(trunk, dev)
    set_device(head, dev)
    del embed, head_w
    cfg = PagedAttentionConfig(block_size=mc["block_size"], max_num_blocks=mc["max_num_blocks"],
                               batch_size=B)
    cache = HIPPagedAttentionKVCache(mc["num_layers"], shape.num_kv_heads, shape.head_dim, cfg,
                                     device=dev)
    prompts = torch.randint(0, V, (B, L), generator=torch.Generator().manual_seed(args.seed + 7))
    # warm-up: a short generation (fills the workspaces, loads the code objects)
    _log("warm-up generation ...")
    greedy_generate(trunk, head, prompts[:, :64], cache, 4)
    cache.reset()
    _log(f"greedy generation: batch {B}, prompts of {L}, {n_new} new tokens ...")
    r = greedy_generate(trunk, head, prompts, cache, n_new)
    decode_tps = B * r.decode_steps / r.decode_s
    ms_step = r.decode_s / r.decode_steps * 1e3
    # bytes of the last decode step (routing of every MoE layer's last step)
    kv_tok = shape.num_kv_heads * shape.head_dim * 2 * 2
    ctx_read = B * (L + n_new - 1)                      # slots read in the last step
    step_bytes = V * H * 2 + B * H * 2                  # lm head + embedding rows
    exp_bytes = 3 * shape.moe_intermediate_size * H * 2
    n_active = []
    for layer in layers:
        step_bytes += shape.attention_weight_bytes() + ctx_read * kv_tok
        if layer.is_dense_layer:
            step_bytes += 3 * mc["dense_intermediate_size"] * H * 2
        else:
            na = int(layer.mlp.last_route.n_segments.item())
            n_active.append(na - shape.num_shared_experts)
            step_bytes += na * exp_bytes + shape.num_experts * H * 4
    gbs = step_bytes / (ms_step * 1e-3) / 1e9
    # the LM head kernel alone (HIP events on its stream), on the last step's hidden rows
    timer = hip_ops.KernelTimer(["lm_head"])
    hip_ops.set_kernel_timer(timer)
    xh = torch.randn(B, H, device=dev).to(torch.bfloat16)
    for _ in range(20):
        head.greedy(xh)
    torch.cuda.synchronize()
    hip_ops.set_kernel_timer(None)
    lm_ms = timer.mean_ms("lm_head")
    lm_gbs = V * H * 2 / (lm_ms * 1e-3) / 1e9
    _log(f"prefill {r.prefill_s * 1e3:.0f} ms ({B * L / r.prefill_s:.0f} tok/s) | decode "
         f"{ms_step:.2f} ms/step, {decode_tps:.0f} tok/s, {gbs:.0f} GB/s | lm head "
         f"{lm_ms * 1e3:.0f} us ({lm_gbs:.0f} GB/s) | active experts per MoE layer "
         f"{min(n_active)}..{max(n_active)}")
    result = {
        "metric": "greedy generate decode tokens/sec @bs64 Ling-mini-2.0-shape full model "
                  "(20 layers, vocab 157184), 1 GPU",
        "value": decode_tps,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": r.decode_steps,
        "warmup": 1,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init bf16 weights (per-layer seeds), random prompt ids",
        "config": {
            "workload": f"greedy generation, {mc['num_layers']} layers (layer 0 dense I=5120, "
                        f"19 MoE), vocab {V}, batch {B} prompts of {L} random ids, {n_new} new "
                        "tokens, paged KV block 32 / 8192 blocks, decode step captured as one "
                        "HIP graph",
            "global_batch": B,
            "prefill_ms": r.prefill_s * 1e3,
            "prefill_tokens_per_s": B * L / r.prefill_s,
            "end_to_end_tokens_per_s": B * n_new / (r.prefill_s + r.decode_s),
            "active_experts_last_step": n_active,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "lm_head_partial_kernel (LM head GEMV + argmax)",
            "achieved": lm_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": lm_gbs / HBM_PEAK_GBS,
            "traffic": None,
            "bytes_per_launch": V * H * 2,
            "avg_launch_us": lm_ms * 1e3,
        },
        "step_roofline": {"bytes_per_step": step_bytes, "achieved": gbs, "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS},
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)


def main():
    args = parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (one GPU only).",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "prefill":
        prefill_main(args)
        return
    if args.workload == "generate":
        generate_main(args)
        return
    decode_main(args, fp8=args.workload == "fp8")


def decode_main(args, fp8: bool) -> None:
    import torch

    import tt_symbiote_amd as ts
    from tt_symbiote_amd import hip_ops
    from tt_symbiote_amd.workloads import (LING_MINI_2, build_decoder_layer, decode_layer_config,
                                           fp8_kv_pools, layer_weights, paged_context)

    dev = torch.device("cuda:0")
    shape = LING_MINI_2
    wl = fp8_workload_config() if fp8 else decode_layer_config("batch32")
    B = wl["batch"]
    _log("building weights and paged context on the GPU ...")
    w = layer_weights(shape, seed=args.seed, device=dev)
    ctx = paged_context(B, wl["ctx_lo"], wl["ctx_hi"], block_size=wl["block_size"],
                        num_kv_heads=shape.num_kv_heads, seed=args.seed + 1, slack=wl["slack"],
                        device=dev)
    x = torch.randn(B, 1, shape.hidden_size, generator=torch.Generator().manual_seed(2)) \
        .to(torch.bfloat16).to(dev)

    layer = build_decoder_layer(w, shape, weight_format="fp8_e4m3" if fp8 else "bf16")
    ts.set_device(layer, dev)
    layer.mlp.keep_last_route = True
    cfg = ts.PagedAttentionConfig(block_size=wl["block_size"], max_num_blocks=ctx.k_pool.shape[0],
                                  batch_size=1)
    cache = ts.HIPPagedAttentionKVCache(1, shape.num_kv_heads, shape.head_dim, cfg,
                                        dtype=torch.float8_e4m3fn if fp8 else torch.bfloat16)
    cache.to_device(dev)
    if fp8:
        kq, ks = fp8_kv_pools(ctx.k_pool)
        vq, vs = fp8_kv_pools(ctx.v_pool)
        cache.key_cache(0).copy_(kq)
        cache.value_cache(0).copy_(hip_ops.fp8_v_pool(vq))
        cache.key_scale(0).copy_(ks)
        cache.value_scale(0).copy_(vs)
        del kq, vq
    else:
        cache.key_cache(0).copy_(ctx.k_pool)
        cache.value_cache(0).copy_(ctx.v_pool)
    cache.set_vllm_page_table(ctx.page_table)
    pos = ctx.positions.to(dev)

    def step():
        return layer(x, past_key_values=cache, cache_position=pos)[0]

    _log(f"warmup {args.warmup} steps ...")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    n_active = int(layer.mlp.last_route.n_segments.item()) - shape.num_shared_experts

    run = step
    graph = None
    per_run = 1
    if not args.eager:
        # capture decode steps (all of their launches, host logic included) as one HIP graph;
        # positions, page table and workspaces are device buffers, so a replay is full steps.
        # Several steps per graph, as the whole model puts its 20 layer steps in one graph:
        # the graph launch gap (about 8 us) is then not charged to every layer step.
        per_run = STEPS_PER_GRAPH if args.steps % STEPS_PER_GRAPH == 0 else 1
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(per_run):
                step()
        torch.cuda.synchronize()
        run = graph.replay
        for _ in range(3):
            run()
        torch.cuda.synchronize()

    # timed region: K steps
    _log(f"timing {args.steps} steps ({'eager' if args.eager else 'graph replay'}, "
         f"{per_run} per launch) ...")
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for _ in range(args.steps // per_run):
        run()
    t_end.record()
    torch.cuda.synchronize()
    ms_per_step = t_start.elapsed_time(t_end) / args.steps
    if args.replays_only:
        _log(f"{ms_per_step * 1e3:.1f} us per step")
        return

    # per-kernel pass: the same steps launched eagerly with HIP events around the dominant
    # kernels (on the stream they are launched on)
    timer = hip_ops.KernelTimer(["moe_gate_up", "moe_down", "paged_gqa_decode"])
    hip_ops.set_kernel_timer(timer)
    torch.cuda.synchronize()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    hip_ops.set_kernel_timer(None)
    gate_up_ms = timer.mean_ms("moe_gate_up")
    down_ms = timer.mean_ms("moe_down")
    attn_ms = timer.mean_ms("paged_gqa_decode")

    stream_gbs = hip_ops.hbm_read_bandwidth(device=dev)
    nbytes = (fp8_algorithmic_bytes if fp8 else algorithmic_bytes)(shape, ctx, n_active, B)
    achieved = nbytes["gate_up"] / (gate_up_ms * 1e-3) / 1e9
    layer_gbs = nbytes["layer"] / (ms_per_step * 1e-3) / 1e9
    _log(f"step {ms_per_step * 1e3:.1f} us | gate_up {gate_up_ms * 1e3:.1f} us "
         f"({achieved:.0f} GB/s) | down {down_ms * 1e3:.1f} us | attention {attn_ms * 1e3:.1f} us "
         f"| active experts {n_active} | layer {layer_gbs:.0f} GB/s | stream read "
         f"{stream_gbs:.0f} GB/s")

    kernel = "moe_gate_up_fp8_kernel" if fp8 else "moe_gate_up_kernel"
    result = {
        "metric": (METRIC if not fp8 else
                   "decode tokens/sec @bs128 fp8 (e4m3 block-scaled experts, e4m3 KV) "
                   "Ling-mini-2.0-shape, 1 GPU; % HBM roofline/layer"),
        "value": B / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 weights and KV, bf16 activations" if fp8 else "bf16",
        "data": ("synthetic: random-init bf16 weights (seed 0) quantised to fp8 e4m3 with "
                 "128x128 block scales; K/V ~ N(0,1) quantised per (block, head)" if fp8 else
                 "synthetic: random-init bf16 weights (seed 0), K/V cache ~ N(0,1)"),
        "config": {
            "workload": ("BailingMoeV2 decoder layer decode step (Ling-mini-2.0 shape), fp8 "
                         "experts + fp8 KV cache, batch 128, cached lengths U[1024,8192], block "
                         "size 32, pool 1.25x shuffled" if fp8 else
                         "BailingMoeV2 decoder layer decode step (Ling-mini-2.0 shape: hidden "
                         "2048, 16q/4kv heads x128, 256 experts top-8 I=512 + 1 shared), batch "
                         "32, cached lengths U[128,4096], block size 32, pool 1.25x shuffled"),
            "global_batch": B,
            "context_tokens": int(ctx.context_lens.sum()),
            "active_experts": n_active,
            "launch": "eager" if args.eager else f"hip_graph ({per_run} steps per graph)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{kernel} (grouped gate/up GEMM + SwiGLU)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(PMC_SUMMARY_FP8 if fp8 else PMC_SUMMARY),
            "bytes_per_launch": nbytes["gate_up"],
            "avg_launch_us": gate_up_ms * 1e3,
        },
        "layer_roofline": {
            "bytes_per_step": nbytes["layer"],
            "achieved": layer_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": layer_gbs / HBM_PEAK_GBS,
            "measured_stream_read_gbs": stream_gbs,
            "frac_of_measured_stream": layer_gbs / stream_gbs,
            "kernel_us": {"moe_gate_up": gate_up_ms * 1e3, "moe_down": down_ms * 1e3,
                          "paged_gqa_decode": attn_ms * 1e3},
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        _log("cpu baseline ...")
        if fp8:
            result["cpu_baseline"] = cpu_baseline_fp8(layer, w, shape, ctx, cache, x,
                                                      args.cpu_steps)
        else:
            result["cpu_baseline"] = cpu_baseline(w, shape, ctx, x, args.cpu_steps)
    print(json.dumps(result), flush=True)


def cpu_baseline_fp8(layer, w_gpu, shape, ctx, cache, x, steps: int) -> dict:
    """The oracle layer on the dequantised weights and pools (the dequantise-then-bf16
    reference), fp32 on the host CPU, on a bounded sample: the first 16 sequences."""
    import types

    import numpy as np
    import torch

    from oracle.fp8 import decode_e4m3, dequant_blocks
    from tt_symbiote_amd import hip_ops

    E = shape.num_experts
    dq = {}
    for name in ("gate_up", "down"):
        bf = layer.mlp._dev[name]
        dq[name] = torch.from_numpy(dequant_blocks(bf.q.view(torch.uint8).cpu().numpy(),
                                                   bf.scale.cpu().numpy())).bfloat16()
    w = dict(w_gpu, gate_up=dq["gate_up"][:E], down=dq["down"][:E],
             shared_gate_up=dq["gate_up"][E], shared_down=dq["down"][E])
    n = min(16, x.shape[0])

    def pool(codes, scales):
        vals = torch.from_numpy(decode_e4m3(codes.contiguous().view(torch.uint8).cpu().numpy()))
        return vals * scales.cpu()[..., None, None]

    sub = types.SimpleNamespace(k_pool=pool(cache.key_cache(0), cache.key_scale(0)),
                                v_pool=pool(hip_ops.fp8_v_rows(cache.value_cache(0)),
                                            cache.value_scale(0)),
                                page_table=ctx.page_table[:n], positions=ctx.positions[:n])
    r = cpu_baseline(w, shape, sub, x[:n], steps, legs=False)
    r["sample"] = (f"{steps} decode steps (median, after 2 warm-up) of the same layer on the "
                   f"dequantised fp8 weights and cache, first {n} of the {x.shape[0]} sequences, "
                   f"fp32 on the host CPU; " + r["sample"].split("; ")[-1])
    return r


if __name__ == "__main__":
    main()
