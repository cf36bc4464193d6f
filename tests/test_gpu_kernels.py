"""Kernel parity on the GPU, through the C ABI, against the oracle.

Integer outputs (router indices, permute) are compared bit for bit with the C oracle; router
weights too (same fp32 operations). Floating-point kernels are compared with fp32 references:
  rmsnorm / prologue / decode / grouped GEMM outputs in bf16: |err| <= 1e-2 + 1e-2*|ref|
  (bf16 rounding of the output is 2^-9 relative);
  the down projection given the kernel's own h: fp32, rtol 1e-4;
  KV cache writes: exact.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import route as R
from oracle.paged_kv import paged_decode_ref
from tt_symbiote_amd import hip_ops
from tt_symbiote_amd.modules.kv_cache import HIPPagedAttentionKVCache, PagedAttentionConfig
from tt_symbiote_amd.workloads import paged_context

pytestmark = pytest.mark.gpu


def _close(got, want, atol=1e-2, rtol=1e-2):
    got = got.float().cpu()
    want = want.float().cpu()
    err = (got - want).abs()
    bound = atol + rtol * want.abs()
    assert bool((err <= bound).all()), \
        f"max err {err.max().item():.3e}, worst excess {(err - bound).max().item():.3e}"


# ------------------------------------------------------------------------------- rmsnorm
@pytest.mark.parametrize("rows,cols", [(1, 2048), (32, 2048), (5, 136), (3, 16384),
                                       (1001, 2048), (6, 3584)])
def test_rmsnorm(device, rows, cols):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 2).bfloat16()
    r = torch.randn(rows, cols, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(cols, generator=g)).bfloat16()
    out = hip_ops.rmsnorm(x.to(device), w.to(device), 1e-6)
    ref = x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    _close(out, ref)
    out2, s = hip_ops.rmsnorm(x.to(device), w.to(device), 1e-6, residual=r.to(device))
    s_ref = x.float() + r.float()
    assert torch.equal(s.cpu(), s_ref)
    ref2 = s_ref.float() * torch.rsqrt(s_ref.float().pow(2).mean(-1, keepdim=True) + 1e-6) \
        * w.float()
    _close(out2, ref2)


@pytest.mark.parametrize("rows,cols", [(9942, 2048), (3, 1024), (5, 136)])
def test_rmsnorm_f32_input(device, rows, cols):
    # fp32 rows (a projection's output) in, bf16 out: one wave per row for widths of 512 * n
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = torch.randn(rows, cols, generator=g) * 3
    w = (1 + 0.1 * torch.randn(cols, generator=g)).bfloat16()
    out = hip_ops.rmsnorm(x.to(device), w.to(device), 1e-6)
    ref = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    _close(out, ref)


# ------------------------------------------------------------------------------- router
ROUTE_CASES = [
    # T, E, n_group, topk_group, top_k, kind
    (1, 256, 8, 4, 8, "randn"),
    (16, 64, 8, 4, 4, "ties"),
    (48, 128, 4, 2, 6, "extreme"),
    (64, 256, 8, 4, 16, "zipf"),        # top-16
    (32, 256, 8, 4, 8, "randn"),
    (64, 256, 8, 4, 8, "randn"),
    (65, 256, 8, 4, 8, "randn"),
    (128, 256, 8, 4, 8, "zipf"),        # the fp8 decode batch
    (129, 256, 8, 4, 8, "ties"),
    (1000, 256, 8, 4, 8, "randn"),
    (9000, 256, 8, 4, 8, "zipf"),
    (300, 64, 8, 4, 4, "randn"),
    (300, 128, 4, 2, 6, "randn"),
    (200, 512, 16, 8, 8, "randn"),
    (1500, 512, 16, 8, 8, "randn"),     # permute in passes of 512 tokens
    (5000, 64, 8, 4, 4, "zipf"),        # three-launch permute over 256-token chunks
    (2049, 256, 8, 4, 8, "ties"),       # one token past the single-workgroup permute
    (4100, 512, 16, 8, 8, "zipf"),      # E = 512: four mask words per expert and chunk
    (2304, 128, 4, 2, 6, "randn"),      # whole chunks only
    (200, 64, 1, 1, 8, "randn"),
    (500, 256, 8, 4, 8, "ties"),
    (100, 256, 8, 4, 8, "extreme"),
    # small batches at the other expert counts
    (17, 64, 8, 4, 4, "randn"),
    (50, 128, 4, 2, 6, "ties"),
    (64, 512, 16, 8, 8, "zipf"),
    (3, 512, 16, 8, 8, "extreme"),
]


def _route_inputs(T, E, kind, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "ties":
        logits = torch.randint(-4, 5, (T, E), generator=g).float() * 0.5
        bias = torch.zeros(E)
    elif kind == "extreme":
        logits = torch.randn(T, E, generator=g) * 60
        bias = torch.randn(E, generator=g) * 0.01
    elif kind == "zipf":
        # expert load skewed ~ rank^-1.1: add log-popularity to the logits
        pop = torch.arange(1, E + 1).float().pow(-1.1)
        logits = torch.randn(T, E, generator=g) + torch.log(pop)[torch.randperm(E, generator=g)]
        bias = torch.randn(E, generator=g) * 0.01
    else:
        logits = torch.randn(T, E, generator=g) * 2
        bias = torch.randn(E, generator=g) * 0.01
    return logits.float().contiguous(), bias.float().contiguous()


@pytest.mark.parametrize("T,E,n_group,topk_group,top_k,kind", ROUTE_CASES)
@pytest.mark.parametrize("with_shared", [True, False])
def test_route_permute_bit_exact(device, T, E, n_group, topk_group, top_k, kind, with_shared):
    logits, bias = _route_inputs(T, E, kind, seed=T * 7 + E)
    kw = dict(n_group=n_group, topk_group=topk_group, top_k=top_k, routed_scale=2.5)
    res = hip_ops.moe_route_permute(logits.to(device), bias.to(device), renormalize=True,
                                    with_shared=with_shared, **kw)
    torch.cuda.synchronize()
    idx_ref, w_ref = R.route_c(logits.numpy(), bias.numpy(), renormalize=True, **kw)
    idx = res.topk_idx.cpu().numpy()
    w = res.topk_w.cpu().numpy()
    assert np.array_equal(idx, idx_ref)
    assert np.array_equal(w.view(np.uint32), w_ref.view(np.uint32)), \
        f"max weight diff {np.abs(w - w_ref).max()}"
    p = R.permute_c(idx_ref, E, with_shared=with_shared)
    assert np.array_equal(res.expert_counts.cpu().numpy(), p["expert_counts"])
    assert np.array_equal(res.expert_offsets.cpu().numpy(), p["expert_offsets"])
    assert np.array_equal(res.sorted_tokens.cpu().numpy(), p["sorted_tokens"])
    assert np.array_equal(res.inv_perm.cpu().numpy(), p["inv_perm"])
    ns = int(res.n_segments.item())
    assert ns == int(p["n_segments"][0])
    for name in ("seg_expert", "seg_offset", "seg_count"):
        assert np.array_equal(getattr(res, name).cpu().numpy()[:ns], p[name][:ns]), name


def test_route_no_renorm(device):
    logits, bias = _route_inputs(40, 256, "randn", seed=3)
    kw = dict(n_group=8, topk_group=4, top_k=8, routed_scale=2.5, renormalize=False)
    res = hip_ops.moe_route_permute(logits.to(device), bias.to(device), **kw)
    idx_ref, w_ref = R.route_c(logits.numpy(), bias.numpy(), **kw)
    assert np.array_equal(res.topk_idx.cpu().numpy(), idx_ref)
    assert np.array_equal(res.topk_w.cpu().numpy(), w_ref)


def test_route_deterministic_across_runs(device):
    logits, bias = _route_inputs(2000, 256, "ties", seed=9)
    kw = dict(n_group=8, topk_group=4, top_k=8, routed_scale=2.5)
    a = hip_ops.moe_route_permute(logits.to(device), bias.to(device), **kw)
    b = hip_ops.moe_route_permute(logits.to(device), bias.to(device), **kw)
    for name in ("topk_idx", "topk_w", "sorted_tokens", "inv_perm"):
        assert torch.equal(getattr(a, name), getattr(b, name))


def test_route_from_logit_parts_bit_exact(device):
    """Four partial logit arrays are summed left to right inside the route kernel; the oracle
    routes the same float32 sum."""
    g = torch.Generator().manual_seed(21)
    parts = (torch.randn(4, 48, 256, generator=g) * 0.7).float()
    bias = (torch.randn(256, generator=g) * 0.01).float()
    kw = dict(n_group=8, topk_group=4, top_k=8, routed_scale=2.5)
    res = hip_ops.moe_route_permute(parts.to(device), bias.to(device), **kw)
    p = parts.numpy()
    logits = ((p[0] + p[1]) + p[2]) + p[3]
    idx_ref, w_ref = R.route_c(logits, bias.numpy(), **kw)
    assert np.array_equal(res.topk_idx.cpu().numpy(), idx_ref)
    assert np.array_equal(res.topk_w.cpu().numpy(), w_ref)


@pytest.mark.parametrize("T,H,E", [(1, 2048, 256), (32, 2048, 256), (40, 512, 64), (128, 2048, 512),
                                   (16, 4096, 128)])
def test_router_logits(device, T, H, E):
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(T, H, generator=g).bfloat16()
    w = (torch.randn(E, H, generator=g) * 0.02).float()
    parts = hip_ops.moe_router_logits(x.to(device), w.to(device))
    assert parts.shape == (4, T, E)
    ref = x.double() @ w.double().T
    got = parts.cpu().double().sum(0)
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)
    # each part is the product over its quarter of H
    q = H // 4
    ref1 = x[:, q:2 * q].double() @ w[:, q:2 * q].double().T
    torch.testing.assert_close(parts[1].cpu().double(), ref1, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("T,H,E", [(300, 2048, 256), (4100, 2048, 256), (129, 512, 64)])
def test_router_logits_split(device, T, H, E):
    g = torch.Generator().manual_seed(T + E + 1)
    x = torch.randn(T, H, generator=g).bfloat16()
    w = (torch.randn(E, H, generator=g) * 0.02).float()
    planes = hip_ops.split_router_weight(w)
    parts = hip_ops.moe_router_logits_split(x.to(device), planes.to(device))
    assert parts.shape == (3, T, E)
    ref = x.double() @ w.double().T
    got = (parts[0].cpu() + parts[1].cpu()) + parts[2].cpu()  # the route kernel's order
    torch.testing.assert_close(got.double(), ref, rtol=1e-5, atol=1e-5)
    # each part is the exact product with its plane (fp32 accumulation only)
    ref_lo = x.double() @ planes[2].double().T
    torch.testing.assert_close(parts[2].cpu().double(), ref_lo, rtol=1e-5, atol=1e-9)
    # same routing as the fp32 router kernel wherever the choice is not a near tie
    bias = torch.zeros(E)
    kw = dict(n_group=8, topk_group=4, top_k=8, routed_scale=2.5)
    r_split = hip_ops.moe_route_permute(parts, bias.to(device), **kw)
    r_fp32 = hip_ops.moe_route_permute(hip_ops.moe_router_logits(x.to(device), w.to(device)),
                                       bias.to(device), **kw)
    same = (r_split.topk_idx.cpu().sort(1).values == r_fp32.topk_idx.cpu().sort(1).values)
    assert same.all(1).float().mean() > 0.999


@pytest.mark.parametrize("M,N,K,bias,out_dtype", [
    (32, 3072, 2048, False, torch.bfloat16),
    (32, 2048, 2048, True, torch.bfloat16),
    (1, 256, 512, False, torch.float32),
    (70, 128, 192, True, torch.float32),
    (64, 2048, 2048, False, torch.float32),      # 32-row passes, weights held in registers
    (100, 512, 1024, True, torch.bfloat16),
    (128, 3072, 2048, True, torch.bfloat16),     # the batch-128 QKV shape
    (77, 2048, 2048, False, torch.float32),      # a partial last pass
])
def test_linear(device, M, N, K, bias, out_dtype):
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    b = (torch.randn(N, generator=g) * 0.1).bfloat16() if bias else None
    out = hip_ops.linear(x.to(device), w.to(device), None if b is None else b.to(device),
                         out_dtype=out_dtype)
    ref = x.float() @ w.float().T + (b.float() if b is not None else 0.0)
    assert out.dtype == out_dtype
    if out_dtype == torch.float32:
        torch.testing.assert_close(out.cpu(), ref, rtol=1e-4, atol=1e-4)
    else:
        _close(out, ref, atol=2e-3, rtol=8e-3)


def _rmsnorm_bf16(x, gamma, eps):
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * r * gamma.float()).bfloat16()


@pytest.mark.parametrize("M,N,K,bias", [(32, 3072, 2048, False), (64, 3072, 2048, False),
                                        (48, 512, 1024, True), (1, 256, 2048, True),
                                        (70, 128, 192, True), (128, 3072, 2048, False),
                                        (97, 2048, 2048, True), (20, 512, 2048, True),
                                        (20, 3072, 2048, True), (33, 3072, 2048, True),
                                        (50, 512, 2048, False)])
def test_rmsnorm_linear(device, M, N, K, bias):
    g = torch.Generator().manual_seed(M * 3 + N + K)
    x = (torch.randn(M, K, generator=g) * 1.5).bfloat16()
    gamma = (1 + 0.1 * torch.randn(K, generator=g)).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    b = (torch.randn(N, generator=g) * 0.1).bfloat16() if bias else None
    out = hip_ops.rmsnorm_linear(x.to(device), gamma.to(device), 1e-6, w.to(device),
                                 None if b is None else b.to(device), out_dtype=torch.float32)
    xn = _rmsnorm_bf16(x, gamma, 1e-6)     # the operand a separate RMSNorm pass would write
    ref = xn.float() @ w.float().T + (b.float() if b is not None else 0.0)
    # the row statistics are summed in another order, which can move an operand by one bf16
    # ulp (2^-8 relative) now and then
    torch.testing.assert_close(out.cpu(), ref, rtol=2e-3, atol=2e-3)
    out_bf = hip_ops.rmsnorm_linear(x.to(device), gamma.to(device), 1e-6, w.to(device),
                                    None if b is None else b.to(device))
    _close(out_bf, ref, atol=3e-3, rtol=8e-3)


def test_rmsnorm_linear_row_blocks_agree(device):
    # up to 32 rows the fused-norm projection runs 16-row blocks as a grid dimension, above 32
    # rows 16-row passes over weights held in registers: the same roundings and summation order
    # per row, so the rows of a batch do not depend on which of them run together
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(64, 2048, generator=g) * 1.5).bfloat16().to(device)
    gamma = (1 + 0.1 * torch.randn(2048, generator=g)).bfloat16().to(device)
    w = (torch.randn(3072, 2048, generator=g) * 0.02).bfloat16().to(device)
    full = hip_ops.rmsnorm_linear(x, gamma, 1e-6, w, None, out_dtype=torch.float32).cpu()
    for m in (1, 15, 20, 32):
        part = hip_ops.rmsnorm_linear(x[:m].contiguous(), gamma, 1e-6, w, None,
                                      out_dtype=torch.float32).cpu()
        assert torch.equal(part, full[:m]), m


@pytest.mark.parametrize("M,N,K", [(32, 2048, 2048), (64, 2048, 2048), (5, 256, 512),
                                   (40, 128, 192), (128, 2048, 2048), (33, 2048, 2048)])
def test_linear_residual(device, M, N, K):
    g = torch.Generator().manual_seed(M + 7 * N + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    b = (torch.randn(N, generator=g) * 0.1).bfloat16()
    res = torch.randn(M, N, generator=g).bfloat16()
    out, parts = hip_ops.linear_residual(x.to(device), w.to(device), res.to(device),
                                         b.to(device))
    ref = x.float() @ w.float().T + b.float() + res.float()
    torch.testing.assert_close(out.cpu(), ref, rtol=1e-4, atol=1e-4)
    ss = out.cpu().double().pow(2).view(M, N // 16, 16).sum(-1).T
    torch.testing.assert_close(parts.cpu().double(), ss, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("T,H,E", [(32, 2048, 256), (1, 2048, 256), (20, 4096, 64)])
def test_router_logits_norm(device, T, H, E):
    g = torch.Generator().manual_seed(T + H + E)
    h = torch.randn(T, H, generator=g) * 1.3
    gamma = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    w = (torch.randn(E, H, generator=g) * 0.02).float()
    ss = h.double().pow(2).view(T, H // 16, 16).sum(-1).T.float().contiguous()
    parts, xn = hip_ops.moe_router_logits_norm(h.to(device), ss.to(device), gamma.to(device),
                                               1e-6, w.to(device))
    xn_ref = _rmsnorm_bf16(h, gamma, 1e-6)
    _close(xn, xn_ref.float(), atol=1e-6, rtol=8e-3)  # at most one bf16 ulp apart
    ref = xn.cpu().double() @ w.double().T            # logits of the operand actually used
    torch.testing.assert_close(parts.cpu().double().sum(0), ref, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------------------- grouped GEMM
def _gemm_case(T, E, H, I, top_k, seed, device, with_shared=True, skew=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16()
    slots = E + (1 if with_shared else 0)
    wgu = (torch.randn(slots, 2 * I, H, generator=g) * 0.05).bfloat16()
    wd = (torch.randn(slots, H, I, generator=g) * 0.05).bfloat16()
    logits = torch.randn(T, E, generator=g) * 2
    if skew:
        logits[:, :4] += 6.0   # a few experts take most tokens
    res = hip_ops.moe_route_permute(logits.to(device), torch.zeros(E, device=device),
                                    n_group=8, topk_group=4, top_k=top_k, routed_scale=2.5,
                                    with_shared=with_shared)
    return x, wgu, wd, res


@pytest.mark.parametrize("kernel", ["stream", "tiled"])
@pytest.mark.parametrize("T,E,H,I,top_k,skew", [
    (1, 64, 256, 128, 4, False),
    (32, 256, 2048, 512, 8, False),
    (7, 64, 512, 192, 4, False),
    (200, 64, 256, 128, 6, True),       # segments of > 64 rows (several passes)
    (700, 64, 512, 256, 8, True),       # segments of several 128-row tiles
    (300, 64, 512, 192, 6, True),       # I not a multiple of the 128 h columns of a tile
    (400, 64, 256, 64, 6, True),        # I = 64: the tiled down GEMM's K loop is one step, in
                                        # thin tiles (at most 64 rows) and whole ones
    # 513 segment entries (E = 512 + shared): the tiled GEMMs leave the persistent kernel for
    # the per-tile lookup kernels (gemm_tile_kernel gate/up, gemm_tile128_kernel down)
    (700, 512, 512, 256, 8, True),      # skewed: segments spanning several 128- and 256-row tiles
    (300, 512, 512, 192, 6, True),      # and I not a multiple of 128
    (40, 512, 512, 128, 8, False),      # many one- and two-row segments
])
def test_grouped_swiglu(device, T, E, H, I, top_k, skew, kernel):
    x, wgu, wd, res = _gemm_case(T, E, H, I, top_k, seed=T + E, device=device, skew=skew)
    h, y = hip_ops.moe_grouped_swiglu(x.to(device), res, wgu.to(device), wd.to(device),
                                      kernel=kernel)
    torch.cuda.synchronize()
    st = res.sorted_tokens.cpu().long()
    ns = int(res.n_segments.item())
    seg_e = res.seg_expert.cpu()[:ns].tolist()
    seg_o = res.seg_offset.cpu()[:ns].tolist()
    seg_c = res.seg_count.cpu()[:ns].tolist()
    hk = h.cpu()
    yk = y.cpu()
    xf = x.float()
    for e, o, c in zip(seg_e, seg_o, seg_c):
        rows = slice(o, o + c)
        xe = xf[st[rows]]
        gate = xe @ wgu[e, :I].float().T
        up = xe @ wgu[e, I:].float().T
        h_ref = F.silu(gate) * up
        _close(hk[rows], h_ref, atol=2e-3, rtol=8e-3)
        y_ref = hk[rows].float() @ wd[e].float().T
        torch.testing.assert_close(yk[rows], y_ref, rtol=1e-4, atol=1e-4)
    if kernel == "tiled":
        # bf16 y: the same fp32 results, rounded once to bf16 (round to nearest even)
        _, yb = hip_ops.moe_grouped_swiglu(x.to(device), res, wgu.to(device), wd.to(device),
                                           kernel=kernel, y_dtype=torch.bfloat16)
        assert yb.dtype == torch.bfloat16
        assert torch.equal(yb.cpu(), yk.bfloat16())


def test_grouped_tiled_workspace_reentrant(device):
    """The tiled grouped GEMMs keep their tile counters in the caller's workspace: two streams
    running prefill-size launches at the same time, each with its own workspace, give the bytes
    of serial runs, and back-to-back launches with different segment lists on one workspace
    leave it zeroed."""
    H, I, E = 2048, 512, 256
    cases = [_gemm_case(T, E, H, I, 8, seed=T, device=device, skew=skew)
             for T, skew in ((1500, True), (900, False))]
    dev_cases = [(x.to(device), res, wgu.to(device), wd.to(device))
                 for x, wgu, wd, res in cases]

    def run(i, ws):
        x, res, wgu, wd = dev_cases[i]
        return hip_ops.moe_grouped_swiglu(x, res, wgu, wd, kernel="tiled",
                                          y_dtype=torch.bfloat16, workspace=ws)

    serial = [tuple(t.clone() for t in run(i, hip_ops.moe_tiled_workspace(device)))
              for i in range(2)]
    # one workspace, different segment lists back to back
    ws = hip_ops.moe_tiled_workspace(device)
    for i in (0, 1, 0, 1, 1, 0):
        h, y = run(i, ws)
        assert torch.equal(h, serial[i][0]) and torch.equal(y, serial[i][1])
    torch.cuda.synchronize()
    assert int(ws.count_nonzero()) == 0
    # two default-priority streams at once, a workspace each
    streams = [torch.cuda.Stream(device), torch.cuda.Stream(device)]
    wss = [hip_ops.moe_tiled_workspace(device) for _ in range(2)]
    torch.cuda.synchronize()
    for rep in range(4):
        outs = [None, None]
        for i in (0, 1):
            with torch.cuda.stream(streams[i]):
                outs[i] = run(i, wss[i])
        torch.cuda.synchronize()
        for i in (0, 1):
            assert torch.equal(outs[i][0], serial[i][0]), (rep, i, "h")
            assert torch.equal(outs[i][1], serial[i][1]), (rep, i, "y")
    assert all(int(w.count_nonzero()) == 0 for w in wss)


def test_grouped_tiled_workspace_checked(device):
    x, wgu, wd, res = _gemm_case(300, 64, 512, 128, 4, seed=1, device=device)
    small = torch.zeros(hip_ops._lib.query("sym_moe_tiled_workspace_bytes") - 4,
                        dtype=torch.uint8, device=device)
    with pytest.raises(hip_ops._lib.SymbioteKernelError, match="workspace"):
        hip_ops.moe_grouped_swiglu(x.to(device), res, wgu.to(device), wd.to(device),
                                   kernel="tiled", workspace=small)


@pytest.mark.parametrize("M,N,K,bias,res,out_dtype", [
    (1000, 3072, 2048, False, False, torch.bfloat16),   # ragged last row tile
    (256, 2048, 2048, True, True, torch.float32),
    (1, 128, 64, False, False, torch.float32),
    (130, 256, 576, True, False, torch.bfloat16),
    (77, 400, 192, True, True, torch.float32),          # N not a multiple of the 256-wide tile
    (300, 16, 128, False, False, torch.bfloat16),
    (8500, 2048, 128, True, True, torch.float32),       # 256 whole tiles + 128-row tail tiles
    (9000, 2304, 128, False, False, torch.bfloat16),    # 252 whole tiles + tail, ragged last tile
])
def test_gemm_tiled(device, M, N, K, bias, res, out_dtype):
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    b = (torch.randn(N, generator=g) * 0.1).bfloat16() if bias else None
    r = torch.randn(M, N, generator=g) if res else None
    out = hip_ops.gemm(a.to(device), w.to(device), None if b is None else b.to(device),
                       None if r is None else r.to(device), out_dtype=out_dtype)
    ref = a.float() @ w.float().T
    if b is not None:
        ref = ref + b.float()
    if r is not None:
        ref = ref + r
    if out_dtype == torch.float32:
        torch.testing.assert_close(out.cpu(), ref, rtol=1e-4, atol=1e-4)
    else:
        _close(out, ref, atol=2e-3, rtol=8e-3)


@pytest.mark.parametrize("M,N,K,bias", [(9942, 2048, 2048, False), (77, 400, 192, True),
                                        (8500, 2048, 128, True)])
def test_gemm_tiled_bf16_residual(device, M, N, K, bias):
    # the prefill dense projection with the layer's bf16 residual added in the epilogue: the
    # same fp32 sum as an fp32 output plus the widened residual, bit for bit
    g = torch.Generator().manual_seed(M * 3 + N + K)
    a = torch.randn(M, K, generator=g).bfloat16().to(device)
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16().to(device)
    b = (torch.randn(N, generator=g) * 0.1).bfloat16().to(device) if bias else None
    r = torch.randn(M, N, generator=g).bfloat16().to(device)
    out = hip_ops.gemm(a, w, b, r, out_dtype=torch.float32)
    plain = hip_ops.gemm(a, w, b, out_dtype=torch.float32)
    assert torch.equal(out.cpu(), plain.cpu() + r.float().cpu())
    ref = a.float().cpu() @ w.float().cpu().T + (b.float().cpu() if bias else 0.0) + r.float().cpu()
    torch.testing.assert_close(out.cpu(), ref, rtol=1e-4, atol=1e-4)
    with pytest.raises(TypeError):
        hip_ops.gemm(a, w, b, r, out_dtype=torch.bfloat16)


def test_combine(device):
    T, E, H, I, K = 32, 256, 2048, 512, 8
    x, wgu, wd, res = _gemm_case(T, E, H, I, K, seed=5, device=device)
    _, y = hip_ops.moe_grouped_swiglu(x.to(device), res, wgu.to(device), wd.to(device))
    resid = torch.randn(T, H, generator=torch.Generator().manual_seed(6))
    out = hip_ops.moe_unpermute_combine(y, res, residual=resid.to(device))
    yc = y.cpu()
    inv = res.inv_perm.cpu().long()
    w = res.topk_w.cpu()
    ref = (yc[inv] * w[..., None]).sum(1) + yc[T * K:T * K + T] + resid
    _close(out, ref, atol=1e-2, rtol=8e-3)
    out2 = hip_ops.moe_unpermute_combine(y, res)
    _close(out2, (yc[inv] * w[..., None]).sum(1) + yc[T * K:T * K + T], atol=1e-2, rtol=8e-3)
    # bf16 y: widened exactly, summed in fp32 as above
    yb = y.bfloat16()
    out3 = hip_ops.moe_unpermute_combine(yb, res, residual=resid.to(device))
    ybc = yb.cpu().float()
    ref3 = (ybc[inv] * w[..., None]).sum(1) + ybc[T * K:T * K + T] + resid
    _close(out3, ref3, atol=1e-2, rtol=8e-3)


# ------------------------------------------------------------------------------- attention
def _dev_ctx(ctx, device):
    return (ctx.k_pool.to(device), ctx.v_pool.to(device), ctx.page_table.to(device),
            ctx.positions.to(device))


@pytest.mark.parametrize("B,Hq,Hkv,bs,lo,hi", [
    (1, 16, 4, 32, 512, 512),
    (32, 16, 4, 32, 128, 4096),
    (4, 8, 4, 16, 0, 40),
    (4, 8, 8, 16, 3, 70),
    (3, 16, 2, 64, 250, 260),
    (5, 16, 16, 32, 1, 300),
    (2, 32, 4, 32, 1000, 3000),
    (48, 16, 4, 32, 100, 1500),    # above 32 sequences: the odd-width grid order
])
def test_paged_decode(device, B, Hq, Hkv, bs, lo, hi):
    ctx = paged_context(B, lo, hi, block_size=bs, num_kv_heads=Hkv, seed=B + Hq + bs)
    q = torch.randn(B, Hq, 128, generator=torch.Generator().manual_seed(1)).bfloat16()
    kp, vp, pt, pos = _dev_ctx(ctx, device)
    scale = 128 ** -0.5
    out = hip_ops.paged_gqa_decode(q.to(device), kp, vp, pt, pos, scale)
    ref = paged_decode_ref(q.float(), ctx.k_pool.float(), ctx.v_pool.float(), ctx.page_table,
                           ctx.positions, scale)
    _close(out, ref, atol=1e-2, rtol=1e-2)


def test_paged_decode_split_boundaries(device):
    # cached lengths around the 256-token split: 255 -> 256 slots, 256 -> 257 slots, ...
    lens = [0, 1, 254, 255, 256, 511, 512, 1023]
    B = len(lens)
    ctxs = [paged_context(1, n, n, block_size=32, num_kv_heads=4, seed=n) for n in lens]
    nb = sum(c.k_pool.shape[0] for c in ctxs)
    kp = torch.cat([c.k_pool for c in ctxs])
    vp = torch.cat([c.v_pool for c in ctxs])
    mb = max(c.page_table.shape[1] for c in ctxs)
    pt = torch.zeros(B, mb, dtype=torch.int32)
    off = 0
    for b, c in enumerate(ctxs):
        pt[b, :c.page_table.shape[1]] = c.page_table[0] + off
        off += c.k_pool.shape[0]
    assert off == nb
    pos = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn(B, 16, 128, generator=torch.Generator().manual_seed(2)).bfloat16()
    out = hip_ops.paged_gqa_decode(q.to(device), kp.to(device), vp.to(device), pt.to(device),
                                   pos.to(device), 0.1)
    ref = paged_decode_ref(q.float(), kp.float(), vp.float(), pt, pos, 0.1)
    _close(out, ref)


def test_paged_decode_block_relabelling_is_bit_exact(device):
    ctx = paged_context(6, 100, 900, block_size=32, num_kv_heads=4, seed=3)
    q = torch.randn(6, 16, 128, generator=torch.Generator().manual_seed(4)).bfloat16().to(device)
    kp, vp, pt, pos = _dev_ctx(ctx, device)
    a = hip_ops.paged_gqa_decode(q, kp, vp, pt, pos, 0.09)
    relabel = torch.randperm(kp.shape[0], generator=torch.Generator().manual_seed(5)).to(device)
    kp2 = torch.empty_like(kp)
    vp2 = torch.empty_like(vp)
    kp2[relabel] = kp
    vp2[relabel] = vp
    b = hip_ops.paged_gqa_decode(q, kp2, vp2, relabel[pt.long()].int(), pos, 0.09)
    assert torch.equal(a, b)


def test_paged_decode_reused_workspace(device):
    # A workspace reused across calls and batch sizes (the cache keeps one) gives identical
    # results: nothing of a previous call's partial results may leak into the next.
    ctx = paged_context(32, 128, 4096, block_size=32, num_kv_heads=4, seed=11)
    kp, vp, pt, pos = _dev_ctx(ctx, device)
    q = torch.randn(32, 16, 128, generator=torch.Generator().manual_seed(12)).bfloat16().to(device)
    cap = pt.shape[1] * 32
    need = hip_ops.paged_decode_workspace_bytes(32, 16, cap)
    ws = torch.full((need,), 0x7F, dtype=torch.uint8, device=device)  # garbage contents
    ref = paged_decode_ref(q.float().cpu(), ctx.k_pool.float(), ctx.v_pool.float(),
                           ctx.page_table, ctx.positions, 0.08)
    first = hip_ops.paged_gqa_decode(q, kp, vp, pt, pos, 0.08, workspace=ws)
    _close(first, ref)
    for _ in range(3):
        again = hip_ops.paged_gqa_decode(q, kp, vp, pt, pos, 0.08, workspace=ws)
        assert torch.equal(again, first)
    # the cache-owned workspace, across batch sizes
    cfg = PagedAttentionConfig(block_size=32, max_num_blocks=kp.shape[0], batch_size=1)
    cache = HIPPagedAttentionKVCache(1, 4, 128, cfg)
    cache.to_device(device)
    cache.key_cache(0).copy_(kp)
    cache.value_cache(0).copy_(vp)
    cache.set_vllm_page_table(pt)
    for bsz in (32, 5, 32, 7):
        o = cache.paged_sdpa_decode(q[:bsz], 0, pos[:bsz], scale=0.08)
        torch.testing.assert_close(o, first[:bsz], rtol=0, atol=0)


def test_kv_write_and_fill(device):
    ctx = paged_context(4, 10, 200, block_size=16, num_kv_heads=4, seed=8)
    kp, vp, pt, pos = _dev_ctx(ctx, device)
    kn = torch.randn(4, 4, 128).bfloat16()
    vn = torch.randn(4, 4, 128).bfloat16()
    hip_ops.paged_kv_write(kn.to(device), vn.to(device), kp, vp, pt, pos)
    kpc, vpc = kp.cpu(), vp.cpu()
    for b in range(4):
        p = int(ctx.positions[b])
        phys = int(ctx.page_table[b, p // 16])
        assert torch.equal(kpc[phys, :, p % 16], kn[b])
        assert torch.equal(vpc[phys, :, p % 16], vn[b])
    # untouched slots unchanged
    mask = torch.ones(kp.shape[0], 4, 16, dtype=torch.bool)
    for b in range(4):
        p = int(ctx.positions[b])
        mask[int(ctx.page_table[b, p // 16]), :, p % 16] = False
    assert torch.equal(kpc[mask], ctx.k_pool[mask])
    # prompt fill of sequence 2 from position 0
    S = int(ctx.positions[2]) + 1
    kf = torch.randn(4, S, 128).bfloat16()
    vf = torch.randn(4, S, 128).bfloat16()
    hip_ops.paged_kv_fill(kf.to(device), vf.to(device), kp, vp, pt, batch_idx=2)
    kpc, vpc = kp.cpu(), vp.cpu()
    for s in range(S):
        phys = int(ctx.page_table[2, s // 16])
        assert torch.equal(kpc[phys, :, s % 16], kf[:, s])
        assert torch.equal(vpc[phys, :, s % 16], vf[:, s])


@pytest.mark.parametrize("rotary_dim,use_norm", [(64, True), (128, True), (64, False)])
def test_decode_prologue(device, rotary_dim, use_norm):
    from oracle.bailing_moe_v2 import apply_partial_rotary

    B, Hq, Hkv, D = 8, 16, 4, 128
    ctx = paged_context(B, 5, 3000, block_size=32, num_kv_heads=Hkv, seed=11)
    kp, vp, pt, pos = _dev_ctx(ctx, device)
    g = torch.Generator().manual_seed(12)
    qkv = torch.randn(B, (Hq + 2 * Hkv) * D, generator=g).bfloat16()
    qn = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    kn = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    theta, max_pos = 1e6, 4096
    inv = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2).float() / rotary_dim))
    fr = torch.arange(max_pos).float()[:, None] * inv[None]
    table = torch.cat([fr.cos(), fr.sin()], 1).contiguous()
    q = hip_ops.attn_decode_prologue(
        qkv.to(device), pos, kp, vp, pt, num_heads=Hq, num_kv_heads=Hkv, rotary_dim=rotary_dim,
        rope_cs=table.to(device), q_norm_w=qn.to(device) if use_norm else None,
        k_norm_w=kn.to(device) if use_norm else None, eps=1e-6)
    # oracle
    x = qkv.float().view(B, Hq + 2 * Hkv, D)
    qr, kr, vr = x[:, :Hq], x[:, Hq:Hq + Hkv], x[:, Hq + Hkv:]

    def norm(t, w):
        return t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()

    if use_norm:
        qr, kr = norm(qr, qn), norm(kr, kn)
    cos = torch.cat([fr[ctx.positions.long()]] * 2, -1).cos()[:, None, :]   # [B,1,rd]
    sin = torch.cat([fr[ctx.positions.long()]] * 2, -1).sin()[:, None, :]
    q_ref, k_ref = apply_partial_rotary(qr.unsqueeze(2), kr.unsqueeze(2), cos, sin)
    _close(q, q_ref[:, :, 0], atol=2e-2, rtol=1e-2)
    kpc, vpc = kp.cpu(), vp.cpu()
    for b in range(B):
        p = int(ctx.positions[b])
        phys = int(ctx.page_table[b, p // 32])
        _close(kpc[phys, :, p % 32], k_ref[b, :, 0], atol=2e-2, rtol=1e-2)
        assert torch.equal(vpc[phys, :, p % 32], vr[b].bfloat16())


@pytest.mark.parametrize("B,Hq,Hkv,rd,use_norm,lo,hi,bs,cap", [
    (8, 16, 4, 64, True, 5, 3000, 32, None),
    (5, 16, 2, 128, False, 0, 300, 16, None),      # 8 q heads per kv head
    (6, 8, 8, 64, True, 250, 600, 64, None),       # 1 q head per kv head
    (6, 16, 4, 64, True, 100, 700, 32, 512),       # some positions beyond the attention cap
    (40, 16, 4, 64, True, 5, 2000, 32, None),      # above 32 sequences: odd-width grid order
])
def test_decode_step_matches_prologue_then_decode(device, B, Hq, Hkv, rd, use_norm, lo, hi, bs,
                                                   cap):
    """The fused step (QK-norm, RoPE, KV write and decode in the split kernel) gives exactly
    the output and the pools of the prologue kernel followed by the decode kernel, including a
    sequence with no position (-1) and one whose new slot has no page-table entry."""
    D = 128
    ctx = paged_context(B, lo, hi, block_size=bs, num_kv_heads=Hkv, seed=B * 7 + Hkv)
    pt = ctx.page_table.clone()
    pos = ctx.positions.clone()
    pos[0] = -1
    last = int(pos[1]) // bs
    pt[1, last] = -1                                  # the new token's block is unmapped
    g = torch.Generator().manual_seed(B + rd)
    qkv = torch.randn(B, (Hq + 2 * Hkv) * D, generator=g).bfloat16().to(device)
    qn = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    kn = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    inv = 1.0 / (1e6 ** (torch.arange(0, rd, 2).float() / rd))
    fr = torch.arange(4096).float()[:, None] * inv[None]
    table = torch.cat([fr.cos(), fr.sin()], 1).contiguous().to(device)
    pt_d, pos_d = pt.to(device), pos.to(device)
    kw = dict(num_heads=Hq, num_kv_heads=Hkv, rotary_dim=rd, rope_cs=table,
              q_norm_w=qn if use_norm else None, k_norm_w=kn if use_norm else None, eps=1e-6)
    max_context = cap or pt.shape[1] * bs
    k1, v1 = ctx.k_pool.to(device), ctx.v_pool.to(device)
    q = hip_ops.attn_decode_prologue(qkv, pos_d, k1, v1, pt_d, **kw)
    ref = hip_ops.paged_gqa_decode(q, k1, v1, pt_d, pos_d, 0.09, max_context=max_context)
    k2, v2 = ctx.k_pool.to(device), ctx.v_pool.to(device)
    out = hip_ops.attn_decode_step(qkv, pos_d, k2, v2, pt_d, 0.09, max_context=max_context, **kw)
    assert torch.equal(out, ref)
    assert torch.equal(k2, k1) and torch.equal(v2, v1)
    assert not bool(out[0].any())                    # no position: zero output


@pytest.mark.parametrize("lens,Hq,Hkv,qscale", [
    ([1, 5, 64, 127, 128, 129, 300], 16, 4, 1.0),
    ([200, 77], 8, 8, 1.0),
    ([513], 16, 2, 1.0),
    ([1500, 37], 16, 4, 4.0),     # many key blocks, peaked softmax (frequent max changes)
])
def test_prefill_attention(device, lens, Hq, Hkv, qscale):
    g = torch.Generator().manual_seed(sum(lens) + Hq)
    T = sum(lens)
    q = (torch.randn(T, Hq, 128, generator=g) * qscale).bfloat16()
    k = torch.randn(T, Hkv, 128, generator=g).bfloat16()
    v = torch.randn(T, Hkv, 128, generator=g).bfloat16()
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    out = hip_ops.prefill_attention(q.to(device), k.to(device), v.to(device), cu.to(device),
                                    max(lens), 0.0884).cpu()
    rep = Hq // Hkv
    for s, L in enumerate(lens):
        a, b = int(cu[s]), int(cu[s + 1])
        qs = q[a:b].float().transpose(0, 1)                       # [Hq, L, D]
        ks = k[a:b].float().transpose(0, 1).repeat_interleave(rep, 0)
        vs = v[a:b].float().transpose(0, 1).repeat_interleave(rep, 0)
        ref = F.scaled_dot_product_attention(qs[None], ks[None], vs[None], is_causal=True,
                                             scale=0.0884)[0].transpose(0, 1)
        _close(out[a:b], ref, atol=1e-2, rtol=1e-2)


def test_prefill_attention_deterministic(device):
    """Repeated launches over many ragged sequences (several workgroups per CU, of different
    lengths) give bit-identical outputs. A row maximum read from the score accumulator before
    the MFMA has written it changes the softmax only in rounding, so only this catches it."""
    lens = [267, 1843, 877, 1609, 2030, 939, 2010, 367]
    g = torch.Generator().manual_seed(11)
    T = sum(lens)
    q = torch.randn(T, 16, 128, generator=g).bfloat16().to(device)
    k = torch.randn(T, 4, 128, generator=g).bfloat16().to(device)
    v = torch.randn(T, 4, 128, generator=g).bfloat16().to(device)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32).to(device)
    ref = hip_ops.prefill_attention(q, k, v, cu, max(lens), 0.0884)
    for _ in range(8):
        assert torch.equal(hip_ops.prefill_attention(q, k, v, cu, max(lens), 0.0884), ref)


def test_prefill_prologue_matches_decode_prologue(device):
    """The packed prefill prologue applies, per token, exactly the decode prologue's arithmetic
    (same kernel); tokens of sequence s land in the pool slots of their positions."""
    lens = [37, 70, 5]
    T = sum(lens)
    Hq, Hkv, D, bs = 16, 4, 128, 32
    nblk = [(L + bs - 1) // bs for L in lens]
    nb = sum(nblk) + 3
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(3)).int()
    pt = torch.zeros(len(lens), max(nblk), dtype=torch.int32)
    o = 0
    for s, n in enumerate(nblk):
        pt[s, :n] = perm[o:o + n]
        o += n
    pos = torch.cat([torch.arange(L) for L in lens]).int()
    sid = torch.cat([torch.full((L,), s) for s, L in enumerate(lens)]).int()
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, generator=g).bfloat16().to(device)
    qn = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    kn = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    inv = 1.0 / (1e6 ** (torch.arange(0, 64, 2).float() / 64))
    fr = torch.arange(512).float()[:, None] * inv[None]
    table = torch.cat([fr.cos(), fr.sin()], 1).contiguous().to(device)
    kw = dict(num_heads=Hq, num_kv_heads=Hkv, rotary_dim=64, rope_cs=table, q_norm_w=qn,
              k_norm_w=kn, eps=1e-6)
    kp = torch.zeros(nb, Hkv, bs, D, dtype=torch.bfloat16, device=device)
    vp = torch.zeros_like(kp)
    q, k, v = hip_ops.attn_prefill_prologue(qkv, pos.to(device), sid.to(device), kp, vp,
                                            pt.to(device), **kw)
    # reference: the decode prologue with one "sequence" per token (its own page-table row)
    kp2 = torch.zeros_like(kp)
    vp2 = torch.zeros_like(kp)
    q2 = hip_ops.attn_decode_prologue(qkv, pos.to(device), kp2, vp2,
                                      pt[sid.long()].contiguous().to(device), **kw)
    assert torch.equal(q, q2)
    assert torch.equal(kp, kp2) and torch.equal(vp, vp2)
    kpc = kp.cpu()
    for t in range(T):
        s, p = int(sid[t]), int(pos[t])
        phys = int(pt[s, p // bs])
        assert torch.equal(kpc[phys, :, p % bs], k[t].cpu())
    assert torch.equal(v.cpu(), qkv.cpu().view(T, Hq + 2 * Hkv, D)[:, Hq + Hkv:])


def test_hbm_read_probe(device):
    # measurement kernel: must read every byte (a rate above the 8 TB/s HBM peak would mean
    # skipped work) and launch cleanly
    gbs = hip_ops.hbm_read_bandwidth(1 << 30, reps=3, device=device)  # 4x the last-level cache
    assert 100.0 < gbs < 8000.0
