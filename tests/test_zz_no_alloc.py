"""The allocation-free paged decode entry point against the workspace one (GPU, through the C
ABI).

sym_paged_gqa_decode_noalloc runs the same kernels as sym_paged_gqa_decode with the split
partials in the library's fixed per-GPU scratch array, so its output must be bit-identical.
Two calls in a row, the second with a smaller batch and shorter contexts (the scratch keeps the
first call's partials: nothing of them may leak into the second), and the second also against
the oracle. A request beyond the scratch size is refused with a clear error before any launch.
"""
import pytest
import torch

from oracle.paged_kv import paged_decode_ref
from tt_symbiote_amd import hip_ops
from tt_symbiote_amd._lib import SymbioteKernelError
from tt_symbiote_amd.workloads import paged_context

pytestmark = pytest.mark.gpu


def _case(device, B, lo, hi, seed):
    ctx = paged_context(B, lo, hi, block_size=32, num_kv_heads=4, seed=seed)
    q = torch.randn(B, 16, 128, generator=torch.Generator().manual_seed(seed + 1)).bfloat16()
    return ctx, q.to(device), (ctx.k_pool.to(device), ctx.v_pool.to(device),
                               ctx.page_table.to(device), ctx.positions.to(device))


def test_noalloc_decode_matches_workspace_entry_point(device):
    scale = 128 ** -0.5
    # first call: the batch-32 decode shape (contexts U[128, 4096]); second: smaller
    for B, lo, hi, seed in ((32, 128, 4096, 21), (5, 1, 700, 22)):
        ctx, q, (kp, vp, pt, pos) = _case(device, B, lo, hi, seed)
        want = hip_ops.paged_gqa_decode(q, kp, vp, pt, pos, scale)
        out = torch.full_like(q, float("nan"))
        got = hip_ops.paged_gqa_decode_noalloc(q, kp, vp, pt, pos, scale, out)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert torch.equal(got, want), f"B={B}: differs from sym_paged_gqa_decode"
        if B == 5:
            ref = paged_decode_ref(q.float().cpu(), ctx.k_pool.float(), ctx.v_pool.float(),
                                   ctx.page_table, ctx.positions, scale)
            err = (got.float().cpu() - ref).abs()
            assert bool((err <= 1e-2 + 1e-2 * ref.abs()).all()), f"max err {err.max():.3e}"


def test_noalloc_decode_rejects_requests_beyond_its_scratch(device):
    # 128 sequences x 16 heads x 512 splits of a 131072-token context: far above 32 MiB
    B, Hq = 128, 16
    q = torch.zeros(B, Hq, 128, dtype=torch.bfloat16, device=device)
    kp = torch.zeros(4, 4, 32, 128, dtype=torch.bfloat16, device=device)
    pt = torch.zeros(B, 4096, dtype=torch.int32, device=device)
    pos = torch.zeros(B, dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    with pytest.raises(SymbioteKernelError, match="scratch"):
        hip_ops.paged_gqa_decode_noalloc(q, kp, kp, pt, pos, 0.1, out)


def test_noalloc_decode_in_a_captured_graph(device):
    """Captured in a HIP graph (the callers it is for) and replayed with new queries and shorter
    contexts written eagerly between replays: every replay equals sym_paged_gqa_decode."""
    scale = 128 ** -0.5
    ctx, q, (kp, vp, pt, pos) = _case(device, 16, 64, 2048, 23)
    out = torch.empty_like(q)
    # the first call locates the scratch array; it runs before the capture, on the side stream
    # the capture uses
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        hip_ops.paged_gqa_decode_noalloc(q, kp, vp, pt, pos, scale, out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        hip_ops.paged_gqa_decode_noalloc(q, kp, vp, pt, pos, scale, out)
    gen = torch.Generator().manual_seed(24)
    base = ctx.positions.clone()
    for rep in range(4):
        q.copy_(torch.randn(tuple(q.shape), generator=gen).bfloat16())
        frac = torch.rand(base.shape, generator=gen) if rep else torch.ones(base.shape)
        pos.copy_((base.float() * frac).to(torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        want = hip_ops.paged_gqa_decode(q, kp, vp, pt, pos, scale)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep} differs from sym_paged_gqa_decode"
