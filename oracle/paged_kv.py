"""Oracle of the paged KV cache and paged GQA decode attention (test infrastructure only).

Restates TTNNPagedAttentionKVCache (ttnn_attention.py:75-371) on CPU tensors:
  pools [num_blocks, Hkv, block_size, D] (ttnn_attention.py:116-137), page table
  [B, blocks_per_seq] (ttnn_attention.py:101-102), paged_update_cache writes slot cur_pos[b]
  (ttnn_attention.py:235-269), paged_scaled_dot_product_attention_decode attends positions
  0..cur_pos[b] inclusive (ttnn_attention.py:288-329, update precedes decode at 2426-2443)
with kv head = q head // (Hq/Hkv) and scale head_dim^-0.5 (ttnn_attention.py:1973).

The attention itself is `torch.nn.functional.scaled_dot_product_attention` on the gathered
rows (a library routine), computed in float32 or float64.
"""
from __future__ import annotations

from typing import List, Optional

import torch
import torch.nn.functional as F


def gather_sequence(pool: torch.Tensor, page_table_row: torch.Tensor, length: int) -> torch.Tensor:
    """Rows 0..length-1 of one sequence: [Hkv, length, D] gathered through the page table."""
    nb, hkv, bs, d = pool.shape
    nblk = (length + bs - 1) // bs
    blocks = page_table_row[:nblk].long()
    rows = pool[blocks]                      # [nblk, Hkv, bs, D]
    rows = rows.permute(1, 0, 2, 3).reshape(hkv, nblk * bs, d)
    return rows[:, :length]


def paged_decode_ref(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                     page_table: torch.Tensor, positions: torch.Tensor, scale: float,
                     dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """q [B, Hq, D] -> out [B, Hq, D] in ``dtype``; sequence b attends slots 0..positions[b]."""
    B, Hq, D = q.shape
    hkv = k_pool.shape[1]
    group = Hq // hkv
    out = torch.zeros(B, Hq, D, dtype=dtype)
    for b in range(B):
        n = int(positions[b]) + 1
        if n <= 0:
            continue
        k = gather_sequence(k_pool, page_table[b], n).to(dtype)
        v = gather_sequence(v_pool, page_table[b], n).to(dtype)
        k = k.repeat_interleave(group, dim=0)   # [Hq, n, D]
        v = v.repeat_interleave(group, dim=0)
        qb = q[b].to(dtype).unsqueeze(1)        # [Hq, 1, D]
        o = F.scaled_dot_product_attention(qb.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                                           scale=scale)
        out[b] = o[0, :, 0]
    return out


def paged_decode_naive(q, k_pool, v_pool, page_table, positions, scale):
    """Explicit per-row loop in float64: softmax(q.k * scale) weighted sum of v, reading
    each slot's physical block by hand. Used to pin :func:`paged_decode_ref`."""
    B, Hq, D = q.shape
    nb, hkv, bs, _ = k_pool.shape
    group = Hq // hkv
    out = torch.zeros(B, Hq, D, dtype=torch.float64)
    for b in range(B):
        n = int(positions[b]) + 1
        for h in range(Hq):
            g = h // group
            scores = []
            for t in range(n):
                phys = int(page_table[b, t // bs])
                kv = k_pool[phys, g, t % bs].double()
                scores.append(float((q[b, h].double() * kv).sum()) * scale)
            m = max(scores)
            ws = [pow(2.718281828459045, s - m) for s in scores]
            tot = sum(ws)
            acc = torch.zeros(D, dtype=torch.float64)
            for t, w in enumerate(ws):
                phys = int(page_table[b, t // bs])
                acc += w * v_pool[phys, g, t % bs].double()
            out[b, h] = acc / tot
    return out


class PagedKVCacheRef:
    """CPU paged cache with the reference's layout, one K and V pool per layer."""

    def __init__(self, k_pools: List[torch.Tensor], v_pools: List[torch.Tensor],
                 page_table: torch.Tensor):
        self.k_pools = k_pools
        self.v_pools = v_pools
        self.page_table = page_table.to(torch.int64)
        self.block_size = k_pools[0].shape[2]

    def write(self, layer: int, positions: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        """k, v [B, Hkv, D] written at slot positions[b] of each sequence."""
        bs = self.block_size
        for b in range(k.shape[0]):
            pos = int(positions[b])
            phys = int(self.page_table[b, pos // bs])
            self.k_pools[layer][phys, :, pos % bs] = k[b].to(self.k_pools[layer].dtype)
            self.v_pools[layer][phys, :, pos % bs] = v[b].to(self.v_pools[layer].dtype)

    def gather(self, layer: int, b: int, length: int):
        return (gather_sequence(self.k_pools[layer], self.page_table[b], length),
                gather_sequence(self.v_pools[layer], self.page_table[b], length))
