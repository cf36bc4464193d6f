"""Paged KV cache on one GPU, with the reference's object API.

Reference: ``PagedAttentionConfig`` and ``TTNNPagedAttentionKVCache``
(ttnn_attention.py:60-371). Same geometry -- per layer one K and one V pool
``[max_num_blocks, num_kv_heads, block_size, head_dim]`` (bf16, zero-initialised) and a page
table ``[batch, blocks_per_sequence]`` int32 mapping logical to physical blocks (identity
``arange`` by default, replaceable with :meth:`set_vllm_page_table`) -- and the same methods:
``to_device``, ``set_vllm_page_table``, ``paged_fill_on_device``, ``paged_update_on_device``,
``paged_sdpa_decode``, ``update_seq_length``, ``get_seq_length``, ``get_max_cache_shape``,
``update`` and ``reset``, with the same host-side counter semantics.

An fp8 variant (``dtype=torch.float8_e4m3fn``) keeps the pools in OCP e4m3fn bytes with one
power-of-two fp32 scale per (block, kv head) per layer (``key_scale`` / ``value_scale``,
``[max_num_blocks, num_kv_heads]``); appends requantise a block's earlier tokens when its scale
grows. Its V pool is dim-major inside each (block, head), ``[max_num_blocks, num_kv_heads,
head_dim, block_size]`` (the operand layout of the attention's P.V; ``hip_ops.fp8_v_rows``
views it as token rows), and block_size is a multiple of 8. The reference's cache is bf16 only;
the format and its rule are this library's.

Differences: pools are torch tensors in HBM (one allocation per pool); the page table is
validated on the host when installed (every entry must name a block of the pool) and copied in
place when its shape is unchanged, so captured HIP graphs that read it stay valid; positions are
per-sequence device int32 tensors, so ragged batches decode without host synchronisation.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch

from .. import hip_ops

try:  # the reference subclasses HF's Cache so HF code accepts the object as past_key_values
    from transformers.cache_utils import Cache as _CacheBase
except Exception:  # pragma: no cover - transformers is optional for the kernels
    _CacheBase = object


@dataclass
class PagedAttentionConfig:
    block_size: int = 64
    max_num_blocks: int = 2048
    batch_size: int = 1

    @property
    def max_seq_length(self) -> int:
        return self.max_num_blocks * self.block_size

    @property
    def blocks_per_sequence(self) -> int:
        return self.max_num_blocks // self.batch_size


class HIPPagedAttentionKVCache(_CacheBase):
    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int,
                 config: PagedAttentionConfig, device=None, dtype: torch.dtype = torch.bfloat16):
        if _CacheBase is not object:
            try:
                super().__init__(layers=[])
            except Exception:
                super().__init__()
        if dtype not in (torch.bfloat16, torch.float8_e4m3fn):
            raise NotImplementedError(f"KV cache dtype {dtype} (bf16 or float8_e4m3fn)")
        if dtype == torch.float8_e4m3fn and (config.block_size % 8 or 256 % config.block_size):
            raise ValueError(f"fp8 KV cache: block_size {config.block_size} must be a multiple "
                             f"of 8 dividing 256")
        if head_dim != hip_ops.HEAD_DIM:
            raise NotImplementedError(f"head_dim {head_dim} (kernels implement {hip_ops.HEAD_DIM})")
        if config.blocks_per_sequence < 1:
            raise ValueError("max_num_blocks must be >= batch_size")
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.config = config
        self.dtype = dtype
        self._device = None
        self._seq_lengths: List[int] = [0] * num_layers
        self._seen_tokens = 0
        self._external_seq_tracking = False
        table = torch.arange(config.batch_size * config.blocks_per_sequence, dtype=torch.int32)
        self.page_table = table.reshape(config.batch_size, config.blocks_per_sequence)
        self._key_cache: List[Optional[torch.Tensor]] = [None] * num_layers
        self._value_cache: List[Optional[torch.Tensor]] = [None] * num_layers
        self._key_scale: List[Optional[torch.Tensor]] = [None] * num_layers
        self._value_scale: List[Optional[torch.Tensor]] = [None] * num_layers
        self._arange: Optional[torch.Tensor] = None
        self._page_table_dev: Optional[torch.Tensor] = None
        self._is_on_device = False
        self._decode_ws: Optional[torch.Tensor] = None
        if device is not None:
            self.to_device(device)

    # ------------------------------------------------------------------ device state
    def to_device(self, device) -> "HIPPagedAttentionKVCache":
        device = torch.device(device)
        if self._is_on_device and self._device == device:
            return self
        shape = (self.config.max_num_blocks, self.num_kv_heads, self.config.block_size,
                 self.head_dim)
        # fp8: V dim-major inside each (block, head), [num_blocks, Hkv, head_dim, block_size]
        v_shape = shape[:2] + (shape[3], shape[2]) if self.is_fp8 else shape
        for i in range(self.num_layers):
            self._key_cache[i] = torch.zeros(shape, dtype=self.dtype, device=device)
            self._value_cache[i] = torch.zeros(v_shape, dtype=self.dtype, device=device)
            if self.is_fp8:
                self._key_scale[i] = torch.zeros(shape[:2], dtype=torch.float32, device=device)
                self._value_scale[i] = torch.zeros(shape[:2], dtype=torch.float32, device=device)
        self._page_table_dev = self.page_table.to(device)
        self._device = device
        self._is_on_device = True
        return self

    def _require_device(self):
        if not self._is_on_device:
            raise RuntimeError("KV cache not on device. Call to_device(device).")

    @property
    def device(self):
        return self._device

    @property
    def is_fp8(self) -> bool:
        return self.dtype == torch.float8_e4m3fn

    def key_scale(self, layer_idx: int) -> Optional[torch.Tensor]:
        """Per-(block, kv head) scales of layer ``layer_idx``'s K pool (None for bf16)."""
        self._require_device()
        return self._key_scale[layer_idx]

    def value_scale(self, layer_idx: int) -> Optional[torch.Tensor]:
        self._require_device()
        return self._value_scale[layer_idx]

    def _cu_arange(self, n: int) -> torch.Tensor:
        """[0, 1, .., n] int32 on the device (one token per sequence), kept for reuse."""
        if self._arange is None or self._arange.numel() < n + 1:
            self._arange = torch.arange(max(n + 1, 2), dtype=torch.int32, device=self._device)
        return self._arange[:n + 1]

    def key_cache(self, layer_idx: int) -> torch.Tensor:
        self._require_device()
        return self._key_cache[layer_idx]

    def value_cache(self, layer_idx: int) -> torch.Tensor:
        self._require_device()
        return self._value_cache[layer_idx]

    @property
    def page_table_device(self) -> torch.Tensor:
        self._require_device()
        return self._page_table_dev

    @property
    def max_context(self) -> int:
        """Largest number of cached tokens a sequence can address through the page table."""
        return int(self.page_table.shape[1]) * self.config.block_size

    def set_vllm_page_table(self, page_table: torch.Tensor) -> "HIPPagedAttentionKVCache":
        """Install an externally managed page table ``[batch, blocks_per_sequence]``."""
        self._require_device()
        if page_table.dim() != 2:
            raise ValueError("page_table must be 2D [batch, blocks_per_sequence], got shape "
                             f"{tuple(page_table.shape)}")
        host = page_table.detach().to("cpu", torch.int32).contiguous()
        if host.numel() and (int(host.min()) < 0 or int(host.max()) >= self.config.max_num_blocks):
            raise ValueError(f"page_table entries must lie in [0, {self.config.max_num_blocks})")
        self.page_table = host
        if self._page_table_dev is not None and self._page_table_dev.shape == host.shape:
            self._page_table_dev.copy_(host)
        else:
            self._page_table_dev = host.to(self._device)
        return self

    # ------------------------------------------------------------------ counters
    def _advance(self, layer_idx: int, n: int) -> None:
        if not self._external_seq_tracking:
            self._seq_lengths[layer_idx] += n
            if layer_idx == 0:
                self._seen_tokens += n

    def advance(self, layer_idx: int, n: int) -> None:
        """Advance layer ``layer_idx``'s counter by ``n`` tokens after a fill or an update,
        unless the caller tracks the counters itself (:meth:`update_seq_length`); the paged
        ops of the attention module call this, as the reference's paged_fill_on_device /
        paged_update_on_device do (ttnn_attention.py:224-233, 259-269)."""
        self._advance(layer_idx, n)

    def set_external_seq_tracking(self, enabled: bool = True) -> None:
        """Hand the counters to the caller (a model loop that calls :meth:`update_seq_length`
        after each layer, outside any captured region) before its first layer runs, so that no
        layer's own fill is counted as well."""
        self._external_seq_tracking = bool(enabled)

    def update_seq_length(self, layer_idx: int, seq_len: int = 1) -> None:
        """Advance the host counters (call from the model loop); switches to external tracking."""
        self._external_seq_tracking = True
        self._seq_lengths[layer_idx] += seq_len
        if layer_idx == 0:
            self._seen_tokens += seq_len

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._seq_lengths[layer_idx]

    def get_max_cache_shape(self) -> Optional[int]:
        return self.config.max_seq_length

    def reset(self) -> None:
        """Reset host counters; device buffers (and their addresses) are kept."""
        self._seq_lengths = [0] * self.num_layers
        self._seen_tokens = 0

    def update(self, key_states, value_states, layer_idx: int, cache_kwargs=None):
        """HF ``Cache.update`` contract for torch layers: counters only (as the reference)."""
        seq_len = key_states.shape[2]
        self._seq_lengths[layer_idx] = seq_len
        if layer_idx == 0:
            self._seen_tokens = seq_len
        return key_states, value_states

    # ------------------------------------------------------------------ paged ops
    def _positions(self, current_pos, batch: int) -> torch.Tensor:
        if not isinstance(current_pos, torch.Tensor):
            current_pos = torch.as_tensor(current_pos)
        pos = current_pos.reshape(-1)
        if pos.numel() == 1 and batch > 1:
            pos = pos.expand(batch)
        if pos.numel() != batch:
            raise ValueError(f"current_pos has {pos.numel()} entries for batch {batch}")
        return pos.to(device=self._device, dtype=torch.int32).contiguous()

    def paged_fill_on_device(self, key_states: torch.Tensor, value_states: torch.Tensor,
                             layer_idx: int, batch_idx: int = 0) -> None:
        """Write a prompt's K/V ``[1, Hkv, S, D]`` (or ``[Hkv, S, D]``) at positions 0..S-1."""
        self._require_device()
        k = key_states[0] if key_states.dim() == 4 else key_states
        v = value_states[0] if value_states.dim() == 4 else value_states
        max_len = self.max_context
        if k.shape[1] > max_len:
            k, v = k[:, :max_len], v[:, :max_len]
        if self.is_fp8:
            k = k.to(torch.bfloat16).contiguous()
            v = v.to(torch.bfloat16).contiguous()
            S = k.shape[1]
            cu = torch.tensor([0, S], dtype=torch.int32, device=self._device)
            rows = self._cu_arange(self.page_table.shape[0])[batch_idx:batch_idx + 1]
            hip_ops.paged_kv_fill_fp8(
                k, v, cu, S, self._key_cache[layer_idx], self._value_cache[layer_idx],
                self._key_scale[layer_idx], self._value_scale[layer_idx], self._page_table_dev,
                layout="htd", seq_rows=rows)
            self._advance(layer_idx, S)
            return
        k = k.to(self.dtype).contiguous()
        v = v.to(self.dtype).contiguous()
        hip_ops.paged_kv_fill(k, v, self._key_cache[layer_idx], self._value_cache[layer_idx],
                              self._page_table_dev, batch_idx, 0)
        self._advance(layer_idx, k.shape[1])

    def paged_update_on_device(self, key_states: torch.Tensor, value_states: torch.Tensor,
                               layer_idx: int, current_pos) -> None:
        """Write one token per sequence: K/V ``[1, B, Hkv, D]`` or ``[B, Hkv, D]``."""
        self._require_device()
        k = key_states[0] if key_states.dim() == 4 else key_states
        v = value_states[0] if value_states.dim() == 4 else value_states
        B = k.shape[0]
        pos = self._positions(current_pos, B)
        if self.is_fp8:
            hip_ops.paged_kv_fill_fp8(
                k.to(torch.bfloat16).contiguous(), v.to(torch.bfloat16).contiguous(),
                self._cu_arange(B), 1, self._key_cache[layer_idx], self._value_cache[layer_idx],
                self._key_scale[layer_idx], self._value_scale[layer_idx], self._page_table_dev,
                start_pos=pos)
            self._advance(layer_idx, 1)
            return
        hip_ops.paged_kv_write(k.to(self.dtype).contiguous(), v.to(self.dtype).contiguous(),
                               self._key_cache[layer_idx], self._value_cache[layer_idx],
                               self._page_table_dev, pos)
        self._advance(layer_idx, 1)

    def decode_workspace(self, batch: int, num_heads: int) -> torch.Tensor:
        """Per-split partial results of the decode kernel (grown on demand, reused)."""
        need = hip_ops.paged_decode_workspace_bytes(batch, num_heads, self.max_context)
        if self._decode_ws is None or self._decode_ws.numel() < need:
            self._decode_ws = torch.empty(need, dtype=torch.uint8, device=self._device)
        return self._decode_ws

    def paged_sdpa_decode(self, query: torch.Tensor, layer_idx: int, current_pos,
                          scale: float = 1.0, program_config=None, compute_kernel_config=None,
                          sliding_window: Optional[int] = None) -> torch.Tensor:
        """Decode attention of ``query`` ``[1, B, Hq, D]`` (or ``[B, Hq, D]``) over slots
        0..current_pos[b]. ``sliding_window`` is accepted and, as in the reference, not
        enforced."""
        self._require_device()
        squeeze = query.dim() == 4
        q = query[0] if squeeze else query
        B, Hq, _ = q.shape
        pos = self._positions(current_pos, B)
        out = hip_ops.paged_gqa_decode(q.to(torch.bfloat16).contiguous(),
                                       self._key_cache[layer_idx],
                                       self._value_cache[layer_idx], self._page_table_dev, pos,
                                       scale, max_context=self.max_context,
                                       workspace=self.decode_workspace(B, Hq),
                                       k_scale=self._key_scale[layer_idx],
                                       v_scale=self._value_scale[layer_idx])
        return out.unsqueeze(0) if squeeze else out
