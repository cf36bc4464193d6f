"""HIP-backed BailingMoeV2 model trunk and LM head, for whole-model decode and greedy generation.

Replaces ``TTNNBailingMoeV2Model`` (modeling_bailing_moe_v2.py:56-334), which swaps the HF
model's embedding, decoder layers and final norm (``from_torch`` 56-95) and runs the layer loop
(97-334, final norm at 262), and the ``lm_head`` linear that the reference maps to a TTNN linear.
HF ``generate`` then reads the logits back and takes the argmax on the host; here
:meth:`HIPLMHead.greedy` takes it on the device (:mod:`tt_symbiote_amd.generate`).

``HIPBailingMoeV2Model.forward(input_ids, cache_position=..., past_key_values=cache)``:
  * seq_len 1 (decode): embedding gather -> each layer's fused decode step -> final RMSNorm;
    without ``cache_position`` / ``position_ids`` the tokens go at the cache's counter
    (``get_seq_length()``), as the reference builds its positions (modeling_bailing_moe_v2.py
    :154-158);
  * seq_len > 1: the batch rows are equal-length prompts at positions 0 .. S-1 (page-table row
    = batch row), run as packed varlen prefill through every layer.
As the reference's layer loop (modeling_bailing_moe_v2.py:244-251), the cache's host counters
are advanced by the model after each layer (``update_seq_length``: the cache switches to
external tracking before the first layer, so no layer is counted twice). Returns the
final-normed hidden states [B, S, H] (bf16) as ``last_hidden_state`` of a ``ModelOutput`` (a
tuple with ``return_dict=False``), as the HF model does.
"""
from __future__ import annotations

from typing import List, Optional

import torch

from .. import hip_ops
from ..core.module import StatefulHIPModule, StatelessHIPModule
from .attention import equal_length_packing, prefill_continues
from .decoder_layer import HIPBailingMoEDecoderLayer


def _model_output(hidden: torch.Tensor, cache):
    """HF's BaseModelOutputWithPast (last_hidden_state, past_key_values), or a tuple when
    transformers is absent."""
    try:
        from transformers.modeling_outputs import BaseModelOutputWithPast
    except Exception:  # pragma: no cover - transformers is optional for the kernels
        return (hidden, cache)
    return BaseModelOutputWithPast(last_hidden_state=hidden, past_key_values=cache)


def _embedding_module(torch_model):
    for name in ("word_embeddings", "embed_tokens"):
        emb = getattr(torch_model, name, None)
        if emb is not None:
            return emb
    raise AttributeError(f"{type(torch_model).__name__} has no word_embeddings / embed_tokens")


class HIPBailingMoeV2Model(StatefulHIPModule):
    def __init__(self):
        super().__init__()
        self.layers: List[HIPBailingMoEDecoderLayer] = []
        self.hidden_size = None
        self.vocab_size = None
        self.eps = 1e-6
        self.config = None
        self._host = {}
        self._dev = {}

    @classmethod
    def from_torch(cls, torch_model):
        emb = _embedding_module(torch_model)
        layers = [layer if isinstance(layer, HIPBailingMoEDecoderLayer)
                  else HIPBailingMoEDecoderLayer.from_torch(layer)
                  for layer in torch_model.layers]
        norm = torch_model.norm
        eps = float(getattr(norm, "variance_epsilon", getattr(norm, "eps", 1e-6)))
        new = cls.from_modules(emb.weight, layers, norm.weight, eps)
        new.config = getattr(torch_model, "config", None)
        new._fallback_torch_layer = torch_model
        return new

    @classmethod
    def from_modules(cls, embed_weight, layers, norm_weight, eps: float = 1e-6):
        new = cls()
        new.layers = list(layers)
        new.vocab_size, new.hidden_size = embed_weight.shape
        new.eps = float(eps)
        new._host = dict(embed=embed_weight, norm=norm_weight)
        return new

    def preprocess_weights_impl(self):
        self._host = {k: v.detach().to(torch.bfloat16).contiguous() for k, v in self._host.items()}
        for layer in self.layers:
            layer.preprocess_weights()
        return super().preprocess_weights_impl()

    def move_weights_to_device_impl(self):
        self._dev = {k: v.to(self.device) for k, v in self._host.items()}
        self._host = {}
        for layer in self.layers:
            if layer.device is None:
                layer.to_device(self.device)
            layer.move_weights_to_device()
        return super().move_weights_to_device_impl()

    def reset_trace_state(self):
        # the layers' KV-slot writes are the only state a step mutates; positions are inputs
        return None

    # ------------------------------------------------------------------ pieces of a step
    def embed(self, ids: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Embedding rows of ids [T] (int32, on the device) -> [T, H] bf16."""
        return hip_ops.embedding(ids, self._dev["embed"], out=out)

    def final_norm(self, h: torch.Tensor) -> torch.Tensor:
        return hip_ops.rmsnorm(h, self._dev["norm"], self.eps)

    def decode_hidden(self, ids: torch.Tensor, positions: torch.Tensor, cache) -> torch.Tensor:
        """One decode step of the trunk: ids [B] int32 at positions [B] -> normed [B, H]."""
        B = ids.numel()
        h = self.embed(ids).view(B, 1, self.hidden_size)
        for layer in self.layers:
            h = layer(h, past_key_values=cache, cache_position=positions)[0]
        return self.final_norm(h.view(B, self.hidden_size))

    def prefill_hidden(self, ids: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                       cache, seq_ids: Optional[torch.Tensor] = None,
                       positions: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Packed prefill of the trunk: ids [T] int32 (sequence s = rows cu_seqlens[s] ..
        cu_seqlens[s+1]-1, positions 0 .. L-1, page-table row seq_ids of its tokens, default s)
        -> normed [T, H]; the prompts' K/V land in the cache."""
        h = self.embed(ids)
        for layer in self.layers:
            h = layer.prefill_varlen(h, cu_seqlens, max_seqlen, cache, positions=positions,
                                     seq_ids=seq_ids)
        return self.final_norm(h)

    # ------------------------------------------------------------------ HF-shaped forward
    def forward(self, input_ids=None, attention_mask=None, position_ids=None,
                past_key_values=None, inputs_embeds=None, cache_position=None,
                return_dict=None, **kwargs):
        if inputs_embeds is not None:
            raise NotImplementedError("inputs_embeds: pass input_ids")
        cache = past_key_values if past_key_values is not None else kwargs.get("past_key_value")
        if cache is None:
            raise NotImplementedError("HIPBailingMoeV2Model needs the paged KV cache "
                                      "(model._tt_kv_cache) as past_key_values")
        ids = torch.as_tensor(input_ids)
        if ids.dim() == 1:
            ids = ids.view(1, -1)
        B, S = ids.shape
        dev = self.device
        ids = ids.to(device=dev, dtype=torch.int32).contiguous()
        cache.set_external_seq_tracking(True)
        if S == 1:
            pos = cache_position if cache_position is not None else position_ids
            if pos is None:
                pos = torch.tensor([cache.get_seq_length(0)])
            pos = torch.as_tensor(pos).reshape(-1)
            if pos.numel() != B:
                pos = pos.expand(B) if pos.numel() == 1 else pos.reshape(B, -1)[:, -1]
            pos = pos.to(device=dev, dtype=torch.int32).contiguous()
            h = self.embed(ids.view(B)).view(B, 1, self.hidden_size)
            for i, layer in enumerate(self.layers):
                h = layer(h, past_key_values=cache, cache_position=pos)[0]
                cache.update_seq_length(i, 1)
            h = self.final_norm(h.view(B, self.hidden_size)).view(B, 1, self.hidden_size)
        else:
            pos = cache_position if cache_position is not None else position_ids
            if prefill_continues(cache, 0, pos):
                raise NotImplementedError("prefill starting at a cached position; prompts "
                                          "start at position 0 (as the reference's prefill)")
            if B > cache.page_table.shape[0]:
                raise ValueError(f"{B} prompts for a page table of {cache.page_table.shape[0]} "
                                 "rows")
            positions, seq_ids, cu = equal_length_packing(B, S, dev)
            h = self.embed(ids.view(B * S))
            for i, layer in enumerate(self.layers):
                h = layer.prefill_varlen(h, cu, S, cache, positions=positions, seq_ids=seq_ids)
                cache.update_seq_length(i, S)
            h = self.final_norm(h).view(B, S, self.hidden_size)
        if return_dict is False:
            return (h, cache)
        return _model_output(h, cache)


class HIPLMHead(StatelessHIPModule):
    """The lm_head linear [V, H] (no bias), with the greedy choice fused on the device."""

    def __init__(self):
        super().__init__()
        self.vocab_size = None
        self.hidden_size = None
        self._host = {}
        self._dev = {}
        self._ws = None

    @classmethod
    def from_torch(cls, linear):
        if getattr(linear, "bias", None) is not None:
            raise NotImplementedError("lm_head with a bias")
        new = cls.from_weight(linear.weight)
        new._fallback_torch_layer = linear
        return new

    @classmethod
    def from_weight(cls, weight):
        new = cls()
        new.vocab_size, new.hidden_size = weight.shape
        new._host = dict(w=weight)
        return new

    def preprocess_weights_impl(self):
        self._host = {k: v.detach().to(torch.bfloat16).contiguous() for k, v in self._host.items()}
        return super().preprocess_weights_impl()

    def move_weights_to_device_impl(self):
        self._dev = {k: v.to(self.device) for k, v in self._host.items()}
        self._host = {}
        # the projection kernels take multiples of 16 output rows: the last vocab % 16 rows get
        # a zero-padded 16-row copy for the logits path
        V, H = self._dev["w"].shape
        tail = V % 16
        if tail:
            pad = torch.zeros(16, H, dtype=torch.bfloat16, device=self.device)
            pad[:tail].copy_(self._dev["w"][V - tail:])
            self._dev["w_tail"] = pad
        return super().move_weights_to_device_impl()

    @property
    def weight(self) -> torch.Tensor:
        return self._dev["w"]

    def workspace(self, batch: int) -> torch.Tensor:
        need = hip_ops.lm_head_greedy_workspace_bytes(batch, self.vocab_size)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws

    def greedy(self, x: torch.Tensor, ids: Optional[torch.Tensor] = None) -> torch.Tensor:
        """argmax over the vocabulary of x [B, H] (bf16, normed) . W^T -> [B] int32."""
        x = x.reshape(-1, self.hidden_size)
        return hip_ops.lm_head_greedy(x, self._dev["w"], ids=ids,
                                      workspace=self.workspace(x.shape[0]))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Logits (fp32) [..., V] for HF-style callers."""
        shape = x.shape
        x2 = x.reshape(-1, self.hidden_size).to(torch.bfloat16).contiguous()
        op = hip_ops.linear if x2.shape[0] <= 64 else hip_ops.gemm
        V = self.vocab_size
        tail = V % 16
        parts = []
        if V - tail:
            parts.append(op(x2, self._dev["w"][:V - tail], None, out_dtype=torch.float32))
        if tail:
            parts.append(op(x2, self._dev["w_tail"], None, out_dtype=torch.float32)[:, :tail])
        out = parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)
        return out.view(*shape[:-1], V)
