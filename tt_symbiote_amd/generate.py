"""Greedy generation on the device.

The reference generates with HF ``GenerationMixin.generate`` (the HF
token loop calls the TTNN model once per token, reads the logits back and takes the argmax on
the host; the model's layer loop is Python, one op dispatch at a time;
modeling_bailing_moe_v2.py:97-334, run_config.py:595-647). Here a batch of prompts is generated
without the host in the loop:

  1. prefill: the prompts, packed varlen in groups of at most ``prefill_tokens`` tokens, go
     through every layer (their K/V land in the paged cache, page-table row = prompt index);
     the last row of each prompt is gathered, normed and greedily decoded into the first new
     token;
  2. decode: one step = embedding of the current tokens -> every layer's fused decode step ->
     final RMSNorm -> LM head with argmax -> ``sym_greedy_advance`` (positions += 1, the token
     stored in the history). The step reads and writes only device buffers, so it is captured
     once as a HIP graph and replayed for every further token.

Prompts of different lengths are supported (each sequence keeps its own position); there is no
stopping criterion (exactly ``max_new_tokens`` per sequence, as the fixed-length benchmark).
The cache's host counters (one per layer, batch-uniform as the reference's) follow sequence 0:
they are advanced with ``update_seq_length`` after the prefill and after the decode steps,
outside the captured graph, as the reference's model loop does (modeling_bailing_moe_v2.py
:244-251).
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch

from . import hip_ops
from .modules.model import HIPBailingMoeV2Model, HIPLMHead


@dataclass
class GreedyResult:
    tokens: torch.Tensor     # [B, max_new_tokens] int32 (host)
    prefill_s: float         # prefill wall time (device-synchronised)
    decode_s: float          # wall time of the decode steps after the first token
    decode_steps: int


class GreedyGenerator:
    """Device buffers and the captured decode step of one batch."""

    def __init__(self, model: HIPBailingMoeV2Model, lm_head: HIPLMHead, cache, batch: int,
                 max_new_tokens: int, use_graph: bool = True):
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be >= 1")
        if cache.page_table.shape[0] < batch:
            raise ValueError(f"the cache's page table has {cache.page_table.shape[0]} rows for "
                             f"a batch of {batch}")
        self.model = model
        self.lm_head = lm_head
        self.cache = cache
        self.batch = batch
        self.max_new_tokens = max_new_tokens
        self.use_graph = use_graph
        dev = model.device
        i32 = dict(dtype=torch.int32, device=dev)
        self.ids = torch.zeros(batch, **i32)          # token fed to the next decode step
        self.positions = torch.zeros(batch, **i32)    # its position
        self.history = torch.zeros(batch, max_new_tokens, **i32)
        self.hist_base = torch.zeros(batch, **i32)    # prompt lengths
        self.graph = None

    # ---------------------------------------------------------------- prefill
    def prefill(self, prompts: Sequence[torch.Tensor], prefill_tokens: int = 16384) -> None:
        """Run the prompts (1-D int tensors) and choose each one's first new token."""
        if len(prompts) != self.batch:
            raise ValueError(f"{len(prompts)} prompts for a batch of {self.batch}")
        lens = [int(p.numel()) for p in prompts]
        if min(lens) < 1:
            raise ValueError("empty prompt")
        if max(lens) + self.max_new_tokens > self.cache.max_context:
            raise ValueError(f"prompt + {self.max_new_tokens} new tokens exceed the cache's "
                             f"{self.cache.max_context} tokens per sequence")
        dev = self.model.device
        s = 0
        while s < self.batch:
            e = s + 1
            total = lens[s]
            while e < self.batch and total + lens[e] <= prefill_tokens:
                total += lens[e]
                e += 1
            group = list(range(s, e))
            ids = torch.cat([prompts[i].reshape(-1).to(torch.int32) for i in group]).to(dev)
            cu_h = torch.tensor([0] + lens[s:e], dtype=torch.int32).cumsum(0, dtype=torch.int32)
            cu = cu_h.to(dev)
            seq = torch.cat([torch.full((lens[i],), i, dtype=torch.int32) for i in group]).to(dev)
            pos = torch.cat([torch.arange(lens[i], dtype=torch.int32) for i in group]).to(dev)
            hn = self.model.prefill_hidden(ids, cu, max(lens[s:e]), self.cache, seq_ids=seq,
                                           positions=pos)
            last = (cu[1:] - 1).contiguous()
            rows = hip_ops.embedding(last, hn)                 # gather each prompt's last row
            self.ids[s:e].copy_(self.lm_head.greedy(rows))
            s = e
        self._count(lens[0])
        lens_d = torch.tensor(lens, dtype=torch.int32, device=dev)
        self.hist_base.copy_(lens_d)
        self.positions.copy_(lens_d - 1)
        hip_ops.greedy_advance(self.ids, self.positions, self.history, self.hist_base)

    def _count(self, n: int) -> None:
        self.cache.set_external_seq_tracking(True)
        for i in range(len(self.model.layers)):
            self.cache.update_seq_length(i, n)

    # ---------------------------------------------------------------- decode
    def _step(self) -> None:
        hn = self.model.decode_hidden(self.ids, self.positions, self.cache)
        self.lm_head.greedy(hn, ids=self.ids)
        hip_ops.greedy_advance(self.ids, self.positions, self.history, self.hist_base)

    def decode(self, n_steps: int) -> None:
        """n_steps decode steps (each appends one token per sequence)."""
        done = 0
        if self.use_graph and self.graph is None and n_steps > 0:
            self._step()          # allocates the grow-only workspaces before capture
            done = 1
            torch.cuda.synchronize()
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self._step()
        for _ in range(n_steps - done):
            if self.graph is not None:
                self.graph.replay()
            else:
                self._step()
        self._count(n_steps)


def greedy_generate(model: HIPBailingMoeV2Model, lm_head: HIPLMHead, prompts, cache,
                    max_new_tokens: int, use_graph: bool = True,
                    prefill_tokens: int = 16384) -> GreedyResult:
    """Greedy-decode ``max_new_tokens`` tokens for each prompt (a [B, L] tensor or a list of 1-D
    tensors) with the paged ``cache`` (row b of its page table serves prompt b)."""
    if isinstance(prompts, torch.Tensor):
        prompts = list(prompts.reshape(prompts.shape[0], -1))
    gen = GreedyGenerator(model, lm_head, cache, len(prompts), max_new_tokens, use_graph)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    gen.prefill(prompts, prefill_tokens)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    gen.decode(max_new_tokens - 1)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    return GreedyResult(gen.history.cpu(), t1 - t0, t2 - t1, max_new_tokens - 1)


def model_parts(hf_model):
    """(trunk, lm_head) of an HF-shaped BailingMoeV2ForCausalLM after apply_recipe."""
    trunk = getattr(hf_model, "model", None)
    head = getattr(hf_model, "lm_head", None)
    if not isinstance(trunk, HIPBailingMoeV2Model) or not isinstance(head, HIPLMHead):
        raise TypeError("apply the recipe (and set_device) first: model.model and model.lm_head "
                        "must be the HIP modules")
    return trunk, head
