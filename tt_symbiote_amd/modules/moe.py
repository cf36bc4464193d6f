"""HIP-backed BailingMoeV2 MoE block (and the dense SwiGLU MLP of the first layers).

Replaces ``TTNNBailingMoE`` (ttnn_moe.py:1494-1647) / ``TTNNMoE.forward`` (1413-1491).
``from_torch`` performs the reference's adaptation (ttnn_moe.py:1557-1647):
``num_experts -> n_routed_experts``, ``num_shared_experts``, ``n_group``, ``topk_group``,
``routed_scaling_factor``, ``moe_intermediate_size``; stacks ``experts[i].gate_proj`` /
``up_proj`` rows into ``gate_up [E, 2I, H]`` (gate rows first) and ``down_proj`` into
``down [E, H, I]``; takes ``gate.expert_bias`` as the score-correction bias (zeros if absent);
forces ``norm_topk_prob`` True (ttnn_moe.py:1532). The shared expert (intermediate
``I * num_shared_experts``) is stored as stack slot ``E`` when its width equals ``I``.

``weight_format="fp8_e4m3"`` stores the routed and shared expert weights as OCP fp8 e4m3fn with
one fp32 scale per 128 x 128 block (quantised once when the weights are prepared); the grouped
kernels dequantise inside the GEMM.

Forward (decode or prefill token counts alike, no host synchronisation):
  logits = x_fp32 W_gate_fp32^T                   fp32 MFMA kernel (four partial sums)
  route  = fused router + top-k + permute kernel  (bit-exact indices)
  h, y   = grouped SwiGLU kernels over the device segment list (+ shared expert)
  out    = unpermute + weighted combine (+ shared) (+ optional residual) kernel
"""
from __future__ import annotations

from typing import Dict

import torch

from .. import hip_ops
from ..core.module import StatelessHIPModule


class HIPBailingMoE(StatelessHIPModule):
    def __init__(self):
        super().__init__()
        self.hidden_size = None
        self.num_experts = None
        self.top_k = None
        self.n_group = None
        self.topk_group = None
        self.routed_scaling_factor = 1.0
        self.intermediate_size = None
        self.has_shared = False
        self.weight_format = "bf16"
        self.keep_last_route = False  # keep the last RouteResult (inspection / tests)
        self.last_route = None
        self._host: Dict[str, torch.Tensor] = {}
        self._dev: Dict[str, torch.Tensor] = {}

    WEIGHT_FORMATS = ("bf16", "fp8_e4m3")

    @classmethod
    def from_torch(cls, torch_moe, weight_format: str = "bf16"):
        cfg = torch_moe.config
        experts = list(torch_moe.experts)
        gate = torch_moe.gate
        bias = getattr(gate, "expert_bias", None)
        if bias is None:
            bias = getattr(gate, "e_score_correction_bias", None)
        if bias is None:
            bias = torch.zeros(gate.weight.shape[0])
        shared = getattr(torch_moe, "shared_experts", None)
        shared_gate_up = shared_down = None
        if shared is not None:
            shared_gate_up = torch.cat([shared.gate_proj.weight.detach(),
                                        shared.up_proj.weight.detach()], dim=0)
            shared_down = shared.down_proj.weight.detach()
        new = cls.from_weights(
            gate_weight=gate.weight, expert_bias=bias, experts=experts,
            shared_gate_up=shared_gate_up, shared_down=shared_down,
            top_k=cfg.num_experts_per_tok, n_group=cfg.n_group, topk_group=cfg.topk_group,
            routed_scaling_factor=cfg.routed_scaling_factor, weight_format=weight_format)
        new._fallback_torch_layer = torch_moe
        return new

    @classmethod
    def from_weights(cls, *, gate_weight, expert_bias, top_k, n_group, topk_group,
                     routed_scaling_factor, w_gate_up=None, w_down=None, experts=None,
                     shared_gate_up=None, shared_down=None, weight_format: str = "bf16"):
        """Build from stacked ``w_gate_up [E, 2I, H]`` / ``w_down [E, H, I]``, or from a list of
        HF expert MLPs (stacked lazily in ``preprocess_weights`` to bound host memory).
        ``weight_format``: "bf16", or "fp8_e4m3" (128 x 128 block-scaled e4m3fn experts)."""
        if weight_format not in cls.WEIGHT_FORMATS:
            raise ValueError(f"weight_format {weight_format!r} not in {cls.WEIGHT_FORMATS}")
        if experts is not None:
            E = len(experts)
            I, H = experts[0].gate_proj.weight.shape
        else:
            E, I2, H = w_gate_up.shape
            I = I2 // 2
            if tuple(w_down.shape) != (E, H, I):
                raise ValueError(f"w_down {tuple(w_down.shape)}, expected {(E, H, I)}")
        if tuple(gate_weight.shape) != (E, H):
            raise ValueError(f"gate weight {tuple(gate_weight.shape)}, expected {(E, H)}")
        if shared_gate_up is not None and tuple(shared_gate_up.shape) != (2 * I, H):
            raise NotImplementedError(
                "shared expert width must equal moe_intermediate_size (num_shared_experts == 1)")
        new = cls()
        new.hidden_size = H
        new.num_experts = E
        new.top_k = int(top_k)
        new.n_group = int(n_group)
        new.topk_group = int(topk_group)
        new.routed_scaling_factor = float(routed_scaling_factor)
        new.intermediate_size = I
        new.has_shared = shared_gate_up is not None
        new.weight_format = weight_format
        new._host = dict(gate_w=gate_weight, bias=expert_bias, gate_up=w_gate_up, down=w_down,
                         experts=experts, shared_gate_up=shared_gate_up, shared_down=shared_down)
        return new

    def preprocess_weights_impl(self):
        h = self._host
        E, I, H = self.num_experts, self.intermediate_size, self.hidden_size
        slots = E + (1 if self.has_shared else 0)
        # stack where the source weights live (host for HF modules; device for tensors that
        # are already resident, which avoids a round trip through host memory)
        src = h["gate_up"] if h["gate_up"] is not None else h["experts"][0].gate_proj.weight
        gate_up = torch.empty(slots, 2 * I, H, dtype=torch.bfloat16, device=src.device)
        down = torch.empty(slots, H, I, dtype=torch.bfloat16, device=src.device)
        if h["experts"] is not None:
            for i, ex in enumerate(h["experts"]):
                gate_up[i, :I] = ex.gate_proj.weight.detach().to(torch.bfloat16)
                gate_up[i, I:] = ex.up_proj.weight.detach().to(torch.bfloat16)
                down[i] = ex.down_proj.weight.detach().to(torch.bfloat16)
        else:
            gate_up[:E] = h["gate_up"].detach().to(torch.bfloat16)
            down[:E] = h["down"].detach().to(torch.bfloat16)
        if self.has_shared:
            gate_up[E] = h["shared_gate_up"].detach().to(torch.bfloat16)
            down[E] = h["shared_down"].detach().to(torch.bfloat16)
        if self.weight_format == "fp8_e4m3":
            gate_up = hip_ops.quantize_block_fp8(gate_up)
            down = hip_ops.quantize_block_fp8(down)
        gate_w = h["gate_w"].detach().float().contiguous()
        self._host = dict(
            gate_w=gate_w, gate_w_planes=hip_ops.split_router_weight(gate_w),
            bias=h["bias"].detach().float().contiguous(),
            gate_up=gate_up, down=down)
        return super().preprocess_weights_impl()

    def move_weights_to_device_impl(self):
        def move(v):
            if isinstance(v, hip_ops.BlockFp8):
                return hip_ops.BlockFp8(v.q.to(self.device), v.scale.to(self.device))
            return v.to(self.device)
        self._dev = {k: move(v) for k, v in self._host.items()}
        self._host = {}
        return super().move_weights_to_device_impl()

    def deallocate_weights_impl(self):
        self._dev = {}
        return super().deallocate_weights_impl()

    def route(self, x: torch.Tensor) -> hip_ops.RouteResult:
        """Router logits (fp32 MFMA, or for many tokens bf16 MFMA tiles over the exact
        three-plane split of the fp32 gate weight) + fused top-k/permute for x [T, H] (bf16)."""
        if x.shape[0] >= hip_ops.ROUTER_SPLIT_MIN_TOKENS:
            logits = hip_ops.moe_router_logits_split(x, self._dev["gate_w_planes"])
        else:
            logits = hip_ops.moe_router_logits(x, self._dev["gate_w"])
        return hip_ops.moe_route_permute(
            logits, self._dev["bias"], n_group=self.n_group, topk_group=self.topk_group,
            top_k=self.top_k, routed_scale=self.routed_scaling_factor, renormalize=True,
            with_shared=self.has_shared)

    def forward(self, hidden_states: torch.Tensor, residual: torch.Tensor = None) -> torch.Tensor:
        """MoE output (bf16); with ``residual`` the result is residual + MoE(x) (one rounding)."""
        shape = hidden_states.shape
        H = shape[-1]
        x = hidden_states.reshape(-1, H)
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        x = x.contiguous()
        res = None
        if residual is not None:
            res = residual.reshape(-1, H).to(torch.float32).contiguous()
        route = self.route(x)
        if self.keep_last_route:
            self.last_route = route
        _, y = hip_ops.moe_grouped_swiglu(x, route, self._dev["gate_up"], self._dev["down"],
                                          y_dtype=_y_dtype(self.weight_format, x.shape[0]))
        out = hip_ops.moe_unpermute_combine(y, route, residual=res)
        return out.view(shape)


    def forward_from_residual(self, h: torch.Tensor, ss_parts: torch.Tensor,
                              norm_weight: torch.Tensor, norm_eps: float) -> torch.Tensor:
        """h + MoE(RMSNorm(h) * norm_weight) (bf16 [T, H]) for the fp32 residual stream h
        [T, H]; ss_parts [n, T] are the partial sums of squares of h's rows. The RMSNorm runs
        inside the router-logits kernel, which also hands the normalised rows to the experts."""
        parts, xn = hip_ops.moe_router_logits_norm(h, ss_parts, norm_weight, norm_eps,
                                                   self._dev["gate_w"])
        route = hip_ops.moe_route_permute(
            parts, self._dev["bias"], n_group=self.n_group, topk_group=self.topk_group,
            top_k=self.top_k, routed_scale=self.routed_scaling_factor, renormalize=True,
            with_shared=self.has_shared)
        if self.keep_last_route:
            self.last_route = route
        _, y = hip_ops.moe_grouped_swiglu(xn, route, self._dev["gate_up"], self._dev["down"])
        return hip_ops.moe_unpermute_combine(y, route, residual=h)


def _y_dtype(weight_format: str, T: int) -> torch.dtype:
    """Expert outputs y in bf16 where the tiled (prefill-size) kernels run: the down GEMM writes
    half the bytes and the combine reads half; it sums in fp32 either way."""
    if weight_format == "bf16" and T >= hip_ops.TILED_MIN_TOKENS:
        return torch.bfloat16
    return torch.float32


class HIPBailingMoeV2MLP(StatelessHIPModule):
    """Dense SwiGLU MLP (layers < first_k_dense_replace), run as one segment of the grouped
    kernels. Replaces TTNNBailingMoeV2MLP (ttnn_moe.py; chosen at
    modeling_bailing_moe_v2.py:388-399)."""

    def __init__(self):
        super().__init__()
        self._host = {}
        self._dev = {}
        self._index_cache = {}

    @classmethod
    def from_torch(cls, torch_mlp):
        new = cls.from_weights(torch_mlp.gate_proj.weight, torch_mlp.up_proj.weight,
                               torch_mlp.down_proj.weight)
        new._fallback_torch_layer = torch_mlp
        return new

    @classmethod
    def from_weights(cls, gate_weight, up_weight, down_weight):
        """gate / up [I, H], down [H, I] (HF nn.Linear layouts)."""
        new = cls()
        new._host = dict(gate=gate_weight, up=up_weight, down=down_weight)
        return new

    def preprocess_weights_impl(self):
        h = self._host
        gate_up = torch.cat([h["gate"].detach(), h["up"].detach()], 0).to(torch.bfloat16)
        self._host = dict(gate_up=gate_up.unsqueeze(0).contiguous(),
                          down=h["down"].detach().to(torch.bfloat16).unsqueeze(0).contiguous())
        return super().preprocess_weights_impl()

    def move_weights_to_device_impl(self):
        self._dev = {k: v.to(self.device) for k, v in self._host.items()}
        self._host = {}
        return super().move_weights_to_device_impl()

    def _route(self, T: int) -> hip_ops.RouteResult:
        r = self._index_cache.get(T)
        if r is None:
            i32 = dict(dtype=torch.int32, device=self.device)
            ar = torch.arange(T, **i32)
            r = hip_ops.RouteResult(
                topk_idx=torch.zeros(T, 1, **i32),
                topk_w=torch.ones(T, 1, dtype=torch.float32, device=self.device),
                expert_counts=torch.tensor([T], **i32),
                expert_offsets=torch.tensor([0, T], **i32),
                sorted_tokens=ar, inv_perm=ar.view(T, 1).clone(),
                seg_expert=torch.tensor([0], **i32), seg_offset=torch.tensor([0], **i32),
                seg_count=torch.tensor([T], **i32), n_segments=torch.tensor([1], **i32),
                with_shared=False)
            self._index_cache[T] = r
        return r

    def forward(self, hidden_states: torch.Tensor, residual: torch.Tensor = None) -> torch.Tensor:
        shape = hidden_states.shape
        H = shape[-1]
        x = hidden_states.reshape(-1, H).to(torch.bfloat16).contiguous()
        route = self._route(x.shape[0])
        _, y = hip_ops.moe_grouped_swiglu(x, route, self._dev["gate_up"], self._dev["down"],
                                          y_dtype=_y_dtype("bf16", x.shape[0]))
        res = None if residual is None else residual.reshape(-1, H).to(torch.float32).contiguous()
        return hip_ops.moe_unpermute_combine(y, route, residual=res).view(shape)
