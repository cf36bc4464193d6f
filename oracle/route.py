"""Oracle of the MoE router and permute (test infrastructure only).

Two restatements of the same reference algorithm, Glm4MoeRouteTokenToExperts.forward
(ttnn_moe.py:413-436) with BailingMoeV2's norm_topk_prob=True (ttnn_moe.py:1532):

* :func:`route_c` / :func:`permute_c` -- the scalar C restatement (moe_route_ref.c): the
  bit-exact contract of the HIP kernel (same sigmoid, lower-index tie break).
* :func:`route_torch` -- the reference's torch formulation line by line (sigmoid, view, topk(2)
  sum, group topk, scatter mask, masked_fill 0.0, topk, gather, normalise, scale), with the
  unspecified torch.topk tie order replaced by a stable descending sort (lower index first).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

from .build import ROUTE_LIB, build

_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(ROUTE_LIB):
            build()
        lib = ctypes.CDLL(ROUTE_LIB)
        lib.oracle_sigmoid.restype = ctypes.c_float
        lib.oracle_sigmoid.argtypes = [ctypes.c_float]
        vp = ctypes.c_void_p
        ci = ctypes.c_int
        lib.oracle_route.restype = ci
        lib.oracle_route.argtypes = [vp, vp, ci, ci, ci, ci, ci, ctypes.c_float, ci, vp, vp]
        lib.oracle_permute.restype = ci
        lib.oracle_permute.argtypes = [vp, ci, ci, ci, ci, vp, vp, vp, vp, vp, vp, vp, vp]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def sigmoid_c(x: np.ndarray) -> np.ndarray:
    """Elementwise oracle sigmoid (scalar loop; small inputs)."""
    lib = _load()
    x = np.asarray(x, dtype=np.float32)
    return np.array([lib.oracle_sigmoid(float(v)) for v in x.ravel()],
                    dtype=np.float32).reshape(x.shape)


def route_c(logits: np.ndarray, bias: np.ndarray, *, n_group: int, topk_group: int, top_k: int,
            routed_scale: float, renormalize: bool = True):
    """Returns (topk_idx int32 [T,K], topk_w float32 [T,K])."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    T, E = logits.shape
    idx = np.zeros((T, top_k), dtype=np.int32)
    w = np.zeros((T, top_k), dtype=np.float32)
    rc = _load().oracle_route(_ptr(logits), _ptr(bias), T, E, n_group, topk_group, top_k,
                              float(routed_scale), 1 if renormalize else 0, _ptr(idx), _ptr(w))
    if rc != 0:
        raise ValueError("oracle_route: invalid arguments")
    return idx, w


def permute_c(topk_idx: np.ndarray, E: int, with_shared: bool = True) -> dict:
    """Stable counting sort of the assignments by (expert, token)."""
    topk_idx = np.ascontiguousarray(topk_idx, dtype=np.int32)
    T, K = topk_idx.shape
    rows = T * K + (T if with_shared else 0)
    out = dict(
        expert_counts=np.zeros(E, np.int32),
        expert_offsets=np.zeros(E + 1, np.int32),
        sorted_tokens=np.zeros(rows, np.int32),
        inv_perm=np.zeros((T, K), np.int32),
        seg_expert=np.zeros(E + 1, np.int32),
        seg_offset=np.zeros(E + 1, np.int32),
        seg_count=np.zeros(E + 1, np.int32),
        n_segments=np.zeros(1, np.int32),
    )
    rc = _load().oracle_permute(
        _ptr(topk_idx), T, K, E, 1 if with_shared else 0, _ptr(out["expert_counts"]),
        _ptr(out["expert_offsets"]), _ptr(out["sorted_tokens"]), _ptr(out["inv_perm"]),
        _ptr(out["seg_expert"]), _ptr(out["seg_offset"]), _ptr(out["seg_count"]),
        _ptr(out["n_segments"]))
    if rc != 0:
        raise ValueError("oracle_permute: invalid arguments")
    return out


def _topk_stable(x: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest entries of each row, ties to the lower index."""
    return torch.sort(x, dim=-1, descending=True, stable=True).indices[..., :k]


def route_torch(logits: torch.Tensor, bias: torch.Tensor, *, n_group: int, topk_group: int,
                top_k: int, routed_scale: float, renormalize: bool = True,
                sigmoid=torch.sigmoid):
    """Glm4MoeRouteTokenToExperts.forward (ttnn_moe.py:413-436), fp32, stable ties."""
    router_logits = sigmoid(logits.float())
    T, E = router_logits.shape
    router_logits_for_choice = router_logits + bias.float()
    group_scores = (
        router_logits_for_choice.view(-1, n_group, E // n_group).topk(2, dim=-1)[0].sum(dim=-1)
    )
    group_idx = _topk_stable(group_scores, topk_group)
    group_mask = torch.zeros_like(group_scores)
    group_mask.scatter_(1, group_idx, 1)
    score_mask = (
        group_mask.unsqueeze(-1).expand(-1, n_group, E // n_group).reshape(-1, E)
    )
    scores_for_choice = router_logits_for_choice.masked_fill(~score_mask.bool(), 0.0)
    topk_indices = _topk_stable(scores_for_choice, top_k)
    topk_weights = router_logits.gather(1, topk_indices)
    if renormalize:
        denominator = topk_weights.sum(dim=-1, keepdim=True) + 1e-20
        topk_weights = topk_weights / denominator
    topk_weights = topk_weights * routed_scale
    return topk_indices, topk_weights


def selection_margins(logits: torch.Tensor, bias: torch.Tensor, *, n_group: int,
                      topk_group: int, top_k: int) -> torch.Tensor:
    """Per token, the smaller of the two decision gaps of the router: between the
    topk_group-th and next group score, and between the top_k-th and next masked expert
    score. A routing difference between two implementations that agree to within
    floating-point rounding is only possible where this margin is tiny."""
    s = torch.sigmoid(logits.double())
    c = s + bias.double()
    T, E = c.shape
    gs = c.view(T, n_group, E // n_group).topk(2, dim=-1)[0].sum(-1)
    gsort = gs.sort(dim=-1, descending=True).values
    gmargin = (gsort[:, topk_group - 1] - gsort[:, topk_group]) if topk_group < n_group \
        else torch.full((T,), float("inf"), dtype=torch.float64)
    keep_idx = gs.topk(topk_group, dim=-1).indices
    mask = torch.zeros_like(gs).scatter_(1, keep_idx, 1).bool()
    m = c.masked_fill(~mask.unsqueeze(-1).expand(-1, -1, E // n_group).reshape(T, E), 0.0)
    msort = m.sort(dim=-1, descending=True).values
    emargin = msort[:, top_k - 1] - msort[:, top_k]
    return torch.minimum(gmargin, emargin)
