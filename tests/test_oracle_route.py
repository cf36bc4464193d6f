"""Pins of the router / permute oracle (CPU).

The reference holds no golden vectors for this path, so the oracle is pinned by:
  * a library implementation of the same algorithm: transformers' DeepseekV3TopkRouter
    (sigmoid + bias, top-2 group sums, group top-k, masked top-k, unbiased weights,
    normalisation, scale) on identical logits;
  * brute force on tiny shapes (enumerate every group subset);
  * hand-derived known answers (tests/golden/router_kat.json);
  * invariants (unique indices, indices inside kept groups, sum of weights = scale, ties to the
    lower index, permute bijection / counts / offsets / order).
"""
import itertools
import json
import os

import numpy as np
import pytest
import torch

from oracle import route as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _logits(T, E, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(T, E, generator=g) * scale).float()


def _bias(E, seed, std=0.05):
    g = torch.Generator().manual_seed(seed + 1000)
    return (torch.randn(E, generator=g) * std).float()


def test_sigmoid_matches_libm_within_2ulp():
    x = np.concatenate([np.linspace(-30, 30, 4001, dtype=np.float32),
                        np.array([0.0, -0.0, 1e-8, -1e-8, 88.0, -88.0, 100.0, -100.0],
                                 dtype=np.float32)])
    got = R.sigmoid_c(x).astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    # denormal-range results (x < -87) compare absolutely
    err = np.abs(got - ref)
    ok = (err <= 2 * ulp) | (err < 1e-37)
    assert ok.all(), f"max ulp error {np.max(err / ulp)} at {x[np.argmax(err / ulp)]}"


@pytest.mark.parametrize("E,n_group,topk_group,top_k", [(256, 8, 4, 8), (64, 8, 4, 4),
                                                         (128, 4, 2, 6), (512, 16, 8, 8),
                                                         (64, 1, 1, 8)])
def test_route_c_matches_torch_restatement(E, n_group, topk_group, top_k):
    logits = _logits(300, E, seed=E + top_k)
    bias = _bias(E, seed=E)
    kw = dict(n_group=n_group, topk_group=topk_group, top_k=top_k, routed_scale=2.5)
    idx_c, w_c = R.route_c(logits.numpy(), bias.numpy(), **kw)
    idx_t, w_t = R.route_torch(logits, bias, **kw)
    margins = R.selection_margins(logits, bias, n_group=n_group, topk_group=topk_group,
                                  top_k=top_k)
    clear = margins > 1e-6
    assert clear.float().mean() > 0.99
    assert np.array_equal(idx_c[clear.numpy()], idx_t.numpy()[clear.numpy()])
    np.testing.assert_allclose(w_c[clear.numpy()], w_t.numpy()[clear.numpy()], rtol=2e-6,
                               atol=1e-7)


def test_route_torch_matches_transformers_deepseek_v3_router():
    from transformers.models.deepseek_v3.configuration_deepseek_v3 import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3TopkRouter

    E, H = 256, 64
    cfg = DeepseekV3Config(hidden_size=H, n_routed_experts=E, num_experts_per_tok=8, n_group=8,
                           topk_group=4, routed_scaling_factor=2.5, norm_topk_prob=True)
    if not hasattr(cfg, "num_local_experts"):
        cfg.num_local_experts = E
    router = DeepseekV3TopkRouter(cfg)
    g = torch.Generator().manual_seed(7)
    with torch.no_grad():
        router.weight.copy_(torch.randn(E, H, generator=g) * 0.3)
        router.e_score_correction_bias.copy_(torch.randn(E, generator=g) * 0.05)
    x = torch.randn(200, H, generator=g)
    logits, w_hf, idx_hf = router(x)
    idx_t, w_t = R.route_torch(logits, router.e_score_correction_bias, n_group=8, topk_group=4,
                               top_k=8, routed_scale=2.5)
    # transformers returns the top-k unsorted: compare as sets, weights matched per expert
    o_hf = idx_hf.sort(dim=-1)
    o_t = idx_t.sort(dim=-1)
    assert torch.equal(o_hf.values, o_t.values)
    torch.testing.assert_close(w_hf.gather(1, o_hf.indices), w_t.gather(1, o_t.indices),
                               rtol=1e-6, atol=1e-7)
    # and the C oracle on the same logits
    idx_c, w_c = R.route_c(logits.detach().numpy(), router.e_score_correction_bias.numpy(),
                           n_group=8, topk_group=4, top_k=8, routed_scale=2.5)
    margins = R.selection_margins(logits.detach(), router.e_score_correction_bias, n_group=8,
                                  topk_group=4, top_k=8)
    clear = (margins > 1e-6).numpy()
    assert np.array_equal(np.sort(idx_c, 1)[clear], o_hf.values.numpy()[clear])


def _brute_force(logits_row, bias, n_group, topk_group, top_k, scale):
    s = 1.0 / (1.0 + np.exp(-logits_row.astype(np.float64)))
    c = s + bias.astype(np.float64)
    E = c.size
    gsz = E // n_group
    gscore = [sorted(c[g * gsz:(g + 1) * gsz])[-2:] for g in range(n_group)]
    gscore = [a + b for a, b in gscore]
    best = None
    for groups in itertools.combinations(range(n_group), topk_group):
        val = sum(gscore[g] for g in groups)
        if best is None or val > best[0] + 1e-15:
            best = (val, groups)
    keep = np.zeros(E, bool)
    for g in best[1]:
        keep[g * gsz:(g + 1) * gsz] = True
    m = np.where(keep, c, 0.0)
    order = sorted(range(E), key=lambda e: (-m[e], e))[:top_k]
    w = s[order] / s[order].sum() * scale
    return np.array(order), w


def test_route_c_matches_brute_force_small():
    E, n_group, topk_group, top_k = 64, 8, 3, 5
    logits = _logits(60, E, seed=3).numpy()
    bias = _bias(E, seed=3).numpy()
    idx_c, w_c = R.route_c(logits, bias, n_group=n_group, topk_group=topk_group, top_k=top_k,
                           routed_scale=1.5)
    for t in range(logits.shape[0]):
        idx_b, w_b = _brute_force(logits[t], bias, n_group, topk_group, top_k, 1.5)
        assert list(idx_c[t]) == list(idx_b)
        np.testing.assert_allclose(w_c[t], w_b, rtol=1e-5)


def test_route_invariants_and_ties():
    E, n_group, topk_group, top_k = 256, 8, 4, 8
    # quantised logits -> many exact ties
    logits = (torch.randint(-4, 5, (500, E), generator=torch.Generator().manual_seed(5))
              .float() * 0.5)
    bias = torch.zeros(E)
    idx, w = R.route_c(logits.numpy(), bias.numpy(), n_group=n_group, topk_group=topk_group,
                       top_k=top_k, routed_scale=2.5)
    idx_t, w_t = R.route_torch(logits, bias, n_group=n_group, topk_group=topk_group,
                               top_k=top_k, routed_scale=2.5)
    assert np.array_equal(idx, idx_t.numpy())          # same tie rule: lower index first
    np.testing.assert_allclose(w.sum(1), 2.5, rtol=1e-6)
    assert (w >= 0).all()
    for t in range(idx.shape[0]):
        assert len(set(idx[t])) == top_k
        s = 1 / (1 + np.exp(-logits[t].numpy()))
        vals = s[idx[t]]
        assert np.all(np.diff(vals) <= 1e-7), "selection must be in descending score order"
        # ties resolved to the lower index
        for a, b in zip(idx[t][:-1], idx[t][1:]):
            if abs(s[a] - s[b]) == 0:
                assert a < b
        groups = set(int(e) // (E // n_group) for e in idx[t])
        assert len(groups) <= topk_group


def test_masked_zero_fill_semantics():
    """Dropped groups score 0.0 (torch form, ttnn_moe.py:429): once the kept groups run out of
    positive corrected scores, experts of dropped groups (score 0.0, lowest index first)
    outrank the kept groups' negative scores."""
    E, n_group, topk_group, top_k = 64, 8, 2, 12
    logits = np.full((1, E), -20.0, np.float32)   # sigmoid ~ 2e-9
    bias = np.full(E, -0.5, np.float32)
    bias[0:8] = 0.3                                 # group 0: score 0.6
    bias[8] = 0.2                                   # group 1: 0.2 + (-0.8) = -0.6
    bias[9:16] = -0.8                               # other groups: -1.0
    idx, _ = R.route_c(logits, bias, n_group=n_group, topk_group=topk_group, top_k=top_k,
                       routed_scale=1.0)
    idx_t, _ = R.route_torch(torch.from_numpy(logits), torch.from_numpy(bias),
                             n_group=n_group, topk_group=topk_group, top_k=top_k,
                             routed_scale=1.0)
    expected = list(range(8)) + [8, 16, 17, 18]
    assert list(idx[0]) == expected
    assert list(idx_t[0].numpy()) == expected


def test_router_known_answers():
    with open(os.path.join(GOLDEN, "router_kat.json")) as f:
        cases = json.load(f)["cases"]
    assert cases
    for case in cases:
        logits = np.array(case["logits"], np.float32)
        bias = np.array(case["bias"], np.float32)
        idx, w = R.route_c(logits, bias, n_group=case["n_group"], topk_group=case["topk_group"],
                           top_k=case["top_k"], routed_scale=case["routed_scale"])
        assert idx.tolist() == case["expected_idx"], case["name"]
        np.testing.assert_allclose(w, np.array(case["expected_w"]), rtol=1e-6, atol=1e-7,
                                   err_msg=case["name"])


@pytest.mark.parametrize("with_shared", [True, False])
def test_permute_invariants(with_shared):
    E, K = 64, 6
    logits = _logits(150, E, seed=11)
    idx, _ = R.route_c(logits.numpy(), np.zeros(E, np.float32), n_group=8, topk_group=4,
                       top_k=K, routed_scale=1.0)
    p = R.permute_c(idx, E, with_shared=with_shared)
    T = idx.shape[0]
    counts = np.bincount(idx.ravel(), minlength=E)
    assert np.array_equal(p["expert_counts"], counts)
    assert np.array_equal(p["expert_offsets"], np.concatenate([[0], np.cumsum(counts)]))
    inv = p["inv_perm"].ravel()
    assert sorted(inv.tolist()) == list(range(T * K))            # bijection
    st = p["sorted_tokens"]
    tok_of_assign = np.repeat(np.arange(T), K)
    assert np.array_equal(st[inv], tok_of_assign)                  # unpermute o permute = id
    # rows sorted by (expert, token)
    expert_of_row = np.empty(T * K, np.int64)
    expert_of_row[inv] = idx.ravel()
    key = expert_of_row * T + st[:T * K]
    assert np.all(np.diff(key) > 0)
    ns = int(p["n_segments"][0])
    active = np.nonzero(counts)[0]
    assert ns == len(active) + (1 if with_shared else 0)
    assert np.array_equal(p["seg_expert"][:len(active)], active)
    assert np.array_equal(p["seg_count"][:len(active)], counts[active])
    assert np.array_equal(p["seg_offset"][:len(active)], p["expert_offsets"][active])
    if with_shared:
        assert (p["seg_expert"][ns - 1], p["seg_offset"][ns - 1], p["seg_count"][ns - 1]) == \
            (E, T * K, T)
        assert np.array_equal(st[T * K:], np.arange(T))


def test_permute_known_answer():
    with open(os.path.join(GOLDEN, "router_kat.json")) as f:
        kat = json.load(f)["permute"]
    p = R.permute_c(np.array(kat["topk_idx"], np.int32), kat["E"], with_shared=True)
    assert p["expert_counts"].tolist() == kat["expert_counts"]
    assert p["expert_offsets"].tolist() == kat["expert_offsets"]
    assert p["sorted_tokens"].tolist() == kat["sorted_tokens"]
    assert p["inv_perm"].tolist() == kat["inv_perm"]
    ns = int(p["n_segments"][0])
    segs = [[int(p["seg_expert"][i]), int(p["seg_offset"][i]), int(p["seg_count"][i])]
            for i in range(ns)]
    assert segs == kat["segments"]
