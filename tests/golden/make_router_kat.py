"""Writes router_kat.json: hand-derived known answers for the MoE router and permute.

Each case is small enough to solve by inspection; the expected expert order below is written
out from that reasoning (not computed by any router implementation). Expected weights are the
float64 values sigmoid(logit[e]) / sum * routed_scale of the selected experts.

  group_limit: E=64, 8 groups of 8, keep 2, top 4. Expert 0 has the largest logit (2.5) but its
    group's second score is sigmoid(-3); group 3 (logits 2.0 at e=26, 1.0 at e=24) and group 5
    (1.5 at e=41, 0.5 at e=40) have the two largest top-2 sums -> [26, 41, 24, 40].
  bias_moves_selection: same logits, bias +0.5 at e=40 and -0.5 at e=24: corrected scores
    40: 1.122, 26: 0.881, 41: 0.818, 24: 0.231 -> [40, 26, 41, 24]; weights still use the
    unbiased sigmoid.
  all_ties: every logit 0 -> every group ties -> groups 0 and 1 kept, experts 0..3 (lower index
    first), equal weights.
  single_expert: top_k = 1 -> weight = routed_scale.
Permute case: T=3, K=2, idx [[2,0],[0,1],[2,1]], E=4, sorted by (expert, token).
"""
import json
import math
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def sig(x):
    return 1.0 / (1.0 + math.exp(-x))


def weights(logits, idx, scale):
    s = [sig(logits[e]) for e in idx]
    tot = sum(s)
    return [v / tot * scale for v in s]


def main():
    E = 64
    base = [-3.0] * E
    base[0] = 2.5
    base[26], base[24] = 2.0, 1.0
    base[41], base[40] = 1.5, 0.5
    cases = []
    idx = [26, 41, 24, 40]
    cases.append(dict(name="group_limit", logits=[base], bias=[0.0] * E, n_group=8,
                      topk_group=2, top_k=4, routed_scale=2.5, expected_idx=[idx],
                      expected_w=[weights(base, idx, 2.5)]))
    bias = [0.0] * E
    bias[40], bias[24] = 0.5, -0.5
    idx = [40, 26, 41, 24]
    cases.append(dict(name="bias_moves_selection", logits=[base], bias=bias, n_group=8,
                      topk_group=2, top_k=4, routed_scale=2.5, expected_idx=[idx],
                      expected_w=[weights(base, idx, 2.5)]))
    zeros = [0.0] * E
    cases.append(dict(name="all_ties", logits=[zeros], bias=[0.0] * E, n_group=8, topk_group=2,
                      top_k=4, routed_scale=2.0, expected_idx=[[0, 1, 2, 3]],
                      expected_w=[[0.5, 0.5, 0.5, 0.5]]))
    cases.append(dict(name="single_expert", logits=[base], bias=[0.0] * E, n_group=8,
                      topk_group=2, top_k=1, routed_scale=2.5, expected_idx=[[26]],
                      expected_w=[[2.5]]))
    permute = dict(topk_idx=[[2, 0], [0, 1], [2, 1]], E=4,
                   expert_counts=[2, 2, 2, 0], expert_offsets=[0, 2, 4, 6, 6],
                   sorted_tokens=[0, 1, 1, 2, 0, 2, 0, 1, 2], inv_perm=[[4, 0], [1, 2], [5, 3]],
                   segments=[[0, 0, 2], [1, 2, 2], [2, 4, 2], [4, 6, 3]])
    with open(os.path.join(HERE, "router_kat.json"), "w") as f:
        json.dump({"cases": cases, "permute": permute}, f, indent=1)


if __name__ == "__main__":
    main()
