/*
 * CPU oracle (test infrastructure only) for the MoE router and permute.
 *
 * Restates, in scalar C, the routing of Glm4MoeRouteTokenToExperts.forward
 * (ttnn_moe.py:413-436) as used by TTNNBailingMoE (ttnn_moe.py:1520-1533):
 *   s = sigmoid(logits)                                  (ttnn_moe.py:414)
 *   c = s + e_score_correction_bias                      (ttnn_moe.py:415)
 *   group score = sum of the top-2 c of each group       (ttnn_moe.py:416-420)
 *   keep the topk_group best groups                      (ttnn_moe.py:421-423)
 *   experts of dropped groups score 0.0                  (ttnn_moe.py:424-429)
 *   idx = top_k experts by score; w = s[idx]             (ttnn_moe.py:430-431)
 *   w /= (sum(w) + 1e-20) when norm_topk_prob; w *= routed_scaling_factor (ttnn_moe.py:432-435)
 * and the token dispatch of TTNNExperts.forward (ttnn_moe.py:1225-1245) as a stable counting
 * sort of the (token, k) assignments by (expert, token).
 *
 * Contract choices the reference leaves open (its torch.topk tie order is unspecified):
 *   ties in group or expert selection go to the lower index; the weight sum runs over k in
 *   selection order; sigmoid is 1/(1+exp(-x)) with the exp below. The HIP kernel implements the
 *   same choices, so integer outputs and weights must agree bit for bit on identical logits.
 *
 * Build: oracle/build.py (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* sigmoid(x) = 1 / (1 + exp(-x)); exp by round(x*log2e) range reduction, two-part ln2,
 * degree-7 Taylor polynomial, exact scaling by 2^n. */
float oracle_sigmoid(float x) {
  float z = -x;
  if (z > 88.5f) return 0.0f;
  if (z < -88.5f) return 1.0f;
  float n = rintf(z * 1.44269502f);
  float r = fmaf(n, -0.693145752f, z);
  r = fmaf(n, -1.42860677e-06f, r);
  float p = fmaf(r, 1.98412698e-04f, 1.38888889e-03f);
  p = fmaf(p, r, 8.33333333e-03f);
  p = fmaf(p, r, 4.16666667e-02f);
  p = fmaf(p, r, 1.66666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  float e = ldexpf(p, (int)n);
  return 1.0f / (1.0f + e);
}

static uint32_t order_bits(float v) {
  float w = v + 0.0f;
  uint32_t u;
  memcpy(&u, &w, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* Returns 0 on success, -1 on invalid arguments. */
int oracle_route(const float* logits, const float* bias, int T, int E, int n_group,
                 int topk_group, int top_k, float routed_scale, int renorm, int32_t* topk_idx,
                 float* topk_w) {
  if (T < 0 || E <= 0 || n_group <= 0 || E % n_group || top_k <= 0 || top_k > E ||
      topk_group <= 0 || topk_group > n_group)
    return -1;
  const int gsz = E / n_group;
  if (gsz < 2) return -1;
  float* s = (float*)malloc(sizeof(float) * E);
  float* c = (float*)malloc(sizeof(float) * E);
  float* m = (float*)malloc(sizeof(float) * E);
  float* gscore = (float*)malloc(sizeof(float) * n_group);
  char* keep = (char*)malloc(n_group);
  char* taken = (char*)malloc(E);
  float* wk = (float*)malloc(sizeof(float) * top_k);
  for (int t = 0; t < T; ++t) {
    const float* row = logits + (size_t)t * E;
    for (int e = 0; e < E; ++e) {
      s[e] = oracle_sigmoid(row[e]);
      c[e] = s[e] + bias[e];
    }
    for (int g = 0; g < n_group; ++g) {
      float t1 = -INFINITY, t2 = -INFINITY;
      for (int j = 0; j < gsz; ++j) {
        const float v = c[g * gsz + j];
        if (v > t1) {
          t2 = t1;
          t1 = v;
        } else if (v > t2) {
          t2 = v;
        }
      }
      gscore[g] = t1 + t2;
    }
    for (int g = 0; g < n_group; ++g) {
      int rank = 0;
      for (int h = 0; h < n_group; ++h)
        rank += (gscore[h] > gscore[g]) || (gscore[h] == gscore[g] && h < g);
      keep[g] = rank < topk_group;
    }
    for (int e = 0; e < E; ++e) {
      m[e] = keep[e / gsz] ? c[e] : 0.0f;
      taken[e] = 0;
    }
    float denom = 0.0f;
    for (int k = 0; k < top_k; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || order_bits(m[e]) > order_bits(m[best])) best = e;
      }
      taken[best] = 1;
      topk_idx[(size_t)t * top_k + k] = best;
      wk[k] = s[best];
      denom = denom + wk[k];
    }
    if (renorm) denom = denom + 1e-20f;
    for (int k = 0; k < top_k; ++k) {
      float w = wk[k];
      if (renorm) w = w / denom;
      topk_w[(size_t)t * top_k + k] = w * routed_scale;
    }
  }
  free(s);
  free(c);
  free(m);
  free(gscore);
  free(keep);
  free(taken);
  free(wk);
  return 0;
}

/* Stable counting sort of assignments a = t*K + k by (expert, token).
 * Outputs: counts[E], offsets[E+1], sorted_tokens[T*K (+T)], inv_perm[T*K],
 * segments (expert, offset, count) for experts with rows, then the shared expert (slot E). */
int oracle_permute(const int32_t* topk_idx, int T, int K, int E, int with_shared,
                   int32_t* counts, int32_t* offsets, int32_t* sorted_tokens, int32_t* inv_perm,
                   int32_t* seg_expert, int32_t* seg_offset, int32_t* seg_count,
                   int32_t* n_segments) {
  if (T < 0 || K <= 0 || E <= 0) return -1;
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (long a = 0; a < (long)T * K; ++a) {
    const int e = topk_idx[a];
    if (e < 0 || e >= E) return -1;
    counts[e]++;
  }
  offsets[0] = 0;
  for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int32_t* fill = (int32_t*)malloc(sizeof(int32_t) * E);
  for (int e = 0; e < E; ++e) fill[e] = offsets[e];
  /* tokens ascending; within a token each expert appears at most once */
  for (int t = 0; t < T; ++t) {
    for (int k = 0; k < K; ++k) {
      const long a = (long)t * K + k;
      const int e = topk_idx[a];
      const int row = fill[e]++;
      sorted_tokens[row] = t;
      inv_perm[a] = row;
    }
  }
  free(fill);
  int ns = 0;
  for (int e = 0; e < E; ++e) {
    if (counts[e] > 0) {
      seg_expert[ns] = e;
      seg_offset[ns] = offsets[e];
      seg_count[ns] = counts[e];
      ns++;
    }
  }
  if (with_shared) {
    for (int t = 0; t < T; ++t) sorted_tokens[T * K + t] = t;
    seg_expert[ns] = E;
    seg_offset[ns] = T * K;
    seg_count[ns] = T;
    ns++;
  }
  n_segments[0] = ns;
  return 0;
}
