// Fused MoE router: sigmoid + expert bias + group-limited top-k + weight normalisation, then a
// deterministic counting-sort permute of the (token, k) assignments by expert.
//
// Reference semantics: Glm4MoeRouteTokenToExperts.forward (ttnn_moe.py:413-436) as used for
// BailingMoeV2 by TTNNBailingMoE (ttnn_moe.py:1520-1533, norm_topk_prob forced True), and the
// token dispatch of TTNNExperts.forward (ttnn_moe.py:1225-1245).
//
// Design (gfx950, wave64):
//   router logits: fp32 MFMA (16x16x4) GEMM writing four partial sums over quarters of H.
//   route kernel (one wave per token, four tokens per workgroup): each lane owns E/64
//     consecutive experts, so a group of E/n_group experts spans a power-of-two run of lanes.
//     Group top-2 merges partners through DPP row operations; group ranking reads the n_group
//     scores with readlane; the final top-k is k rounds of a wave-wide max of order-preserving
//     value bits (DPP inside each 16-lane row, readlane across rows) followed by a ballot for
//     the lowest lane holding it, so ties pick the lower expert index.
//   permute kernel (one workgroup): per-expert counts and offsets, then each chunk of 64
//     tokens folded into one 64-bit token mask per expert (LDS atomic OR, order independent);
//     every assignment's row = expert offset + earlier chunks + popcount of earlier tokens in
//     its own chunk mask. The result does not depend on scheduling order: bit-exact across runs.
//
// Floating point: contraction is disabled in this file so the sigmoid below (own Cody-Waite exp,
// explicit fma) and every add/divide are the IEEE operations the CPU oracle performs.
#pragma clang fp contract(off)

#include "common.h"

namespace sym {

// sigmoid(x) = 1 / (1 + exp(-x)); exp by round(x*log2e) range reduction with a two-part ln2 and a
// degree-7 Taylor polynomial on |r| <= ln2/2 (relative error < 6e-8), scaled by ldexp.
// Branch-free: the argument is clamped to [-88.5, 88.5] and the saturated results are selected
// afterwards (0 for -x > 88.5, 1 for -x < -88.5), the same values as a branchy evaluation.
__device__ __forceinline__ float route_sigmoid(float x) {
  const float z = -x;
  const float zc = fminf(fmaxf(z, -88.5f), 88.5f);
  const float n = rintf(zc * 1.44269502f);
  float r = fmaf(n, -0.693145752f, zc);
  r = fmaf(n, -1.42860677e-06f, r);
  float p = fmaf(r, 1.98412698e-04f, 1.38888889e-03f);
  p = fmaf(p, r, 8.33333333e-03f);
  p = fmaf(p, r, 4.16666667e-02f);
  p = fmaf(p, r, 1.66666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const float e = ldexpf(p, (int)n);
  const float sg = 1.0f / (1.0f + e);
  return z > 88.5f ? 0.0f : (z < -88.5f ? 1.0f : sg);
}

// Order-preserving map float -> uint32 (larger float -> larger uint); -0.0 is folded onto +0.0.
__device__ __forceinline__ uint32_t order_bits(float v) {
  uint32_t u = __float_as_uint(v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int kMaxTopK = 32;
constexpr int kLogitParts = 4;  // partial sums written by the router-logits kernel

// ---- wave64 cross-lane helpers built on DPP row operations (VALU latency) and readlane ----
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within each 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within each 16

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __uint_as_float(dpp32<CTRL>(__float_as_uint(v)));
}
// (t1, t2) <- the two largest of the union of this lane's pair and the partner's pair.
__device__ __forceinline__ void top2_merge(float& t1, float& t2, float o1, float o2) {
  const float n1 = fmaxf(t1, o1);
  const float n2 = fmaxf(fminf(t1, o1), fmaxf(t2, o2));
  t1 = n1;
  t2 = n2;
}

// Route one token with the calling wave (all 64 lanes). Lane l owns experts l*EPL .. l*EPL+EPL-1.
// The partner patterns used for the group top-2 (xor 1, xor 2, half mirror, mirror, then xor 16
// and xor 32) always pair disjoint lane sets, so no expert is counted twice.
// Logits of token t for this lane's experts: all partial sums loaded unconditionally (one
// batch of EPL * kLogitParts loads, parts past n_parts repeat the last one and are not added),
// then added left to right. (A load under q < n_parts would be waited for at the end of its
// branch: one round trip per part.)
template <int EPL>
__device__ __forceinline__ void load_token_logits(const float* __restrict__ logits, int n_parts,
                                                  size_t part_stride, int t, int E, int lane,
                                                  float (&parts)[kLogitParts][EPL]) {
#pragma unroll
  for (int q = 0; q < kLogitParts; ++q)
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      parts[q][j] = logits[(size_t)min(q, n_parts - 1) * part_stride + (size_t)t * E + lane * EPL + j];
}

template <int EPL>
__device__ __forceinline__ void route_token(const float (&parts)[kLogitParts][EPL], int n_parts,
                                            const float* bv, int E, int n_group, int topk_group,
                                            int top_k, float routed_scale, int renorm, int lane,
                                            int& my_idx, float& my_w) {
  const int gsz = E / n_group;
  const int lpg = gsz / EPL;
  const int my_group = lane / lpg;
  float s[EPL], c[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    float x = parts[0][j];
#pragma unroll
    for (int q = 1; q < kLogitParts; ++q) {
      if (q < n_parts) x = x + parts[q][j];
    }
    s[j] = route_sigmoid(x);
    c[j] = s[j] + bv[j];
  }
  // largest and second largest c of this lane (branch-free; same values as a running update)
  float t1 = -INFINITY, t2 = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const float v = c[j];
    t2 = fmaxf(t2, fminf(t1, v));
    t1 = fmaxf(t1, v);
  }
  if (lpg >= 2) top2_merge(t1, t2, dppf<kDppXor1>(t1), dppf<kDppXor1>(t2));
  if (lpg >= 4) top2_merge(t1, t2, dppf<kDppXor2>(t1), dppf<kDppXor2>(t2));
  if (lpg >= 8) top2_merge(t1, t2, dppf<kDppHalfMirror>(t1), dppf<kDppHalfMirror>(t2));
  if (lpg >= 16) top2_merge(t1, t2, dppf<kDppMirror>(t1), dppf<kDppMirror>(t2));
  if (lpg >= 32) top2_merge(t1, t2, __shfl_xor(t1, 16), __shfl_xor(t2, 16));
  if (lpg >= 64) top2_merge(t1, t2, __shfl_xor(t1, 32), __shfl_xor(t2, 32));
  const float gscore = t1 + t2;

  int rank = 0;
  for (int g = 0; g < n_group; ++g) {
    const float o = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gscore), g * lpg));
    rank += (o > gscore) || (o == gscore && g < my_group);
  }
  const bool keep = rank < topk_group;

  // top-k over the kept experts: k rounds of (largest value, lowest expert index on ties).
  // Round: wave max of the order-preserving value bits (DPP in rows, readlane across rows),
  // then the lowest lane holding that value (ballot + find-first-one) and the lowest of its
  // experts with it; that expert's value is cleared to 0 (below every real value's bits).
  uint32_t kv[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) kv[j] = order_bits(keep ? c[j] : 0.0f);
  float denom = 0.0f;
  my_idx = 0;
  my_w = 0.0f;
  for (int k = 0; k < top_k; ++k) {
    uint32_t lb = kv[0];
#pragma unroll
    for (int j = 1; j < EPL; ++j) lb = max(lb, kv[j]);
    uint32_t m = max(lb, dpp32<kDppXor1>(lb));
    m = max(m, dpp32<kDppXor2>(m));
    m = max(m, dpp32<kDppHalfMirror>(m));
    m = max(m, dpp32<kDppMirror>(m));
    const uint32_t best =
        max(max((uint32_t)__builtin_amdgcn_readlane((int)m, 0),
                (uint32_t)__builtin_amdgcn_readlane((int)m, 16)),
            max((uint32_t)__builtin_amdgcn_readlane((int)m, 32),
                (uint32_t)__builtin_amdgcn_readlane((int)m, 48)));
    const unsigned long long holders = __ballot(lb == best);
    const int owner = __ffsll((long long)holders) - 1;
    int jl = EPL - 1;
#pragma unroll
    for (int j = EPL - 2; j >= 0; --j) jl = kv[j] == best ? j : jl;
    float sl = s[0];
#pragma unroll
    for (int j = 1; j < EPL; ++j) sl = jl == j ? s[j] : sl;
    const int jj = __builtin_amdgcn_readlane(jl, owner);
    const float sv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sl), owner));
    if (lane == owner) {
#pragma unroll
      for (int j = 0; j < EPL; ++j) kv[j] = j == jj ? 0u : kv[j];
    }
    denom = denom + sv;
    if (lane == k) {
      my_idx = owner * EPL + jj;
      my_w = sv;
    }
  }
  if (renorm) {
    denom = denom + 1e-20f;
    my_w = my_w / denom;
  }
  my_w = my_w * routed_scale;
}

// Routes one token per wave (four per workgroup): writes the token's top-k experts (in
// selection order) and their weights.
template <int EPL>
__global__ __launch_bounds__(256) void moe_route_kernel(
    const float* __restrict__ logits, int n_parts, const float* __restrict__ bias, int T, int E,
    int n_group, int topk_group, int top_k, float routed_scale, int renorm,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float parts[kLogitParts][EPL];
  load_token_logits<EPL>(logits, n_parts, (size_t)T * E, t, E, lane, parts);
  float bv[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) bv[j] = bias[lane * EPL + j];
  int my_idx;
  float my_w;
  route_token<EPL>(parts, n_parts, bv, E, n_group, topk_group, top_k, routed_scale, renorm, lane,
                   my_idx, my_w);
  if (lane < top_k) {
    topk_idx[(size_t)t * top_k + lane] = my_idx;
    topk_w[(size_t)t * top_k + lane] = my_w;
  }
}

// Exclusive scan of one int per thread over the workgroup (up to 1024 threads).
__device__ int block_exclusive_scan(int v, int* s_wave, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int n = __shfl_up(x, off);
    if (lane >= off) x += n;
  }
  if (lane == 63) s_wave[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < nwaves ? s_wave[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int n = __shfl_up(w, off);
      if (lane >= off) w += n;
    }
    if (lane < nwaves) s_wave[lane] = w;
  }
  __syncthreads();
  const int before = wave > 0 ? s_wave[wave - 1] : 0;
  *total = s_wave[nwaves - 1];
  __syncthreads();
  return before + x - v;
}

// Counting-sort permute of all (token, k) assignments by expert, in one workgroup of 1024
// threads (thread e owns expert e for the per-expert steps):
//   1. per-expert counts (LDS atomics), exclusive scan -> expert offsets; a second scan over
//      "expert has tokens" gives the compacted segment list (routed experts ascending, then the
//      shared-expert segment over rows T*K .. T*K+T-1 in token order);
//   2. tokens in passes of kMaskWords / E chunks of 64: each chunk's routing folded into one
//      64-bit token mask per expert (atomic OR, order independent); an assignment's row is its
//      expert's offset + the expert's tokens in earlier chunks + popcount of the lower tokens of
//      its own chunk mask, i.e. rows of an expert follow token order.
// No step depends on scheduling order, so the result is bit-exact across runs.
constexpr int kMaskWords = 4096;  // LDS mask words per pass
constexpr int kPermuteThreads = 1024;

__global__ __launch_bounds__(kPermuteThreads) void moe_permute_kernel(
    const int32_t* __restrict__ topk_idx, int T, int K, int E, int with_shared,
    int32_t* __restrict__ expert_counts, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ sorted_tokens, int32_t* __restrict__ inv_perm,
    int32_t* __restrict__ seg_expert, int32_t* __restrict__ seg_offset,
    int32_t* __restrict__ seg_count, int32_t* __restrict__ n_segments) {
  __shared__ unsigned long long s_mask[kMaskWords];
  __shared__ int s_pre[kMaskWords];
  __shared__ int s_base[kPermuteThreads];  // per expert: count, then next free row
  __shared__ int s_wave[16];
  const int tid = threadIdx.x;
  const int e = tid;
  const int TK = T * K;

  if (e < E) s_base[e] = 0;
  __syncthreads();
  for (int a = tid; a < TK; a += kPermuteThreads) atomicAdd(&s_base[topk_idx[a]], 1);
  __syncthreads();
  const int cnt = e < E ? s_base[e] : 0;
  int total = 0;
  const int off = block_exclusive_scan(cnt, s_wave, &total);
  int n_routed = 0;
  const int flag = (e < E && cnt > 0) ? 1 : 0;
  const int slot = block_exclusive_scan(flag, s_wave, &n_routed);
  if (e < E) {
    s_base[e] = off;
    expert_counts[e] = cnt;
    expert_offsets[e] = off;
    if (flag) {
      seg_expert[slot] = e;
      seg_offset[slot] = off;
      seg_count[slot] = cnt;
    }
  }
  if (tid == 0) {
    expert_offsets[E] = total;
    if (with_shared) {
      seg_expert[n_routed] = E;
      seg_offset[n_routed] = TK;
      seg_count[n_routed] = T;
    }
    n_segments[0] = n_routed + (with_shared ? 1 : 0);
  }
  if (with_shared)
    for (int t = tid; t < T; t += kPermuteThreads) sorted_tokens[TK + t] = t;

  const int cpp = kMaskWords / E;  // chunks per pass
  for (int t0 = 0; t0 < T; t0 += cpp * 64) {
    const int nt = min(T - t0, cpp * 64);
    const int nch = (nt + 63) >> 6;
    for (int i = tid; i < nch * E; i += kPermuteThreads) s_mask[i] = 0ull;
    __syncthreads();
    const int a0 = t0 * K, a1 = (t0 + nt) * K;
    for (int a = a0 + tid; a < a1; a += kPermuteThreads) {
      const int tl = a / K - t0;
      atomicOr(&s_mask[(tl >> 6) * E + topk_idx[a]], 1ull << (tl & 63));
    }
    __syncthreads();
    if (e < E) {
      int run = s_base[e];
      for (int c = 0; c < nch; ++c) {
        s_pre[c * E + e] = run;
        run += __popcll(s_mask[c * E + e]);
      }
      s_base[e] = run;
    }
    __syncthreads();
    for (int a = a0 + tid; a < a1; a += kPermuteThreads) {
      const int t = a / K;
      const int tl = t - t0;
      const int ex = topk_idx[a];
      const int bit = tl & 63;
      const unsigned long long m = s_mask[(tl >> 6) * E + ex];
      const unsigned long long lower = bit ? (m & ((1ull << bit) - 1ull)) : 0ull;
      const int row = s_pre[(tl >> 6) * E + ex] + __popcll(lower);
      sorted_tokens[row] = t;
      inv_perm[a] = row;
    }
    __syncthreads();
  }
}

// Permute of many tokens across the GPU (the same outputs as moe_permute_kernel, bit for bit),
// in three launches over chunks of kChunkTokens tokens:
//   1. moe_permute_count_kernel: per (chunk, expert) assignment counts (LDS atomics);
//   2. moe_permute_scan_kernel (one workgroup, thread e owns expert e): each expert's exclusive
//      prefix over the chunks (in place), its total count, the expert offsets and the segment
//      list exactly as moe_permute_kernel builds them;
//   3. moe_permute_scatter_kernel: per chunk, one 64-bit token mask per (64 tokens, expert)
//      (atomic OR, order independent); an assignment's row is its expert's offset + the expert's
//      tokens in earlier chunks + those in earlier words of this chunk + popcount of the lower
//      tokens of its own word, i.e. rows of an expert follow token order.
constexpr int kChunkTokens = 256;
constexpr int kChunkWords = kChunkTokens / 64;
constexpr int kPermuteSingleMaxTokens = 2048;  // above this the three-launch permute runs

__global__ __launch_bounds__(256) void moe_permute_count_kernel(
    const int32_t* __restrict__ topk_idx, int T, int K, int E, int32_t* __restrict__ chunk_cnt) {
  __shared__ int s_cnt[512];
  const int c = blockIdx.x, tid = threadIdx.x;
  for (int e = tid; e < E; e += 256) s_cnt[e] = 0;
  __syncthreads();
  const int a0 = c * kChunkTokens * K, a1 = min(T, (c + 1) * kChunkTokens) * K;
  for (int a = a0 + tid; a < a1; a += 256) atomicAdd(&s_cnt[topk_idx[a]], 1);
  __syncthreads();
  for (int e = tid; e < E; e += 256) chunk_cnt[(size_t)c * E + e] = s_cnt[e];
}

__global__ __launch_bounds__(kPermuteThreads) void moe_permute_scan_kernel(
    int T, int K, int E, int with_shared, int n_chunks, int32_t* __restrict__ chunk_cnt,
    int32_t* __restrict__ expert_counts, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ sorted_tokens, int32_t* __restrict__ seg_expert,
    int32_t* __restrict__ seg_offset, int32_t* __restrict__ seg_count,
    int32_t* __restrict__ n_segments) {
  __shared__ int s_wave[16];
  const int tid = threadIdx.x;
  const int e = tid;
  const int TK = T * K;
  int cnt = 0;
  if (e < E)
    for (int c0 = 0; c0 < n_chunks; c0 += 8) {
      // the loads of 8 chunks are issued before any store (the stores could alias them)
      int v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[i] = c0 + i < n_chunks ? chunk_cnt[(size_t)(c0 + i) * E + e] : 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (c0 + i < n_chunks) chunk_cnt[(size_t)(c0 + i) * E + e] = cnt;
        cnt += v[i];
      }
    }
  int total = 0;
  const int off = block_exclusive_scan(cnt, s_wave, &total);
  int n_routed = 0;
  const int flag = (e < E && cnt > 0) ? 1 : 0;
  const int slot = block_exclusive_scan(flag, s_wave, &n_routed);
  if (e < E) {
    expert_counts[e] = cnt;
    expert_offsets[e] = off;
    if (flag) {
      seg_expert[slot] = e;
      seg_offset[slot] = off;
      seg_count[slot] = cnt;
    }
  }
  if (tid == 0) {
    expert_offsets[E] = total;
    if (with_shared) {
      seg_expert[n_routed] = E;
      seg_offset[n_routed] = TK;
      seg_count[n_routed] = T;
    }
    n_segments[0] = n_routed + (with_shared ? 1 : 0);
  }
  if (with_shared)
    for (int t = tid; t < T; t += kPermuteThreads) sorted_tokens[TK + t] = t;
}

__global__ __launch_bounds__(256) void moe_permute_scatter_kernel(
    const int32_t* __restrict__ topk_idx, int T, int K, int E,
    const int32_t* __restrict__ chunk_cnt, const int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ sorted_tokens, int32_t* __restrict__ inv_perm) {
  __shared__ unsigned long long s_mask[kChunkWords * 512];
  __shared__ int s_base[512];
  const int c = blockIdx.x, tid = threadIdx.x;
  const int t0 = c * kChunkTokens;
  for (int i = tid; i < kChunkWords * E; i += 256) s_mask[i] = 0ull;
  for (int e = tid; e < E; e += 256)
    s_base[e] = expert_offsets[e] + chunk_cnt[(size_t)c * E + e];
  __syncthreads();
  const int a0 = t0 * K, a1 = min(T, t0 + kChunkTokens) * K;
  for (int a = a0 + tid; a < a1; a += 256) {
    const int tl = a / K - t0;
    atomicOr(&s_mask[(tl >> 6) * E + topk_idx[a]], 1ull << (tl & 63));
  }
  __syncthreads();
  for (int a = a0 + tid; a < a1; a += 256) {
    const int t = a / K;
    const int tl = t - t0;
    const int ex = topk_idx[a];
    const int w = tl >> 6, bit = tl & 63;
    int row = s_base[ex];
    for (int ww = 0; ww < w; ++ww) row += __popcll(s_mask[ww * E + ex]);
    const unsigned long long m = s_mask[w * E + ex];
    row += __popcll(bit ? (m & ((1ull << bit) - 1ull)) : 0ull);
    sorted_tokens[row] = t;
    inv_perm[a] = row;
  }
}

// Router logits in fp32 with v_mfma_f32_16x16x4_f32: parts[q][t][e] = sum over the q-th
// quarter of H of x[t][k] * w[e][k]. One workgroup of 8 waves per (16 experts, quarter of H);
// each wave owns H/32 consecutive k of the quarter and issues its weight loads (16 bytes per lane
// per 16-wide k chunk: 4 consecutive k of weight row l%16) four chunks at a time ahead of the
// activation loads; the 8 partial accumulators reduce through LDS. The 4 MFMAs of a 16-wide
// k chunk use one element each of the lane's 4 consecutive k, so A and B agree on the k order.
// NORM: the activations are the fp32 residual stream h [T, H] and the kernel applies the
// RMSNorm in front: r[t] = rsqrt(sum(ss_parts[:, t]) / H + eps) from the per-16-column sums of
// squares written by the producer of h, and the operand is bf16(h * r * gamma) (the rounding of
// a separate RMSNorm pass), upcast. The workgroups of the first expert tile also store that
// normalised row (bf16) for the expert GEMMs.
constexpr int kLogitWaves = 8;
constexpr int kLogitRows = 32;  // token rows per pass at most (two 16-row tiles)

// NT 16-row tiles per workgroup (grid z = passes of 16 * NT rows): a decode batch of up to 32
// tokens takes one tile per workgroup, so its 256 experts x 4 quarters of H spread over 128
// workgroups instead of 64.
template <bool NORM, int NT>
__global__ __launch_bounds__(kLogitWaves * 64) void moe_router_logits_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ hres,
    const float* __restrict__ ss_parts, int n_ss, const uint16_t* __restrict__ gamma, float eps,
    const float* __restrict__ w, int T, int H, int E, float* __restrict__ parts,
    uint16_t* __restrict__ xn_out) {
  __shared__ float s_red[kLogitWaves][NT][4][64];
  __shared__ float s_r[kLogitRows];
  const int ntile = blockIdx.x;
  const int q = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int quarter = H >> 2;
  const int sub = quarter / kLogitWaves;              // a multiple of 16 (H % 512 == 0)
  const int k_beg = q * quarter + wave * sub + kq * 4;
  const int nk = sub >> 4;                            // 16-wide k chunks of this wave
  const float* wr = w + (size_t)(ntile * 16 + r16) * H + k_beg;
  // one pass of kLogitRows tokens per workgroup (grid z), so long prompts spread over many
  // workgroups
  {
    const int mb = blockIdx.z * 16 * NT;
    float rm[2] = {1.f, 1.f};
    // rows past T repeat the last row; their results are dropped
    const int m0 = min(mb + r16, T - 1), m1 = min(mb + 16 + r16, T - 1);
    floatx4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    // NORM: the first 128 partial sums of squares of the pass's rows (16 threads per row, each
    // every 16th), issued before the weight and activation loads: loads complete in order, so
    // the rows' r is then reduced while those are still arriving
    const int ss_row = min(mb + (threadIdx.x >> 4), T - 1);
    const int ss_c = threadIdx.x & 15;
    float ss0[8];
    if constexpr (NORM) {
#pragma unroll
      for (int j = 0; j < 8; ++j) ss0[j] = ss_parts[(size_t)min(ss_c + 16 * j, n_ss - 1) * T + ss_row];
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int kc = 0; kc < nk; kc += 4) {
      // a group of up to 4 chunks: weights, activations (and gamma) issued first; chunks past
      // the range repeat the last chunk's loads and contribute zero (no branch, which would let
      // the compiler sink their loads behind the first MFMAs)
      float4 b[4];
      float4 hv[NT][4];
      uint2 xv[NT][4], gv[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        b[c] = *reinterpret_cast<const float4*>(wr + 16 * min(kc + c, nk - 1));
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const size_t off = (size_t)(t ? m1 : m0) * H + k_beg + 16 * min(kc + c, nk - 1);
          if constexpr (NORM) hv[t][c] = *reinterpret_cast<const float4*>(hres + off);
          else xv[t][c] = *reinterpret_cast<const uint2*>(x + off);
        }
      if constexpr (NORM) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          gv[c] = *reinterpret_cast<const uint2*>(gamma + k_beg + 16 * min(kc + c, nk - 1));
        if (kc == 0) {
          // r of the pass's rows: 16 threads per row, each summing every 16th partial sum
          const int row = ss_row;
          const int c = ss_c;
          float t = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) t += c + 16 * j < n_ss ? ss0[j] : 0.f;
          for (int i0 = c + 128; i0 < n_ss; i0 += 128) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const int i = i0 + 16 * j;
              v[j] = ss_parts[(size_t)min(i, n_ss - 1) * T + row];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 8; ++j) t += i0 + 16 * j < n_ss ? v[j] : 0.f;
          }
          t += __shfl_xor(t, 1);
          t += __shfl_xor(t, 2);
          t += __shfl_xor(t, 4);
          t += __shfl_xor(t, 8);
          if (c == 0) s_r[threadIdx.x >> 4] = rsqrtf(t / (float)H + eps);
          __syncthreads();
          rm[0] = s_r[r16];
          rm[1] = s_r[(NT - 1) * 16 + r16];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      float a[NT][4][4];
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if constexpr (NORM) {
            const float r = rm[t];
            a[t][c][0] = bf16_to_f32(f32_to_bf16(hv[t][c].x * r * bf16_lo(gv[c].x)));
            a[t][c][1] = bf16_to_f32(f32_to_bf16(hv[t][c].y * r * bf16_hi(gv[c].x)));
            a[t][c][2] = bf16_to_f32(f32_to_bf16(hv[t][c].z * r * bf16_lo(gv[c].y)));
            a[t][c][3] = bf16_to_f32(f32_to_bf16(hv[t][c].w * r * bf16_hi(gv[c].y)));
          } else {
            a[t][c][0] = bf16_lo(xv[t][c].x);
            a[t][c][1] = bf16_hi(xv[t][c].x);
            a[t][c][2] = bf16_lo(xv[t][c].y);
            a[t][c][3] = bf16_hi(xv[t][c].y);
          }
        }
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float z = kc + c < nk ? 1.f : 0.f;
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][c][0] * z, b[c].x, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][c][1] * z, b[c].y, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][c][2] * z, b[c].z, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][c][3] * z, b[c].w, acc[t], 0, 0, 0);
        }
      if constexpr (NORM) {
        if (xn_out && ntile == 0) {
          // the normalised rows, for the expert GEMMs
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              if (kc + c < nk && mb + t * 16 + r16 < T) {
                const int k = k_beg + 16 * (kc + c);
                uint2 o;
                o.x = pack_bf16x2(a[t][c][0], a[t][c][1]);
                o.y = pack_bf16x2(a[t][c][2], a[t][c][3]);
                *reinterpret_cast<uint2*>(xn_out + (size_t)(t ? m1 : m0) * H + k) = o;
              }
            }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_red[wave][t][i][lane] = acc[t][i];
    __syncthreads();
    if (threadIdx.x < 256 * NT) {
      // tile t = tid / 256, element i of lane l's fragment
      const int t = threadIdx.x >> 8;
      const int l = threadIdx.x & 63;
      const int i = (threadIdx.x >> 6) & 3;
      const int row = mb + t * 16 + 4 * (l >> 4) + i;
      float v = 0.f;
#pragma unroll
      for (int wv = 0; wv < kLogitWaves; ++wv) v += s_red[wv][t][i][l];
      if (row < T) parts[((size_t)q * T + row) * E + ntile * 16 + (l & 15)] = v;
    }
  }
}

}  // namespace sym

using namespace sym;

extern "C" size_t sym_moe_route_workspace_bytes(int T, int E) {
  // up to kPermuteSingleMaxTokens tokens the permute keeps its state in LDS; above, the
  // per-(chunk, expert) prefix counts of the three-launch permute
  if (T <= kPermuteSingleMaxTokens || E <= 0) return 0;
  return (size_t)((T + kChunkTokens - 1) / kChunkTokens) * E * sizeof(int32_t);
}

static int check_router_logits(const char* what, int T, int H, int E) {
  SYM_REQUIRE(T >= 0, SYM_ERR_INVALID, "%s: T=%d < 0", what, T);
  SYM_REQUIRE(H > 0 && H % 512 == 0, SYM_ERR_UNSUPPORTED,
              "%s: H=%d must be a positive multiple of 512", what, H);
  SYM_REQUIRE(E > 0 && E % 16 == 0 && E / 16 <= 65535, SYM_ERR_UNSUPPORTED,
              "%s: E=%d must be a positive multiple of 16", what, E);
  return SYM_OK;
}

extern "C" int sym_moe_router_logits(const void* x, const float* w, int T, int H, int E,
                                     float* parts, void* stream) {
  int rc = check_router_logits("moe_router_logits", T, H, E);
  if (rc || T == 0) return rc;
  SYM_REQUIRE(x && w && parts, SYM_ERR_INVALID, "moe_router_logits: null pointer argument");
  (void)hipGetLastError();
  SYM_REQUIRE((T + kLogitRows - 1) / kLogitRows <= 65535, SYM_ERR_UNSUPPORTED,
              "moe_router_logits: T=%d too large", T);
  if (T <= 32)
    hipLaunchKernelGGL((moe_router_logits_kernel<false, 1>),
                       dim3(E / 16, kLogitParts, (T + 15) / 16), dim3(kLogitWaves * 64), 0,
                       (hipStream_t)stream, (const uint16_t*)x, (const float*)nullptr,
                       (const float*)nullptr, 0, (const uint16_t*)nullptr, 0.f, w, T, H, E,
                       parts, (uint16_t*)nullptr);
  else
    hipLaunchKernelGGL((moe_router_logits_kernel<false, 2>),
                       dim3(E / 16, kLogitParts, (T + kLogitRows - 1) / kLogitRows),
                       dim3(kLogitWaves * 64), 0, (hipStream_t)stream, (const uint16_t*)x,
                       (const float*)nullptr, (const float*)nullptr, 0,
                       (const uint16_t*)nullptr, 0.f, w, T, H, E, parts, (uint16_t*)nullptr);
  return sym_host::check_launch("moe_router_logits_kernel");
}

extern "C" int sym_moe_router_logits_norm(const float* h, const float* ss_parts, int n_ss,
                                          const void* gamma, float eps, const float* w, int T,
                                          int H, int E, float* parts, void* xn_out,
                                          void* stream) {
  int rc = check_router_logits("moe_router_logits_norm", T, H, E);
  if (rc || T == 0) return rc;
  SYM_REQUIRE(h && ss_parts && gamma && w && parts, SYM_ERR_INVALID,
              "moe_router_logits_norm: null pointer argument");
  SYM_REQUIRE(n_ss >= 1, SYM_ERR_INVALID, "moe_router_logits_norm: n_ss=%d", n_ss);
  (void)hipGetLastError();
  SYM_REQUIRE((T + kLogitRows - 1) / kLogitRows <= 65535, SYM_ERR_UNSUPPORTED,
              "moe_router_logits_norm: T=%d too large", T);
  if (T <= 32)
    hipLaunchKernelGGL((moe_router_logits_kernel<true, 1>),
                       dim3(E / 16, kLogitParts, (T + 15) / 16), dim3(kLogitWaves * 64), 0,
                       (hipStream_t)stream, (const uint16_t*)nullptr, h, ss_parts, n_ss,
                       (const uint16_t*)gamma, eps, w, T, H, E, parts, (uint16_t*)xn_out);
  else
    hipLaunchKernelGGL((moe_router_logits_kernel<true, 2>),
                       dim3(E / 16, kLogitParts, (T + kLogitRows - 1) / kLogitRows),
                       dim3(kLogitWaves * 64), 0, (hipStream_t)stream, (const uint16_t*)nullptr,
                       h, ss_parts, n_ss, (const uint16_t*)gamma, eps, w, T, H, E, parts,
                       (uint16_t*)xn_out);
  return sym_host::check_launch("moe_router_logits_kernel");
}

extern "C" int sym_moe_route_permute(const float* logits, int n_logit_parts, const float* bias,
                                     int T, int E, int n_group, int topk_group, int top_k,
                                     float routed_scale, int renormalize, int with_shared,
                                     int32_t* topk_idx, float* topk_w, int32_t* expert_counts,
                                     int32_t* expert_offsets, int32_t* sorted_tokens,
                                     int32_t* inv_perm, int32_t* seg_expert, int32_t* seg_offset,
                                     int32_t* seg_count, int32_t* n_segments, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  SYM_REQUIRE(T >= 0, SYM_ERR_INVALID, "moe_route_permute: T=%d < 0", T);
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(logits && bias && topk_idx && topk_w && expert_counts && expert_offsets &&
                  sorted_tokens && inv_perm && seg_expert && seg_offset && seg_count &&
                  n_segments,
              SYM_ERR_INVALID, "moe_route_permute: null pointer argument");
  SYM_REQUIRE(n_logit_parts >= 1 && n_logit_parts <= kLogitParts, SYM_ERR_INVALID,
              "moe_route_permute: n_logit_parts=%d out of [1,%d]", n_logit_parts, kLogitParts);
  SYM_REQUIRE(E == 64 || E == 128 || E == 256 || E == 512, SYM_ERR_UNSUPPORTED,
              "moe_route_permute: E=%d not in {64,128,256,512}", E);
  SYM_REQUIRE(n_group >= 1 && E % n_group == 0, SYM_ERR_INVALID,
              "moe_route_permute: n_group=%d does not divide E=%d", n_group, E);
  const int epl = E / 64;
  const int gsz = E / n_group;
  SYM_REQUIRE(gsz >= 2 && gsz % epl == 0, SYM_ERR_UNSUPPORTED,
              "moe_route_permute: group size %d must be >= 2 and a multiple of %d", gsz, epl);
  const int lpg = gsz / epl;
  SYM_REQUIRE((lpg & (lpg - 1)) == 0, SYM_ERR_UNSUPPORTED,
              "moe_route_permute: lanes per group %d is not a power of two", lpg);
  SYM_REQUIRE(top_k >= 1 && top_k <= kMaxTopK && top_k <= E, SYM_ERR_INVALID,
              "moe_route_permute: top_k=%d out of range", top_k);
  SYM_REQUIRE(topk_group >= 1 && topk_group <= n_group, SYM_ERR_INVALID,
              "moe_route_permute: topk_group=%d out of range [1,%d]", topk_group, n_group);
  SYM_REQUIRE(top_k <= topk_group * gsz, SYM_ERR_INVALID,
              "moe_route_permute: top_k=%d exceeds the experts of the kept groups", top_k);
  SYM_REQUIRE((long long)T * top_k + T < (1ll << 30), SYM_ERR_INVALID,
              "moe_route_permute: T=%d too large", T);
  const size_t ws_need = sym_moe_route_workspace_bytes(T, E);
  SYM_REQUIRE(ws_need == 0 || (workspace && workspace_bytes >= ws_need), SYM_ERR_WORKSPACE,
              "moe_route_permute: workspace of %zu bytes needed for T=%d (got %zu)", ws_need, T,
              workspace ? workspace_bytes : (size_t)0);

  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  const dim3 grid((T + 3) / 4), block(256);
#define SYM_LAUNCH_ROUTE(EE)                                                                    \
  hipLaunchKernelGGL(moe_route_kernel<EE>, grid, block, 0, s, logits, n_logit_parts, bias, T, E, \
                     n_group, topk_group, top_k, routed_scale, renormalize, topk_idx, topk_w)
  switch (epl) {
    case 1: SYM_LAUNCH_ROUTE(1); break;
    case 2: SYM_LAUNCH_ROUTE(2); break;
    case 4: SYM_LAUNCH_ROUTE(4); break;
    default: SYM_LAUNCH_ROUTE(8); break;
  }
#undef SYM_LAUNCH_ROUTE
  int rc = sym_host::check_launch("moe_route_kernel");
  if (rc) return rc;
  if (ws_need == 0) {
    hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(kPermuteThreads), 0, s, topk_idx, T,
                       top_k, E, with_shared, expert_counts, expert_offsets, sorted_tokens,
                       inv_perm, seg_expert, seg_offset, seg_count, n_segments);
    return sym_host::check_launch("moe_permute_kernel");
  }
  const int n_chunks = (T + kChunkTokens - 1) / kChunkTokens;
  int32_t* chunk_cnt = (int32_t*)workspace;
  hipLaunchKernelGGL(moe_permute_count_kernel, dim3(n_chunks), dim3(256), 0, s, topk_idx, T, top_k,
                     E, chunk_cnt);
  rc = sym_host::check_launch("moe_permute_count_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(moe_permute_scan_kernel, dim3(1), dim3(kPermuteThreads), 0, s, T, top_k, E,
                     with_shared, n_chunks, chunk_cnt, expert_counts, expert_offsets,
                     sorted_tokens, seg_expert, seg_offset, seg_count, n_segments);
  rc = sym_host::check_launch("moe_permute_scan_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(moe_permute_scatter_kernel, dim3(n_chunks), dim3(256), 0, s, topk_idx, T,
                     top_k, E, chunk_cnt, expert_offsets, sorted_tokens, inv_perm);
  return sym_host::check_launch("moe_permute_scatter_kernel");
}
