// Fused MoE router: sigmoid + expert bias + group-limited top-k + weight normalisation, then a
// deterministic counting-sort permute of the (token, k) assignments by expert.
//
// Reference semantics: Glm4MoeRouteTokenToExperts.forward (ttnn_moe.py:413-436) as used for
// BailingMoeV2 by TTNNBailingMoE (ttnn_moe.py:1520-1533, norm_topk_prob forced True), and the
// token dispatch of TTNNExperts.forward (ttnn_moe.py:1225-1245).
//
// Design (gfx950, wave64):
//   kernel 1 (one workgroup per chunk of 64 tokens, one wave per token at a time): each lane owns
//     E/64 consecutive experts, so a group of E/n_group experts spans a power-of-two run of lanes.
//     Group top-2 is a butterfly over those lanes; group ranking reads the n_group scores with
//     lane broadcasts; the final top-k is k rounds of a wave-wide max over 64-bit keys
//     (order-preserving float bits << 32 | (0xFFFF - expert)), which makes ties pick the lower
//     expert index. The chunk's routing is folded into one 64-bit token mask per expert (LDS
//     atomic OR, order independent).
//   kernel 2 (one workgroup): per-expert prefix over chunks, exclusive scan over experts, then
//     every assignment's row = expert offset + earlier chunks + popcount of earlier tokens in its
//     own chunk mask. The result does not depend on scheduling order: bit-exact across runs.
//
// Floating point: contraction is disabled in this file so the sigmoid below (own Cody-Waite exp,
// explicit fma) and every add/divide are the IEEE operations the CPU oracle performs.
#pragma clang fp contract(off)

#include "common.h"

namespace sym {

// sigmoid(x) = 1 / (1 + exp(-x)); exp by round(x*log2e) range reduction with a two-part ln2 and a
// degree-7 Taylor polynomial on |r| <= ln2/2 (relative error < 6e-8), scaled by ldexp.
__device__ __forceinline__ float route_sigmoid(float x) {
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

// Order-preserving map float -> uint32 (larger float -> larger uint); -0.0 is folded onto +0.0.
__device__ __forceinline__ uint32_t order_bits(float v) {
  uint32_t u = __float_as_uint(v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int off) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl_xor(lo, off);
  hi = __shfl_xor(hi, off);
  return ((uint64_t)hi << 32) | lo;
}

constexpr int kChunk = 64;      // tokens per chunk (one bit each in a u64 mask)
constexpr int kRouteThreads = 1024;
constexpr int kMaxTopK = 32;

template <int EPL>
__global__ __launch_bounds__(kRouteThreads) void moe_route_chunk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int T, int E, int n_group,
    int topk_group, int top_k, float routed_scale, int renorm, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_w, unsigned long long* __restrict__ chunk_mask,
    int32_t* __restrict__ chunk_cnt) {
  __shared__ unsigned long long s_mask[64 * EPL];
  __shared__ int32_t s_idx[kChunk * kMaxTopK];

  const int chunk = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;

  for (int e = tid; e < E; e += blockDim.x) s_mask[e] = 0ull;

  const int gsz = E / n_group;  // experts per group
  const int lpg = gsz / EPL;    // lanes per group (power of two)
  const int my_group = lane / lpg;

  float bv[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) bv[j] = bias[lane * EPL + j];

  const int tok0 = chunk * kChunk;
  const int ntok = min(kChunk, T - tok0);

  for (int tl = wave; tl < ntok; tl += nwaves) {
    const int t = tok0 + tl;
    const float* lrow = logits + (size_t)t * E + lane * EPL;
    float s[EPL], c[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      s[j] = route_sigmoid(lrow[j]);
      c[j] = s[j] + bv[j];
    }

    // group score = largest + second largest c of the group
    float t1 = -INFINITY, t2 = -INFINITY;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const float v = c[j];
      if (v > t1) {
        t2 = t1;
        t1 = v;
      } else if (v > t2) {
        t2 = v;
      }
    }
    for (int off = 1; off < lpg; off <<= 1) {
      const float o1 = __shfl_xor(t1, off);
      const float o2 = __shfl_xor(t2, off);
      const float n1 = fmaxf(t1, o1);
      const float n2 = fmaxf(fminf(t1, o1), fmaxf(t2, o2));
      t1 = n1;
      t2 = n2;
    }
    const float gscore = t1 + t2;

    // rank of this lane's group among all groups (ties: lower group first)
    int rank = 0;
    for (int g = 0; g < n_group; ++g) {
      const float o = __shfl(gscore, g * lpg);
      rank += (o > gscore) || (o == gscore && g < my_group);
    }
    const bool keep = rank < topk_group;

    unsigned long long key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const float m = keep ? c[j] : 0.0f;
      key[j] = ((unsigned long long)order_bits(m) << 32) |
               (unsigned long long)(0xFFFFu - (uint32_t)(lane * EPL + j));
    }

    float denom = 0.0f;
    int my_idx = 0;
    float my_w = 0.0f;
    for (int k = 0; k < top_k; ++k) {
      unsigned long long best = 0ull;
#pragma unroll
      for (int j = 0; j < EPL; ++j) best = key[j] > best ? key[j] : best;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = shfl_xor_u64(best, off);
        best = o > best ? o : best;
      }
      const int e = (int)(0xFFFFu - (uint32_t)(best & 0xFFFFull));
      const int owner = e / EPL;
      const int jj = e - owner * EPL;
      float sv = 0.0f;
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        if (j == jj) sv = s[j];
      }
      if (lane == owner) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
          if (j == jj) key[j] = 0ull;
        }
      }
      sv = __shfl(sv, owner);
      denom = denom + sv;
      if (lane == k) {
        my_idx = e;
        my_w = sv;
      }
    }
    if (renorm) {
      denom = denom + 1e-20f;
      my_w = my_w / denom;
    }
    my_w = my_w * routed_scale;
    if (lane < top_k) {
      topk_idx[(size_t)t * top_k + lane] = my_idx;
      topk_w[(size_t)t * top_k + lane] = my_w;
      s_idx[tl * top_k + lane] = my_idx;
    }
  }
  __syncthreads();
  for (int a = tid; a < ntok * top_k; a += blockDim.x) {
    const int tl = a / top_k;
    atomicOr(&s_mask[s_idx[a]], 1ull << tl);
  }
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) {
    const unsigned long long m = s_mask[e];
    chunk_mask[(size_t)chunk * E + e] = m;
    chunk_cnt[(size_t)chunk * E + e] = __popcll(m);
  }
}

// Exclusive scan of one int per thread over a workgroup of up to 1024 threads.
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

__global__ __launch_bounds__(kRouteThreads) void moe_permute_kernel(
    const int32_t* __restrict__ topk_idx, int T, int K, int E, int n_chunks,
    const unsigned long long* __restrict__ chunk_mask, const int32_t* __restrict__ chunk_cnt,
    int32_t* __restrict__ chunk_pre, int with_shared, int32_t* __restrict__ expert_counts,
    int32_t* __restrict__ expert_offsets, int32_t* __restrict__ sorted_tokens,
    int32_t* __restrict__ inv_perm, int32_t* __restrict__ seg_expert,
    int32_t* __restrict__ seg_offset, int32_t* __restrict__ seg_count,
    int32_t* __restrict__ n_segments) {
  __shared__ int s_off[1024];
  __shared__ int s_wave[16];
  const int tid = threadIdx.x;
  const int e = tid;

  int cnt = 0;
  if (e < E) {
    for (int c = 0; c < n_chunks; ++c) {
      const int v = chunk_cnt[(size_t)c * E + e];
      chunk_pre[(size_t)c * E + e] = cnt;
      cnt += v;
    }
  }
  int total = 0;
  const int off = block_exclusive_scan(cnt, s_wave, &total);
  int n_routed = 0;
  const int flag = (e < E && cnt > 0) ? 1 : 0;
  const int slot = block_exclusive_scan(flag, s_wave, &n_routed);
  if (e < E) {
    s_off[e] = off;
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
      seg_offset[n_routed] = T * K;
      seg_count[n_routed] = T;
    }
    n_segments[0] = n_routed + (with_shared ? 1 : 0);
  }
  __syncthreads();

  for (int a = tid; a < T * K; a += blockDim.x) {
    const int t = a / K;
    const int ex = topk_idx[a];
    const int c = t >> 6;
    const int bit = t & 63;
    const unsigned long long m = chunk_mask[(size_t)c * E + ex];
    const unsigned long long lower = bit ? (m & ((1ull << bit) - 1ull)) : 0ull;
    const int row = s_off[ex] + chunk_pre[(size_t)c * E + ex] + __popcll(lower);
    sorted_tokens[row] = t;
    inv_perm[a] = row;
  }
  if (with_shared) {
    for (int t = tid; t < T; t += blockDim.x) sorted_tokens[T * K + t] = t;
  }
}

}  // namespace sym

using namespace sym;

extern "C" size_t sym_moe_route_workspace_bytes(int T, int E) {
  if (T <= 0 || E <= 0) return 0;
  const size_t chunks = (size_t)(T + kChunk - 1) / kChunk;
  // chunk masks (u64) + chunk counts (i32) + chunk prefixes (i32), each [chunks, E]
  return chunks * (size_t)E * (8 + 4 + 4) + 256;
}

extern "C" int sym_moe_route_permute(const float* logits, const float* bias, int T, int E,
                                     int n_group, int topk_group, int top_k, float routed_scale,
                                     int renormalize, int with_shared, int32_t* topk_idx,
                                     float* topk_w, int32_t* expert_counts,
                                     int32_t* expert_offsets, int32_t* sorted_tokens,
                                     int32_t* inv_perm, int32_t* seg_expert, int32_t* seg_offset,
                                     int32_t* seg_count, int32_t* n_segments, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  SYM_REQUIRE(T >= 0, SYM_ERR_INVALID, "moe_route_permute: T=%d < 0", T);
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(logits && bias && topk_idx && topk_w && expert_counts && expert_offsets &&
                  sorted_tokens && inv_perm && seg_expert && seg_offset && seg_count &&
                  n_segments && workspace,
              SYM_ERR_INVALID, "moe_route_permute: null pointer argument");
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
  const size_t need = sym_moe_route_workspace_bytes(T, E);
  SYM_REQUIRE(workspace_bytes >= need, SYM_ERR_WORKSPACE,
              "moe_route_permute: workspace %zu < required %zu", workspace_bytes, need);

  const int n_chunks = (T + kChunk - 1) / kChunk;
  char* ws = (char*)workspace;
  unsigned long long* chunk_mask = (unsigned long long*)ws;
  int32_t* chunk_cnt = (int32_t*)(ws + (size_t)n_chunks * E * 8);
  int32_t* chunk_pre = chunk_cnt + (size_t)n_chunks * E;

  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  const dim3 grid(n_chunks), block(kRouteThreads);
  switch (epl) {
    case 1:
      hipLaunchKernelGGL(moe_route_chunk_kernel<1>, grid, block, 0, s, logits, bias, T, E, n_group,
                         topk_group, top_k, routed_scale, renormalize, topk_idx, topk_w,
                         chunk_mask, chunk_cnt);
      break;
    case 2:
      hipLaunchKernelGGL(moe_route_chunk_kernel<2>, grid, block, 0, s, logits, bias, T, E, n_group,
                         topk_group, top_k, routed_scale, renormalize, topk_idx, topk_w,
                         chunk_mask, chunk_cnt);
      break;
    case 4:
      hipLaunchKernelGGL(moe_route_chunk_kernel<4>, grid, block, 0, s, logits, bias, T, E, n_group,
                         topk_group, top_k, routed_scale, renormalize, topk_idx, topk_w,
                         chunk_mask, chunk_cnt);
      break;
    default:
      hipLaunchKernelGGL(moe_route_chunk_kernel<8>, grid, block, 0, s, logits, bias, T, E, n_group,
                         topk_group, top_k, routed_scale, renormalize, topk_idx, topk_w,
                         chunk_mask, chunk_cnt);
      break;
  }
  int rc = sym_host::check_launch("moe_route_chunk_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(1024), 0, s, topk_idx, T, top_k, E, n_chunks,
                     chunk_mask, chunk_cnt, chunk_pre, with_shared, expert_counts, expert_offsets,
                     sorted_tokens, inv_perm, seg_expert, seg_offset, seg_count, n_segments);
  return sym_host::check_launch("moe_permute_kernel");
}
