// Paged GQA decode attention over a block-table KV cache, plus the decode prologue
// (per-head QK RMSNorm, split-half partial RoPE, paged KV write) and the cache write/fill ops.
//
// Reference semantics:
//   TTNNPagedAttentionKVCache (ttnn_attention.py:75-371): pools [num_blocks, Hkv, block_size, D],
//   page table [B, blocks_per_seq]; paged_update_on_device (235-269) writes slot cur_pos[b];
//   paged_sdpa_decode (288-329) attends positions 0..cur_pos[b] inclusive with
//   scale = head_dim^-0.5 (ttnn_attention.py:1973), GQA kv head = q head / (Hq/Hkv).
//   Decode prologue order qkv -> split -> qk_norm -> rope -> paged update
//   (ttnn_attention.py:2329-2431); RMSNorm formula ttnn_normalization.py:54-68; RoPE
//   split-half form TorchRotaryPositionEmbedding (ttnn_rope.py:23-62), partial rotary on the
//   first rotary_dim dims, inv_freq = theta^-(2i/rotary_dim) (ttnn_rope.py:304).
//
// Decode kernel design (gfx950): split-K ("flash decoding"). One workgroup (4 waves) owns one
// (sequence, kv head, 256-token split): it loads the G = Hq/Hkv query heads of that kv head once
// and streams the split's K then V rows exactly once. A K/V row of 128 bf16 is 256 contiguous
// bytes; 16 lanes x 16 bytes cover a row, so one wave-wide load covers 4 consecutive tokens of
// a block (1 KB contiguous). QK dots reduce over the 16 lanes of a token with xor shuffles;
// scores live in LDS (G x 256 fp32), softmax statistics are workgroup reductions, and P.V
// accumulates per lane in registers with a final cross-lane/cross-wave reduction. Each split
// writes an unnormalised partial output and its (max, sum) in the log2 domain; a merge kernel
// combines the splits with the log-sum-exp rule. Splits past a sequence's length exit at once.
#include "common.h"

namespace sym {

constexpr int kHeadDim = 128;
constexpr int kSplit = 256;  // tokens per split
constexpr int kAttnThreads = 256;

// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attn_decode_prologue_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const float* __restrict__ rope_cs, int max_pos,
    const int32_t* __restrict__ positions, int Hq, int Hkv, int rd, float eps, int use_qk_norm,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int32_t* __restrict__ block_tables, int mbps, int block_size, int num_blocks) {
  const int b = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  const int nh = Hq + 2 * Hkv;
  const int pos = positions[b];
  const int half = rd >> 1;

  int phys = -1;
  int off = 0;
  if (pos >= 0) {
    const int blk = pos / block_size;
    off = pos - blk * block_size;
    if (blk < mbps) {
      const int p = block_tables[(size_t)b * mbps + blk];
      if (p >= 0 && p < num_blocks) phys = p;
    }
  }
  const bool rope_ok = pos >= 0 && pos < max_pos;

  for (int h = wave; h < nh; h += nwaves) {
    const uint16_t* src = qkv + ((size_t)b * nh + h) * kHeadDim;
    float x0 = bf16_to_f32(src[lane]);
    float x1 = bf16_to_f32(src[lane + 64]);
    const bool is_q = h < Hq;
    const bool is_v = h >= Hq + Hkv;
    if (!is_v) {
      if (use_qk_norm) {
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float r = rsqrtf(ss * (1.0f / kHeadDim) + eps);
        const uint16_t* w = is_q ? qn_w : kn_w;
        x0 = x0 * r * bf16_to_f32(w[lane]);
        x1 = x1 * r * bf16_to_f32(w[lane + 64]);
      }
      if (rope_ok && rd > 0) {
        // element i lives in lane i % 64, slot i / 64
        const int i0 = lane, i1 = lane + 64;
        const int p0 = i0 < half ? i0 + half : i0 - half;
        const int p1 = i1 < half ? i1 + half : i1 - half;
        const float a0 = __shfl(x0, p0 & 63), b0 = __shfl(x1, p0 & 63);
        const float a1 = __shfl(x0, p1 & 63), b1 = __shfl(x1, p1 & 63);
        const float y0 = (p0 >> 6) ? b0 : a0;  // value of element p0
        const float y1 = (p1 >> 6) ? b1 : a1;
        const float* cs = rope_cs + (size_t)pos * rd;  // [cos(half) | sin(half)]
        float n0 = x0, n1 = x1;
        if (i0 < rd) {
          const int f = i0 < half ? i0 : i0 - half;
          const float c = cs[f], s = cs[half + f];
          n0 = i0 < half ? x0 * c - y0 * s : x0 * c + y0 * s;
        }
        if (i1 < rd) {
          const int f = i1 < half ? i1 : i1 - half;
          const float c = cs[f], s = cs[half + f];
          n1 = i1 < half ? x1 * c - y1 * s : x1 * c + y1 * s;
        }
        x0 = n0;
        x1 = n1;
      }
    }
    if (is_q) {
      uint16_t* dst = q_out + ((size_t)b * Hq + h) * kHeadDim;
      dst[lane] = f32_to_bf16(x0);
      dst[lane + 64] = f32_to_bf16(x1);
    } else if (phys >= 0) {
      const int g = is_v ? h - Hq - Hkv : h - Hq;
      uint16_t* pool = is_v ? v_pool : k_pool;
      uint16_t* dst = pool + (((size_t)phys * Hkv + g) * block_size + off) * kHeadDim;
      dst[lane] = f32_to_bf16(x0);
      dst[lane + 64] = f32_to_bf16(x1);
    }
  }
}

// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void paged_kv_write_kernel(
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ positions, int Hkv,
    int block_size, int mbps, int num_blocks) {
  const int b = blockIdx.x;
  const int pos = positions[b];
  if (pos < 0) return;
  const int blk = pos / block_size;
  if (blk >= mbps) return;
  const int phys = block_tables[(size_t)b * mbps + blk];
  if (phys < 0 || phys >= num_blocks) return;
  const int off = pos - blk * block_size;
  const int n = Hkv * kHeadDim;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int g = i / kHeadDim, d = i - g * kHeadDim;
    const size_t dst = (((size_t)phys * Hkv + g) * block_size + off) * kHeadDim + d;
    k_pool[dst] = k_new[(size_t)b * n + i];
    v_pool[dst] = v_new[(size_t)b * n + i];
  }
}

__global__ __launch_bounds__(256) void paged_kv_fill_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint16_t* __restrict__ k_pool,
    uint16_t* __restrict__ v_pool, const int32_t* __restrict__ bt_row, int start_pos, int S,
    int Hkv, int block_size, int mbps, int num_blocks) {
  // grid: (S, Hkv); k, v [Hkv, S, D]
  const int s = blockIdx.x, g = blockIdx.y;
  const int pos = start_pos + s;
  const int blk = pos / block_size;
  if (blk >= mbps) return;
  const int phys = bt_row[blk];
  if (phys < 0 || phys >= num_blocks) return;
  const int off = pos - blk * block_size;
  const size_t dst = (((size_t)phys * Hkv + g) * block_size + off) * kHeadDim;
  const size_t src = ((size_t)g * S + s) * kHeadDim;
  for (int d = threadIdx.x; d < kHeadDim; d += blockDim.x) {
    k_pool[dst + d] = k[src + d];
    v_pool[dst + d] = v[src + d];
  }
}

// ---------------------------------------------------------------------------------------------
template <int G>
__global__ __launch_bounds__(kAttnThreads) void paged_decode_split_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int32_t* __restrict__ block_tables,
    const int32_t* __restrict__ positions, int Hkv, int block_size, int mbps, int num_blocks,
    float scale_log2, float* __restrict__ ws_o, float* __restrict__ ws_ml, int max_splits) {
  constexpr int D = kHeadDim;
  __shared__ float s_q[G][D];
  __shared__ float s_p[G][kSplit];
  __shared__ float s_red[4][G][D];
  __shared__ float s_stat[G][4];
  __shared__ int s_bt[kSplit];   // physical block of each token (always a valid block)
  __shared__ int s_ok[kSplit];   // token is inside the split and its page-table entry is valid

  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int Hq = Hkv * G;
  const int ctx = positions[b] + 1;
  const int t0 = split * kSplit;
  if (t0 >= ctx) return;
  const int t1 = min(ctx, t0 + kSplit);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = lane & 15;  // 8 dims: sub*8 .. sub*8+7
  const int tq = lane >> 4;   // token within a group of 4

  for (int i = tid; i < G * D; i += kAttnThreads) {
    const int h = i / D, d = i - h * D;
    s_q[h][d] = bf16_to_f32(q[((size_t)b * Hq + g * G + h) * D + d]) * scale_log2;
  }
  // Physical block of every token of the split. Tokens past the sequence read the split's
  // last valid token instead (an in-bounds row already being loaded) and are masked out, so
  // every K/V load below is unconditional.
  {
    const int t = t0 + tid;
    const int tc = min(t, t1 - 1);
    const int blk = tc / block_size;
    int p = blk < mbps ? block_tables[(size_t)b * mbps + blk] : -1;
    const bool valid = t < t1 && p >= 0 && p < num_blocks;
    if (p < 0 || p >= num_blocks) p = 0;
    s_bt[tid] = p;
    s_ok[tid] = valid;
  }
  __syncthreads();

  float qr[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) qr[h][i] = s_q[h][sub * 8 + i];

  // Issue every K and V load of this wave's 64 tokens up front (16 + 16 loads of 16 bytes per
  // lane); V arrives while the scores and the softmax statistics are computed.
  uint4 kreg[16], vreg[16];
  size_t roff[16];
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int tl = wave * 64 + it * 4 + tq;
    const int tc = min(t0 + tl, t1 - 1);
    roff[it] = (((size_t)s_bt[tl] * Hkv + g) * block_size + (tc - (tc / block_size) * block_size)) *
                   D + sub * 8;
  }
#pragma unroll
  for (int it = 0; it < 16; ++it) kreg[it] = *reinterpret_cast<const uint4*>(k_pool + roff[it]);
#pragma unroll
  for (int it = 0; it < 16; ++it) vreg[it] = *reinterpret_cast<const uint4*>(v_pool + roff[it]);

  // ---- scores ----
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int tl = wave * 64 + it * 4 + tq;
    float kf[8];
    unpack8(kreg[it], kf);
    float dot[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) d = fmaf(qr[h][i], kf[i], d);
      dot[h] = d;
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) dot[h] += __shfl_xor(dot[h], o);
    }
    if (sub == 0) {
      const bool valid = s_ok[tl] != 0;
#pragma unroll
      for (int h = 0; h < G; ++h) s_p[h][tl] = valid ? dot[h] : -INFINITY;
    }
  }
  __syncthreads();

  // ---- softmax statistics over the split (log2 domain) ----
  float mx[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float m = wave_max(s_p[h][tid]);
    if (lane == 0) s_stat[h][wave] = m;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; ++h)
    mx[h] = fmaxf(fmaxf(s_stat[h][0], s_stat[h][1]), fmaxf(s_stat[h][2], s_stat[h][3]));
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float v = s_p[h][tid];
    const float p = (mx[h] == -INFINITY || v == -INFINITY) ? 0.f : exp2f(v - mx[h]);
    s_p[h][tid] = p;
    const float l = wave_sum(p);
    if (lane == 0) s_stat[h][wave] = l;
  }
  __syncthreads();

  // ---- P.V ----
  float acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int tl = wave * 64 + it * 4 + tq;
    float vf[8];
    unpack8(vreg[it], vf);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float p = s_p[h][tl];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(p, vf[i], acc[h][i]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = acc[h][i];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[h][i] = v;
    }
  if (tq == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) s_red[wave][h][sub * 8 + i] = acc[h][i];
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += kAttnThreads) {
    const int h = i / D, d = i - h * D;
    const float o = (s_red[0][h][d] + s_red[1][h][d]) + (s_red[2][h][d] + s_red[3][h][d]);
    ws_o[(((size_t)b * Hq + g * G + h) * max_splits + split) * D + d] = o;
  }
  if (tid < G) {
    const float l = (s_stat[tid][0] + s_stat[tid][1]) + (s_stat[tid][2] + s_stat[tid][3]);
    float* ml = ws_ml + (((size_t)b * Hq + g * G + tid) * max_splits + split) * 2;
    ml[0] = mx[tid];
    ml[1] = l;
  }
}

__global__ __launch_bounds__(kHeadDim) void paged_decode_merge_kernel(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    const int32_t* __restrict__ positions, int Hq, int max_splits, uint16_t* __restrict__ out) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int ctx = positions[b] + 1;
  const int ns = min(max_splits, max(0, (ctx + kSplit - 1) / kSplit));
  const size_t base = ((size_t)b * Hq + h) * max_splits;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, ws_ml[(base + s) * 2]);
  float L = 0.f, o = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < ns; ++s) {
      const float m = ws_ml[(base + s) * 2];
      const float w = m == -INFINITY ? 0.f : exp2f(m - M);
      L += w * ws_ml[(base + s) * 2 + 1];
      o += w * ws_o[(base + s) * kHeadDim + d];
    }
  }
  out[((size_t)b * Hq + h) * kHeadDim + d] = f32_to_bf16(L > 0.f ? o / L : 0.f);
}

}  // namespace sym

using namespace sym;

static int check_cache_args(const char* what, int B, int Hkv, int head_dim, int block_size,
                            int mbps, int num_blocks) {
  SYM_REQUIRE(B >= 0 && Hkv >= 1 && block_size >= 1 && mbps >= 1 && num_blocks >= 1,
              SYM_ERR_INVALID, "%s: bad sizes B=%d Hkv=%d block_size=%d mbps=%d num_blocks=%d",
              what, B, Hkv, block_size, mbps, num_blocks);
  SYM_REQUIRE(head_dim == kHeadDim, SYM_ERR_UNSUPPORTED, "%s: head_dim=%d (only 128)", what,
              head_dim);
  return SYM_OK;
}

extern "C" int sym_attn_decode_prologue(const void* qkv, const void* q_norm_w,
                                        const void* k_norm_w, const float* rope_cs, int max_pos,
                                        const int32_t* positions, int B, int Hq, int Hkv,
                                        int head_dim, int rotary_dim, float eps, int use_qk_norm,
                                        void* q_out, void* k_pool, void* v_pool,
                                        const int32_t* block_tables, int max_blocks_per_seq,
                                        int block_size, int num_blocks, void* stream) {
  int rc = check_cache_args("attn_decode_prologue", B, Hkv, head_dim, block_size,
                            max_blocks_per_seq, num_blocks);
  if (rc) return rc;
  if (B == 0) return SYM_OK;
  SYM_REQUIRE(qkv && positions && q_out && k_pool && v_pool && block_tables, SYM_ERR_INVALID,
              "attn_decode_prologue: null pointer argument");
  SYM_REQUIRE(Hq >= Hkv && Hq % Hkv == 0, SYM_ERR_INVALID,
              "attn_decode_prologue: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  SYM_REQUIRE(rotary_dim >= 0 && rotary_dim <= head_dim && rotary_dim % 2 == 0, SYM_ERR_INVALID,
              "attn_decode_prologue: rotary_dim=%d", rotary_dim);
  SYM_REQUIRE(rotary_dim == 0 || (rope_cs && max_pos > 0), SYM_ERR_INVALID,
              "attn_decode_prologue: rope table missing");
  SYM_REQUIRE(!use_qk_norm || (q_norm_w && k_norm_w), SYM_ERR_INVALID,
              "attn_decode_prologue: qk-norm weights missing");
  (void)hipGetLastError();
  hipLaunchKernelGGL(attn_decode_prologue_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)qkv, (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w,
                     rope_cs, max_pos, positions, Hq, Hkv, rotary_dim, eps, use_qk_norm,
                     (uint16_t*)q_out, (uint16_t*)k_pool, (uint16_t*)v_pool, block_tables,
                     max_blocks_per_seq, block_size, num_blocks);
  return sym_host::check_launch("attn_decode_prologue_kernel");
}

extern "C" int sym_paged_kv_write(const void* k_new, const void* v_new, void* k_pool,
                                  void* v_pool, const int32_t* block_tables,
                                  const int32_t* positions, int B, int Hkv, int head_dim,
                                  int block_size, int max_blocks_per_seq, int num_blocks,
                                  void* stream) {
  int rc = check_cache_args("paged_kv_write", B, Hkv, head_dim, block_size, max_blocks_per_seq,
                            num_blocks);
  if (rc) return rc;
  if (B == 0) return SYM_OK;
  SYM_REQUIRE(k_new && v_new && k_pool && v_pool && block_tables && positions, SYM_ERR_INVALID,
              "paged_kv_write: null pointer argument");
  (void)hipGetLastError();
  hipLaunchKernelGGL(paged_kv_write_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)k_new, (const uint16_t*)v_new, (uint16_t*)k_pool,
                     (uint16_t*)v_pool, block_tables, positions, Hkv, block_size,
                     max_blocks_per_seq, num_blocks);
  return sym_host::check_launch("paged_kv_write_kernel");
}

extern "C" int sym_paged_kv_fill(const void* k, const void* v, void* k_pool, void* v_pool,
                                 const int32_t* block_tables, int batch_idx, int start_pos, int S,
                                 int Hkv, int head_dim, int block_size, int max_blocks_per_seq,
                                 int num_blocks, void* stream) {
  int rc = check_cache_args("paged_kv_fill", 1, Hkv, head_dim, block_size, max_blocks_per_seq,
                            num_blocks);
  if (rc) return rc;
  SYM_REQUIRE(S >= 0 && start_pos >= 0 && batch_idx >= 0, SYM_ERR_INVALID,
              "paged_kv_fill: S=%d start_pos=%d batch_idx=%d", S, start_pos, batch_idx);
  if (S == 0) return SYM_OK;
  SYM_REQUIRE(k && v && k_pool && v_pool && block_tables, SYM_ERR_INVALID,
              "paged_kv_fill: null pointer argument");
  SYM_REQUIRE((long long)start_pos + S <= (long long)max_blocks_per_seq * block_size,
              SYM_ERR_INVALID, "paged_kv_fill: positions %d..%d exceed the page table", start_pos,
              start_pos + S - 1);
  SYM_REQUIRE(S <= 65535 * 64, SYM_ERR_INVALID, "paged_kv_fill: S=%d too large", S);
  (void)hipGetLastError();
  hipLaunchKernelGGL(paged_kv_fill_kernel, dim3(S, Hkv), dim3(128), 0, (hipStream_t)stream,
                     (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)k_pool, (uint16_t*)v_pool,
                     block_tables + (size_t)batch_idx * max_blocks_per_seq, start_pos, S, Hkv,
                     block_size, max_blocks_per_seq, num_blocks);
  return sym_host::check_launch("paged_kv_fill_kernel");
}

extern "C" size_t sym_paged_gqa_decode_workspace_bytes(int B, int Hq, int head_dim,
                                                       int max_context) {
  if (B <= 0 || Hq <= 0 || head_dim <= 0 || max_context <= 0) return 0;
  const size_t splits = (size_t)(max_context + kSplit - 1) / kSplit;
  return (size_t)B * Hq * splits * ((size_t)head_dim + 2) * sizeof(float) + 256;
}

extern "C" int sym_paged_gqa_decode(const void* q, const void* k_pool, const void* v_pool,
                                    const int32_t* block_tables, const int32_t* positions, int B,
                                    int Hq, int Hkv, int head_dim, int block_size,
                                    int max_blocks_per_seq, int num_blocks, int max_context,
                                    float scale, void* workspace, size_t workspace_bytes,
                                    void* out, void* stream) {
  int rc = check_cache_args("paged_gqa_decode", B, Hkv, head_dim, block_size, max_blocks_per_seq,
                            num_blocks);
  if (rc) return rc;
  if (B == 0) return SYM_OK;
  SYM_REQUIRE(q && k_pool && v_pool && block_tables && positions && workspace && out,
              SYM_ERR_INVALID, "paged_gqa_decode: null pointer argument");
  SYM_REQUIRE(Hq >= Hkv && Hq % Hkv == 0, SYM_ERR_INVALID,
              "paged_gqa_decode: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  const int G = Hq / Hkv;
  SYM_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, SYM_ERR_UNSUPPORTED,
              "paged_gqa_decode: group size %d not in {1,2,4,8}", G);
  SYM_REQUIRE(max_context >= 1 && (long long)max_context <= (long long)max_blocks_per_seq * block_size,
              SYM_ERR_INVALID, "paged_gqa_decode: max_context=%d outside (0, %d]", max_context,
              max_blocks_per_seq * block_size);
  SYM_REQUIRE(B <= 65535 && Hkv <= 65535, SYM_ERR_INVALID, "paged_gqa_decode: grid too large");
  const size_t need = sym_paged_gqa_decode_workspace_bytes(B, Hq, head_dim, max_context);
  SYM_REQUIRE(workspace_bytes >= need, SYM_ERR_WORKSPACE,
              "paged_gqa_decode: workspace %zu < required %zu", workspace_bytes, need);
  const int max_splits = (max_context + kSplit - 1) / kSplit;
  float* ws_o = (float*)workspace;
  float* ws_ml = ws_o + (size_t)B * Hq * max_splits * head_dim;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  const dim3 grid(max_splits, Hkv, B), block(kAttnThreads);
  const uint16_t* qq = (const uint16_t*)q;
  const uint16_t* kp = (const uint16_t*)k_pool;
  const uint16_t* vp = (const uint16_t*)v_pool;
#define SYM_LAUNCH_DECODE(GG)                                                                   \
  hipLaunchKernelGGL(paged_decode_split_kernel<GG>, grid, block, 0, s, qq, kp, vp, block_tables, \
                     positions, Hkv, block_size, max_blocks_per_seq, num_blocks, scale_log2, ws_o, \
                     ws_ml, max_splits)
  switch (G) {
    case 1: SYM_LAUNCH_DECODE(1); break;
    case 2: SYM_LAUNCH_DECODE(2); break;
    case 4: SYM_LAUNCH_DECODE(4); break;
    default: SYM_LAUNCH_DECODE(8); break;
  }
#undef SYM_LAUNCH_DECODE
  rc = sym_host::check_launch("paged_decode_split_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(paged_decode_merge_kernel, dim3(Hq, B), dim3(kHeadDim), 0, s, ws_o, ws_ml,
                     positions, Hq, max_splits, (uint16_t*)out);
  return sym_host::check_launch("paged_decode_merge_kernel");
}
