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
// Decode kernel design (gfx950): split-K ("flash decoding"). One workgroup
// (4 waves) owns one (sequence, kv head, 256-token split): it loads the G = Hq/Hkv query heads
// of that kv head once and streams the split's K and V rows exactly once, all loads issued up
// front. Scores come from MFMA (query heads as the rows of the A operand), live in LDS
// (G x 256 fp32) for the workgroup softmax, and P.V accumulates per lane on the VALU. A merge
// kernel combines the splits of each sequence with the log-sum-exp rule. Splits past a
// sequence's length exit at once.
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
// Split-K decode. Workgroup = (split of 256 tokens, kv head g, sequence b), 4 waves x 64 tokens.
//   QK^T on MFMA: per 16-token tile, S[head][token] = Q[16 x 128] . K^T[128 x 16] as four
//   v_mfma_f32_16x16x32_bf16 (query heads are rows 0..G-1 of the A operand; lane l streams
//   dims 8*(l/16) + 32*j of token l%16, so one wave-wide load covers 64 contiguous bytes of 16
//   K rows). P.V on the VALU: a lane owns 8 dims of one token per step (16 lanes per token).
//   All K and V loads of the wave are issued before the first use.
// Each split writes its unnormalised output and (max, sum) in the log2 domain for the merge
// kernel; a sequence with a single split writes its normalised output directly. (Merging in the
// last split to finish would need a device-scope release per workgroup; on this chip that
// writes back the XCD's L2 each time and costs more than the separate merge launch.)
template <int G>
__global__ __launch_bounds__(kAttnThreads) void paged_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int32_t* __restrict__ block_tables,
    const int32_t* __restrict__ positions, int Hkv, int block_size, int mbps, int num_blocks,
    int max_context, float scale_log2, float* __restrict__ ws_o, float* __restrict__ ws_ml,
    int max_splits, uint16_t* __restrict__ out) {
  constexpr int D = kHeadDim;
  __shared__ float s_p[G][kSplit];
  __shared__ float s_red[4][G][D];
  __shared__ float s_stat[G][4];
  __shared__ float s_fin[2][G];
  __shared__ unsigned s_row[kSplit];  // K/V pool row of each token (always an in-bounds row)
  __shared__ int s_ok[kSplit];        // token is inside the split and its page-table entry is valid

  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int Hq = Hkv * G;
  const int tid = threadIdx.x;
  const int ctx = min(positions[b] + 1, max_context);
  if (ctx <= 0) {
    // nothing cached (position < 0): the output is zero
    if (split == 0)
      for (int i = tid; i < G * D; i += kAttnThreads)
        out[((size_t)b * Hq + g * G) * D + i] = 0;
    return;
  }
  const int t0 = split * kSplit;
  if (t0 >= ctx) return;
  const int t1 = min(ctx, t0 + kSplit);
  const int nsplit = (ctx + kSplit - 1) / kSplit;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int kg = lane >> 4;

  {
    // Pool row of every token of the split. Tokens past the sequence read the split's last
    // token instead, and tokens of an invalid page-table entry read block 0, so every K/V load
    // below is unconditional and in bounds; both are masked out of the softmax.
    const int t = t0 + tid;
    const int tc = min(t, t1 - 1);
    const int blk = tc / block_size;
    int pb = blk < mbps ? block_tables[(size_t)b * mbps + blk] : -1;
    const bool valid = t < t1 && pb >= 0 && pb < num_blocks;
    if (pb < 0 || pb >= num_blocks) pb = 0;
    s_row[tid] = (unsigned)(((size_t)pb * Hkv + g) * block_size + (tc - blk * block_size));
    s_ok[tid] = valid;
  }
  // query fragments (A operand): head r16 (rows >= G are zero), dims 8*kg + 32*j
  uint4 qa[4];
  {
    const uint16_t* qr = q + ((size_t)b * Hq + g * G + min(r16, G - 1)) * D + 8 * kg;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 32 * j);
      qa[j] = r16 < G ? v : make_uint4(0, 0, 0, 0);
    }
  }
  __syncthreads();

  auto row_offset = [&](int tl) -> size_t { return (size_t)s_row[tl] * D; };
  // K in the MFMA B layout: tile tt of 16 tokens, token r16, dims 8*kg + 32*j
  uint4 kb[4][4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const uint16_t* kr = k_pool + row_offset(wave * 64 + tt * 16 + r16) + 8 * kg;
#pragma unroll
    for (int j = 0; j < 4; ++j) kb[tt][j] = *reinterpret_cast<const uint4*>(kr + 32 * j);
  }
  // V for P.V: step it covers tokens it*4 + kg (4 per step), lane r16 owns dims r16*8 .. +8
  uint4 vreg[16];
#pragma unroll
  for (int it = 0; it < 16; ++it)
    vreg[it] = *reinterpret_cast<const uint4*>(v_pool + row_offset(wave * 64 + it * 4 + kg) +
                                               r16 * 8);

  // ---- scores on MFMA ----
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    floatx4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) sacc = mfma16x16x32(qa[j], kb[tt][j], sacc);
    const int tl = wave * 64 + tt * 16 + r16;
    const bool valid = s_ok[tl] != 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kg + i;
      if (h < G) s_p[h][tl] = valid ? sacc[i] * scale_log2 : -INFINITY;
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
    const float pr = (mx[h] == -INFINITY || v == -INFINITY) ? 0.f : exp2f(v - mx[h]);
    s_p[h][tid] = pr;
    const float l = wave_sum(pr);
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
    const int tl = wave * 64 + it * 4 + kg;
    float vf[8];
    unpack8(vreg[it], vf);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float pr = s_p[h][tl];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(pr, vf[i], acc[h][i]);
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
  if (kg == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) s_red[wave][h][r16 * 8 + i] = acc[h][i];
  }
  if (tid < G) {
    s_fin[0][tid] = mx[tid];
    s_fin[1][tid] = (s_stat[tid][0] + s_stat[tid][1]) + (s_stat[tid][2] + s_stat[tid][3]);
  }
  __syncthreads();

  if (nsplit == 1) {
    for (int i = tid; i < G * D; i += kAttnThreads) {
      const int h = i / D, d = i - h * D;
      const float o = (s_red[0][h][d] + s_red[1][h][d]) + (s_red[2][h][d] + s_red[3][h][d]);
      const float L = s_fin[1][h];
      out[((size_t)b * Hq + g * G + h) * D + d] = f32_to_bf16(L > 0.f ? o / L : 0.f);
    }
    return;
  }

  // this split's unnormalised output and (max, sum); the merge kernel combines the splits
  for (int i = tid; i < G * D; i += kAttnThreads) {
    const int h = i / D, d = i - h * D;
    const float o = (s_red[0][h][d] + s_red[1][h][d]) + (s_red[2][h][d] + s_red[3][h][d]);
    ws_o[(((size_t)b * Hq + g * G + h) * max_splits + split) * D + d] = o;
  }
  if (tid < G) {
    float* ml = ws_ml + (((size_t)b * Hq + g * G + tid) * max_splits + split) * 2;
    ml[0] = s_fin[0][tid];
    ml[1] = s_fin[1][tid];
  }
}

// Merge of the splits of a sequence with more than one split (log-sum-exp rule), one wave per
// (sequence, query head): lane l owns dims 2l, 2l+1; the split weights 2^(m_s - M) are computed
// one split per lane and broadcast, and the partial-output loads of 8 splits are issued at once.
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    const int32_t* __restrict__ positions, int B, int Hq, int max_context, int max_splits,
    uint16_t* __restrict__ out) {
  constexpr int D = kHeadDim;
  const int lane = threadIdx.x & 63;
  const int idx = blockIdx.x * 4 + (threadIdx.x >> 6);  // b * Hq + head
  if (idx >= B * Hq) return;
  const int ctx = min(positions[idx / Hq] + 1, max_context);
  const int nsplit = ctx <= 0 ? 0 : (ctx + kSplit - 1) / kSplit;
  if (nsplit <= 1) return;  // written directly by the split kernel
  const float2* ml = reinterpret_cast<const float2*>(ws_ml) + (size_t)idx * max_splits;
  const float2* po = reinterpret_cast<const float2*>(ws_o) + (size_t)idx * max_splits * (D / 2) + lane;
  float M = -INFINITY;
  for (int s = lane; s < nsplit; s += 64) M = fmaxf(M, ml[s].x);
  M = wave_max(M);
  float L = 0.f, ox = 0.f, oy = 0.f;
  for (int c = 0; c < nsplit; c += 64) {
    float w = 0.f;
    if (c + lane < nsplit) {
      const float2 v = ml[c + lane];
      w = (v.x == -INFINITY) ? 0.f : exp2f(v.x - M);
      L = fmaf(w, v.y, L);
    }
    const int n = min(64, nsplit - c);
    int j = 0;
    for (; j + 8 <= n; j += 8) {
      float2 pv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) pv[u] = po[(size_t)(c + j + u) * (D / 2)];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float wj = __shfl(w, j + u);
        ox = fmaf(wj, pv[u].x, ox);
        oy = fmaf(wj, pv[u].y, oy);
      }
    }
    for (; j < n; ++j) {
      const float2 pv = po[(size_t)(c + j) * (D / 2)];
      const float wj = __shfl(w, j);
      ox = fmaf(wj, pv.x, ox);
      oy = fmaf(wj, pv.y, oy);
    }
  }
  L = wave_sum(L);
  reinterpret_cast<uint32_t*>(out)[(size_t)idx * (D / 2) + lane] =
      L > 0.f ? pack_bf16x2(ox / L, oy / L) : 0u;
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
  SYM_REQUIRE((unsigned long long)num_blocks * Hkv * block_size <= 0xFFFFFFFFull,
              SYM_ERR_UNSUPPORTED, "%s: pool of %llu rows per K/V (at most 2^32 - 1)", what,
              (unsigned long long)num_blocks * Hkv * block_size);
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
  // partial outputs and (max, sum) of every split
  return (size_t)B * Hq * splits * ((size_t)head_dim + 2) * sizeof(float);
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
  hipLaunchKernelGGL(paged_decode_kernel<GG>, grid, block, 0, s, qq, kp, vp, block_tables,       \
                     positions, Hkv, block_size, max_blocks_per_seq, num_blocks, max_context,    \
                     scale_log2, ws_o, ws_ml, max_splits, (uint16_t*)out)
  switch (G) {
    case 1: SYM_LAUNCH_DECODE(1); break;
    case 2: SYM_LAUNCH_DECODE(2); break;
    case 4: SYM_LAUNCH_DECODE(4); break;
    default: SYM_LAUNCH_DECODE(8); break;
  }
#undef SYM_LAUNCH_DECODE
  rc = sym_host::check_launch("paged_decode_kernel");
  if (rc || max_splits == 1) return rc;
  hipLaunchKernelGGL(paged_decode_merge_kernel, dim3((B * Hq + 3) / 4), dim3(256), 0, s, ws_o,
                     ws_ml, positions, B, Hq, max_context, max_splits, (uint16_t*)out);
  return sym_host::check_launch("paged_decode_merge_kernel");
}
