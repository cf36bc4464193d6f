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
// of that kv head once and streams the split's K and V rows exactly once, K issued up front and
// V after the scores. Scores come from MFMA (query heads as the rows of the A operand), live in
// LDS (G x 256 fp32) for the workgroup softmax, and P.V runs on the MFMA too (P of the lane's
// tokens as the A operand, the V elements it loaded as B, with matching k orders). A merge
// kernel combines the splits of each sequence with the log-sum-exp rule. Splits past a
// sequence's length exit at once.
#include <mutex>

#include "common.h"

namespace sym {

constexpr int kHeadDim = 128;
constexpr int kTPW = 64;           // tokens per wave in the split kernel
constexpr int kSplit = 4 * kTPW;  // tokens per split (one workgroup of 4 waves)
// The fp8 cache's split kernel: tokens per wave (a wave of 128 tokens fits the bf16 kernel's
// registers, but measured slower: 225 against 199 us at batch 128 with 1024-8192 contexts).
constexpr int kTPW8 = 64;
constexpr int kSplit8 = 4 * kTPW8;
static_assert(kSplit <= kSplit8, "the decode workspace (kSplit-token splits) must hold the fp8 kernel's");
// fp8 split kernel: V is loaded after the scores (into the registers K used) and the kernel is
// held to 6 workgroups per CU at up to 4 query heads per kv head (80 VGPRs with P.V on MFMA, 2
// of them spilled: 164 against 170 us at 5 per CU, 82 VGPRs, at batch 128 with 1024-8192
// contexts); 8 heads per kv head keep the default. (With P.V on the VALU: late V and 5 per CU,
// 92 VGPRs, 197 us; late V alone at 4 per CU 218 us; V with K 210 us.)
constexpr int kFp8MinBlocks = 6;
constexpr int kBf16MinBlocks = 1;
constexpr int kAttnThreads = 256;

// ---------------------------------------------------------------------------------------------
// QK RMSNorm (optional) and split-half partial RoPE of one head, held by a wave as
// x0 = dim `lane`, x1 = dim `lane + 64`. norm: x * rsqrt(mean(x^2) + eps) * w in fp32 (one
// rounding at the end, by the caller); RoPE over dims [0, rd): for i < rd/2,
// y_i = x_i cos - x_{i+rd/2} sin and y_{i+rd/2} = x_{i+rd/2} cos + x_i sin, with
// cs = [cos(pos f_0..) | sin(pos f_0..)] the table row of the position.
// The per-lane operands (norm weights, cos/sin of the lane's two dims) are loaded separately
// from the arithmetic, so a kernel can issue those loads early.
struct RopeLane {
  float c0, s0, c1, s1;  // cos/sin for dims lane and lane + 64 (unused past rd)
};

__device__ __forceinline__ RopeLane load_rope_lane(const float* __restrict__ cs, int rd,
                                                   int lane) {
  RopeLane r{1.f, 0.f, 1.f, 0.f};
  if (cs && rd > 0) {
    const int half = rd >> 1;
    const int i0 = lane, i1 = lane + 64;
    const int f0 = i0 < half ? i0 : i0 - half;
    const int f1 = i1 < half ? i1 : i1 - half;
    if (i0 < rd) { r.c0 = cs[f0]; r.s0 = cs[half + f0]; }
    if (i1 < rd) { r.c1 = cs[f1]; r.s1 = cs[half + f1]; }
  }
  return r;
}

// Branch-free form for a kernel that issues these loads early: cs must point at rd readable
// floats (a table row, or any rd floats when RoPE is off; the values are then not used).
__device__ __forceinline__ RopeLane load_rope_lane_nobranch(const float* __restrict__ cs,
                                                            int rd, int lane) {
  const int half = max(rd >> 1, 1);
  const int i0 = lane, i1 = lane + 64;
  const int f0 = min(i0 < half ? i0 : i0 - half, half - 1);
  const int f1 = min(i1 < half ? i1 : i1 - half, half - 1);
  return RopeLane{cs[f0], cs[half + f0], cs[f1], cs[half + f1]};
}

// Stand-ins the fused kernel reads when QK-norm or RoPE is off, so its early loads need no
// branches (1.0 in bf16; 256 zero floats).
__device__ const uint16_t kOnesBf16[kHeadDim] = {
#define SYM_ONE8 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80
    SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8,
    SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8, SYM_ONE8
#undef SYM_ONE8
};
__device__ const float kZeroRope[2 * kHeadDim] = {};

__device__ __forceinline__ void qk_norm_rope(float& x0, float& x1, bool norm, float w0, float w1,
                                             float eps, bool rope, const RopeLane& rl, int rd,
                                             int lane) {
  // no contraction: the prologue kernel and the fused decode step round identically
#pragma clang fp contract(off)
  if (norm) {
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float r = rsqrtf(ss * (1.0f / kHeadDim) + eps);
    x0 = x0 * r * w0;
    x1 = x1 * r * w1;
  }
  if (rope && rd > 0) {
    const int half = rd >> 1;
    // element i lives in lane i % 64, slot i / 64
    const int i0 = lane, i1 = lane + 64;
    const int p0 = i0 < half ? i0 + half : i0 - half;
    const int p1 = i1 < half ? i1 + half : i1 - half;
    const float a0 = __shfl(x0, p0 & 63), b0 = __shfl(x1, p0 & 63);
    const float a1 = __shfl(x0, p1 & 63), b1 = __shfl(x1, p1 & 63);
    const float y0 = (p0 >> 6) ? b0 : a0;  // value of element p0
    const float y1 = (p1 >> 6) ? b1 : a1;
    float n0 = x0, n1 = x1;
    if (i0 < rd) n0 = i0 < half ? x0 * rl.c0 - y0 * rl.s0 : x0 * rl.c0 + y0 * rl.s0;
    if (i1 < rd) n1 = i1 < half ? x1 * rl.c1 - y1 * rl.s1 : x1 * rl.c1 + y1 * rl.s1;
    x0 = n0;
    x1 = n1;
  }
}

// Physical block of the slot of `pos` in sequence b, or -1 (position < 0, beyond the page table,
// or an entry outside [0, num_blocks)); *off gets the slot's offset in the block.
__device__ __forceinline__ int slot_block(const int32_t* __restrict__ block_tables, int b,
                                          int pos, int mbps, int block_size, int num_blocks,
                                          int* off) {
  if (pos < 0) return -1;
  const int blk = pos / block_size;
  *off = pos - blk * block_size;
  if (blk >= mbps) return -1;
  const int p = block_tables[(size_t)b * mbps + blk];
  return (p >= 0 && p < num_blocks) ? p : -1;
}

// Row b of qkv is one token: its position is positions[b], its page-table row is
// bt_rows[b] (or b when bt_rows is null: one token per sequence, the decode case). q goes to
// q_out; k and v go to the pools and, when k_out / v_out are given, also to [rows, Hkv, 128].
__global__ __launch_bounds__(256) void attn_decode_prologue_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const float* __restrict__ rope_cs, int max_pos,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ bt_rows, int Hq, int Hkv,
    int rd, float eps, int use_qk_norm, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out, uint16_t* __restrict__ k_pool,
    uint16_t* __restrict__ v_pool, const int32_t* __restrict__ block_tables, int mbps,
    int block_size, int num_blocks) {
  const int b = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  const int nh = Hq + 2 * Hkv;
  const int pos = positions[b];
  const int btr = bt_rows ? bt_rows[b] : b;
  int off = 0;
  const int phys = slot_block(block_tables, btr, pos, mbps, block_size, num_blocks, &off);
  const bool rope = pos >= 0 && pos < max_pos;
  const RopeLane rl = load_rope_lane(rope ? rope_cs + (size_t)pos * rd : nullptr, rd, lane);

  for (int h = wave; h < nh; h += nwaves) {
    const uint16_t* src = qkv + ((size_t)b * nh + h) * kHeadDim;
    float x0 = bf16_to_f32(src[lane]);
    float x1 = bf16_to_f32(src[lane + 64]);
    const bool is_q = h < Hq;
    const bool is_v = h >= Hq + Hkv;
    if (!is_v) {
      const uint16_t* w = is_q ? qn_w : kn_w;
      const float w0 = use_qk_norm ? bf16_to_f32(w[lane]) : 1.f;
      const float w1 = use_qk_norm ? bf16_to_f32(w[lane + 64]) : 1.f;
      qk_norm_rope(x0, x1, use_qk_norm != 0, w0, w1, eps, rope, rl, rd, lane);
    }
    if (is_q) {
      uint16_t* dst = q_out + ((size_t)b * Hq + h) * kHeadDim;
      dst[lane] = f32_to_bf16(x0);
      dst[lane + 64] = f32_to_bf16(x1);
    } else {
      const int g = is_v ? h - Hq - Hkv : h - Hq;
      uint16_t* kv_out = is_v ? v_out : k_out;
      if (kv_out) {
        uint16_t* dst = kv_out + ((size_t)b * Hkv + g) * kHeadDim;
        dst[lane] = f32_to_bf16(x0);
        dst[lane + 64] = f32_to_bf16(x1);
      }
      if (phys >= 0 && k_pool) {
        uint16_t* pool = is_v ? v_pool : k_pool;
        uint16_t* dst = pool + (((size_t)phys * Hkv + g) * block_size + off) * kHeadDim;
        dst[lane] = f32_to_bf16(x0);
        dst[lane + 64] = f32_to_bf16(x1);
      }
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
//   All K loads of the wave are issued before the first use, and all V loads right after the
//   scores (the softmax statistics are reduced while they arrive).
// Each split writes its unnormalised output and (max, sum) in the log2 domain for the merge
// kernel; a sequence with a single split writes its normalised output directly. (Merging in the
// last split to finish would need a device-scope release per workgroup; on this chip that
// writes back the XCD's L2 each time and costs more than the separate merge launch.)
// Inputs of the fused decode step: q, k and v of the new token come packed in qkv [B, Hq+2Hkv,
// 128] (bf16) and go through QK-norm and RoPE inside the attention kernel.
struct FusedQKV {
  const uint16_t* qkv;
  const uint16_t* qn_w;  // null: no QK-norm
  const uint16_t* kn_w;
  const float* rope_cs;  // [max_pos, rd] = [cos | sin]
  int max_pos;
  int rd;
  float eps;
};

// Max / sum over the 16 lanes of each row of the wave (DPP: xor 1, xor 2, half-mirror, mirror;
// every lane of the row ends with the row's value).
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_row<0xB1>(v));
  v = fmaxf(v, dpp_row<0x4E>(v));
  v = fmaxf(v, dpp_row<0x141>(v));
  return fmaxf(v, dpp_row<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_row<0xB1>(v);
  v += dpp_row<0x4E>(v);
  v += dpp_row<0x141>(v);
  return v + dpp_row<0x140>(v);
}

// Live workgroups first. With compact set, the workgroup with linear id L (x fastest over the
// grid (splits, Hkv, B)) takes kv head L % Hkv and item L / Hkv, where sequence b owns
// max(ceil(ctx_b / S), 1) consecutive items in sequence order (one for a sequence with nothing
// cached, which writes the zero output): the workgroups of absent splits all come after the
// live ones in dispatch order instead of between them. Lane l reads the positions of sequences
// 4l .. 4l + 3 (B <= 256); a prefix scan over the lanes and a ballot find the item's sequence.
// Returns false past the last item. Results are wave-uniform.
__device__ __forceinline__ bool decode_item(const int32_t* __restrict__ positions, int B,
                                            int max_context, int S, int Hkv, int& split, int& g,
                                            int& b) {
  const int L = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  g = L % Hkv;
  const int item = L / Hkv;
  const int lane = threadIdx.x & 63;
  int cnt[4], pre[4], run = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int sq = lane * 4 + i;
    int c = 0;
    if (sq < B) {
      const int ctx = min(positions[sq] + 1, max_context);
      c = ctx <= 0 ? 1 : (ctx + S - 1) / S;
    }
    cnt[i] = c;
    pre[i] = run;
    run += c;
  }
  int x = run;  // inclusive scan over the lanes
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (item >= __shfl(x, 63)) return false;
  const int excl = x - run;
  const int l = __ffsll((long long)__ballot(item >= excl && item < x)) - 1;
  int bb = 0, sp = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int st = __shfl(excl + pre[i], l);
    const int c = __shfl(cnt[i], l);
    if (item >= st && item < st + c) {
      bb = l * 4 + i;
      sp = item - st;
    }
  }
  b = __builtin_amdgcn_readfirstlane(bb);
  split = __builtin_amdgcn_readfirstlane(sp);
  return true;
}

template <int G, int TPW, bool FUSED>
__global__ __launch_bounds__(kAttnThreads, kBf16MinBlocks) void paged_decode_kernel(
    const uint16_t* __restrict__ q, FusedQKV fq, uint16_t* __restrict__ k_pool,
    uint16_t* __restrict__ v_pool, const int32_t* __restrict__ block_tables,
    const int32_t* __restrict__ positions, int Hkv, int block_size, int mbps, int num_blocks,
    int max_context, float scale_log2, float* __restrict__ ws_o, float* __restrict__ ws_ml,
    int max_splits, uint16_t* __restrict__ out, int compact) {
  constexpr int D = kHeadDim;
  constexpr int SPLIT = 4 * TPW;   // tokens per workgroup
  constexpr int KT = TPW / 16;     // 16-token MFMA tiles per wave
  constexpr int VS = TPW / 4;      // P.V steps per wave (4 tokens per step)
  __shared__ __align__(16) uint16_t s_q[FUSED ? G : 1][D];     // normalised, rotated q heads
  __shared__ __align__(16) uint16_t s_new[FUSED ? 2 : 1][D];   // new token's k and v
  __shared__ float s_p[G][SPLIT];
  __shared__ float s_red[4][G][D];
  __shared__ float s_stat[2][G][4];  // each wave's max and sum of its tokens, per head
  __shared__ unsigned s_row[SPLIT];  // K/V pool row of each token (always an in-bounds row)
  __shared__ int s_ok[SPLIT];        // token is inside the split and its page-table entry is valid

  int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  if (compact && !decode_item(positions, gridDim.z, max_context, SPLIT, Hkv, split, g, b)) return;
  const int Hq = Hkv * G;
  const int tid = threadIdx.x;
  const int pos = positions[b];
  const int ctx = min(pos + 1, max_context);
  if (ctx <= 0) {
    // nothing cached (position < 0): the output is zero
    if (split == 0)
      for (int i = tid; i < G * D; i += kAttnThreads)
        out[((size_t)b * Hq + g * G) * D + i] = 0;
    return;
  }
  const int t0 = split * SPLIT;
  if (t0 >= ctx) return;
  const int t1 = min(ctx, t0 + SPLIT);
  const int nsplit = (ctx + SPLIT - 1) / SPLIT;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int kg = lane >> 4;

  // Fused step: this wave's heads of the new token (q heads g*G .. g*G+G-1 and, in the
  // workgroup of the sequence's last split, k and v of kv head g). Their qkv rows are loaded
  // first, so that waiting for them later does not wait for the K/V rows issued after them.
  constexpr int JPW = FUSED ? (G + 2 + 3) / 4 : 1;  // head jobs per wave
  const bool writer = FUSED && split == (ctx - 1) / SPLIT;
  const int n_jobs = writer ? G + 2 : G;
  float hx[JPW][2];
  float wq[2] = {1.f, 1.f}, wk[2] = {1.f, 1.f};
  RopeLane rl{1.f, 0.f, 1.f, 0.f};
  const bool rope = FUSED && pos < fq.max_pos;
  if constexpr (FUSED) {
    const int nh = Hq + 2 * Hkv;
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) {
      const int job = min(wave + 4 * jj, n_jobs - 1);
      const int h = job < G ? g * G + job : (job == G ? Hq + g : Hq + Hkv + g);
      const uint16_t* src = fq.qkv + ((size_t)b * nh + h) * D;
      hx[jj][0] = bf16_to_f32(src[lane]);
      hx[jj][1] = bf16_to_f32(src[lane + 64]);
    }
    const uint16_t* qw = fq.qn_w ? fq.qn_w : kOnesBf16;
    const uint16_t* kw = fq.qn_w ? fq.kn_w : kOnesBf16;
    wq[0] = bf16_to_f32(qw[lane]);
    wq[1] = bf16_to_f32(qw[lane + 64]);
    wk[0] = bf16_to_f32(kw[lane]);
    wk[1] = bf16_to_f32(kw[lane + 64]);
    rl = load_rope_lane_nobranch(rope ? fq.rope_cs + (size_t)pos * fq.rd : kZeroRope, fq.rd,
                                 lane);
  }
  if (tid < SPLIT) {
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
  // query fragments (A operand) of the plain kernel: head r16 (rows >= G are zero), dims
  // 8*kg + 32*j
  uint4 qa[4];
  if constexpr (!FUSED) {
    const uint16_t* qr = q + ((size_t)b * Hq + g * G + min(r16, G - 1)) * D + 8 * kg;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 32 * j);
      qa[j] = r16 < G ? v : make_uint4(0, 0, 0, 0);
    }
  }
  if constexpr (FUSED) {
    // the head rows and norm/RoPE operands arrive with the page table (one round trip), before
    // the K/V loads are issued
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) asm volatile("" ::"v"(hx[jj][0]), "v"(hx[jj][1]));
    asm volatile("" ::"v"(wq[0]), "v"(wq[1]), "v"(wk[0]), "v"(wk[1]), "v"(rl.c0), "v"(rl.s0),
                 "v"(rl.c1), "v"(rl.s1));
  }
  __syncthreads();

  const int wt0 = wave * TPW;  // this wave's first token in the split
  auto row_offset = [&](int tl) -> size_t { return (size_t)s_row[tl] * D; };
  // K in the MFMA B layout: tile tt of 16 tokens, token r16, dims 8*kg + 32*j
  uint4 kb[KT][4];
#pragma unroll
  for (int tt = 0; tt < KT; ++tt) {
    const uint16_t* kr = k_pool + row_offset(wt0 + tt * 16 + r16) + 8 * kg;
#pragma unroll
    for (int j = 0; j < 4; ++j) kb[tt][j] = *reinterpret_cast<const uint4*>(kr + 32 * j);
  }
  // V for P.V, in flight together with K: step it covers tokens it*4 + kg (4 per step), lane r16
  // owns dims r16*8 .. +8 (the new token's row, on the writer, is substituted where V is used)
  uint4 vreg[VS];
  if constexpr (FUSED) {
    // QK-norm + RoPE of this wave's heads (K loads in flight), into LDS; the writer also
    // stores k and v into the pool slot of the new token
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) {
      const int job = wave + 4 * jj;
      if (job < n_jobs) {
        float x0 = hx[jj][0], x1 = hx[jj][1];
        if (job <= G)
          qk_norm_rope(x0, x1, fq.qn_w != nullptr, job < G ? wq[0] : wk[0],
                       job < G ? wq[1] : wk[1], fq.eps, rope, rl, fq.rd, lane);
        const uint16_t y0 = f32_to_bf16(x0), y1 = f32_to_bf16(x1);
        uint16_t* dst = job < G ? s_q[job] : s_new[job - G];
        dst[lane] = y0;
        dst[lane + 64] = y1;
        if (job >= G) {
          int off = 0;
          const int phys = slot_block(block_tables, b, pos, mbps, block_size, num_blocks, &off);
          if (phys >= 0) {
            uint16_t* pool = job == G ? k_pool : v_pool;
            uint16_t* pd = pool + (((size_t)phys * Hkv + g) * block_size + off) * D;
            pd[lane] = y0;
            pd[lane + 64] = y1;
          }
        }
      }
    }
    __syncthreads();
    const uint16_t* qr = &s_q[min(r16, G - 1)][8 * kg];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 32 * j);
      qa[j] = r16 < G ? v : make_uint4(0, 0, 0, 0);
    }
  }
  // the new token's rows come from LDS (the pool slot is being written by this workgroup)
  const bool patch_new = FUSED && writer && pos < t1;
  if (patch_new) {
    const int tn = pos - t0;
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
      if (wt0 + tt * 16 + r16 == tn)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          kb[tt][j] = *reinterpret_cast<const uint4*>(&s_new[0][8 * kg + 32 * j]);
  }

  // ---- scores on MFMA: lane (kg, r16) holds heads 4 kg + i of token wt0 + 16 tt + r16 ----
  float sc[KT][4];
#pragma unroll
  for (int tt = 0; tt < KT; ++tt) {
    floatx4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) sacc = mfma16x16x32(qa[j], kb[tt][j], sacc);
    const bool valid = s_ok[wt0 + tt * 16 + r16] != 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[tt][i] = valid ? sacc[i] * scale_log2 : -INFINITY;
  }
#pragma unroll
  for (int it = 0; it < VS; ++it)
    vreg[it] = *reinterpret_cast<const uint4*>(v_pool + row_offset(wt0 + it * 4 + kg) + r16 * 8);
  const int tn = patch_new ? pos - t0 : -1;
  const uint4 v_new = patch_new ? *reinterpret_cast<const uint4*>(&s_new[1][r16 * 8])
                                : make_uint4(0u, 0u, 0u, 0u);

  // ---- softmax of this wave's tokens (log2 domain, relative to the wave's own maximum), in
  // the score layout: each row of 16 lanes reduces its heads over its tokens with DPP. The
  // probabilities go to s_p for the P.V operand; s_p is written and read by this wave only (LDS
  // operations of a wave complete in order), so no workgroup barrier: the four waves' (max, sum)
  // pairs are combined once, after P.V. ----
  float mrow[4], lrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float m = sc[0][i];
#pragma unroll
    for (int tt = 1; tt < KT; ++tt) m = fmaxf(m, sc[tt][i]);
    mrow[i] = row16_max(m);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float l = 0.f;
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) {
      const float v = sc[tt][i];
      const float pr = (mrow[i] == -INFINITY || v == -INFINITY) ? 0.f : fast_exp2(v - mrow[i]);
      sc[tt][i] = pr;
      l += pr;
    }
    lrow[i] = row16_sum(l);
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int tt = 0; tt < KT; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kg + i;
      if (h < G) s_p[h][wt0 + tt * 16 + r16] = sc[tt][i];
    }
  asm volatile("" ::: "memory");
  // head h's statistics live in lane 16 * (h / 4) (row h / 4, slot h % 4)
  float mw[G], lw[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    mw[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mrow[h % 4]), 16 * (h / 4)));
    lw[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lrow[h % 4]), 16 * (h / 4)));
  }

  // ---- P.V on MFMA ----
  // k-step ks covers steps it = 8 ks .. 8 ks + 7: lane group kg holds tokens wt0 + 4 it + kg, lane
  // r16 dims r16*8 .. +7 of each (vreg[it]). The MFMA's k and n orders only have to agree between
  // its operands, so MFMA c of the step takes, as column n = r16, dim r16*8 + c: B = element c of
  // the lane's 8 tokens (v_perm of the 16-bit halves, it ascending), A = P of the same 8 tokens
  // for head r16 (rows >= G zero). Lane (kg, r16) then holds rows 4 kg + i (heads) of the dims
  // r16*8 + c in acc[c][i]: the layout the VALU version had after reducing over kg.
  floatx4 pacc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) pacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < VS / 8; ++ks) {
    float pf[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) pf[m] = s_p[min(r16, G - 1)][wt0 + 4 * (8 * ks + m) + kg];
    uint4 pa = make_uint4(pack_bf16x2(pf[0], pf[1]), pack_bf16x2(pf[2], pf[3]),
                          pack_bf16x2(pf[4], pf[5]), pack_bf16x2(pf[6], pf[7]));
    if (r16 >= G) pa = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      // 16-bit element c of vreg[it] is half c % 2 of word c / 2
      const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
      const uint4* v0 = &vreg[8 * ks];
      auto word = [&](int m) -> uint32_t {
        const uint4 x = wt0 + 4 * (8 * ks + m) + kg == tn ? v_new : v0[m];
        return (c >> 1) == 0 ? x.x : (c >> 1) == 1 ? x.y : (c >> 1) == 2 ? x.z : x.w;
      };
      const uint4 vb = make_uint4(__builtin_amdgcn_perm(word(1), word(0), sel),
                                  __builtin_amdgcn_perm(word(3), word(2), sel),
                                  __builtin_amdgcn_perm(word(5), word(4), sel),
                                  __builtin_amdgcn_perm(word(7), word(6), sel));
      pacc[c] = mfma16x16x32(pa, vb, pacc[c]);
      // one operand built at a time (building them all first needs 32 more registers)
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kg + i;
      if (h < G) s_red[wave][h][r16 * 8 + c] = pacc[c][i];
    }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s_stat[0][h][wave] = mw[h];
      s_stat[1][h][wave] = lw[h];
    }
  }
  __syncthreads();

  // the split's maximum M over the waves' maxima and each wave's weight 2^(m_w - M) (0 for a
  // wave without a valid token), the split's sum, and its output for head h, dim d
  auto split_stats = [&](int h, float (&f)[4], float& M, float& L) {
    M = fmaxf(fmaxf(s_stat[0][h][0], s_stat[0][h][1]), fmaxf(s_stat[0][h][2], s_stat[0][h][3]));
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float m = s_stat[0][h][w];
      f[w] = m == -INFINITY ? 0.f : fast_exp2(m - M);
    }
    L = (f[0] * s_stat[1][h][0] + f[1] * s_stat[1][h][1]) +
        (f[2] * s_stat[1][h][2] + f[3] * s_stat[1][h][3]);
  };
  auto split_out = [&](int h, int d, const float (&f)[4]) {
    return (f[0] * s_red[0][h][d] + f[1] * s_red[1][h][d]) +
           (f[2] * s_red[2][h][d] + f[3] * s_red[3][h][d]);
  };

  if (nsplit == 1) {
    for (int i = tid; i < G * D; i += kAttnThreads) {
      const int h = i / D, d = i - h * D;
      float f[4], M, L;
      split_stats(h, f, M, L);
      const float o = split_out(h, d, f);
      out[((size_t)b * Hq + g * G + h) * D + d] = f32_to_bf16(L > 0.f ? o / L : 0.f);
    }
    return;
  }

  // this split's unnormalised output and (max, sum); the merge kernel combines the splits
  for (int i = tid; i < G * D; i += kAttnThreads) {
    const int h = i / D, d = i - h * D;
    float f[4], M, L;
    split_stats(h, f, M, L);
    ws_o[(((size_t)b * Hq + g * G + h) * max_splits + split) * D + d] = split_out(h, d, f);
  }
  if (tid < G) {
    float f[4], M, L;
    split_stats(tid, f, M, L);
    float* ml = ws_ml + (((size_t)b * Hq + g * G + tid) * max_splits + split) * 2;
    ml[0] = M;
    ml[1] = L;
  }
}

// Merge of the splits of a sequence with more than one split (log-sum-exp rule), one wave per
// (sequence, query head): lane l owns dims 2l, 2l+1; the split weights 2^(m_s - M) are computed
// one split per lane and broadcast. The partial outputs of the first kMergeBatch splits do not
// depend on the weights: they are loaded together with the (max, sum) pairs, right after the
// sequence length, so that a merge of up to kMergeBatch splits waits for two round trips.
__global__ __launch_bounds__(64) void paged_decode_merge_kernel(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    const int32_t* __restrict__ positions, int B, int Hq, int max_context, int max_splits,
    int split_tokens, uint16_t* __restrict__ out) {
  constexpr int D = kHeadDim;
  const int lane = threadIdx.x & 63;
  const int idx = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);  // b * Hq + head
  if (idx >= B * Hq) return;
  const int ctx = min(positions[idx / Hq] + 1, max_context);
  const int nsplit = ctx <= 0 ? 0 : (ctx + split_tokens - 1) / split_tokens;
  if (nsplit <= 1) return;  // written directly by the split kernel
  const float2* ml = reinterpret_cast<const float2*>(ws_ml) + (size_t)idx * max_splits;
  const float2* po = reinterpret_cast<const float2*>(ws_o) + (size_t)idx * max_splits * (D / 2) + lane;
  constexpr int kMergeBatch = 32;
  const float2 ml0 = ml[min(lane, nsplit - 1)];  // split `lane`'s (max, sum) (lane < nsplit)
  float2 pv0[kMergeBatch];  // splits past nsplit repeat the last one (in bounds, not used)
#pragma unroll
  for (int u = 0; u < kMergeBatch; ++u) pv0[u] = po[(size_t)min(u, nsplit - 1) * (D / 2)];
  float M = lane < nsplit ? ml0.x : -INFINITY;
  for (int s = lane + 64; s < nsplit; s += 64) M = fmaxf(M, ml[s].x);
  M = wave_max(M);
  float L = 0.f, ox = 0.f, oy = 0.f;
  for (int c = 0; c < nsplit; c += 64) {
    float w = 0.f;
    if (c + lane < nsplit) {
      const float2 v = c == 0 ? ml0 : ml[c + lane];
      w = (v.x == -INFINITY) ? 0.f : fast_exp2(v.x - M);
      L = fmaf(w, v.y, L);
    }
    const int n = min(64, nsplit - c);
    int j = 0;
    if (c == 0) {
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const float wj = __shfl(w, u);
        if (u < n) {
          ox = fmaf(wj, pv0[u].x, ox);
          oy = fmaf(wj, pv0[u].y, oy);
        }
      }
      j = min(n, kMergeBatch);
    }
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

// ---------------------------------------------------------------------------------------------
// fp8 e4m3fn KV cache: K pool [num_blocks, Hkv, block_size, 128] and V pool
// [num_blocks, Hkv, 128, block_size] of e4m3fn bytes (V dim-major inside each (block, head):
// the bytes of one dim for consecutive slots are contiguous, which is the layout of the P.V
// MFMA operand), and one fp32 scale per (block, kv head), scales [num_blocks, Hkv]; a stored
// value is byte value * scale. block_size is a multiple of 8 that divides 256.
// Scales are powers of two. Appending tokens to a block (prefill fill or the decode write):
//   s_new = max(s_old, pow2_ceil(amax(new tokens) / 448))     (s_old = 0 for an empty block)
//   if the block already holds tokens and s_new > s_old, each of their bytes c becomes
//   e4m3(value(c) * (s_old / s_new)) (an exact exponent shift except where a value turns
//   subnormal); the new tokens are e4m3(x / s_new) with x their bf16 values.
// So no value is ever clamped, and the scale of a block is fixed once the block is full.

__device__ __forceinline__ float pow2_ceil_f32(float y) {
  if (y == 0.f) return 0.f;
  if (y < 1.17549435e-38f) return 1.17549435e-38f;  // 2^-126
  const uint32_t b = __float_as_uint(y);
  if ((b & 0x7fffffu) == 0) return y;
  return __uint_as_float((b & 0x7f800000u) + 0x00800000u);
}

// value(c) * r for the 4 bytes of w, re-encoded (r <= 1: no clamp needed).
__device__ __forceinline__ uint32_t fp8x4_rescale(uint32_t w, float r) {
  const floatx2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
  const floatx2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
  return f32x4_to_fp8x4(lo.x * r, lo.y * r, hi.x * r, hi.y * r);
}

// value(c) * r for one byte c, re-encoded (r <= 1).
__device__ __forceinline__ uint8_t fp8_rescale1(uint8_t c, float r) {
  const floatx2 v = __builtin_amdgcn_cvt_pk_f32_fp8((uint32_t)c, false);
  return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(v.x * r, 0.f, 0, false) & 0xff);
}

// Byte mask of 8 flags: byte i (lo word bytes 0-3, hi word bytes 4-7) is 0xff when bit i of m
// is set. (m & 0xf) * 0x00204081 moves bit i to bit 8i (the other partial products land
// elsewhere), & 0x01010101 keeps those, * 0xff fills the bytes.
__device__ __forceinline__ uint2 byte_mask8(uint32_t m) {
  const uint32_t lo = (((m & 0xfu) * 0x00204081u) & 0x01010101u) * 0xffu;
  const uint32_t hi = ((((m >> 4) & 0xfu) * 0x00204081u) & 0x01010101u) * 0xffu;
  return make_uint2(lo, hi);
}

// Fill: grid (ceil(max_seqlen / block_size) + 1, Hkv, n_seqs), 256 threads; workgroup = the
// j-th block touched by sequence s for kv head g. Sequence s holds tokens cu[s] + i, i < L, at
// positions start[s] + i (start null: from 0), in page-table row s; the 128 bf16 dims of token
// t, head g start at element t * tok_stride + g * head_stride of k / v. Each (block, head) is
// owned by one workgroup.
__global__ __launch_bounds__(256) void paged_kv_fill_fp8_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, long long tok_stride,
    long long head_stride, const int32_t* __restrict__ cu_seqlens,
    const int32_t* __restrict__ start_pos, const int32_t* __restrict__ seq_rows, int n_rows,
    int Hkv, uint8_t* __restrict__ k_pool, uint8_t* __restrict__ v_pool,
    float* __restrict__ k_scale, float* __restrict__ v_scale,
    const int32_t* __restrict__ block_tables, int mbps, int block_size, int num_blocks) {
  __shared__ float s_amax[2][4];
  const int j = blockIdx.x, g = blockIdx.y, sq = blockIdx.z;
  const int c0 = cu_seqlens[sq];
  const int L = cu_seqlens[sq + 1] - c0;
  const int start = start_pos ? start_pos[sq] : 0;
  const int row = seq_rows ? seq_rows[sq] : sq;  // page-table row of the sequence
  if (L <= 0 || start < 0 || row < 0 || row >= n_rows) return;
  const int blk = start / block_size + j;
  const int p0 = max(start, blk * block_size);
  const int p1 = min(start + L, (blk + 1) * block_size);
  if (p0 >= p1 || blk >= mbps) return;
  const int phys = block_tables[(size_t)row * mbps + blk];
  if (phys < 0 || phys >= num_blocks) return;
  const int n_old = p0 - blk * block_size;
  const int n_new = p1 - p0;
  const int tid = threadIdx.x;
  const int nchunk = n_new * (kHeadDim / 8);  // 8 dims per chunk
  const size_t tok0 = (size_t)c0 + (p0 - start);
  auto src_off = [&](int c) -> size_t {
    return (tok0 + c / 16) * (size_t)tok_stride + (size_t)g * head_stride + (c % 16) * 8;
  };
  float ak = 0.f, av = 0.f;
  for (int c = tid; c < nchunk; c += 256) {
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(k + src_off(c)), f);
#pragma unroll
    for (int i = 0; i < 8; ++i) ak = fmaxf(ak, fabsf(f[i]));
    unpack8(*reinterpret_cast<const uint4*>(v + src_off(c)), f);
#pragma unroll
    for (int i = 0; i < 8; ++i) av = fmaxf(av, fabsf(f[i]));
  }
  ak = wave_max(ak);
  av = wave_max(av);
  if ((tid & 63) == 0) {
    s_amax[0][tid >> 6] = ak;
    s_amax[1][tid >> 6] = av;
  }
  const size_t sidx = (size_t)phys * Hkv + g;
  const float sk_old = n_old > 0 ? k_scale[sidx] : 0.f;
  const float sv_old = n_old > 0 ? v_scale[sidx] : 0.f;
  __syncthreads();
  ak = fmaxf(fmaxf(s_amax[0][0], s_amax[0][1]), fmaxf(s_amax[0][2], s_amax[0][3]));
  av = fmaxf(fmaxf(s_amax[1][0], s_amax[1][1]), fmaxf(s_amax[1][2], s_amax[1][3]));
  const float sk = fmaxf(sk_old, pow2_ceil_f32(ak / kFp8Max));
  const float sv = fmaxf(sv_old, pow2_ceil_f32(av / kFp8Max));
  uint8_t* kb = k_pool + sidx * block_size * kHeadDim;
  uint8_t* vb = v_pool + sidx * block_size * kHeadDim;
  // requantise the block's earlier tokens where the scale grew
  const int nw_old = n_old * (kHeadDim / 4);
  if (sk > sk_old && n_old > 0) {
    const float r = sk_old / sk;
    uint32_t* w = reinterpret_cast<uint32_t*>(kb);
    for (int i = tid; i < nw_old; i += 256) w[i] = fp8x4_rescale(w[i], r);
  }
  if (sv > sv_old && n_old > 0) {
    // V is dim-major: the earlier tokens are bytes [0, n_old) of each of the 128 dim rows
    const float r = sv_old / sv;
    for (int i = tid; i < n_old * kHeadDim; i += 256) {
      const int d = i / n_old, sl = i - d * n_old;
      uint8_t* pv = vb + (size_t)d * block_size + sl;
      *pv = fp8_rescale1(*pv, r);
    }
  }
  // the new tokens
  for (int c = tid; c < nchunk; c += 256) {
    const size_t dst = (size_t)(n_old + c / 16) * kHeadDim + (c % 16) * 8;
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(k + src_off(c)), f);
    uint2 q = make_uint2(0u, 0u);
    if (sk > 0.f) {
      q.x = f32x4_to_fp8x4(clamp_fp8(f[0] / sk), clamp_fp8(f[1] / sk), clamp_fp8(f[2] / sk),
                           clamp_fp8(f[3] / sk));
      q.y = f32x4_to_fp8x4(clamp_fp8(f[4] / sk), clamp_fp8(f[5] / sk), clamp_fp8(f[6] / sk),
                           clamp_fp8(f[7] / sk));
    }
    *reinterpret_cast<uint2*>(kb + dst) = q;
    unpack8(*reinterpret_cast<const uint4*>(v + src_off(c)), f);
    q = make_uint2(0u, 0u);
    if (sv > 0.f) {
      q.x = f32x4_to_fp8x4(clamp_fp8(f[0] / sv), clamp_fp8(f[1] / sv), clamp_fp8(f[2] / sv),
                           clamp_fp8(f[3] / sv));
      q.y = f32x4_to_fp8x4(clamp_fp8(f[4] / sv), clamp_fp8(f[5] / sv), clamp_fp8(f[6] / sv),
                           clamp_fp8(f[7] / sv));
    }
    // dim-major V: byte i of the chunk goes to dim (c % 16) * 8 + i, slot n_old + c / 16
    uint8_t* vd = vb + (size_t)((c % 16) * 8) * block_size + n_old + c / 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vd[(size_t)i * block_size] = (uint8_t)(q.x >> (8 * i));
      vd[(size_t)(i + 4) * block_size] = (uint8_t)(q.y >> (8 * i));
    }
  }
  if (tid == 0) {
    k_scale[sidx] = sk;
    v_scale[sidx] = sv;
  }
}

// The decode write of one head of the new token by one wave: x0 / x1 are dims lane / lane+64
// (bf16 values as floats); appended to (block phys, head g) at slot off by the rule above.
__device__ __forceinline__ void fp8_append_token(uint8_t* __restrict__ pool,
                                                 float* __restrict__ scales, int phys, int g,
                                                 int Hkv, int block_size, int off, float x0,
                                                 float x1, int lane, bool dim_major) {
  const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  const size_t sidx = (size_t)phys * Hkv + g;
  const float s_old = off > 0 ? scales[sidx] : 0.f;
  const float s_new = fmaxf(s_old, pow2_ceil_f32(amax / kFp8Max));
  uint8_t* blk = pool + sidx * block_size * kHeadDim;
  if (off > 0 && s_new > s_old) {
    const float r = s_old / s_new;
    if (dim_major) {
      // the earlier tokens are bytes [0, off) of each of the 128 dim rows
      for (int i = lane; i < off * kHeadDim; i += 64) {
        const int d = i / off, sl = i - d * off;
        uint8_t* p = blk + (size_t)d * block_size + sl;
        *p = fp8_rescale1(*p, r);
      }
    } else {
      uint32_t* w = reinterpret_cast<uint32_t*>(blk);
      for (int i = lane; i < off * (kHeadDim / 4); i += 64) w[i] = fp8x4_rescale(w[i], r);
    }
  }
  uint32_t q = 0;
  if (s_new > 0.f)
    q = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clamp_fp8(x0 / s_new), clamp_fp8(x1 / s_new),
                                                  0, false);
  if (dim_major) {
    blk[(size_t)lane * block_size + off] = (uint8_t)(q & 0xffu);
    blk[(size_t)(lane + 64) * block_size + off] = (uint8_t)((q >> 8) & 0xffu);
  } else {
    blk[(size_t)off * kHeadDim + lane] = (uint8_t)(q & 0xffu);
    blk[(size_t)off * kHeadDim + lane + 64] = (uint8_t)((q >> 8) & 0xffu);
  }
  if (lane == 0) scales[sidx] = s_new;
}

// Split-K decode over the fp8 cache, same workgroup shape and outputs as paged_decode_kernel.
//   K in the MFMA B layout: lane l holds bytes [32*(l/16), +32) of token l%16 of a 16-token tile
//   (two 16-byte loads); MFMA j takes its bytes 8j .. 8j+7, converted exactly to bf16, against
//   the query dims 32*(l/16) + 8j .. +7 from LDS. P.V on MFMA too: per 32-token k-step the A
//   operand is P (query heads as rows, bf16, lanes of rows >= G zero) and the B operand of
//   column tile j is V dim-major: lane l takes the 8 bytes of dim 16j + l%16 for the tokens
//   8*(l/16) .. +7 of the k-step (one aligned 8-byte piece of a block's dim row), bytes of
//   tokens outside the sequence zeroed. A token's K scale multiplies its score and its V scale
//   its probability in P.V (the softmax sum uses the unscaled probability), so the dequantised
//   values are never formed. In the fused step the workgroup of the sequence's last split first appends the new
//   token's k and v to the pool (with any requantisation of its block), then reads the split
//   from the pool like every other workgroup; a block never straddles two splits (block_size
//   divides 256, and the split is a multiple of 256 tokens), so no other workgroup reads the
//   block being rewritten. A thread owns split / 256 tokens in the softmax.
template <int G, bool FUSED>
__global__ __launch_bounds__(kAttnThreads, G >= 8 ? 1 : kFp8MinBlocks) void paged_decode_fp8_kernel(
    const uint16_t* __restrict__ q, FusedQKV fq, uint8_t* __restrict__ k_pool,
    uint8_t* __restrict__ v_pool, float* __restrict__ k_scale, float* __restrict__ v_scale,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ positions, int Hkv,
    int block_size, int mbps, int num_blocks, int max_context, float scale_log2,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, int max_splits,
    uint16_t* __restrict__ out, int compact) {
  constexpr int D = kHeadDim;
  constexpr int TPW = kTPW8;
  constexpr int SPLIT = kSplit8;
  constexpr int KT = TPW / 16;                 // 16-token K tiles per wave
  constexpr int TPT = SPLIT / kAttnThreads;    // tokens per thread in the softmax
  __shared__ __align__(16) uint16_t s_q[G][D];
  __shared__ __align__(16) float s_p[G][SPLIT];
  __shared__ float s_red[4][G][D];
  __shared__ float s_stat[2][G][4];  // each wave's max and sum of its tokens, per head
  __shared__ unsigned s_row[SPLIT];

  int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  if (compact && !decode_item(positions, gridDim.z, max_context, SPLIT, Hkv, split, g, b)) return;
  const int Hq = Hkv * G;
  const int tid = threadIdx.x;
  const int pos = positions[b];
  const int ctx = min(pos + 1, max_context);
  if (ctx <= 0) {
    if (split == 0)
      for (int i = tid; i < G * D; i += kAttnThreads)
        out[((size_t)b * Hq + g * G) * D + i] = 0;
    return;
  }
  const int t0 = split * SPLIT;
  if (t0 >= ctx) return;
  const int t1 = min(ctx, t0 + SPLIT);
  const int nsplit = (ctx + SPLIT - 1) / SPLIT;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int kg = lane >> 4;

  constexpr int JPW = FUSED ? (G + 2 + 3) / 4 : 1;
  const bool writer = FUSED && split == (ctx - 1) / SPLIT;
  const int n_jobs = writer ? G + 2 : G;
  float hx[JPW][2];
  float wq[2] = {1.f, 1.f}, wk[2] = {1.f, 1.f};
  RopeLane rl{1.f, 0.f, 1.f, 0.f};
  const bool rope = FUSED && pos < fq.max_pos;
  if constexpr (FUSED) {
    const int nh = Hq + 2 * Hkv;
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) {
      const int job = min(wave + 4 * jj, n_jobs - 1);
      const int h = job < G ? g * G + job : (job == G ? Hq + g : Hq + Hkv + g);
      const uint16_t* src = fq.qkv + ((size_t)b * nh + h) * D;
      hx[jj][0] = bf16_to_f32(src[lane]);
      hx[jj][1] = bf16_to_f32(src[lane + 64]);
    }
    const uint16_t* qw = fq.qn_w ? fq.qn_w : kOnesBf16;
    const uint16_t* kw = fq.qn_w ? fq.kn_w : kOnesBf16;
    wq[0] = bf16_to_f32(qw[lane]);
    wq[1] = bf16_to_f32(qw[lane + 64]);
    wk[0] = bf16_to_f32(kw[lane]);
    wk[1] = bf16_to_f32(kw[lane + 64]);
    rl = load_rope_lane_nobranch(rope ? fq.rope_cs + (size_t)pos * fq.rd : kZeroRope, fq.rd,
                                 lane);
  } else {
    if (tid < G * 16) {
      const int h = tid >> 4, c = tid & 15;
      *reinterpret_cast<uint4*>(&s_q[h][c * 8]) = *reinterpret_cast<const uint4*>(
          q + ((size_t)b * Hq + g * G + h) * D + c * 8);
    }
  }
  // tokens t0 + tid + 256 j of the split: their pool rows (always in bounds) and validity
  bool my_ok[TPT];
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    const int tl = tid + kAttnThreads * j;
    const int t = t0 + tl;
    const int tc = min(t, t1 - 1);
    const int blk = tc / block_size;
    int pb = blk < mbps ? block_tables[(size_t)b * mbps + blk] : -1;
    my_ok[j] = t < t1 && pb >= 0 && pb < num_blocks;
    if (pb < 0 || pb >= num_blocks) pb = 0;
    s_row[tl] = (unsigned)(((size_t)pb * Hkv + g) * block_size + (tc - blk * block_size));
  }
  const unsigned long long okw = __ballot(my_ok[0]);  // validity of this wave's 64 tokens
  if constexpr (FUSED) {
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) asm volatile("" ::"v"(hx[jj][0]), "v"(hx[jj][1]));
    asm volatile("" ::"v"(wq[0]), "v"(wq[1]), "v"(wk[0]), "v"(wk[1]), "v"(rl.c0), "v"(rl.s0),
                 "v"(rl.c1), "v"(rl.s1));
  }
  __syncthreads();

  const int wt0 = wave * TPW;
  uint4 kb[KT][2];
  // P.V operands: k-step ks covers tokens wt0 + 32 ks .. +31; lane l's 8 tokens start at
  // wt0 + 32 ks + 8 kg, all in one block (block_size % 8 == 0, aligned). A group past the
  // sequence reads the aligned piece of the split's last token (its row in s_row), in bounds.
  static_assert(TPW == 64 && TPT == 1, "P.V MFMA tiling assumes 64 tokens per wave");
  constexpr int KS = TPW / 32;
  uint2 vreg[KS][D / 16];
  // K and V scales of the tokens wt0 + 16 tt + r16 this lane holds scores of: the scale index
  // (block, head) is the pool row / block_size (a power of two)
  const int bs_log2 = 31 - __clz(block_size);
  float ksc[KT], vsc[KT];
  auto load_v = [&]() {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const unsigned row = s_row[wt0 + 32 * ks + 8 * kg];
      const unsigned o = row & (unsigned)(block_size - 1);
      const uint8_t* vb = v_pool + (size_t)(row - o) * D + (o & ~7u) + (size_t)r16 * block_size;
#pragma unroll
      for (int j = 0; j < D / 16; ++j)
        vreg[ks][j] = *reinterpret_cast<const uint2*>(vb + (size_t)(16 * j) * block_size);
    }
  };
  auto issue_loads = [&]() {
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) {
      const unsigned row = s_row[wt0 + tt * 16 + r16];
      const uint8_t* kr = k_pool + (size_t)row * D + 32 * kg;
      kb[tt][0] = *reinterpret_cast<const uint4*>(kr);
      kb[tt][1] = *reinterpret_cast<const uint4*>(kr + 16);
      ksc[tt] = k_scale[row >> bs_log2];
      vsc[tt] = v_scale[row >> bs_log2];
    }
  };
  if (!writer) issue_loads();
  if constexpr (FUSED) {
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) {
      const int job = wave + 4 * jj;
      if (job < n_jobs) {
        float x0 = hx[jj][0], x1 = hx[jj][1];
        if (job <= G)
          qk_norm_rope(x0, x1, fq.qn_w != nullptr, job < G ? wq[0] : wk[0],
                       job < G ? wq[1] : wk[1], fq.eps, rope, rl, fq.rd, lane);
        const uint16_t y0 = f32_to_bf16(x0), y1 = f32_to_bf16(x1);
        if (job < G) {
          s_q[job][lane] = y0;
          s_q[job][lane + 64] = y1;
        } else {
          int off = 0;
          const int phys = slot_block(block_tables, b, pos, mbps, block_size, num_blocks, &off);
          if (phys >= 0)
            fp8_append_token(job == G ? k_pool : v_pool, job == G ? k_scale : v_scale, phys, g,
                             Hkv, block_size, off, bf16_to_f32(y0), bf16_to_f32(y1), lane,
                             job != G);
        }
      }
    }
    // the appended token (and any requantised rows) are visible to the whole workgroup after
    // the barrier
    __syncthreads();
    if (writer) issue_loads();
  }
  uint4 qa[4];
  {
    const uint16_t* qr = &s_q[min(r16, G - 1)][32 * kg];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 8 * j);
      qa[j] = r16 < G ? v : make_uint4(0, 0, 0, 0);
    }
  }

  // ---- scores on MFMA: lane (kg, r16) holds heads 4 kg + i of token wt0 + 16 tt + r16 ----
  float sc[KT][4];
#pragma unroll
  for (int tt = 0; tt < KT; ++tt) {
    floatx4 sacc = {0.f, 0.f, 0.f, 0.f};
    sacc = mfma16x16x32(qa[0], fp8x8_to_bf16x8(kb[tt][0].x, kb[tt][0].y), sacc);
    sacc = mfma16x16x32(qa[1], fp8x8_to_bf16x8(kb[tt][0].z, kb[tt][0].w), sacc);
    sacc = mfma16x16x32(qa[2], fp8x8_to_bf16x8(kb[tt][1].x, kb[tt][1].y), sacc);
    sacc = mfma16x16x32(qa[3], fp8x8_to_bf16x8(kb[tt][1].z, kb[tt][1].w), sacc);
    const bool valid = (okw >> (tt * 16 + r16)) & 1ull;
    const float f = ksc[tt] * scale_log2;
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[tt][i] = valid ? sacc[i] * f : -INFINITY;
  }
  load_v();  // into the registers K used; arrives during the softmax

  // ---- softmax of this wave's tokens (log2 domain, relative to the wave's own maximum), in
  // the score layout: each row of 16 lanes reduces its heads over its tokens with DPP. P (times
  // the token's V scale) goes to s_p for the P.V operand; s_p is written and read by this wave
  // only (LDS operations of a wave complete in order), so no workgroup barrier: the four waves'
  // (max, sum) pairs are combined once, after P.V. ----
  float mrow[4], lrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float m = sc[0][i];
#pragma unroll
    for (int tt = 1; tt < KT; ++tt) m = fmaxf(m, sc[tt][i]);
    mrow[i] = row16_max(m);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float l = 0.f;
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) {
      const float v = sc[tt][i];
      const float pr = (mrow[i] == -INFINITY || v == -INFINITY) ? 0.f : fast_exp2(v - mrow[i]);
      sc[tt][i] = pr * vsc[tt];
      l += pr;
    }
    lrow[i] = row16_sum(l);
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int tt = 0; tt < KT; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kg + i;
      if (h < G) s_p[h][wt0 + tt * 16 + r16] = sc[tt][i];
    }
  asm volatile("" ::: "memory");
  // head h's statistics live in lane 16 * (h / 4) (row h / 4, slot h % 4)
  float mw[G], lw[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    mw[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mrow[h % 4]), 16 * (h / 4)));
    lw[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lrow[h % 4]), 16 * (h / 4)));
  }

  // ---- P.V on MFMA: O[head][dim] += P[head][token] . V[token][dim] per 32-token k-step ----
  floatx4 oacc[D / 16];
#pragma unroll
  for (int j = 0; j < D / 16; ++j) oacc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int tl0 = wt0 + 32 * ks + 8 * kg;
    // A: P of head r16 (P already carries the V scale) for the lane's 8 tokens, in bf16
    const float4 p0 = *reinterpret_cast<const float4*>(&s_p[min(r16, G - 1)][tl0]);
    const float4 p1 = *reinterpret_cast<const float4*>(&s_p[min(r16, G - 1)][tl0 + 4]);
    uint4 pa = make_uint4(pack_bf16x2(p0.x, p0.y), pack_bf16x2(p0.z, p0.w),
                          pack_bf16x2(p1.x, p1.y), pack_bf16x2(p1.z, p1.w));
    if (r16 >= G) pa = make_uint4(0u, 0u, 0u, 0u);
    // bytes of tokens outside the sequence (or of an invalid block) are zeroed: their P is 0,
    // and a slot never written may hold any byte
    const uint2 m = byte_mask8((uint32_t)(okw >> (32 * ks + 8 * kg)) & 0xffu);
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      const uint2 w = make_uint2(vreg[ks][j].x & m.x, vreg[ks][j].y & m.y);
      oacc[j] = mfma16x16x32(pa, fp8x8_to_bf16x8(w.x, w.y), oacc[j]);
    }
  }
  // lane l holds rows 4*(l/16) + i (heads) of column 16j + l%16
#pragma unroll
  for (int j = 0; j < D / 16; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kg + i;
      if (h < G) s_red[wave][h][16 * j + r16] = oacc[j][i];
    }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s_stat[0][h][wave] = mw[h];
      s_stat[1][h][wave] = lw[h];
    }
  }
  __syncthreads();

  // the split's maximum M over the waves' maxima and each wave's weight 2^(m_w - M) (0 for a
  // wave without a valid token), the split's sum, and its output for head h, dim d
  auto split_stats = [&](int h, float (&f)[4], float& M, float& L) {
    M = fmaxf(fmaxf(s_stat[0][h][0], s_stat[0][h][1]), fmaxf(s_stat[0][h][2], s_stat[0][h][3]));
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float m = s_stat[0][h][w];
      f[w] = m == -INFINITY ? 0.f : fast_exp2(m - M);
    }
    L = (f[0] * s_stat[1][h][0] + f[1] * s_stat[1][h][1]) +
        (f[2] * s_stat[1][h][2] + f[3] * s_stat[1][h][3]);
  };
  auto split_out = [&](int h, int d, const float (&f)[4]) {
    return (f[0] * s_red[0][h][d] + f[1] * s_red[1][h][d]) +
           (f[2] * s_red[2][h][d] + f[3] * s_red[3][h][d]);
  };

  if (nsplit == 1) {
    for (int i = tid; i < G * D; i += kAttnThreads) {
      const int h = i / D, d = i - h * D;
      float f[4], M, L;
      split_stats(h, f, M, L);
      const float o = split_out(h, d, f);
      out[((size_t)b * Hq + g * G + h) * D + d] = f32_to_bf16(L > 0.f ? o / L : 0.f);
    }
    return;
  }
  for (int i = tid; i < G * D; i += kAttnThreads) {
    const int h = i / D, d = i - h * D;
    float f[4], M, L;
    split_stats(h, f, M, L);
    ws_o[(((size_t)b * Hq + g * G + h) * max_splits + split) * D + d] = split_out(h, d, f);
  }
  if (tid < G) {
    float f[4], M, L;
    split_stats(tid, f, M, L);
    float* ml = ws_ml + (((size_t)b * Hq + g * G + tid) * max_splits + split) * 2;
    ml[0] = M;
    ml[1] = L;
  }
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
                     rope_cs, max_pos, positions, (const int32_t*)nullptr, Hq, Hkv, rotary_dim,
                     eps, use_qk_norm, (uint16_t*)q_out, (uint16_t*)nullptr, (uint16_t*)nullptr,
                     (uint16_t*)k_pool, (uint16_t*)v_pool, block_tables, max_blocks_per_seq,
                     block_size, num_blocks);
  return sym_host::check_launch("attn_decode_prologue_kernel");
}

extern "C" int sym_attn_prefill_prologue(const void* qkv, const void* q_norm_w,
                                         const void* k_norm_w, const float* rope_cs, int max_pos,
                                         const int32_t* positions, const int32_t* seq_ids, int T,
                                         int Hq, int Hkv, int head_dim, int rotary_dim, float eps,
                                         int use_qk_norm, void* q_out, void* k_out, void* v_out,
                                         void* k_pool, void* v_pool, const int32_t* block_tables,
                                         int max_blocks_per_seq, int block_size, int num_blocks,
                                         void* stream) {
  int rc = check_cache_args("attn_prefill_prologue", T, Hkv, head_dim, block_size,
                            max_blocks_per_seq, num_blocks);
  if (rc) return rc;
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(qkv && positions && seq_ids && q_out && k_out && v_out && block_tables,
              SYM_ERR_INVALID, "attn_prefill_prologue: null pointer argument");
  SYM_REQUIRE((k_pool == nullptr) == (v_pool == nullptr), SYM_ERR_INVALID,
              "attn_prefill_prologue: k_pool and v_pool must both be given or both be null");
  SYM_REQUIRE(Hq >= Hkv && Hq % Hkv == 0, SYM_ERR_INVALID,
              "attn_prefill_prologue: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  SYM_REQUIRE(rotary_dim >= 0 && rotary_dim <= head_dim && rotary_dim % 2 == 0, SYM_ERR_INVALID,
              "attn_prefill_prologue: rotary_dim=%d", rotary_dim);
  SYM_REQUIRE(rotary_dim == 0 || (rope_cs && max_pos > 0), SYM_ERR_INVALID,
              "attn_prefill_prologue: rope table missing");
  SYM_REQUIRE(!use_qk_norm || (q_norm_w && k_norm_w), SYM_ERR_INVALID,
              "attn_prefill_prologue: qk-norm weights missing");
  (void)hipGetLastError();
  hipLaunchKernelGGL(attn_decode_prologue_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)qkv, (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w,
                     rope_cs, max_pos, positions, seq_ids, Hq, Hkv, rotary_dim, eps, use_qk_norm,
                     (uint16_t*)q_out, (uint16_t*)k_out, (uint16_t*)v_out, (uint16_t*)k_pool,
                     (uint16_t*)v_pool, block_tables, max_blocks_per_seq, block_size, num_blocks);
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

// Argument checks and launch of the split kernel (plain or fused with the prologue) and the
// merge kernel.
// k_scale / v_scale non-null: the pools are fp8 e4m3fn with per-(block, head) scales.
static int launch_decode(const char* what, const void* q, const FusedQKV* fq, void* k_pool,
                         void* v_pool, float* k_scale, float* v_scale,
                         const int32_t* block_tables, const int32_t* positions, int B, int Hq,
                         int Hkv, int head_dim, int block_size, int max_blocks_per_seq,
                         int num_blocks, int max_context, float scale, void* workspace,
                         size_t workspace_bytes, void* out, void* stream) {
  int rc = check_cache_args(what, B, Hkv, head_dim, block_size, max_blocks_per_seq, num_blocks);
  if (rc) return rc;
  if (B == 0) return SYM_OK;
  SYM_REQUIRE((q || fq) && k_pool && v_pool && block_tables && positions && workspace && out,
              SYM_ERR_INVALID, "%s: null pointer argument", what);
  const bool fp8 = k_scale != nullptr;
  SYM_REQUIRE(fp8 == (v_scale != nullptr), SYM_ERR_INVALID, "%s: k_scale and v_scale", what);
  SYM_REQUIRE(!fp8 || (kSplit8 % block_size == 0 && block_size % 8 == 0), SYM_ERR_UNSUPPORTED,
              "%s: fp8 cache needs block_size a multiple of 8 dividing %d (got %d)", what, kSplit8,
              block_size);
  SYM_REQUIRE(Hq >= Hkv && Hq % Hkv == 0, SYM_ERR_INVALID, "%s: Hq=%d not a multiple of Hkv=%d",
              what, Hq, Hkv);
  const int G = Hq / Hkv;
  SYM_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, SYM_ERR_UNSUPPORTED,
              "%s: group size %d not in {1,2,4,8}", what, G);
  SYM_REQUIRE(max_context >= 1 && (long long)max_context <= (long long)max_blocks_per_seq * block_size,
              SYM_ERR_INVALID, "%s: max_context=%d outside (0, %d]", what, max_context,
              max_blocks_per_seq * block_size);
  SYM_REQUIRE(B <= 65535 && Hkv <= 65535, SYM_ERR_INVALID, "%s: grid too large", what);
  const size_t need = sym_paged_gqa_decode_workspace_bytes(B, Hq, head_dim, max_context);
  SYM_REQUIRE(workspace_bytes >= need, SYM_ERR_WORKSPACE, "%s: workspace %zu < required %zu",
              what, workspace_bytes, need);
  const int split_tokens = fp8 ? kSplit8 : kSplit;
  const int max_splits = (max_context + split_tokens - 1) / split_tokens;
  float* ws_o = (float*)workspace;
  float* ws_ml = ws_o + (size_t)B * Hq * max_splits * head_dim;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  // Workgroups are spread over the XCDs and their shader engines in linear-id order, so a split
  // dimension that is a multiple of 32 puts split s of every (kv head, sequence) row on the same
  // XCD / engine slot: the low splits (present in every sequence) pile onto a quarter of the
  // CUs while the high ones (mostly past the end) leave others idle. An odd width rotates the
  // mapping from row to row; the extra split starts at or past max_context and exits at once.
  // (fp8 batch 128, 1024-8192 tokens: 32 -> 33 splits, 153 -> 123 us.)
  const dim3 grid(max_splits | 1, Hkv, B), block(kAttnThreads);
  // live workgroups first in dispatch order (decode_item), for the bf16 cache up to 32
  // sequences: batch 32 with 128-4096 cached tokens (about one round of workgroups), split kernel
  // 26.6-26.7 against 27.6-27.7 us. With several rounds the odd-width grid order is faster: the
  // whole model at batch 64 with 2048-2176 tokens, 6.63-6.64 against 6.67 ms per step; the fp8
  // cache's batch 128 with 1024-8192 tokens, 115.3-116.5 against 120.6-120.9 us.
  const int compact = !fp8 && B <= 32 ? 1 : 0;
  const uint16_t* qq = (const uint16_t*)q;
  uint16_t* kp = (uint16_t*)k_pool;
  uint16_t* vp = (uint16_t*)v_pool;
  const FusedQKV f = fq ? *fq : FusedQKV{};
  uint8_t* kp8 = (uint8_t*)k_pool;
  uint8_t* vp8 = (uint8_t*)v_pool;
#define SYM_LAUNCH_DECODE(GG, FF)                                                               \
  if (fp8)                                                                                      \
    hipLaunchKernelGGL((paged_decode_fp8_kernel<GG, FF>), grid, block, 0, s, qq, f, kp8, vp8,   \
                       k_scale, v_scale, block_tables, positions, Hkv, block_size,              \
                       max_blocks_per_seq, num_blocks, max_context, scale_log2, ws_o, ws_ml,    \
                       max_splits, (uint16_t*)out, compact);                                    \
  else                                                                                          \
    hipLaunchKernelGGL((paged_decode_kernel<GG, kTPW, FF>), grid, block, 0, s, qq, f, kp, vp,   \
                       block_tables, positions, Hkv, block_size, max_blocks_per_seq,            \
                       num_blocks, max_context, scale_log2, ws_o, ws_ml, max_splits,            \
                       (uint16_t*)out, compact)
#define SYM_LAUNCH_DECODE_G(FF)               \
  switch (G) {                                \
    case 1: SYM_LAUNCH_DECODE(1, FF); break;  \
    case 2: SYM_LAUNCH_DECODE(2, FF); break;  \
    case 4: SYM_LAUNCH_DECODE(4, FF); break;  \
    default: SYM_LAUNCH_DECODE(8, FF); break; \
  }
  if (fq) {
    SYM_LAUNCH_DECODE_G(true);
  } else {
    SYM_LAUNCH_DECODE_G(false);
  }
#undef SYM_LAUNCH_DECODE_G
#undef SYM_LAUNCH_DECODE
  rc = sym_host::check_launch(fp8 ? "paged_decode_fp8_kernel" : "paged_decode_kernel");
  if (rc || max_splits == 1) return rc;
  // one wave per workgroup: the (sequence, head) merges spread over as many CUs as possible
  hipLaunchKernelGGL(paged_decode_merge_kernel, dim3(B * Hq), dim3(64), 0, s, ws_o, ws_ml,
                     positions, B, Hq, max_context, max_splits, split_tokens, (uint16_t*)out);
  return sym_host::check_launch("paged_decode_merge_kernel");
}

extern "C" int sym_paged_gqa_decode(const void* q, const void* k_pool, const void* v_pool,
                                    const int32_t* block_tables, const int32_t* positions, int B,
                                    int Hq, int Hkv, int head_dim, int block_size,
                                    int max_blocks_per_seq, int num_blocks, int max_context,
                                    float scale, void* workspace, size_t workspace_bytes,
                                    void* out, void* stream) {
  SYM_REQUIRE(B <= 0 || q, SYM_ERR_INVALID, "paged_gqa_decode: null pointer argument");
  // the plain kernel only reads the pools
  return launch_decode("paged_gqa_decode", q, nullptr, const_cast<void*>(k_pool),
                       const_cast<void*>(v_pool), nullptr, nullptr, block_tables, positions, B,
                       Hq, Hkv, head_dim,
                       block_size, max_blocks_per_seq, num_blocks, max_context, scale, workspace,
                       workspace_bytes, out, stream);
}

// ---------------------------------------------------------------------------------------------
// Allocation-free decode. The per-split partial results live in this file-scope device array
// instead of a caller workspace: one copy per GPU, held until the process ends. The host never
// passes the array's name to a kernel (in host code it is only a stand-in for the symbol); each
// device's copy is located once with hipGetSymbolAddress and that address is used. Nothing in it
// needs initial contents: the split kernel writes every (sequence, head, split) entry that the
// merge kernel reads, and a sequence with a single split never touches it.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};
}  // namespace

// Address of the current device's scratch copy (located on the first call on that device).
static int noalloc_scratch(const char* what, void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  SYM_REQUIRE(e == hipSuccess, SYM_ERR_LAUNCH, "%s: hipGetDevice: %s", what,
              hipGetErrorString(e));
  SYM_REQUIRE(dev >= 0 && dev < kMaxDevices, SYM_ERR_UNSUPPORTED, "%s: device %d", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    SYM_REQUIRE(e == hipSuccess && p, SYM_ERR_LAUNCH,
                "%s: hipGetSymbolAddress(scratch) on device %d: %s", what, dev,
                hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return SYM_OK;
}

extern "C" int sym_paged_gqa_decode_noalloc(const void* q, const void* k_pool,
                                            const void* v_pool, const int32_t* block_tables,
                                            const int32_t* positions, int B, int Hq, int Hkv,
                                            int head_dim, int block_size,
                                            int max_blocks_per_seq, int num_blocks,
                                            int max_context, float scale, void* out,
                                            void* stream) {
  const char* what = "paged_gqa_decode_noalloc";
  SYM_REQUIRE(B <= 0 || q, SYM_ERR_INVALID, "%s: null pointer argument", what);
  const size_t need = sym_paged_gqa_decode_workspace_bytes(B, Hq, head_dim, max_context);
  SYM_REQUIRE(need <= kNoAllocScratchBytes, SYM_ERR_WORKSPACE,
              "%s: B=%d x Hq=%d x %d splits of the context need %zu bytes of scratch, above the "
              "fixed %zu (use sym_paged_gqa_decode with a caller workspace)",
              what, B, Hq, (max_context + kSplit - 1) / kSplit, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  int rc = noalloc_scratch(what, &ws);
  if (rc) return rc;
  return launch_decode(what, q, nullptr, const_cast<void*>(k_pool), const_cast<void*>(v_pool),
                       nullptr, nullptr, block_tables, positions, B, Hq, Hkv, head_dim,
                       block_size, max_blocks_per_seq, num_blocks, max_context, scale, ws,
                       kNoAllocScratchBytes, out, stream);
}

extern "C" int sym_attn_decode_step(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                    const float* rope_cs, int max_pos, const int32_t* positions,
                                    int B, int Hq, int Hkv, int head_dim, int rotary_dim,
                                    float eps, int use_qk_norm, void* k_pool, void* v_pool,
                                    const int32_t* block_tables, int max_blocks_per_seq,
                                    int block_size, int num_blocks, int max_context, float scale,
                                    void* workspace, size_t workspace_bytes, void* out,
                                    void* stream) {
  SYM_REQUIRE(B <= 0 || qkv, SYM_ERR_INVALID, "attn_decode_step: null pointer argument");
  SYM_REQUIRE(rotary_dim >= 0 && rotary_dim <= head_dim && rotary_dim % 2 == 0, SYM_ERR_INVALID,
              "attn_decode_step: rotary_dim=%d", rotary_dim);
  SYM_REQUIRE(rotary_dim == 0 || (rope_cs && max_pos > 0), SYM_ERR_INVALID,
              "attn_decode_step: rope table missing");
  SYM_REQUIRE(!use_qk_norm || (q_norm_w && k_norm_w), SYM_ERR_INVALID,
              "attn_decode_step: QK-norm weights missing");
  const FusedQKV fq{(const uint16_t*)qkv,
                    use_qk_norm ? (const uint16_t*)q_norm_w : nullptr,
                    use_qk_norm ? (const uint16_t*)k_norm_w : nullptr,
                    rotary_dim ? rope_cs : nullptr,
                    rotary_dim ? max_pos : 0,
                    rotary_dim,
                    eps};
  return launch_decode("attn_decode_step", nullptr, &fq, k_pool, v_pool, nullptr, nullptr,
                       block_tables, positions, B, Hq, Hkv, head_dim, block_size,
                       max_blocks_per_seq, num_blocks, max_context, scale, workspace,
                       workspace_bytes, out, stream);
}

extern "C" int sym_paged_gqa_decode_fp8(const void* q, const void* k_pool, const void* v_pool,
                                        const float* k_scale, const float* v_scale,
                                        const int32_t* block_tables, const int32_t* positions,
                                        int B, int Hq, int Hkv, int head_dim, int block_size,
                                        int max_blocks_per_seq, int num_blocks, int max_context,
                                        float scale, void* workspace, size_t workspace_bytes,
                                        void* out, void* stream) {
  SYM_REQUIRE(B <= 0 || (q && k_scale && v_scale), SYM_ERR_INVALID,
              "paged_gqa_decode_fp8: null pointer argument");
  // the plain kernel only reads the pools and scales
  return launch_decode("paged_gqa_decode_fp8", q, nullptr, const_cast<void*>(k_pool),
                       const_cast<void*>(v_pool), const_cast<float*>(k_scale),
                       const_cast<float*>(v_scale), block_tables, positions, B, Hq, Hkv,
                       head_dim, block_size, max_blocks_per_seq, num_blocks, max_context, scale,
                       workspace, workspace_bytes, out, stream);
}

extern "C" int sym_attn_decode_step_fp8(const void* qkv, const void* q_norm_w,
                                        const void* k_norm_w, const float* rope_cs, int max_pos,
                                        const int32_t* positions, int B, int Hq, int Hkv,
                                        int head_dim, int rotary_dim, float eps, int use_qk_norm,
                                        void* k_pool, void* v_pool, float* k_scale,
                                        float* v_scale, const int32_t* block_tables,
                                        int max_blocks_per_seq, int block_size, int num_blocks,
                                        int max_context, float scale, void* workspace,
                                        size_t workspace_bytes, void* out, void* stream) {
  SYM_REQUIRE(B <= 0 || (qkv && k_scale && v_scale), SYM_ERR_INVALID,
              "attn_decode_step_fp8: null pointer argument");
  SYM_REQUIRE(rotary_dim >= 0 && rotary_dim <= head_dim && rotary_dim % 2 == 0, SYM_ERR_INVALID,
              "attn_decode_step_fp8: rotary_dim=%d", rotary_dim);
  SYM_REQUIRE(rotary_dim == 0 || (rope_cs && max_pos > 0), SYM_ERR_INVALID,
              "attn_decode_step_fp8: rope table missing");
  SYM_REQUIRE(!use_qk_norm || (q_norm_w && k_norm_w), SYM_ERR_INVALID,
              "attn_decode_step_fp8: QK-norm weights missing");
  const FusedQKV fq{(const uint16_t*)qkv,
                    use_qk_norm ? (const uint16_t*)q_norm_w : nullptr,
                    use_qk_norm ? (const uint16_t*)k_norm_w : nullptr,
                    rotary_dim ? rope_cs : nullptr,
                    rotary_dim ? max_pos : 0,
                    rotary_dim,
                    eps};
  return launch_decode("attn_decode_step_fp8", nullptr, &fq, k_pool, v_pool, k_scale, v_scale,
                       block_tables, positions, B, Hq, Hkv, head_dim, block_size,
                       max_blocks_per_seq, num_blocks, max_context, scale, workspace,
                       workspace_bytes, out, stream);
}

extern "C" int sym_paged_kv_fill_fp8(const void* k, const void* v, long long tok_stride,
                                     long long head_stride, const int32_t* cu_seqlens,
                                     const int32_t* start_pos, const int32_t* seq_rows,
                                     int n_seqs, int max_seqlen, int Hkv, int head_dim,
                                     void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                                     const int32_t* block_tables, int page_table_rows,
                                     int max_blocks_per_seq, int block_size, int num_blocks,
                                     void* stream) {
  int rc = check_cache_args("paged_kv_fill_fp8", n_seqs, Hkv, head_dim, block_size,
                            max_blocks_per_seq, num_blocks);
  if (rc) return rc;
  SYM_REQUIRE(max_seqlen >= 0, SYM_ERR_INVALID, "paged_kv_fill_fp8: max_seqlen=%d", max_seqlen);
  if (n_seqs == 0 || max_seqlen == 0) return SYM_OK;
  SYM_REQUIRE(k && v && cu_seqlens && k_pool && v_pool && k_scale && v_scale && block_tables,
              SYM_ERR_INVALID, "paged_kv_fill_fp8: null pointer argument");
  SYM_REQUIRE(kSplit8 % block_size == 0 && block_size % 8 == 0, SYM_ERR_UNSUPPORTED,
              "paged_kv_fill_fp8: block_size=%d must be a multiple of 8 dividing %d", block_size,
              kSplit8);
  SYM_REQUIRE(n_seqs <= 65535 && Hkv <= 65535, SYM_ERR_INVALID, "paged_kv_fill_fp8: grid");
  SYM_REQUIRE(page_table_rows >= 1 && (seq_rows || n_seqs <= page_table_rows), SYM_ERR_INVALID,
              "paged_kv_fill_fp8: %d sequences for a page table of %d rows", n_seqs,
              page_table_rows);
  SYM_REQUIRE(tok_stride > 0 && head_stride > 0 && tok_stride % 8 == 0 && head_stride % 8 == 0,
              SYM_ERR_INVALID, "paged_kv_fill_fp8: strides %lld, %lld must be positive multiples"
              " of 8", tok_stride, head_stride);
  const int gx = (max_seqlen + block_size - 1) / block_size + 1;
  (void)hipGetLastError();
  hipLaunchKernelGGL(paged_kv_fill_fp8_kernel, dim3(gx, Hkv, n_seqs), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)k, (const uint16_t*)v, tok_stride,
                     head_stride, cu_seqlens, start_pos, seq_rows, page_table_rows, Hkv,
                     (uint8_t*)k_pool, (uint8_t*)v_pool, k_scale, v_scale, block_tables,
                     max_blocks_per_seq, block_size, num_blocks);
  return sym_host::check_launch("paged_kv_fill_fp8_kernel");
}
