// Prefill attention: causal GQA flash attention over packed variable-length sequences, and the
// prefill prologue (QK-norm, partial RoPE and the paged KV write of every token).
//
// Reference: the prefill branch of TTNNBailingMoEAttention (ttnn_attention.py:2153-2230: QKV,
// QK-norm, RoPE, paged_fill_on_device of the sequence's K/V, causal SDPA), generalised from the
// reference's batch_idx-0-only prefill (ttnn_attention.py:2205-2210) to packed sequences given by
// cu_seqlens (positions 0 .. L-1 of each sequence).
//
// Attention design (gfx950): one workgroup of 4 waves per (128-query block, query head,
// sequence); each wave owns 32 queries (two 16-query tiles) and keeps its Q fragments in
// registers. Key blocks of 64 tokens are staged in LDS (K row-major, V transposed). The wave
// computes the transposed scores S^T = K Q^T on v_mfma_f32_16x16x32_bf16, so a lane holds 16
// keys of one query per tile: the online softmax (log2 domain) reduces a query over the lane's
// own values and two xor shuffles, and the exponentiated scores, packed to bf16, are already the
// B operand of O^T += V^T P^T (the MFMA's k index is free to follow the score layout: lane group
// kq takes keys 4kq .. 4kq+3 of two adjacent 16-key tiles, and reads the matching V^T columns as
// two 8-byte pieces). Only key blocks at or before the query block are visited, and only the
// blocks that cross the diagonal or the sequence end are masked.
#include "common.h"

namespace sym {

constexpr int kPD = 128;           // head dim
constexpr int kPQ = 128;           // queries per workgroup
constexpr int kPK = 64;            // keys per block
constexpr int kPKStride = kPD + 8; // LDS row stride of K (elements)
constexpr float kLazyMax = 8.f;      // log2 headroom of the lazily rescaled softmax
constexpr int kPVStride = kPK + 4; // LDS row stride of V^T: 34 dwords, so the 16 rows of an
                                   // 8-byte fragment read start in distinct bank pairs

// 16 bytes as a native vector (an array of these stays in registers across the key-block loop;
// one of HIP's uint4 struct was left in scratch memory)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads of one key block (keys k0 .. k0+63 of a sequence, clamped to its last key L-1) for the
// staging below: kreg[j] = K chunk (idx%16) of key idx/16, vreg[i][u] = V chunk idx/32 of key
// 2(idx%32)+u, with idx = tid + 256j (resp. 256i). k / v point at the sequence's first token of
// this kv head.
__device__ __forceinline__ void load_kv_block(const uint16_t* __restrict__ k,
                                              const uint16_t* __restrict__ v, int Hkv, int L,
                                              int k0, int tid, u32x4 (&kreg)[4],
                                              u32x4 (&vreg)[2][2]) {
  // element offsets from the sequence's first row in 32 bits with 24-bit multiplies (the host
  // checks max_seqlen * Hkv * 128 < 2^31)
  const unsigned row = (unsigned)Hkv * kPD;
  const int kk = k0 + (tid >> 4), kc = (tid & 15) * 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const unsigned kr = (unsigned)min(kk + 16 * j, L - 1);
    kreg[j] = *reinterpret_cast<const u32x4*>(k + (__umul24(kr, row) + kc));
  }
  const int vk = k0 + 2 * (tid & 31), vc = (tid >> 5) * 8;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const unsigned kr = (unsigned)min(vk + u, L - 1);
      vreg[i][u] = *reinterpret_cast<const u32x4*>(v + (__umul24(kr, row) + vc + 64 * i));
    }
  }
}

// Stores one key block's registers (from load_kv_block) into an LDS stage:
//   K: item j = tid + 256j is (key idx/16, 16-byte chunk idx%16), stored row-major;
//   V: item i = tid + 256i is (key pair p = idx%32, chunk c = idx/32): the chunk of keys 2p and
//      2p+1 is transposed into 8 dwords (dim c*8+e: key 2p in the low half, 2p+1 in the high
//      half), so the 32 lanes of a pair-row write 128 contiguous bytes of sVt (no bank
//      conflicts).
__device__ __forceinline__ void stage_kv_block(uint16_t* __restrict__ sK,
                                               uint16_t* __restrict__ sVt, int tid,
                                               const u32x4 (&kreg)[4],
                                               const u32x4 (&vreg)[2][2]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = tid + 256 * j;
    *reinterpret_cast<u32x4*>(&sK[(idx >> 4) * kPKStride + (idx & 15) * 8]) = kreg[j];
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + 256 * i;
    const int p = idx & 31, c = idx >> 5;
    const u32x4 a = vreg[i][0], b = vreg[i][1];
    uint32_t* dst = reinterpret_cast<uint32_t*>(&sVt[(c * 8) * kPVStride + 2 * p]);
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
      // dims 2mm (low halves) and 2mm+1 (high halves) of keys 2p (low) and 2p+1 (high)
      dst[(2 * mm) * (kPVStride / 2)] = __builtin_amdgcn_perm(b[mm], a[mm], 0x05040100u);
      dst[(2 * mm + 1) * (kPVStride / 2)] = __builtin_amdgcn_perm(b[mm], a[mm], 0x07060302u);
    }
  }
}

// Maximum over lanes l, l^16, l^32, l^48 (the four lanes that hold one query's keys) with the
// gfx950 cross-row swaps: v_permlane32_swap of x with itself leaves x of lane l^32 in the other
// register of the pair (likewise v_permlane16_swap for l^16), all in VALU.
__device__ __forceinline__ float max_over_rows(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const float a0 = __uint_as_float(a[0]), a1 = __uint_as_float(a[1]);
  const float y = a0 > a1 ? a0 : a1;
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false,
                                                  false);
  const float b0 = __uint_as_float(b[0]), b1 = __uint_as_float(b[1]);
  return b0 > b1 ? b0 : b1;
}

__global__ __launch_bounds__(256, 2) void prefill_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const int32_t* __restrict__ cu_seqlens, int Hq, int Hkv,
    float scale_log2, uint16_t* __restrict__ out) {
  // two stages: block kb+1 is stored while block kb is read
  __shared__ __align__(16) uint16_t sK[2][kPK * kPKStride];
  __shared__ __align__(16) uint16_t sVt[2][kPD * kPVStride];

  // Query blocks in decreasing order over the whole grid (z slowest): the blocks with the most
  // key blocks under the causal mask, of every sequence and head, are dispatched first and the
  // short ones fill the tail. Heads vary fastest, so consecutive workgroups (dealt round-robin
  // to the XCDs) carry the same amount of work.
  const int qb = gridDim.z - 1 - blockIdx.z, h = blockIdx.x, sq = blockIdx.y;
  const int s0 = cu_seqlens[sq];
  const int L = cu_seqlens[sq + 1] - s0;
  const int q0 = qb * kPQ;
  if (q0 >= L) return;
  const int g = h / (Hq / Hkv);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar mask branches
  const int r16 = lane & 15, kq = lane >> 4;

  // Q fragments (B operand of S^T): column r16 = query q0 + wave*32 + t*16 + r16 (clamped),
  // dims 8*kq + 32*c
  const int wq0 = q0 + wave * 32;
  int qrow[2];
  uint4 qf[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    qrow[t] = wq0 + t * 16 + r16;
    const int qi = min(qrow[t], L - 1);
    const uint16_t* qr = q + ((size_t)(s0 + qi) * Hq + h) * kPD + 8 * kq;
#pragma unroll
    for (int c = 0; c < 4; ++c) qf[t][c] = *reinterpret_cast<const uint4*>(qr + 32 * c);
  }
  // O^T: lane holds dims d*16 + 4*kq + i of its query (tile t)
  floatx4 o[2][8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int d = 0; d < 8; ++d) o[t][d] = floatx4{0.f, 0.f, 0.f, 0.f};
  // running max (log2 domain) of the lane's query (the same in its 4 lanes r16 + 16*kq) and the
  // lane's share of its running sum (the four shares are added after the last key block: every
  // rescale multiplies all four by the same factor)
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};

  const int q_last = min(q0 + kPQ, L) - 1;
  const int nkb = q_last / kPK + 1;
  // Key block kb is read from stage kb&1 while block kb+1, loaded into registers during block
  // kb-1, is stored into the other stage and block kb+2 is loaded; one barrier per block (the
  // stage written during block kb was last read during block kb-1, before that block's barrier).
  u32x4 kreg[4], vreg[2][2];
  const uint16_t* kbase = k + ((size_t)s0 * Hkv + g) * kPD;
  const uint16_t* vbase = v + ((size_t)s0 * Hkv + g) * kPD;
  load_kv_block(kbase, vbase, Hkv, L, 0, tid, kreg, vreg);
  stage_kv_block(sK[0], sVt[0], tid, kreg, vreg);
  if (nkb > 1) load_kv_block(kbase, vbase, Hkv, L, kPK, tid, kreg, vreg);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * kPK;
    const uint16_t* cK = sK[kb & 1];
    const uint16_t* cVt = sVt[kb & 1];
    // ---- S^T = K Q^T: lane holds keys k0 + 16j + 4*kq + i of query qrow[t] ----
    floatx4 sc[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[t][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint4 kf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        kf[j] = *reinterpret_cast<const uint4*>(&cK[(j * 16 + r16) * kPKStride + 8 * kq + 32 * c]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[t][j] = mfma16x16x32(kf[j], qf[t][c], sc[t][j]);
    }
    if (kb + 1 < nkb) {
      stage_kv_block(sK[(kb + 1) & 1], sVt[(kb + 1) & 1], tid, kreg, vreg);
      if (kb + 2 < nkb) load_kv_block(kbase, vbase, Hkv, L, k0 + 2 * kPK, tid, kreg, vreg);
    }
    // keys past a query of this wave (the diagonal) or past the sequence are masked
    const bool masked = k0 + kPK - 1 > wq0 || k0 + kPK > L;
    uint4 pf[2][2];  // P^T operands: [t][32-key chunk]
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (masked) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = k0 + 16 * j + 4 * kq + i;
            if (key > qrow[t] || key >= L) sc[t][j][i] = -INFINITY;
          }
      }
      float mx = sc[t][0][0];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[t][j][i]);
      mx = max_over_rows(mx);
      // Lazy rescaling: the running max (log2 domain) moves only when a score exceeds it by more
      // than kLazyMax, so the weights stay below 2^kLazyMax and most blocks skip the rescale of
      // the output; the result is the same softmax. Key 0 of block 0 is visible to every query,
      // so the max is finite from the first block on.
      const float mxs = mx * scale_log2;
      const bool grow = mxs > m[t] + kLazyMax;  // true on the first block (m = -inf)
      const float mn = grow ? mxs : m[t];
      const float alpha = grow ? fast_exp2(m[t] - mn) : 1.f;
      float rs = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pj = fast_exp2(fmaf(sc[t][j][i], scale_log2, -mn));
          sc[t][j][i] = pj;
          rs += pj;
        }
      m[t] = mn;
      l[t] = l[t] * alpha + rs;
      if (__any(alpha != 1.f)) {
#pragma unroll
        for (int d = 0; d < 8; ++d)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[t][d][i] *= alpha;
      }
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
        pf[t][cc] = make_uint4(pack_bf16x2(sc[t][2 * cc][0], sc[t][2 * cc][1]),
                               pack_bf16x2(sc[t][2 * cc][2], sc[t][2 * cc][3]),
                               pack_bf16x2(sc[t][2 * cc + 1][0], sc[t][2 * cc + 1][1]),
                               pack_bf16x2(sc[t][2 * cc + 1][2], sc[t][2 * cc + 1][3]));
    }
    // ---- O^T += V^T P^T: A = V^T rows d*16 + r16, keys 32cc + 4kq + {0..3, 16..19} ----
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const uint16_t* vr = &cVt[(d * 16 + r16) * kPVStride + 32 * cc + 4 * kq];
        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16);
        const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int t = 0; t < 2; ++t) o[t][d] = mfma16x16x32(vf, pf[t][cc], o[t][d]);
      }
    }
    __syncthreads();  // every wave is done with stage kb&1 and has stored block kb+1
  }
  // ---- normalise and store: lane holds dims d*16 + 4*kq + i of query qrow[t] ----
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float lt = l[t] + __shfl_xor(l[t], 16);
    lt += __shfl_xor(lt, 32);
    if (qrow[t] < L) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      uint16_t* orow = out + ((size_t)(s0 + qrow[t]) * Hq + h) * kPD + 4 * kq;
#pragma unroll
      for (int d = 0; d < 8; ++d)
        *reinterpret_cast<uint2*>(orow + d * 16) =
            make_uint2(pack_bf16x2(o[t][d][0] * inv, o[t][d][1] * inv),
                       pack_bf16x2(o[t][d][2] * inv, o[t][d][3] * inv));
    }
  }
}

}  // namespace sym

using namespace sym;

extern "C" int sym_prefill_attention(const void* q, const void* k, const void* v,
                                     const int32_t* cu_seqlens, int n_seqs, int max_seqlen,
                                     int Hq, int Hkv, int head_dim, float scale, void* out,
                                     void* stream) {
  SYM_REQUIRE(n_seqs >= 0 && max_seqlen >= 0, SYM_ERR_INVALID,
              "prefill_attention: n_seqs=%d max_seqlen=%d", n_seqs, max_seqlen);
  if (n_seqs == 0 || max_seqlen == 0) return SYM_OK;
  SYM_REQUIRE(q && k && v && cu_seqlens && out, SYM_ERR_INVALID,
              "prefill_attention: null pointer argument");
  SYM_REQUIRE(head_dim == kPD, SYM_ERR_UNSUPPORTED, "prefill_attention: head_dim=%d (only 128)",
              head_dim);
  SYM_REQUIRE(Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0 && Hq <= 65535, SYM_ERR_INVALID,
              "prefill_attention: Hq=%d Hkv=%d", Hq, Hkv);
  SYM_REQUIRE(n_seqs <= 65535 && (max_seqlen + kPQ - 1) / kPQ <= 65535, SYM_ERR_INVALID,
              "prefill_attention: n_seqs=%d max_seqlen=%d", n_seqs, max_seqlen);
  SYM_REQUIRE((long long)max_seqlen * Hkv * kPD < (1LL << 31), SYM_ERR_UNSUPPORTED,
              "prefill_attention: max_seqlen=%d x Hkv=%d too large", max_seqlen, Hkv);
  (void)hipGetLastError();
  hipLaunchKernelGGL(prefill_attention_kernel, dim3(Hq, n_seqs, (max_seqlen + kPQ - 1) / kPQ),
                     dim3(256), 0, (hipStream_t)stream, (const uint16_t*)q, (const uint16_t*)k,
                     (const uint16_t*)v, cu_seqlens, Hq, Hkv, scale * 1.4426950408889634f,
                     (uint16_t*)out);
  return sym_host::check_launch("prefill_attention_kernel");
}
