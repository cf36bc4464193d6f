// Prefill attention: causal GQA flash attention over packed variable-length sequences, and the
// prefill prologue (QK-norm, partial RoPE and the paged KV write of every token).
//
// Reference: the prefill branch of TTNNBailingMoEAttention (ttnn_attention.py:2153-2230: QKV,
// QK-norm, RoPE, paged_fill_on_device of the sequence's K/V, causal SDPA), generalised from the
// reference's batch_idx-0-only prefill (ttnn_attention.py:2205-2210) to packed sequences given by
// cu_seqlens (positions 0 .. L-1 of each sequence).
//
// Attention design (gfx950): one workgroup of 4 waves per (128-query block, query head,
// sequence); each wave owns 32 query rows (two 16-row MFMA tiles) and keeps its Q fragments in
// registers. Key blocks of 64 tokens are staged in LDS (K row-major, V transposed so the
// P.V operand reads 16 contiguous bytes); S = Q K^T and O += P V run on
// v_mfma_f32_16x16x32_bf16; the online softmax (log2 domain) reduces each row over the 16
// lanes that hold it with xor shuffles; P goes through a per-wave LDS tile from the MFMA output
// layout to the operand layout. Only key blocks at or before the query block are visited.
#include "common.h"

namespace sym {

constexpr int kPD = 128;           // head dim
constexpr int kPQ = 128;           // queries per workgroup
constexpr int kPK = 64;            // keys per block
constexpr int kPKStride = kPD + 8; // LDS row stride of K (elements)
constexpr int kPVStride = kPK + 8; // LDS row stride of transposed V
constexpr int kPPStride = kPK + 8; // LDS row stride of a wave's P tile

__global__ __launch_bounds__(256) void prefill_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const int32_t* __restrict__ cu_seqlens, int Hq, int Hkv,
    float scale_log2, uint16_t* __restrict__ out) {
  __shared__ __align__(16) uint16_t sK[kPK * kPKStride];
  __shared__ __align__(16) uint16_t sVt[kPD * kPVStride];
  __shared__ __align__(16) uint16_t sP[4][32 * kPPStride];

  const int qb = blockIdx.x, h = blockIdx.y, sq = blockIdx.z;
  const int s0 = cu_seqlens[sq];
  const int L = cu_seqlens[sq + 1] - s0;
  const int q0 = qb * kPQ;
  if (q0 >= L) return;
  const int g = h / (Hq / Hkv);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r16 = lane & 15, kq = lane >> 4;

  // Q fragments (A operand): row tile t, query q0 + wave*32 + t*16 + r16 (clamped), dims
  // 8*kq + 32*c
  uint4 qa[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int qi = min(q0 + wave * 32 + t * 16 + r16, L - 1);
    const uint16_t* qr = q + ((size_t)(s0 + qi) * Hq + h) * kPD + 8 * kq;
#pragma unroll
    for (int c = 0; c < 4; ++c) qa[t][c] = *reinterpret_cast<const uint4*>(qr + 32 * c);
  }
  floatx4 o[2][8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int d = 0; d < 8; ++d) o[t][d] = floatx4{0.f, 0.f, 0.f, 0.f};
  // running max / sum of the 4 rows 4*kq + i of each row tile (identical in the 16 lanes of a
  // row group)
  float m[2][4], l[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m[t][i] = -INFINITY;
      l[t][i] = 0.f;
    }

  const int q_last = min(q0 + kPQ, L) - 1;
  const int nkb = q_last / kPK + 1;
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * kPK;
    // ---- stage K (row-major) and V (transposed) of keys k0 .. k0+63 (clamped rows) ----
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int idx = tid + 256 * j;        // 64 keys x 16 chunks of 8 dims
      const int key = idx >> 4, ch = idx & 15;
      const int kr = min(k0 + key, L - 1);
      const size_t src = ((size_t)(s0 + kr) * Hkv + g) * kPD + ch * 8;
      *reinterpret_cast<uint4*>(&sK[key * kPKStride + ch * 8]) =
          *reinterpret_cast<const uint4*>(k + src);
      const uint4 vv = *reinterpret_cast<const uint4*>(v + src);
      const uint16_t* ve = reinterpret_cast<const uint16_t*>(&vv);
#pragma unroll
      for (int e = 0; e < 8; ++e) sVt[(ch * 8 + e) * kPVStride + key] = ve[e];
    }
    __syncthreads();
    // ---- S = Q K^T for this wave's 32 rows x 64 keys ----
    floatx4 sc[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[t][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint4 kbf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        kbf[j] = *reinterpret_cast<const uint4*>(&sK[(j * 16 + r16) * kPKStride + 8 * kq + 32 * c]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[t][j] = mfma16x16x32(qa[t][c], kbf[j], sc[t][j]);
    }
    // ---- online softmax: lane holds rows 4*kq + i, key column j*16 + r16 ----
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qi = q0 + wave * 32 + t * 16 + 4 * kq + i;
        float x[4];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int kj = k0 + j * 16 + r16;
          x[j] = (kj <= qi && kj < L) ? sc[t][j][i] * scale_log2 : -INFINITY;
          mx = fmaxf(mx, x[j]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 1));
        mx = fmaxf(mx, __shfl_xor(mx, 2));
        mx = fmaxf(mx, __shfl_xor(mx, 4));
        mx = fmaxf(mx, __shfl_xor(mx, 8));
        const float mn = fmaxf(m[t][i], mx);
        const float alpha = mn == -INFINITY ? 1.f : exp2f(m[t][i] - mn);
        float rs = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float pj = mn == -INFINITY ? 0.f : exp2f(x[j] - mn);
          x[j] = pj;
          rs += pj;
        }
        rs += __shfl_xor(rs, 1);
        rs += __shfl_xor(rs, 2);
        rs += __shfl_xor(rs, 4);
        rs += __shfl_xor(rs, 8);
        m[t][i] = mn;
        l[t][i] = l[t][i] * alpha + rs;
#pragma unroll
        for (int d = 0; d < 8; ++d) o[t][d][i] *= alpha;
        // P (bf16) into this wave's LDS tile: row t*16 + 4*kq + i, key j*16 + r16
#pragma unroll
        for (int j = 0; j < 4; ++j)
          sP[wave][(t * 16 + 4 * kq + i) * kPPStride + j * 16 + r16] = f32_to_bf16(x[j]);
      }
    }
    // P is written and read by different lanes of this wave: the wavefront-scope fence keeps
    // the compiler from moving the reads above the writes (a wave's LDS operations run in order)
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // ---- O += P V (P rows as A: row r16, keys 8*kq + 32*c; V^T rows as B) ----
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      uint4 pa[2], vb[8];
#pragma unroll
      for (int t = 0; t < 2; ++t)
        pa[t] = *reinterpret_cast<const uint4*>(&sP[wave][(t * 16 + r16) * kPPStride + 8 * kq + 32 * c]);
#pragma unroll
      for (int d = 0; d < 8; ++d)
        vb[d] = *reinterpret_cast<const uint4*>(&sVt[(d * 16 + r16) * kPVStride + 8 * kq + 32 * c]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int d = 0; d < 8; ++d) o[t][d] = mfma16x16x32(pa[t], vb[d], o[t][d]);
    }
  }
  // ---- normalise and store: lane holds rows 4*kq + i, dim d*16 + r16 ----
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qi = q0 + wave * 32 + t * 16 + 4 * kq + i;
      if (qi < L) {
        const float inv = l[t][i] > 0.f ? 1.f / l[t][i] : 0.f;
        uint16_t* orow = out + ((size_t)(s0 + qi) * Hq + h) * kPD;
#pragma unroll
        for (int d = 0; d < 8; ++d) orow[d * 16 + r16] = f32_to_bf16(o[t][d][i] * inv);
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
  SYM_REQUIRE(n_seqs <= 65535, SYM_ERR_INVALID, "prefill_attention: n_seqs=%d", n_seqs);
  (void)hipGetLastError();
  hipLaunchKernelGGL(prefill_attention_kernel, dim3((max_seqlen + kPQ - 1) / kPQ, Hq, n_seqs),
                     dim3(256), 0, (hipStream_t)stream, (const uint16_t*)q, (const uint16_t*)k,
                     (const uint16_t*)v, cu_seqlens, Hq, Hkv, scale * 1.4426950408889634f,
                     (uint16_t*)out);
  return sym_host::check_launch("prefill_attention_kernel");
}
