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

constexpr int kPD = 128;              // head dim
constexpr int kPQ = 128;              // queries per workgroup
constexpr int kPK = 64;               // keys per block
constexpr int kRowElems = kPD;        // one key's 128 dims (256 bytes) per LDS row
constexpr int kStageElems = kPK * kRowElems;  // one operand (K or V) of one key block: 16 KB
constexpr float kLazyMax = 8.f;       // log2 headroom of the lazily rescaled softmax

// LDS layout of a key block: K and V row-major (row r = key k0 + r, 256 bytes), their 16-byte
// chunks c stored at slot c ^ swizzle(r) of the row, so that both kinds of fragment read touch
// distinct banks without padding (which the LDS-DMA's contiguous 1 KB writes cannot leave):
//   K: swizzle r & 15      - the 16 rows of a K fragment read (one chunk each) hit 16 slots;
//   V: swizzle 2 * (r & 7) - a transposed V read (16 rows x 32 bytes) hits every slot twice.
__device__ __forceinline__ int k_slot(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int v_slot(int r, int c) { return c ^ ((r & 7) << 1); }

// Instruction order of one overlapped stretch: NR groups of (RD LDS reads, then MPG times one
// MFMA followed by NV VALU instructions), so the softmax of one half issues between the MFMAs
// of the other.
template <int NR, int RD, int MPG, int NV>
__device__ __forceinline__ void interleave_mfma_valu() {
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if constexpr (RD > 0) __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);  // LDS reads
#pragma unroll
    for (int i = 0; i < MPG; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);  // VALU
    }
  }
}

// Makes the P^T operands of a half exist at this point: without it the compiler sinks the
// exponentials below the rescale branch, out of the stretch where they overlap the MFMAs.
__device__ __forceinline__ void pin_operands(const uint4 (&p)[2]) {
  asm volatile("" ::"v"(p[0].x), "v"(p[0].y), "v"(p[0].z), "v"(p[0].w), "v"(p[1].x),
               "v"(p[1].y), "v"(p[1].z), "v"(p[1].w));
}

// v_max_f32 / v_max3_f32 without the canonicalising maxima that fmaxf adds for operands the
// compiler cannot prove canonical (the scores hold no NaN)
__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Maxima of both query tiles over the four lanes l, l^16, l^32, l^48 that hold one query's keys,
// with the gfx950 cross-row swaps: v_permlane32_swap of (x0, x1) pairs the upper half of x0
// with the lower half of x1, so one maximum reduces tile 0 over l^32 in lanes 0-31 and tile 1
// in lanes 32-63; a v_permlane16_swap step reduces over l^16, and a last v_permlane32_swap
// hands each tile's result to all 64 lanes.
__device__ __forceinline__ void max_over_rows2(float& x0, float& x1) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x0), __float_as_uint(x1), false,
                                                  false);
  const float z = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(z), __float_as_uint(z), false,
                                                  false);
  const float w = vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(w), __float_as_uint(w), false,
                                                  false);
  x0 = __uint_as_float(c[0]);
  x1 = __uint_as_float(c[1]);
}

__global__ __launch_bounds__(256, 2) void prefill_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const int32_t* __restrict__ cu_seqlens, int Hq, int Hkv,
    float scale_log2, uint16_t* __restrict__ out) {
  // two stages of (K, V): block kb+1 is loaded into one while block kb is read from the other
  __shared__ __align__(16) uint16_t lds[2][2][kStageElems];

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
  // running max (log2 domain) of the lane's query (the same in its 4 lanes r16 + 16*kq), and the
  // running sum of its weights: ls = ONES P^T on the MFMA (a 16 x 32 A operand of bf16 ones), so
  // every element of ls[t] is the sum over the bf16 weights that O^T accumulates
  float m[2] = {-INFINITY, -INFINITY};
  floatx4 ls[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
  const uint4 ones = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);

  const int q_last = min(q0 + kPQ, L) - 1;
  const int nkb = q_last / kPK + 1;

  // LDS-DMA of key block kb_ (keys past the sequence clamped to its last) into stage kb_ & 1:
  // wave w moves rows 16w .. 16w+15 of K and of V, 4 rows (1 KB) per instruction; lane (row
  // lane/16, slot lane%16) fetches the chunk that the slot holds. Byte offsets from the
  // sequence's first row fit in 32 bits (the host checks max_seqlen * Hkv * 128 < 2^31).
  const uint16_t* kbase = k + ((size_t)s0 * Hkv + g) * kPD;
  const uint16_t* vbase = v + ((size_t)s0 * Hkv + g) * kPD;
  const uint32_t row_bytes = (uint32_t)Hkv * kPD * 2;
  const size_t block_elems = (size_t)kPK * Hkv * kPD;  // one key block of this sequence
  uint32_t k_src[4], v_src[4];  // lane's byte offsets within a block (row r, slot lane%16)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * wave + 4 * i + (lane >> 4);
    k_src[i] = r * row_bytes + 16 * k_slot(r, lane & 15);
    v_src[i] = r * row_bytes + 16 * v_slot(r, lane & 15);
  }
  auto load_block = [&](int kb_) {
    uint16_t* st = &lds[kb_ & 1][0][0];
    const uint16_t* kb_k = kbase + kb_ * block_elems;
    const uint16_t* kb_v = vbase + kb_ * block_elems;
    if ((kb_ + 1) * kPK <= L) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dma16(kb_k, k_src[i], st + (16 * wave + 4 * i) * kRowElems);
        dma16(kb_v, v_src[i], st + kStageElems + (16 * wave + 4 * i) * kRowElems);
      }
    } else {  // the sequence's last block: rows past it repeat its last key
      const int last = L - 1 - kb_ * kPK;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * wave + 4 * i + (lane >> 4);
        const uint32_t row = (uint32_t)min(r, last) * row_bytes;
        dma16(kb_k, row + 16 * k_slot(r, lane & 15), st + (16 * wave + 4 * i) * kRowElems);
        dma16(kb_v, row + 16 * v_slot(r, lane & 15),
              st + kStageElems + (16 * wave + 4 * i) * kRowElems);
      }
    }
  };

  // Fragment addresses within a stage (elements):
  //   K (A operand of S^T, rows 32h + 16jj + r16, dims 8kq + 32c): chunk kq + 4c of that row;
  //   V (read transposed: lane s = r16 of group kq addresses key 4kq + s/4 (+ 32h, + 16 for
  //   the upper four keys), dims 16d + 4(s%4) .. +3, and receives keys 4kq .. 4kq+3 of dim
  //   16d + r16 - the A operand of O^T += V^T P^T in the key order of the score layout).
  int k_off[4], v_off[8];
#pragma unroll
  for (int c = 0; c < 4; ++c) k_off[c] = r16 * kRowElems + 8 * k_slot(r16, kq + 4 * c);
  const int vr = 4 * kq + (r16 >> 2);
#pragma unroll
  for (int d = 0; d < 8; ++d)
    v_off[d] = kStageElems + vr * kRowElems + 8 * v_slot(vr, 2 * d + ((r16 >> 1) & 1)) +
               4 * (r16 & 1);

  // One key block in two 32-key halves h: S^T of half 1 is issued while the softmax of half 0
  // runs, and O^T += V^T P^T of half 0 while the softmax of half 1 runs, so a wave's MFMAs and
  // VALU work overlap. MASK (the block crosses the diagonal or the sequence end) is a template
  // flag so that each half's MFMAs and softmax form one branch-free stretch of code.
  auto block = [&](auto mask_tag, int kb) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int k0 = kb * kPK;
    if (kb + 1 < nkb) load_block(kb + 1);
    const uint16_t* st = &lds[kb & 1][0][0];
    // S^T of half h: sh[t][jj] holds keys k0 + 32h + 16jj + 4*kq + i of query qrow[t]
    auto scores = [&](int hh, floatx4 (&sh)[2][2]) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) sh[t][jj] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        uint4 kf[2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          kf[jj] = *reinterpret_cast<const uint4*>(
              st + k_off[c] + (32 * hh + 16 * jj) * kRowElems);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) sh[t][jj] = mfma16x16x32(kf[jj], qf[t][c], sh[t][jj]);
      }
    };
    // Online softmax of half hh (log2 domain, lazily rescaled: the running max moves only when
    // a score exceeds it by more than kLazyMax, so the weights stay below 2^kLazyMax; the
    // result is the same softmax). Key 0 of block 0 is visible to every query, so the max is
    // finite from the first half on. Leaves the P^T operands in pf, the rescale factors in al.
    auto softmax = [&](int hh, floatx4 (&sh)[2][2], uint4 (&pf)[2], float (&al)[2]) {
      float mx[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if constexpr (MASK) {
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = k0 + 32 * hh + 16 * jj + 4 * kq + i;
              if (key > qrow[t] || key >= L) sh[t][jj][i] = -INFINITY;
            }
        }
        mx[t] = vmax(vmax3(sh[t][0][0], sh[t][0][1], sh[t][0][2]),
                     vmax3(sh[t][0][3], sh[t][1][0], vmax3(sh[t][1][1], sh[t][1][2], sh[t][1][3])));
      }
      max_over_rows2(mx[0], mx[1]);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float mxs = mx[t] * scale_log2;
        const bool grow = mxs > m[t] + kLazyMax;  // true on the first half (m = -inf)
        const float mn = grow ? mxs : m[t];
        al[t] = grow ? fast_exp2(m[t] - mn) : 1.f;
        m[t] = mn;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
          for (int i = 0; i < 4; ++i) sh[t][jj][i] = fast_exp2(fmaf(sh[t][jj][i], scale_log2, -mn));
        pf[t] = make_uint4(pack_bf16x2(sh[t][0][0], sh[t][0][1]),
                           pack_bf16x2(sh[t][0][2], sh[t][0][3]),
                           pack_bf16x2(sh[t][1][0], sh[t][1][1]),
                           pack_bf16x2(sh[t][1][2], sh[t][1][3]));
      }
    };
    auto rescale = [&](const float (&al)[2]) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
        if (__any(al[t] != 1.f)) {
#pragma unroll
          for (int d = 0; d < 8; ++d)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[t][d][i] *= al[t];
#pragma unroll
          for (int i = 0; i < 4; ++i) ls[t][i] *= al[t];
        }
    };
    // O^T += V^T P^T of half hh: A = V^T rows 16d + r16, keys 32hh + 4kq + {0..3, 16..19}
    auto pv = [&](int hh, const uint4 (&pf)[2]) {
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const uint2 lo = lds_read_tr16(st + v_off[d] + (32 * hh) * kRowElems);
        const uint2 hi = lds_read_tr16(st + v_off[d] + (32 * hh + 16) * kRowElems);
        const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int t = 0; t < 2; ++t) o[t][d] = mfma16x16x32(vf, pf[t], o[t][d]);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) ls[t] = mfma16x16x32(ones, pf[t], ls[t]);
    };
    floatx4 s0[2][2], s1[2][2];
    uint4 p0[2], p1[2];
    float a0[2], a1[2];
    scores(0, s0);
    __builtin_amdgcn_sched_barrier(0);
    scores(1, s1);
    softmax(0, s0, p0, a0);
    interleave_mfma_valu<4, 2, 4, 6>();
    pin_operands(p0);
    __builtin_amdgcn_sched_barrier(0);
    rescale(a0);
    __builtin_amdgcn_sched_barrier(0);
    pv(0, p0);
    softmax(1, s1, p1, a1);
    interleave_mfma_valu<8, 2, 2, 6>();
    interleave_mfma_valu<1, 0, 2, 6>();
    pin_operands(p1);
    __builtin_amdgcn_sched_barrier(0);
    rescale(a1);
    pv(1, p1);
    // this wave's DMA of block kb+1 has landed and its reads of stage kb&1 are done; after the
    // barrier every wave's are
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  load_block(0);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  // Blocks from kb_mask on hold keys past a query of this wave (the diagonal) or past the
  // sequence and are masked: two loops in sequence (one branch between the two block bodies in
  // every iteration makes the register allocator spill). Every wave runs nkb blocks in all.
  const int kb_mask = min(min(wq0 + 1, L) / kPK, nkb);
  int kb = 0;
  for (; kb < kb_mask; ++kb) block(std::false_type{}, kb);
  for (; kb < nkb; ++kb) block(std::true_type{}, kb);

  // ---- normalise and store: lane holds dims d*16 + 4*kq + i of query qrow[t] ----
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const float lt = ls[t][0];
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
