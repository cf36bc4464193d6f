// Prefill attention: causal GQA flash attention over packed variable-length sequences, and the
// prefill prologue (QK-norm, partial RoPE and the paged KV write of every token).
//
// Reference: the prefill branch of TTNNBailingMoEAttention (ttnn_attention.py:2153-2230: QKV,
// QK-norm, RoPE, paged_fill_on_device of the sequence's K/V, causal SDPA), generalised from the
// reference's batch_idx-0-only prefill (ttnn_attention.py:2205-2210) to packed sequences given by
// cu_seqlens (positions 0 .. L-1 of each sequence).
//
// Attention design (gfx950): one workgroup of 4 waves per (128-query block, query head,
// sequence); each wave owns 32 queries and keeps their Q fragments in registers. Key blocks of 64
// tokens are moved by LDS-DMA into one of two LDS stages (K and V row-major, XOR-swizzled) while
// the previous block is computed. The wave computes the transposed scores S^T = K Q^T on
// v_mfma_f32_32x32x16_bf16 (two 32-key tiles), so a lane holds 16 keys of one query per tile and
// lane l^32 the other 16: the online softmax (log2 domain, lazily rescaled) reduces a query over
// the lane's own values and one cross-half swap, and the exponentiated scores, packed to bf16,
// are already the B operand of O^T += V^T P^T (the MFMA's k index follows the score layout), whose
// A operand comes from transposing LDS reads of row-major V. A key block is computed in two 32-key
// halves so that one half's softmax issues between the other half's MFMAs. Only key blocks at or
// before the query block are visited, and only the blocks that cross the diagonal or the sequence
// end are masked.
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
//   V: swizzle 4 * (r & 3) - a transposed V read (per 32 lanes: 4 rows x 64 bytes) hits
//                            4 distinct 64-byte windows.
__device__ __forceinline__ int k_slot(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int v_slot(int r, int c) { return c ^ ((r & 3) << 2); }

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

// Maximum over lanes l and l^32 (the two lanes that hold one query's keys): v_permlane32_swap
// of x with itself leaves the other half's value in the second register of the pair.
// (Maxima are written as compiler-visible operations, never as inline asm, here and below: the
// compiler inserts no wait states before inline asm that reads an MFMA result, so such an asm
// could read the accumulator before the MFMA has written it.)
__device__ __forceinline__ float max_over_halves(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const float a0 = __uint_as_float(a[0]), a1 = __uint_as_float(a[1]);
  return a0 > a1 ? a0 : a1;
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
  const int n32 = lane & 31, hp = lane >> 5;  // the lane's query column and key half

  // Q fragments (B operand of S^T): column n32 = query q0 + wave*32 + n32 (clamped), dims
  // 16c + 8hp .. +7
  const int wq0 = q0 + wave * 32;
  const int qrow = wq0 + n32;
  uint4 qf[8];
  {
    const uint16_t* qr = q + ((size_t)(s0 + min(qrow, L - 1)) * Hq + h) * kPD + 8 * hp;
#pragma unroll
    for (int c = 0; c < 8; ++c) qf[c] = *reinterpret_cast<const uint4*>(qr + 16 * c);
  }
  // O^T tiles dt: lane holds dims 32dt + 8j + 4hp + i of query qrow in element 4j + i
  floatx16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
  // running max (log2 domain) of the lane's query (the same in lanes l and l^32) and the lane's
  // share of its running sum (the two shares are added after the last key block: every rescale
  // multiplies both by the same factor)
  float m = -INFINITY, l = 0.f;

  const int q_last = min(q0 + kPQ, L) - 1;
  const int nkb = q_last / kPK + 1;

  // LDS-DMA of key block kb_ (keys past the sequence clamped to its last) into stage kb_ & 1:
  // wave w moves rows 16w .. 16w+15 of K and of V, 4 rows (1 KB) per instruction; lane (row
  // lane/16, slot lane%16) fetches the chunk that the slot holds. Byte offsets within a block fit
  // in 32 bits (the host checks max_seqlen * Hkv * 128 < 2^31).
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
  //   K (A operand of S^T, row 32kt + n32, dims 16c + 8hp .. +7): chunk 2c + hp of that row;
  //   V (read transposed: lane s of 16-lane group G addresses key row 4(G/2) + s/4 (+ 32kt +
  //   16p, + 8 for the upper four keys), dims 32dt + 16(G%2) + 4(s%4) .. +3, and receives keys
  //   4hp .. 4hp+3 of dim 32dt + n32: the A operand of O^T += V^T P^T in the score layout's key
  //   order).
  int k_off[8], v_off[4];
#pragma unroll
  for (int c = 0; c < 8; ++c) k_off[c] = n32 * kRowElems + 8 * k_slot(n32, 2 * c + hp);
  {
    const int G = lane >> 4, sl = lane & 15;
    const int vr = 4 * (G >> 1) + (sl >> 2);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      v_off[dt] = kStageElems + vr * kRowElems +
                  8 * v_slot(vr, 4 * dt + 2 * (G & 1) + ((sl >> 1) & 1)) + 4 * (sl & 1);
  }

  // One key block in two 32-key halves kt: S^T of half 1 is issued while the softmax of half 0
  // runs, and O^T += V^T P^T of half 0 while the softmax of half 1 runs. MASK (the block crosses
  // the diagonal or the sequence end) is a template flag so that each half's MFMAs and softmax
  // form one branch-free stretch of code.
  auto block = [&](auto mask_tag, int kb) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int k0 = kb * kPK;
    if (kb + 1 < nkb) load_block(kb + 1);
    const uint16_t* st = &lds[kb & 1][0][0];
    // S^T of half kt: lane holds keys k0 + 32kt + 8j + 4hp + i of query qrow (element 4j + i)
    auto scores = [&](int kt) {
      floatx16 sc;
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        uint4 kf = *reinterpret_cast<const uint4*>(st + k_off[c] + 32 * kt * kRowElems);
        sc = mfma32x32x16(kf, qf[c], sc);
        // With a zero accumulator the compiler may give the 16-register result the registers of
        // the (then dead) A operand. An asm that reads and writes kf after the MFMA keeps kf live
        // across it (and cannot move above it), so the two stay apart.
        if (c == 0) asm volatile("" : "+v"(kf.x), "+v"(kf.y), "+v"(kf.z), "+v"(kf.w));
      }
      return sc;
    };
    // Online softmax of half kt (log2 domain, lazily rescaled: the running max moves only when a
    // score exceeds it by more than kLazyMax, so the weights stay below 2^kLazyMax; the result
    // is the same softmax). Key 0 of block 0 is visible to every query, so the max is finite
    // from the first half on. Returns the P^T operands (k-steps of keys 16p .. 16p+15) and
    // leaves the rescale factor in al.
    auto softmax = [&](int kt, floatx16& sc, uint4 (&pf)[2], float& al) {
      if constexpr (MASK) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = k0 + 32 * kt + 8 * j + 4 * hp + i;
            if (key > qrow || key >= L) sc[4 * j + i] = -INFINITY;
          }
      }
      float mx = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                       fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
      mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(sc[8], sc[9]), fmaxf(sc[10], sc[11])),
                           fmaxf(fmaxf(sc[12], sc[13]), fmaxf(sc[14], sc[15]))));
      mx = max_over_halves(mx);
      const float mxs = mx * scale_log2;
      const bool grow = mxs > m + kLazyMax;  // true on the first half (m = -inf)
      const float mn = grow ? mxs : m;
      al = grow ? fast_exp2(m - mn) : 1.f;
      m = mn;
      float rs = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sc[e] = fast_exp2(fmaf(sc[e], scale_log2, -mn));
        rs += sc[e];
      }
      l = l * al + rs;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
        pf[pp] = make_uint4(pack_bf16x2(sc[8 * pp + 0], sc[8 * pp + 1]),
                            pack_bf16x2(sc[8 * pp + 2], sc[8 * pp + 3]),
                            pack_bf16x2(sc[8 * pp + 4], sc[8 * pp + 5]),
                            pack_bf16x2(sc[8 * pp + 6], sc[8 * pp + 7]));
    };
    auto rescale = [&](float al) {
      if (__any(al != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[dt][e] *= al;
      }
    };
    // O^T += V^T P^T of half kt: k-step p covers keys 32kt + 16p + {4hp .. 4hp+3, 8+4hp .. 11+4hp}
    auto pv = [&](int kt, const uint4 (&pf)[2]) {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const uint16_t* vp = st + v_off[dt] + (32 * kt + 16 * pp) * kRowElems;
          const uint2 lo = lds_read_tr16(vp);
          const uint2 hi = lds_read_tr16(vp + 8 * kRowElems);
          o[dt] = mfma32x32x16(make_uint4(lo.x, lo.y, hi.x, hi.y), pf[pp], o[dt]);
        }
    };
    uint4 p0[2], p1[2];
    float a0, a1;
    floatx16 s0 = scores(0);
    __builtin_amdgcn_sched_barrier(0);
    floatx16 s1 = scores(1);
    softmax(0, s0, p0, a0);
    interleave_mfma_valu<8, 1, 1, 8>();
    pin_operands(p0);
    __builtin_amdgcn_sched_barrier(0);
    rescale(a0);
    __builtin_amdgcn_sched_barrier(0);
    pv(0, p0);
    softmax(1, s1, p1, a1);
    interleave_mfma_valu<8, 2, 1, 8>();
    pin_operands(p1);
    __builtin_amdgcn_sched_barrier(0);
    rescale(a1);
    pv(1, p1);
    // this wave's DMA of block kb+1 has landed and its reads of stage kb&1 are done; after the
    // barrier every wave's are
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  load_block(0);
  // The compiler's own wait for the Q loads, here: it cannot see the waits inside the asm below
  // and would otherwise place them in the key-block loop, where they would also wait for the
  // next block's DMA.
#pragma unroll
  for (int c = 0; c < 8; ++c) asm volatile("" ::"v"(qf[c].x), "v"(qf[c].y), "v"(qf[c].z), "v"(qf[c].w));
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  // Blocks from kb_mask on hold keys past a query of this wave (the diagonal) or past the
  // sequence and are masked: two loops in sequence (one branch between the two block bodies in
  // every iteration makes the register allocator spill). Every wave runs nkb blocks in all.
  const int kb_mask = min(min(wq0 + 1, L) / kPK, nkb);
  int kb = 0;
  for (; kb < kb_mask; ++kb) block(std::false_type{}, kb);
  for (; kb < nkb; ++kb) block(std::true_type{}, kb);

  // ---- normalise and store: lane holds dims 32dt + 8j + 4hp + i of query qrow ----
  {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false,
                                                    false);
    const float lt = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    if (qrow < L) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      uint16_t* orow = out + ((size_t)(s0 + qrow) * Hq + h) * kPD + 4 * hp;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<uint2*>(orow + 32 * dt + 8 * j) =
              make_uint2(pack_bf16x2(o[dt][4 * j] * inv, o[dt][4 * j + 1] * inv),
                         pack_bf16x2(o[dt][4 * j + 2] * inv, o[dt][4 * j + 3] * inv));
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
