// Model ends of the greedy decode loop: the token embedding gather, the LM head with the greedy
// (argmax) choice fused in, and the per-step bookkeeping of positions and generated tokens.
//
// Reference: TTNNBailingMoeV2Model swaps the embedding and the final norm of the HF model
// (modeling_bailing_moe_v2.py:56-95, forward 97-334, final norm 262); the lm_head is a TTNN
// linear; HF GenerationMixin.generate reads the logits back and takes argmax on the host
// (greedy). Here the argmax runs on the device and only token ids leave it.
//
// LM head design (gfx950): at decode the head is a skinny GEMM that streams the [V, H] weight
// once (157184 x 2048 bf16 = 644 MB for Ling-mini-2.0). A workgroup of 8 waves owns 128 vocab
// rows; each wave streams 16 rows over all of H (lane l: 32 contiguous bytes of row l % 16 per
// 64-wide K step, the B operand of v_mfma_f32_16x16x32_bf16). The token rows (up to 64 per
// pass, the A operand) are staged in LDS 256 columns at a time, once per workgroup, while the
// chunk's weight loads are in flight, so the 8 waves share one read of them. The logits never
// go to memory: the wave reduces its 16 columns to (max, lowest index) per token row with lane
// shuffles, the workgroup reduces its 8 waves through LDS and writes one partial per
// (workgroup, row); a second kernel reduces the partials of a row. Ties resolve to the lowest
// vocab index (torch.argmax's rule).
#include "common.h"

namespace sym {

constexpr int kLmWaves = 8;
constexpr int kLmThreads = kLmWaves * 64;
constexpr int kLmRowsPerWG = kLmWaves * 16;  // vocab rows per workgroup
constexpr int kLmKC = 256;                   // K chunk of the token rows staged in LDS
constexpr int kLmXStride = kLmKC + 8;        // LDS row stride (528 B: conflict-free b128 reads)

__global__ __launch_bounds__(256) void embedding_gather_kernel(
    const int32_t* __restrict__ ids, const uint16_t* __restrict__ table, int H, int V,
    uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int id = ids[t];
  const bool ok = id >= 0 && id < V;
  const uint4* src = reinterpret_cast<const uint4*>(table + (size_t)(ok ? id : 0) * H);
  uint4* dst = reinterpret_cast<uint4*>(out + (size_t)t * H);
  for (int c = threadIdx.x; c < H / 8; c += 256) dst[c] = ok ? src[c] : make_uint4(0, 0, 0, 0);
}

// (value, index) of the larger logit; equal values keep the lower index
__device__ __forceinline__ void arg_better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

template <int MT>
__global__ __launch_bounds__(kLmThreads) void lm_head_partial_kernel(
    const uint16_t* __restrict__ x, int B, int H, const uint16_t* __restrict__ w, int V,
    float* __restrict__ part_val, int* __restrict__ part_idx) {
  __shared__ __align__(16) uint16_t s_x[2 * 16 * MT * kLmXStride];
  __shared__ float s_val[kLmWaves][16 * MT];
  __shared__ int s_idx[kLmWaves][16 * MT];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int vcol = blockIdx.x * kLmRowsPerWG + wave * 16 + r16;   // this lane's vocab column
  const uint16_t* wr = w + (size_t)min(vcol, V - 1) * H + kq * 16;
  constexpr int kXLoads = 16 * MT * (kLmKC / 8) / kLmThreads;      // 16-byte pieces per thread
  for (int mb = 0; mb < B; mb += 16 * MT) {
    floatx4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int kc = 0; kc < H; kc += kLmKC) {
      // this chunk's weights first (in flight while the token rows are staged)
      uint4 b[kLmKC / 64][2];
#pragma unroll
      for (int s = 0; s < kLmKC / 64; ++s) {
        b[s][0] = *reinterpret_cast<const uint4*>(wr + kc + s * 64);
        b[s][1] = *reinterpret_cast<const uint4*>(wr + kc + s * 64 + 8);
      }
      // stage the chunk of token rows into the LDS buffer of this chunk's parity (last read
      // two chunks ago, before the previous chunk's barrier)
      uint16_t* sx = s_x + ((kc / kLmKC) & 1) * (16 * MT * kLmXStride);
      const int c8 = (tid % (kLmKC / 8)) * 8;
      uint4 xv[kXLoads];
#pragma unroll
      for (int j = 0; j < kXLoads; ++j) {
        const int row = tid / (kLmKC / 8) + j * (kLmThreads / (kLmKC / 8));
        xv[j] = *reinterpret_cast<const uint4*>(x + (size_t)min(mb + row, B - 1) * H + kc + c8);
      }
#pragma unroll
      for (int j = 0; j < kXLoads; ++j) {
        const int row = tid / (kLmKC / 8) + j * (kLmThreads / (kLmKC / 8));
        *reinterpret_cast<uint4*>(&sx[row * kLmXStride + c8]) = xv[j];
      }
      __syncthreads();
#pragma unroll
      for (int s = 0; s < kLmKC / 64; ++s)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint16_t* ar = &sx[(mt * 16 + r16) * kLmXStride + s * 64 + kq * 16];
          const uint4 a0 = *reinterpret_cast<const uint4*>(ar);
          const uint4 a1 = *reinterpret_cast<const uint4*>(ar + 8);
          acc[mt] = mfma16x16x32(a0, b[s][0], acc[mt]);
          acc[mt] = mfma16x16x32(a1, b[s][1], acc[mt]);
        }
    }
    // lane holds logits of token rows 4*kq + i (tile mt), vocab column vcol: reduce the
    // wave's 16 columns per row over the 16 lanes of the row group
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float bv = vcol < V ? acc[mt][i] : -INFINITY;
        int bi = vcol < V ? vcol : 0x7fffffff;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
          const float ov = __shfl_xor(bv, off);
          const int oi = __shfl_xor(bi, off);
          arg_better(bv, bi, ov, oi);
        }
        if (r16 == 0) {
          s_val[wave][mt * 16 + 4 * kq + i] = bv;
          s_idx[wave][mt * 16 + 4 * kq + i] = bi;
        }
      }
    __syncthreads();
    if (tid < 16 * MT) {
      const int row = mb + tid;
      float bv = s_val[0][tid];
      int bi = s_idx[0][tid];
#pragma unroll
      for (int wv = 1; wv < kLmWaves; ++wv) arg_better(bv, bi, s_val[wv][tid], s_idx[wv][tid]);
      if (row < B) {
        part_val[(size_t)blockIdx.x * B + row] = bv;
        part_idx[(size_t)blockIdx.x * B + row] = bi;
      }
    }
  }
}

// One workgroup per token row: the best of the row's partials.
__global__ __launch_bounds__(256) void lm_head_reduce_kernel(
    const float* __restrict__ part_val, const int* __restrict__ part_idx, int n_parts, int B,
    int32_t* __restrict__ ids) {
  __shared__ float s_val[4];
  __shared__ int s_idx[4];
  const int row = blockIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int p = threadIdx.x; p < n_parts; p += 256)
    arg_better(bv, bi, part_val[(size_t)p * B + row], part_idx[(size_t)p * B + row]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    arg_better(bv, bi, ov, oi);
  }
  if ((threadIdx.x & 63) == 0) {
    s_val[threadIdx.x >> 6] = bv;
    s_idx[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    bv = s_val[0];
    bi = s_idx[0];
#pragma unroll
    for (int wv = 1; wv < 4; ++wv) arg_better(bv, bi, s_val[wv], s_idx[wv]);
    ids[row] = bi;
  }
}

// positions[b] += 1 (the position of the token just chosen); that token goes to column
// positions[b] - hist_base[b] of its history row when the column is inside [0, hist_cols).
__global__ __launch_bounds__(256) void greedy_advance_kernel(
    const int32_t* __restrict__ ids, int B, int32_t* __restrict__ positions,
    int32_t* __restrict__ history, const int32_t* __restrict__ hist_base, int hist_cols) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  if (b >= B) return;
  const int p = positions[b] + 1;
  positions[b] = p;
  if (history) {
    const int col = p - hist_base[b];
    if (col >= 0 && col < hist_cols) history[(size_t)b * hist_cols + col] = ids[b];
  }
}

}  // namespace sym

using namespace sym;

extern "C" int sym_embedding_bf16(const int32_t* ids, const void* table, int T, int H, int V,
                                  void* out, void* stream) {
  SYM_REQUIRE(T >= 0 && H > 0 && V > 0, SYM_ERR_INVALID, "embedding: T=%d H=%d V=%d", T, H, V);
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(ids && table && out, SYM_ERR_INVALID, "embedding: null pointer argument");
  SYM_REQUIRE(H % 8 == 0, SYM_ERR_UNSUPPORTED, "embedding: H=%d must be a multiple of 8", H);
  (void)hipGetLastError();
  hipLaunchKernelGGL(embedding_gather_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream, ids,
                     (const uint16_t*)table, H, V, (uint16_t*)out);
  return sym_host::check_launch("embedding_gather_kernel");
}

extern "C" size_t sym_lm_head_greedy_workspace_bytes(int B, int V) {
  if (B <= 0 || V <= 0) return 0;
  const size_t parts = (size_t)(V + kLmRowsPerWG - 1) / kLmRowsPerWG;
  return parts * (size_t)B * (sizeof(float) + sizeof(int));
}

extern "C" int sym_lm_head_greedy(const void* x, const void* w, int B, int H, int V,
                                  void* workspace, size_t workspace_bytes, int32_t* ids,
                                  void* stream) {
  SYM_REQUIRE(B >= 0 && H > 0 && V > 0, SYM_ERR_INVALID, "lm_head_greedy: B=%d H=%d V=%d", B, H,
              V);
  if (B == 0) return SYM_OK;
  SYM_REQUIRE(x && w && workspace && ids, SYM_ERR_INVALID, "lm_head_greedy: null pointer");
  SYM_REQUIRE(H % kLmKC == 0, SYM_ERR_UNSUPPORTED,
              "lm_head_greedy: H=%d must be a multiple of %d", H, kLmKC);
  const size_t need = sym_lm_head_greedy_workspace_bytes(B, V);
  SYM_REQUIRE(workspace_bytes >= need, SYM_ERR_WORKSPACE,
              "lm_head_greedy: workspace %zu < required %zu", workspace_bytes, need);
  const int parts = (V + kLmRowsPerWG - 1) / kLmRowsPerWG;
  float* pv = (float*)workspace;
  int* pi = (int*)(pv + (size_t)parts * B);
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  if (B <= 16)
    hipLaunchKernelGGL((lm_head_partial_kernel<1>), dim3(parts), dim3(kLmThreads), 0, s,
                       (const uint16_t*)x, B, H, (const uint16_t*)w, V, pv, pi);
  else if (B <= 32)
    hipLaunchKernelGGL((lm_head_partial_kernel<2>), dim3(parts), dim3(kLmThreads), 0, s,
                       (const uint16_t*)x, B, H, (const uint16_t*)w, V, pv, pi);
  else
    hipLaunchKernelGGL((lm_head_partial_kernel<4>), dim3(parts), dim3(kLmThreads), 0, s,
                       (const uint16_t*)x, B, H, (const uint16_t*)w, V, pv, pi);
  int rc = sym_host::check_launch("lm_head_partial_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(lm_head_reduce_kernel, dim3(B), dim3(256), 0, s, pv, pi, parts, B, ids);
  return sym_host::check_launch("lm_head_reduce_kernel");
}

extern "C" int sym_greedy_advance(const int32_t* ids, int B, int32_t* positions,
                                  int32_t* history, const int32_t* hist_base, int hist_cols,
                                  void* stream) {
  SYM_REQUIRE(B >= 0 && hist_cols >= 0, SYM_ERR_INVALID, "greedy_advance: B=%d hist_cols=%d", B,
              hist_cols);
  if (B == 0) return SYM_OK;
  SYM_REQUIRE(ids && positions, SYM_ERR_INVALID, "greedy_advance: null pointer argument");
  SYM_REQUIRE(!history || hist_base, SYM_ERR_INVALID, "greedy_advance: history without base");
  (void)hipGetLastError();
  hipLaunchKernelGGL(greedy_advance_kernel, dim3((B + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, ids, B, positions, history, hist_base, hist_cols);
  return sym_host::check_launch("greedy_advance_kernel");
}
