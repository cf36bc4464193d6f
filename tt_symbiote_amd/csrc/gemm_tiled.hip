// Tiled bf16 GEMMs for prefill-size problems (MFMA-bound): dense projections and the grouped
// expert GEMMs over ragged, expert-sorted rows.
//
// Reference: the projections of TTNNBailingMoEAttention (ttnn_attention.py:2001-2011) at
// sequence length > 1, and the expert sparse_matmuls of TTNNExperts.forward
// (ttnn_moe.py:1250-1289) with the shared expert (ttnn_moe.py:656-675), for prefill batches.
//
// Design (gfx950): a workgroup of 4 waves computes a 128 x 128 output tile; each wave owns a
// 64 x 64 quadrant as 4 x 4 v_mfma_f32_16x16x32_bf16 tiles (64 accumulator registers). The K
// loop moves 64 columns per step: every thread loads 4 x 16 bytes of the A tile and 4 x 16
// bytes of the B tile (8 threads per 128-byte row, coalesced), stores them to LDS (rows padded
// to 144 bytes so the 16 rows of an MFMA fragment read fall in distinct banks), and the loads of
// step k+1 are in flight while step k's 32 MFMAs per wave run from LDS.
//   DENSE:   out[M, N] = A[M, K] . W[N, K]^T (+ bias) (+ residual fp32), bf16 or fp32 out.
//   GATE_UP: rows of a segment gather x[sorted_tokens[row]]; the B tile holds 64 gate rows and
//            the matching 64 up rows of the expert, so each wave's quadrant pairs 32 gate with 32
//            up columns and the epilogue writes h = silu(gate) * up (bf16).
//   DOWN:    rows of a segment are h rows (contiguous); y = h . W_down^T (fp32).
// Grouped modes: the workgroup's row tile is found from the device-side segment list (prefix
// of ceil(count / 128) over the segments, in LDS); workgroups past the last tile exit.
#include "common.h"

namespace sym {

constexpr int kTM = 128, kTN = 128, kTK = 64;
constexpr int kTileThreads = 256;
constexpr int kLdsStride = kTK + 8;  // bf16 elements per LDS row (144 bytes)
constexpr int kMaxGemmSegments = 4096;

enum TileMode { kDense = 0, kGateUp = 1, kDown = 2 };

struct TileArgs {
  const uint16_t* a;        // DENSE/DOWN: rows [., K]; GATE_UP: x [T, K]
  const uint16_t* w;        // DENSE: [N, K]; GATE_UP: [S, 2I, K]; DOWN: [S, N, K]
  const uint16_t* bias;     // DENSE, optional [N]
  const float* residual;    // DENSE, optional [M, N] fp32
  const int32_t* sorted_tokens;
  const int32_t* seg_expert;
  const int32_t* seg_offset;
  const int32_t* seg_count;
  const int32_t* n_segments;
  int M, N, K;              // GATE_UP: N = I (h columns); DOWN: N = H
  uint16_t* out_bf16;
  float* out_f32;
};

__device__ __forceinline__ uint4 ld_g16(const uint16_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

template <int MODE>
__global__ __launch_bounds__(kTileThreads) void gemm_tile_kernel(TileArgs p) {
  __shared__ __align__(16) uint16_t sA[kTM * kLdsStride];
  __shared__ __align__(16) uint16_t sB[kTN * kLdsStride];
  __shared__ int s_tile_start[MODE == kDense ? 1 : kMaxGemmSegments + 1];
  __shared__ int s_info[4];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int r16 = lane & 15, kq = lane >> 4;
  const int K = p.K;

  // ---- locate the tile ----
  int row0, rows, e = 0;  // first output row, valid rows in the tile, expert
  const int ct = blockIdx.x;
  if constexpr (MODE == kDense) {
    row0 = blockIdx.y * kTM;
    rows = min(kTM, p.M - row0);
  } else {
    const int nseg = p.n_segments[0];
    if (wave == 0) {
      int run = 0;
      for (int s0 = 0; s0 < nseg; s0 += 64) {
        const int s = s0 + lane;
        const int nt = s < nseg ? (p.seg_count[s] + kTM - 1) / kTM : 0;
        int x = nt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int y = __shfl_up(x, off);
          if (lane >= off) x += y;
        }
        if (s < nseg) s_tile_start[s] = run + x - nt;
        run += __shfl(x, 63);
      }
      if (lane == 0) s_tile_start[nseg] = run;
    }
    __syncthreads();
    const int g = blockIdx.y;
    if (g >= s_tile_start[nseg]) return;
    if (tid == 0) s_info[0] = 0;
    __syncthreads();
    for (int s = tid; s < nseg; s += kTileThreads)
      if (s_tile_start[s] <= g && g < s_tile_start[s + 1]) s_info[0] = s;
    __syncthreads();
    const int seg = s_info[0];
    const int rt = g - s_tile_start[seg];
    e = p.seg_expert[seg];
    row0 = p.seg_offset[seg] + rt * kTM;
    rows = min(kTM, p.seg_count[seg] - rt * kTM);
  }

  // ---- global -> register mapping: thread loads rows (tid/8) + 32j, 16-byte chunk tid%8 ----
  const int lrow = tid >> 3, lchunk = tid & 7;
  const uint16_t* a_ptr[4];
  const uint16_t* b_ptr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = min(lrow + 32 * j, rows - 1);  // rows past the tile repeat its last row
    size_t arow;
    if constexpr (MODE == kGateUp) arow = (size_t)p.sorted_tokens[row0 + r];
    else arow = (size_t)(row0 + r);
    a_ptr[j] = p.a + arow * K + lchunk * 8;
    const int br = lrow + 32 * j;  // B tile row 0..127
    size_t brow;
    if constexpr (MODE == kGateUp) {
      // 64 gate rows then the matching 64 up rows of expert e
      const int col = ct * 64 + (br & 63);
      brow = (size_t)e * 2 * p.N + (br < 64 ? col : p.N + col);
    } else if constexpr (MODE == kDown) {
      brow = (size_t)e * p.N + ct * kTN + br;
    } else {
      brow = (size_t)(ct * kTN + br);
    }
    b_ptr[j] = p.w + brow * K + lchunk * 8;
  }

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  uint4 ra[4], rb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ra[j] = ld_g16(a_ptr[j]);
    rb[j] = ld_g16(b_ptr[j]);
  }
  // B fragment rows of this wave's 4 column tiles
  int brow_frag[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (MODE == kGateUp)
      brow_frag[j] = (j < 2 ? 0 : 64) + wn * 32 + (j & 1) * 16 + r16;
    else
      brow_frag[j] = wn * 64 + j * 16 + r16;
  }

  const int nk = K / kTK;
  for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *reinterpret_cast<uint4*>(&sA[(lrow + 32 * j) * kLdsStride + lchunk * 8]) = ra[j];
      *reinterpret_cast<uint4*>(&sB[(lrow + 32 * j) * kLdsStride + lchunk * 8]) = rb[j];
    }
    __syncthreads();
    if (kt + 1 < nk) {
      const int k = (kt + 1) * kTK;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ra[j] = ld_g16(a_ptr[j] + k);
        rb[j] = ld_g16(b_ptr[j] + k);
      }
    }
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const int ko = kh * 32 + kq * 8;
      uint4 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        fa[i] = *reinterpret_cast<const uint4*>(&sA[(wm * 64 + i * 16 + r16) * kLdsStride + ko]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[j] = *reinterpret_cast<const uint4*>(&sB[brow_frag[j] * kLdsStride + ko]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(fa[i], fb[j], acc[i][j]);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds rows 4*(l/16)+q, column l%16 of each 16 x 16 tile ----
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = wm * 64 + i * 16 + kq * 4 + q;
      if (r >= rows) continue;
      const size_t orow = (size_t)(row0 + r);
      if constexpr (MODE == kGateUp) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float g = acc[i][j][q], u = acc[i][j + 2][q];
          const int col = ct * 64 + wn * 32 + j * 16 + r16;
          p.out_bf16[orow * p.N + col] = f32_to_bf16(g / (1.0f + expf(-g)) * u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int col = ct * kTN + wn * 64 + j * 16 + r16;
          float v = acc[i][j][q];
          if constexpr (MODE == kDense) {
            if (p.bias) v += bf16_to_f32(p.bias[col]);
            if (p.residual) v += p.residual[orow * p.N + col];
          }
          if (p.out_f32) p.out_f32[orow * p.N + col] = v;
          else p.out_bf16[orow * p.N + col] = f32_to_bf16(v);
        }
      }
    }
  }
}

}  // namespace sym

using namespace sym;

extern "C" int sym_gemm_bf16(const void* a, const void* w, const void* bias, const float* residual,
                             int M, int N, int K, void* out, int out_fp32, void* stream) {
  SYM_REQUIRE(M >= 0, SYM_ERR_INVALID, "gemm_bf16: M=%d < 0", M);
  if (M == 0) return SYM_OK;
  SYM_REQUIRE(a && w && out, SYM_ERR_INVALID, "gemm_bf16: null pointer argument");
  SYM_REQUIRE(N > 0 && N % kTN == 0 && N / kTN <= 2147483647, SYM_ERR_UNSUPPORTED,
              "gemm_bf16: N=%d must be a positive multiple of %d", N, kTN);
  SYM_REQUIRE(K > 0 && K % kTK == 0, SYM_ERR_UNSUPPORTED,
              "gemm_bf16: K=%d must be a positive multiple of %d", K, kTK);
  SYM_REQUIRE((M + kTM - 1) / kTM <= 65535, SYM_ERR_UNSUPPORTED, "gemm_bf16: M=%d too large", M);
  TileArgs p{};
  p.a = (const uint16_t*)a;
  p.w = (const uint16_t*)w;
  p.bias = (const uint16_t*)bias;
  p.residual = residual;
  p.M = M;
  p.N = N;
  p.K = K;
  p.out_bf16 = out_fp32 ? nullptr : (uint16_t*)out;
  p.out_f32 = out_fp32 ? (float*)out : nullptr;
  (void)hipGetLastError();
  hipLaunchKernelGGL((gemm_tile_kernel<kDense>), dim3(N / kTN, (M + kTM - 1) / kTM),
                     dim3(kTileThreads), 0, (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile_kernel");
}

static int check_grouped(const char* what, int T, int H, int I, int rows, int max_segments) {
  SYM_REQUIRE(T >= 0 && rows >= 0, SYM_ERR_INVALID, "%s: T=%d rows=%d", what, T, rows);
  SYM_REQUIRE(H > 0 && H % kTN == 0, SYM_ERR_UNSUPPORTED, "%s: H=%d must be a multiple of %d",
              what, H, kTN);
  SYM_REQUIRE(I > 0 && I % 64 == 0, SYM_ERR_UNSUPPORTED, "%s: I=%d must be a multiple of 64",
              what, I);
  SYM_REQUIRE(max_segments >= 1 && max_segments <= kMaxGemmSegments, SYM_ERR_INVALID,
              "%s: max_segments=%d out of range", what, max_segments);
  SYM_REQUIRE((long long)rows / kTM + max_segments <= 65535, SYM_ERR_UNSUPPORTED,
              "%s: %d rows too many", what, rows);
  return SYM_OK;
}

extern "C" int sym_moe_gate_up_tiled(const void* x, int T, int H, int I, int rows,
                                     const int32_t* sorted_tokens, const int32_t* seg_expert,
                                     const int32_t* seg_offset, const int32_t* seg_count,
                                     const int32_t* n_segments, int max_segments,
                                     const void* w_gate_up, void* h, void* stream) {
  int rc = check_grouped("moe_gate_up_tiled", T, H, I, rows, max_segments);
  if (rc || rows == 0 || T == 0) return rc;
  SYM_REQUIRE(x && sorted_tokens && seg_expert && seg_offset && seg_count && n_segments &&
                  w_gate_up && h,
              SYM_ERR_INVALID, "moe_gate_up_tiled: null pointer argument");
  SYM_REQUIRE(H % kTK == 0, SYM_ERR_UNSUPPORTED, "moe_gate_up_tiled: H=%d", H);
  TileArgs p{};
  p.a = (const uint16_t*)x;
  p.w = (const uint16_t*)w_gate_up;
  p.sorted_tokens = sorted_tokens;
  p.seg_expert = seg_expert;
  p.seg_offset = seg_offset;
  p.seg_count = seg_count;
  p.n_segments = n_segments;
  p.M = rows;
  p.N = I;
  p.K = H;
  p.out_bf16 = (uint16_t*)h;
  (void)hipGetLastError();
  hipLaunchKernelGGL((gemm_tile_kernel<kGateUp>), dim3(I / 64, rows / kTM + max_segments),
                     dim3(kTileThreads), 0, (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile_kernel");
}

extern "C" int sym_moe_down_tiled(const void* h, int T, int H, int I, int rows,
                                  const int32_t* seg_expert, const int32_t* seg_offset,
                                  const int32_t* seg_count, const int32_t* n_segments,
                                  int max_segments, const void* w_down, float* y, void* stream) {
  int rc = check_grouped("moe_down_tiled", T, H, I, rows, max_segments);
  if (rc || rows == 0 || T == 0) return rc;
  SYM_REQUIRE(h && seg_expert && seg_offset && seg_count && n_segments && w_down && y,
              SYM_ERR_INVALID, "moe_down_tiled: null pointer argument");
  TileArgs p{};
  p.a = (const uint16_t*)h;
  p.w = (const uint16_t*)w_down;
  p.seg_expert = seg_expert;
  p.seg_offset = seg_offset;
  p.seg_count = seg_count;
  p.n_segments = n_segments;
  p.M = rows;
  p.N = H;
  p.K = I;
  p.out_f32 = y;
  (void)hipGetLastError();
  hipLaunchKernelGGL((gemm_tile_kernel<kDown>), dim3(H / kTN, rows / kTM + max_segments),
                     dim3(kTileThreads), 0, (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile_kernel");
}
