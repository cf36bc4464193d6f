// Skinny bf16 GEMMs for the decode projections: out[M, N] = x[M, K] . w[N, K]^T (+ bias[N]),
// optionally with the RMSNorm of x fused in front and the residual add + the next RMSNorm's
// statistics fused behind.
//
// Reference: the fused query_key_value projection and the dense output projection of
// TTNNBailingMoEAttention._forward_decode_paged (ttnn_attention.py:2324, 2459), weights built at
// ttnn_attention.py:2001-2011; the decoder layer's input_layernorm before the attention and the
// residual add + post_attention_layernorm after it (modeling_bailing_moe_v2.py:440-468;
// RMSNorm of DeepseekV2RMSNorm, ttnn_normalization.py:54-68).
//
// Design (gfx950): at decode sizes (M = batch <= 64) a projection streams its weights once. One
// workgroup of 8 waves owns 16 output columns; the waves split K into contiguous K-step ranges
// (K = 2048: 4 steps of 64 each, one batch of loads), issue the weight loads and then the
// activation loads of a batch before its v_mfma_f32_16x16x32_bf16 (weight rows as the B
// operand, MT 16-row tiles of x as A), and reduce their partial accumulators through LDS.
//   NORM: the workgroup first reads its rows' activations once more for the sum of squares
//         (8 waves x their K range, reduced through LDS), then forms the MFMA operand
//         bf16(x * r * gamma) in registers: the same rounding as a separate RMSNorm pass.
//   RES:  the epilogue adds bias and the bf16 residual in fp32, writes the fp32 row and each
//         row's sum of squares over the workgroup's 16 columns (the statistics of the next
//         RMSNorm, finished by its consumer).
#include "common.h"

namespace sym {

constexpr int kLinWaves = 8;
constexpr int kLinThreads = kLinWaves * 64;

__device__ __forceinline__ uint4 ldg16(const uint16_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// bf16(x * r * g) for 8 packed bf16 x and g values (left-to-right products, as the RMSNorm
// kernel).
__device__ __forceinline__ uint4 scale8(uint4 xv, uint4 gv, float r) {
  float xf[8], gf[8];
  unpack8(xv, xf);
  unpack8(gv, gf);
  uint4 o;
  o.x = pack_bf16x2(xf[0] * r * gf[0], xf[1] * r * gf[1]);
  o.y = pack_bf16x2(xf[2] * r * gf[2], xf[3] * r * gf[3]);
  o.z = pack_bf16x2(xf[4] * r * gf[4], xf[5] * r * gf[5]);
  o.w = pack_bf16x2(xf[6] * r * gf[6], xf[7] * r * gf[7]);
  return o;
}

__device__ __forceinline__ float sumsq8(uint4 v) {
  float f[8];
  unpack8(v, f);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s = fmaf(f[i], f[i], s);
  return s;
}

// One batch of S K-steps starting at step st: weight loads, activation loads (and gamma when
// NORM), then the MFMAs.
template <int MT, int S, bool NORM>
__device__ __forceinline__ void proj_batch(const uint16_t* __restrict__ wr,
                                           const uint16_t* const (&xr)[MT],
                                           const uint16_t* __restrict__ gr, const float (&rr)[MT],
                                           int st, int nmt, floatx4 (&acc)[MT]) {
  uint4 b[S][2], a[MT][S][2], gm[NORM ? S : 1][2];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int k = (st + s) << 6;
    b[s][0] = ldg16(wr + k);
    b[s][1] = ldg16(wr + k + 8);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int k = (st + s) << 6;
      a[mt][s][0] = ldg16(xr[mt] + k);
      a[mt][s][1] = ldg16(xr[mt] + k + 8);
    }
  if constexpr (NORM) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int k = (st + s) << 6;
      gm[s][0] = ldg16(gr + k);
      gm[s][1] = ldg16(gr + k + 8);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // every tile is computed (rows past M repeat row M-1; their results are dropped): a branch
  // on the tile count would let the compiler sink the tile's loads behind the first MFMAs
  (void)nmt;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      uint4 a0 = a[mt][s][0], a1 = a[mt][s][1];
      if constexpr (NORM) {
        a0 = scale8(a0, gm[s][0], rr[mt]);
        a1 = scale8(a1, gm[s][1], rr[mt]);
      }
      acc[mt] = mfma16x16x32(a0, b[s][0], acc[mt]);
      acc[mt] = mfma16x16x32(a1, b[s][1], acc[mt]);
    }
  }
}

// Sum of squares of this lane's row (tile mt) over S K-steps starting at st (loads batched).
template <int MT, int S>
__device__ __forceinline__ void sumsq_batch(const uint16_t* const (&xr)[MT], int st,
                                            float (&ss)[MT]) {
  uint4 a[MT][S][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int k = (st + s) << 6;
      a[mt][s][0] = ldg16(xr[mt] + k);
      a[mt][s][1] = ldg16(xr[mt] + k + 8);
    }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < S; ++s) ss[mt] += sumsq8(a[mt][s][0]) + sumsq8(a[mt][s][1]);
}

template <int MT, int U, bool NORM, bool RES>
__global__ __launch_bounds__(kLinThreads) void proj_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, int M, int N, int K, const uint16_t* __restrict__ gamma,
    float eps, const uint16_t* __restrict__ residual, float* __restrict__ sumsq_parts,
    uint16_t* __restrict__ out_bf16, float* __restrict__ out_f32) {
  __shared__ float s_red[kLinWaves][MT][4][64];
  __shared__ float s_ss[NORM ? kLinWaves : 1][16 * MT];
  __shared__ float s_r[16 * MT];
  // gamma of the single-batch path (K = 64 * U * kLinWaves), staged once per workgroup
  __shared__ __align__(16) uint16_t s_g[NORM ? 64 * U * kLinWaves : 1];
  const int col0 = blockIdx.x * 16;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int nsteps = K >> 6;
  const int s_beg = (wave * nsteps) / kLinWaves;
  const int s_end = ((wave + 1) * nsteps) / kLinWaves;
  const uint16_t* wr = w + (size_t)(col0 + r16) * K + kq * 16;
  const uint16_t* gr = NORM ? gamma + kq * 16 : nullptr;
  // RES: this thread's residual element of the first pass is requested before the weights (it
  // does not depend on them), so the epilogue does not wait a round trip for it after the
  // reduction barrier; later passes (M above 16 * MT * gridDim.y) load theirs there
  float res_first = 0.f;
  if constexpr (RES) {
    if (threadIdx.x < 256 * MT) {
      const int l = threadIdx.x & 63;
      const int row = blockIdx.y * 16 * MT + (threadIdx.x >> 8) * 16 + 4 * (l >> 4) +
                      ((threadIdx.x >> 6) & 3);
      if (row < M) res_first = bf16_to_f32(residual[(size_t)row * N + col0 + (l & 15)]);
    }
  }

  for (int mb = blockIdx.y * 16 * MT; mb < M; mb += gridDim.y * 16 * MT) {
    const int nmt = min(MT, (M - mb + 15) >> 4);
    floatx4 acc[MT];
    const uint16_t* xr[MT];
    float rr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      // rows past M read row M-1 (in bounds); their outputs are dropped
      xr[mt] = x + (size_t)min(mb + mt * 16 + r16, M - 1) * K + kq * 16;
      rr[mt] = 1.f;
    }
    bool done = false;
    if constexpr (NORM) {
      if (nsteps == U * kLinWaves) {
        // one batch per wave: activations, gamma and weights in flight together; the sums of
        // squares come from the activation registers, and the same registers feed the MFMAs.
        // The activations are issued first, so the norm statistics (which wait for them only;
        // loads complete in order) are reduced while the weights are still arriving. The wave's
        // 512 bytes of gamma take one load (lane l: k = 4l .. 4l+3 of its range) into LDS, read
        // back after the statistics barrier: the MFMA layout would need eight loads in which
        // 16 lanes each read the same address, which cost about 1 us of load issue.
        uint4 b[U][2], a[MT][U][2], gm[U][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int s = 0; s < U; ++s) {
            const int k = (s_beg + s) << 6;
            a[mt][s][0] = ldg16(xr[mt] + k);
            a[mt][s][1] = ldg16(xr[mt] + k + 8);
          }
        const int kw = s_beg << 6;  // this wave's first k
        const uint2 gl = *reinterpret_cast<const uint2*>(gamma + kw + 4 * lane);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < U; ++s) {
          const int k = (s_beg + s) << 6;
          b[s][0] = ldg16(wr + k);
          b[s][1] = ldg16(wr + k + 8);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          float v = 0.f;
#pragma unroll
          for (int s = 0; s < U; ++s) v += sumsq8(a[mt][s][0]) + sumsq8(a[mt][s][1]);
          v += __shfl_xor(v, 16);
          v += __shfl_xor(v, 32);
          if (kq == 0) s_ss[wave][mt * 16 + r16] = v;
        }
        *reinterpret_cast<uint2*>(&s_g[kw + 4 * lane]) = gl;
        __syncthreads();
        if (threadIdx.x < 16 * MT) {
          float t = 0.f;
#pragma unroll
          for (int i = 0; i < kLinWaves; ++i) t += s_ss[i][threadIdx.x];
          s_r[threadIdx.x] = rsqrtf(t / (float)K + eps);
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < U; ++s) {
          const int k = ((s_beg + s) << 6) + kq * 16;
          gm[s][0] = *reinterpret_cast<const uint4*>(&s_g[k]);
          gm[s][1] = *reinterpret_cast<const uint4*>(&s_g[k + 8]);
        }
        // normalised rows in place, one K-step at a time (a scheduling barrier after each
        // keeps the compiler from converting all of them ahead of the MFMAs)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const float r = s_r[mt * 16 + r16];
#pragma unroll
          for (int s = 0; s < U; ++s) {
            a[mt][s][0] = scale8(a[mt][s][0], gm[s][0], r);
            a[mt][s][1] = scale8(a[mt][s][1], gm[s][1], r);
            acc[mt] = mfma16x16x32(a[mt][s][0], b[s][0], acc[mt]);
            acc[mt] = mfma16x16x32(a[mt][s][1], b[s][1], acc[mt]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        done = true;
      }
    }
    if (!done) {
      if constexpr (NORM) {
        // sum of squares of each row over this wave's K range, then over the 8 waves
        float ss[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) ss[mt] = 0.f;
        {
          int st = s_beg;
          for (; st + U <= s_end; st += U) sumsq_batch<MT, U>(xr, st, ss);
          for (; st < s_end; ++st) sumsq_batch<MT, 1>(xr, st, ss);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          float v = ss[mt];
          v += __shfl_xor(v, 16);
          v += __shfl_xor(v, 32);
          if (kq == 0) s_ss[wave][mt * 16 + r16] = v;
        }
        __syncthreads();
        if (threadIdx.x < 16 * MT) {
          float t = 0.f;
#pragma unroll
          for (int i = 0; i < kLinWaves; ++i) t += s_ss[i][threadIdx.x];
          s_r[threadIdx.x] = rsqrtf(t / (float)K + eps);
        }
        __syncthreads();
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) rr[mt] = s_r[mt * 16 + r16];
      }
      int st = s_beg;
      for (; st + U <= s_end; st += U) proj_batch<MT, U, NORM>(wr, xr, gr, rr, st, nmt, acc);
      for (; st < s_end; ++st) proj_batch<MT, 1, NORM>(wr, xr, gr, rr, st, nmt, acc);
    }

#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_red[wave][mt][i][lane] = acc[mt][i];
    __syncthreads();
    // 256 fragment elements per tile; a 512-thread workgroup covers two tiles per round (the
    // round count is uniform, so the shuffles below see whole waves)
    for (int e = threadIdx.x; e < 256 * MT; e += kLinThreads) {
      // thread -> element i of lane l's fragment of tile mt: row 4*(l/16)+i, column l%16
      const int mt = e >> 8;
      const int l = e & 63;
      const int i = (e >> 6) & 3;
      const int row = mb + mt * 16 + 4 * (l >> 4) + i;
      const int col = col0 + (l & 15);
      float v = 0.f;
#pragma unroll
      for (int wv = 0; wv < kLinWaves; ++wv) v += s_red[wv][mt][i][l];
      if (bias) v += bf16_to_f32(bias[col]);
      const bool ok = row < M;
      if constexpr (RES) {
        if (ok) {
          v += (mb == blockIdx.y * 16 * MT && e == (int)threadIdx.x)
                   ? res_first
                   : bf16_to_f32(residual[(size_t)row * N + col]);
          out_f32[(size_t)row * N + col] = v;
        }
        // sum of squares over the 16 columns of this row (16 consecutive lanes)
        float q = ok ? v * v : 0.f;
        q += __shfl_xor(q, 1);
        q += __shfl_xor(q, 2);
        q += __shfl_xor(q, 4);
        q += __shfl_xor(q, 8);
        if (ok && (l & 15) == 0) sumsq_parts[(size_t)blockIdx.x * M + row] = q;
      } else if (ok) {
        if (out_f32) out_f32[(size_t)row * N + col] = v;
        else out_bf16[(size_t)row * N + col] = f32_to_bf16(v);
      }
    }
    __syncthreads();
  }
}

// Rows in passes of 16 * MT rows for M > 32 with K = 64 * 4 * kLinWaves, workgroup y of the grid
// taking passes y, y + gridDim.y, ...: each wave's weights for its 4 K-steps are loaded once and
// stay in registers for every pass of the workgroup. The next pass's activations
// are requested into the same registers as soon as the current pass's MFMAs have read them, so
// they arrive during the cross-wave reduction and the stores; the epilogue's bias and residual
// are requested when the pass starts. (The general kernel above re-streams the weights and
// waits for every load in every pass.)
template <bool NORM, bool RES, int MT = 2>
__global__ __launch_bounds__(kLinThreads) void proj_rows_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, int M, int N, int K, const uint16_t* __restrict__ gamma,
    float eps, const uint16_t* __restrict__ residual, float* __restrict__ sumsq_parts,
    uint16_t* __restrict__ out_bf16, float* __restrict__ out_f32) {
  constexpr int U = 4;
  static_assert(256 * MT <= kLinThreads, "at most one output element per thread and pass");
  __shared__ float s_red[kLinWaves][MT][4][64];
  __shared__ float s_ss[NORM ? kLinWaves : 1][16 * MT];
  __shared__ float s_r[16 * MT];
  // gamma (K = 64 * U * kLinWaves values), staged once: each wave stores its 512 bytes with
  // one load before the first pass's statistics barrier, and every pass reads it from LDS
  __shared__ __align__(16) uint16_t s_g[NORM ? 64 * U * kLinWaves : 1];
  const int col0 = blockIdx.x * 16;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int k0 = wave * U * 64 + kq * 16;  // this lane's first element of the wave's K range
  const uint16_t* wr = w + (size_t)(col0 + r16) * K + k0;
  // this thread's output element of each pass: element i of lane l's fragment of tile mt
  // (with MT = 1 the upper 4 waves have no element: the store is wave-uniformly skipped)
  const bool e_any = threadIdx.x < 256 * MT;
  const int e_mt = min((int)(threadIdx.x >> 8), MT - 1), e_l = threadIdx.x & 63,
            e_i = (threadIdx.x >> 6) & 3;
  const int e_row = e_mt * 16 + 4 * (e_l >> 4) + e_i;  // + mb
  const int e_col = col0 + (e_l & 15);

  uint4 b[U][2];
#pragma unroll
  for (int s = 0; s < U; ++s) {
    b[s][0] = ldg16(wr + s * 64);
    b[s][1] = ldg16(wr + s * 64 + 8);
  }
  // rows past M read row M - 1 (in bounds); their outputs are dropped
  uint4 a[MT][U][2];
  auto load_rows = [&](int mb) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint16_t* xr = x + (size_t)min(mb + mt * 16 + r16, M - 1) * K + k0;
#pragma unroll
      for (int s = 0; s < U; ++s) {
        a[mt][s][0] = ldg16(xr + s * 64);
        a[mt][s][1] = ldg16(xr + s * 64 + 8);
      }
    }
  };
  // workgroup y of the grid takes passes y, y + gridDim.y, ...
  const int mb0 = blockIdx.y * 16 * MT, mstep = gridDim.y * 16 * MT;
  load_rows(mb0);
  if constexpr (NORM) {
    const uint2 gl = *reinterpret_cast<const uint2*>(gamma + wave * U * 64 + 4 * lane);
    *reinterpret_cast<uint2*>(&s_g[wave * U * 64 + 4 * lane]) = gl;
  }
  const float bias_v = bias ? bf16_to_f32(bias[e_col]) : 0.f;

  for (int mb = mb0; mb < M; mb += mstep) {
    const int row = mb + e_row;
    const bool ok = e_any && row < M;
    float res_v = 0.f;
    if constexpr (RES) res_v = ok ? bf16_to_f32(residual[(size_t)row * N + e_col]) : 0.f;
    floatx4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
    if constexpr (NORM) {
      // gamma comes from LDS in each pass (after the statistics barrier below), rather than
      // held in registers: they go to the weights
      uint4 gm[U][2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float v = 0.f;
#pragma unroll
        for (int s = 0; s < U; ++s) v += sumsq8(a[mt][s][0]) + sumsq8(a[mt][s][1]);
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (kq == 0) s_ss[wave][mt * 16 + r16] = v;
      }
      __syncthreads();
      if (threadIdx.x < 16 * MT) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < kLinWaves; ++i) t += s_ss[i][threadIdx.x];
        s_r[threadIdx.x] = rsqrtf(t / (float)K + eps);
      }
      __syncthreads();
      // normalised rows in place, one K-step at a time (a scheduling barrier after each keeps
      // the compiler from converting all of them ahead of the MFMAs); with one row tile per
      // pass gamma is read from LDS per step, which holds one step's fragments in registers
      if constexpr (MT == 1) {
        const float r = s_r[r16];
#pragma unroll
        for (int s = 0; s < U; ++s) {
          const uint4 g0 = *reinterpret_cast<const uint4*>(&s_g[k0 + s * 64]);
          const uint4 g1 = *reinterpret_cast<const uint4*>(&s_g[k0 + s * 64 + 8]);
          a[0][s][0] = scale8(a[0][s][0], g0, r);
          a[0][s][1] = scale8(a[0][s][1], g1, r);
          acc[0] = mfma16x16x32(a[0][s][0], b[s][0], acc[0]);
          acc[0] = mfma16x16x32(a[0][s][1], b[s][1], acc[0]);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int s = 0; s < U; ++s) {
          gm[s][0] = *reinterpret_cast<const uint4*>(&s_g[k0 + s * 64]);
          gm[s][1] = *reinterpret_cast<const uint4*>(&s_g[k0 + s * 64 + 8]);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const float r = s_r[mt * 16 + r16];
#pragma unroll
          for (int s = 0; s < U; ++s) {
            a[mt][s][0] = scale8(a[mt][s][0], gm[s][0], r);
            a[mt][s][1] = scale8(a[mt][s][1], gm[s][1], r);
            acc[mt] = mfma16x16x32(a[mt][s][0], b[s][0], acc[mt]);
            acc[mt] = mfma16x16x32(a[mt][s][1], b[s][1], acc[mt]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int s = 0; s < U; ++s) {
          acc[mt] = mfma16x16x32(a[mt][s][0], b[s][0], acc[mt]);
          acc[mt] = mfma16x16x32(a[mt][s][1], b[s][1], acc[mt]);
        }
    }
    // the MFMAs have read the rows: the next pass's rows go into the same registers now
    if (mb + mstep < M) load_rows(mb + mstep);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_red[wave][mt][i][lane] = acc[mt][i];
    __syncthreads();
    float v = bias_v;
#pragma unroll
    for (int wv = 0; wv < kLinWaves; ++wv) v += s_red[wv][e_mt][e_i][e_l];
    if (!e_any) {
      __syncthreads();
      continue;
    }
    if constexpr (RES) {
      v += res_v;
      if (ok) out_f32[(size_t)row * N + e_col] = v;
      // sum of squares over the 16 columns of this row (16 consecutive lanes)
      float q = ok ? v * v : 0.f;
      q += __shfl_xor(q, 1);
      q += __shfl_xor(q, 2);
      q += __shfl_xor(q, 4);
      q += __shfl_xor(q, 8);
      if (ok && (e_l & 15) == 0) sumsq_parts[(size_t)blockIdx.x * M + row] = q;
    } else if (ok) {
      if (out_f32) out_f32[(size_t)row * N + e_col] = v;
      else out_bf16[(size_t)row * N + e_col] = f32_to_bf16(v);
    }
    __syncthreads();
  }
}

}  // namespace sym

using namespace sym;

static int check_proj(const char* what, const void* x, const void* w, int M, int N, int K) {
  SYM_REQUIRE(M >= 0, SYM_ERR_INVALID, "%s: M=%d < 0", what, M);
  SYM_REQUIRE(M == 0 || (x && w), SYM_ERR_INVALID, "%s: null pointer argument", what);
  SYM_REQUIRE(N > 0 && N % 16 == 0 && N / 16 <= 2147483647, SYM_ERR_UNSUPPORTED,
              "%s: N=%d must be a positive multiple of 16", what, N);
  SYM_REQUIRE(K > 0 && K % 64 == 0, SYM_ERR_UNSUPPORTED,
              "%s: K=%d must be a positive multiple of 64", what, K);
  return SYM_OK;
}

template <bool NORM, bool RES>
static void launch_proj(const void* x, const void* w, const void* bias, int M, int N, int K,
                        const void* gamma, float eps, const void* residual, float* sumsq_parts,
                        void* out_bf16, float* out_f32, hipStream_t s) {
  // Above 32 rows with K = 2048: row passes over weights held in registers, the passes spread
  // over a second grid dimension (the weights of a column tile are re-read from L2 by its
  // row-block workgroups, which share an XCD: N / 16 is a multiple of 8). Without the norm: one
  // 32-row pass per workgroup (dense 2048 x 2048 at 128 rows: 19.7 -> 13.4 us). With the norm
  // fused: two 16-row passes per workgroup, 128 VGPRs so that two workgroups share a CU (QKV
  // 3072 x 2048 at 128 rows: 25.4 us with 32-row passes in one row block, 25.7 with one 16-row
  // pass per workgroup, 21.7); up to 64 rows one 16-row pass per workgroup is faster (QKV at 64
  // rows: 15.3 against 16.1 us for two passes). Other K above 32 rows: passes of 64 rows (32
  // with the norm fused, whose single-batch path a 64-row pass would leave: 24.4 against 18.7 us
  // for 3072 x 2048 at 64 rows), each streaming the weights.
  if (M > 32 && K == 64 * 4 * kLinWaves && NORM)
    hipLaunchKernelGGL((proj_rows_kernel<NORM, RES, 1>),
                       dim3(N / 16, M <= 64 ? (M + 15) / 16 : (M + 31) / 32),
                       dim3(kLinThreads), 0, s, (const uint16_t*)x, (const uint16_t*)w,
                       (const uint16_t*)bias, M, N, K, (const uint16_t*)gamma, eps,
                       (const uint16_t*)residual, sumsq_parts, (uint16_t*)out_bf16, out_f32);
  else if (M > 32 && K == 64 * 4 * kLinWaves)
    hipLaunchKernelGGL((proj_rows_kernel<NORM, RES, 2>), dim3(N / 16, (M + 31) / 32),
                       dim3(kLinThreads), 0, s, (const uint16_t*)x, (const uint16_t*)w,
                       (const uint16_t*)bias, M, N, K, (const uint16_t*)gamma, eps,
                       (const uint16_t*)residual, sumsq_parts, (uint16_t*)out_bf16, out_f32);
  else if (M > 32 && !NORM)
    hipLaunchKernelGGL((proj_kernel<4, 4, NORM, RES>), dim3(N / 16), dim3(kLinThreads), 0, s,
                       (const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)bias, M, N, K,
                       (const uint16_t*)gamma, eps, (const uint16_t*)residual, sumsq_parts,
                       (uint16_t*)out_bf16, out_f32);
  else if (!NORM)
    // 16-row blocks as a second grid dimension: each workgroup reads half the activations of a
    // 32-row batch and the grid doubles (dense 2048 x 2048 at 32 rows: 8.3 -> 6.7 us). With the
    // norm fused the 16-row kernel needs 172 VGPRs (2 rounds of workgroups), so it keeps 32.
    hipLaunchKernelGGL((proj_kernel<1, 4, NORM, RES>), dim3(N / 16, (M + 15) / 16),
                       dim3(kLinThreads), 0, s, (const uint16_t*)x, (const uint16_t*)w,
                       (const uint16_t*)bias, M, N, K, (const uint16_t*)gamma, eps,
                       (const uint16_t*)residual, sumsq_parts, (uint16_t*)out_bf16, out_f32);
  else
    hipLaunchKernelGGL((proj_kernel<2, 4, NORM, RES>), dim3(N / 16), dim3(kLinThreads), 0, s,
                       (const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)bias, M, N, K,
                       (const uint16_t*)gamma, eps, (const uint16_t*)residual, sumsq_parts,
                       (uint16_t*)out_bf16, out_f32);
}

extern "C" int sym_linear_bf16(const void* x, const void* w, const void* bias, int M, int N,
                               int K, void* out, int out_fp32, void* stream) {
  int rc = check_proj("linear_bf16", x, w, M, N, K);
  if (rc || M == 0) return rc;
  SYM_REQUIRE(out, SYM_ERR_INVALID, "linear_bf16: null pointer argument");
  (void)hipGetLastError();
  launch_proj<false, false>(x, w, bias, M, N, K, nullptr, 0.f, nullptr, nullptr,
                            out_fp32 ? nullptr : out, out_fp32 ? (float*)out : nullptr,
                            (hipStream_t)stream);
  return sym_host::check_launch("proj_kernel");
}

extern "C" int sym_rmsnorm_linear_bf16(const void* x, const void* gamma, float eps,
                                       const void* w, const void* bias, int M, int N, int K,
                                       void* out, int out_fp32, void* stream) {
  int rc = check_proj("rmsnorm_linear_bf16", x, w, M, N, K);
  if (rc || M == 0) return rc;
  SYM_REQUIRE(gamma && out, SYM_ERR_INVALID, "rmsnorm_linear_bf16: null pointer argument");
  (void)hipGetLastError();
  launch_proj<true, false>(x, w, bias, M, N, K, gamma, eps, nullptr, nullptr,
                           out_fp32 ? nullptr : out, out_fp32 ? (float*)out : nullptr,
                           (hipStream_t)stream);
  return sym_host::check_launch("proj_kernel");
}

extern "C" int sym_linear_residual_bf16(const void* x, const void* w, const void* bias,
                                        const void* residual, int M, int N, int K, float* out,
                                        float* sumsq_parts, void* stream) {
  int rc = check_proj("linear_residual_bf16", x, w, M, N, K);
  if (rc || M == 0) return rc;
  SYM_REQUIRE(residual && out && sumsq_parts, SYM_ERR_INVALID,
              "linear_residual_bf16: null pointer argument");
  (void)hipGetLastError();
  launch_proj<false, true>(x, w, bias, M, N, K, nullptr, 0.f, residual, sumsq_parts, nullptr,
                           out, (hipStream_t)stream);
  return sym_host::check_launch("proj_kernel");
}
