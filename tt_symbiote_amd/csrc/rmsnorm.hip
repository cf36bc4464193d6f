// Row RMSNorm with an optional fused residual add, bf16 or fp32 in, fp32 statistics.
// Reference: the decoder layer's input_layernorm / post_attention_layernorm and residual adds
// (modeling_bailing_moe_v2.py:440-468), RMSNorm formula of DeepseekV2RMSNorm
// (ttnn_normalization.py:54-68):
//   s   = x + residual                    (fp32; written to residual_out as the layer's
//                                          residual stream, no intermediate bf16 rounding)
//   out = bf16(weight * s * rsqrt(mean(s^2) + eps))
// cols = 512 * NP (NP <= 8): one wave per row, 4 rows per workgroup; lane l owns the 8
// consecutive columns 8 (64 p + l) .. +7 of chunk p, all NP chunks loaded before any use, and the
// row's sum of squares is a wave reduction (no LDS, no barrier). A prompt of ~10 k rows is then
// ~2.5 k workgroups instead of one 256-thread workgroup per row (bf16 rows of 2048, 9942 rows:
// 22.1 -> 17.3 us).
// Other widths: one workgroup per row; each thread owns 8 consecutive columns per pass.
#include "common.h"

namespace sym {

constexpr int kNormThreads = 256;
constexpr int kNormMaxPasses = 8;  // cols <= 256 * 8 * 8 = 16384

// 8 consecutive values of a row as fp32: one 16-byte load of bf16, two of fp32
__device__ __forceinline__ void load8(const uint16_t* p, float (&v)[8]) {
  unpack8(*reinterpret_cast<const uint4*>(p), v);
}
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// TX: uint16_t (bf16 x) or float (fp32 x, e.g. a projection's fp32 output)
template <typename TX>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const TX* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ w, int cols, float eps, uint16_t* __restrict__ out,
    float* __restrict__ res_out) {
  __shared__ float s_part[kNormThreads / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const size_t base = (size_t)row * cols;
  float v[kNormMaxPasses][8];
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < kNormMaxPasses; ++p) {
    const int c = (p * kNormThreads + tid) * 8;
    if (c < cols) {
      load8(x + base + c, v[p]);
      if (res) {
        float r[8];
        unpack8(*reinterpret_cast<const uint4*>(res + base + c), r);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[p][i] += r[i];
        float4* dst = reinterpret_cast<float4*>(res_out + base + c);
        dst[0] = make_float4(v[p][0], v[p][1], v[p][2], v[p][3]);
        dst[1] = make_float4(v[p][4], v[p][5], v[p][6], v[p][7]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(v[p][i], v[p][i], ss);
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += s_part[i];
  const float r = rsqrtf(tot / (float)cols + eps);
#pragma unroll
  for (int p = 0; p < kNormMaxPasses; ++p) {
    const int c = (p * kNormThreads + tid) * 8;
    if (c < cols) {
      float wf[8];
      unpack8(*reinterpret_cast<const uint4*>(w + c), wf);
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = v[p][i] * r * wf[i];
      uint4 q;
      q.x = pack_bf16x2(o[0], o[1]);
      q.y = pack_bf16x2(o[2], o[3]);
      q.z = pack_bf16x2(o[4], o[5]);
      q.w = pack_bf16x2(o[6], o[7]);
      *reinterpret_cast<uint4*>(out + base + c) = q;
    }
  }
}

template <typename TX, int NP>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(
    const TX* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ w, int rows, int cols, float eps, uint16_t* __restrict__ out,
    float* __restrict__ res_out) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves: no barrier below
  const int lane = threadIdx.x & 63;
  const size_t base = (size_t)row * cols;
  float v[NP][8];
#pragma unroll
  for (int p = 0; p < NP; ++p) load8(x + base + (p * 64 + lane) * 8, v[p]);
  if (res) {
    uint4 rv[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
      rv[p] = *reinterpret_cast<const uint4*>(res + base + (p * 64 + lane) * 8);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float r[8];
      unpack8(rv[p], r);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[p][i] += r[i];
      float4* dst = reinterpret_cast<float4*>(res_out + base + (p * 64 + lane) * 8);
      dst[0] = make_float4(v[p][0], v[p][1], v[p][2], v[p][3]);
      dst[1] = make_float4(v[p][4], v[p][5], v[p][6], v[p][7]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(v[p][i], v[p][i], ss);
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)cols + eps);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int c = (p * 64 + lane) * 8;
    float wf[8];
    unpack8(*reinterpret_cast<const uint4*>(w + c), wf);
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = v[p][i] * r * wf[i];
    uint4 q;
    q.x = pack_bf16x2(o[0], o[1]);
    q.y = pack_bf16x2(o[2], o[3]);
    q.z = pack_bf16x2(o[4], o[5]);
    q.w = pack_bf16x2(o[6], o[7]);
    *reinterpret_cast<uint4*>(out + base + c) = q;
  }
}

}  // namespace sym

using namespace sym;

// the wave-per-row kernel for cols = 512 * NP, NP <= 8; false for other widths
template <typename TX>
static bool launch_rows(const TX* x, const uint16_t* res, const uint16_t* w, int rows, int cols,
                        float eps, uint16_t* out, float* res_out, hipStream_t s) {
  if (cols % 512 != 0 || cols > 4096) return false;
  const dim3 grid((rows + 3) / 4), block(256);
  switch (cols / 512) {
#define SYM_NORM_ROWS(NP)                                                                     \
  case NP:                                                                                    \
    hipLaunchKernelGGL((rmsnorm_rows_kernel<TX, NP>), grid, block, 0, s, x, res, w, rows, cols, \
                       eps, out, res_out);                                                    \
    return true;
    SYM_NORM_ROWS(1) SYM_NORM_ROWS(2) SYM_NORM_ROWS(3) SYM_NORM_ROWS(4)
    SYM_NORM_ROWS(5) SYM_NORM_ROWS(6) SYM_NORM_ROWS(7) SYM_NORM_ROWS(8)
#undef SYM_NORM_ROWS
  }
  return false;
}

extern "C" int sym_rmsnorm_bf16(const void* x, const void* residual, const void* weight, int rows,
                                int cols, float eps, void* out, float* residual_out, void* stream) {
  SYM_REQUIRE(rows >= 0, SYM_ERR_INVALID, "rmsnorm: rows=%d < 0", rows);
  if (rows == 0) return SYM_OK;
  SYM_REQUIRE(x && weight && out, SYM_ERR_INVALID, "rmsnorm: null pointer argument");
  SYM_REQUIRE(!residual || residual_out, SYM_ERR_INVALID,
              "rmsnorm: residual given without residual_out");
  SYM_REQUIRE(cols > 0 && cols % 8 == 0 && cols <= kNormThreads * 8 * kNormMaxPasses,
              SYM_ERR_UNSUPPORTED, "rmsnorm: cols=%d (multiple of 8, <= %d)", cols,
              kNormThreads * 8 * kNormMaxPasses);
  (void)hipGetLastError();
  if (!launch_rows((const uint16_t*)x, (const uint16_t*)residual, (const uint16_t*)weight, rows,
                   cols, eps, (uint16_t*)out, residual_out, (hipStream_t)stream))
    hipLaunchKernelGGL(rmsnorm_kernel<uint16_t>, dim3(rows), dim3(kNormThreads), 0,
                       (hipStream_t)stream, (const uint16_t*)x, (const uint16_t*)residual,
                       (const uint16_t*)weight, cols, eps, (uint16_t*)out, residual_out);
  return sym_host::check_launch("rmsnorm_kernel");
}

extern "C" int sym_rmsnorm_f32(const float* x, const void* residual, const void* weight, int rows,
                               int cols, float eps, void* out, float* residual_out,
                               void* stream) {
  SYM_REQUIRE(rows >= 0, SYM_ERR_INVALID, "rmsnorm_f32: rows=%d < 0", rows);
  if (rows == 0) return SYM_OK;
  SYM_REQUIRE(x && weight && out, SYM_ERR_INVALID, "rmsnorm_f32: null pointer argument");
  SYM_REQUIRE(!residual || residual_out, SYM_ERR_INVALID,
              "rmsnorm_f32: residual given without residual_out");
  SYM_REQUIRE(cols > 0 && cols % 8 == 0 && cols <= kNormThreads * 8 * kNormMaxPasses,
              SYM_ERR_UNSUPPORTED, "rmsnorm_f32: cols=%d (multiple of 8, <= %d)", cols,
              kNormThreads * 8 * kNormMaxPasses);
  SYM_REQUIRE(((uintptr_t)x & 15) == 0 && (!residual_out || ((uintptr_t)residual_out & 15) == 0),
              SYM_ERR_INVALID, "rmsnorm_f32: x and residual_out must be 16-byte aligned");
  (void)hipGetLastError();
  if (!launch_rows(x, (const uint16_t*)residual, (const uint16_t*)weight, rows, cols, eps,
                   (uint16_t*)out, residual_out, (hipStream_t)stream))
    hipLaunchKernelGGL(rmsnorm_kernel<float>, dim3(rows), dim3(kNormThreads), 0,
                       (hipStream_t)stream, x, (const uint16_t*)residual,
                       (const uint16_t*)weight, cols, eps, (uint16_t*)out, residual_out);
  return sym_host::check_launch("rmsnorm_kernel");
}
