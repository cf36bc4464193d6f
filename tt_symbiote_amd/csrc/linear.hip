// Skinny bf16 GEMM for the decode projections: out[M, N] = x[M, K] . w[N, K]^T (+ bias[N]).
//
// Reference: the fused query_key_value projection and the dense output projection of
// TTNNBailingMoEAttention._forward_decode_paged (ttnn_attention.py:2324, 2459), weights built at
// ttnn_attention.py:2001-2011.
//
// Design (gfx950): at decode sizes (M = batch <= 64) the GEMM streams its weights once. One
// workgroup owns 16 output columns; its 4 waves split K into contiguous K-step ranges, issue the
// weight and activation loads of U K-steps per batch before their MFMAs
// (v_mfma_f32_16x16x32_bf16, weight rows as the B operand, up to MT 16-row tiles of x as A), and
// reduce their partial accumulators through LDS. Output in bf16 or fp32.
#include "common.h"

namespace sym {

template <int MT, int U>
__global__ __launch_bounds__(256) void linear_bf16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, int M, int N, int K, uint16_t* __restrict__ out_bf16,
    float* __restrict__ out_f32) {
  __shared__ float s_red[4][MT][4][64];
  const int col0 = blockIdx.x * 16;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int nsteps = K >> 6;
  const int s_beg = (wave * nsteps) >> 2;
  const int s_end = ((wave + 1) * nsteps) >> 2;
  const uint16_t* wr = w + (size_t)(col0 + r16) * K + kq * 16;

  for (int mb = 0; mb < M; mb += 16 * MT) {
    const int nmt = min(MT, (M - mb + 15) >> 4);
    floatx4 acc[MT];
    const uint16_t* xr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      // rows past M read row M-1 (in bounds); their outputs are dropped
      xr[mt] = x + (size_t)min(mb + mt * 16 + r16, M - 1) * K + kq * 16;
    }
    int st = s_beg;
    for (; st + U <= s_end; st += U) {
      uint4 b[U][2], a[MT][U][2];
#pragma unroll
      for (int s = 0; s < U; ++s) {
        const int k = (st + s) << 6;
        b[s][0] = *reinterpret_cast<const uint4*>(wr + k);
        b[s][1] = *reinterpret_cast<const uint4*>(wr + k + 8);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int s = 0; s < U; ++s) {
          const int k = (st + s) << 6;
          a[mt][s][0] = *reinterpret_cast<const uint4*>(xr[mt] + k);
          a[mt][s][1] = *reinterpret_cast<const uint4*>(xr[mt] + k + 8);
        }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (mt < nmt) {
#pragma unroll
          for (int s = 0; s < U; ++s) {
            acc[mt] = mfma16x16x32(a[mt][s][0], b[s][0], acc[mt]);
            acc[mt] = mfma16x16x32(a[mt][s][1], b[s][1], acc[mt]);
          }
        }
      }
    }
    for (; st < s_end; ++st) {
      const int k = st << 6;
      const uint4 b0 = *reinterpret_cast<const uint4*>(wr + k);
      const uint4 b1 = *reinterpret_cast<const uint4*>(wr + k + 8);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 a0 = *reinterpret_cast<const uint4*>(xr[mt] + k);
        const uint4 a1 = *reinterpret_cast<const uint4*>(xr[mt] + k + 8);
        if (mt < nmt) {
          acc[mt] = mfma16x16x32(a0, b0, acc[mt]);
          acc[mt] = mfma16x16x32(a1, b1, acc[mt]);
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (mt < nmt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s_red[wave][mt][i][lane] = acc[mt][i];
      }
    }
    __syncthreads();
    {
      const int l = threadIdx.x & 63;
      const int i = threadIdx.x >> 6;
      const int col = col0 + (l & 15);
      const float bv = bias ? bf16_to_f32(bias[col]) : 0.f;
      for (int mt = 0; mt < nmt; ++mt) {
        const int row = mb + mt * 16 + 4 * (l >> 4) + i;
        const float v = (s_red[0][mt][i][l] + s_red[1][mt][i][l]) +
                        (s_red[2][mt][i][l] + s_red[3][mt][i][l]) + bv;
        if (row < M) {
          if (out_f32) out_f32[(size_t)row * N + col] = v;
          else out_bf16[(size_t)row * N + col] = f32_to_bf16(v);
        }
      }
    }
    __syncthreads();
  }
}

}  // namespace sym

using namespace sym;

extern "C" int sym_linear_bf16(const void* x, const void* w, const void* bias, int M, int N,
                               int K, void* out, int out_fp32, void* stream) {
  SYM_REQUIRE(M >= 0, SYM_ERR_INVALID, "linear_bf16: M=%d < 0", M);
  if (M == 0) return SYM_OK;
  SYM_REQUIRE(x && w && out, SYM_ERR_INVALID, "linear_bf16: null pointer argument");
  SYM_REQUIRE(N > 0 && N % 16 == 0, SYM_ERR_UNSUPPORTED,
              "linear_bf16: N=%d must be a positive multiple of 16", N);
  SYM_REQUIRE(K > 0 && K % 64 == 0, SYM_ERR_UNSUPPORTED,
              "linear_bf16: K=%d must be a positive multiple of 64", K);
  (void)hipGetLastError();
  hipLaunchKernelGGL((linear_bf16_kernel<2, 4>), dim3(N / 16), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)bias, M, N, K,
                     out_fp32 ? nullptr : (uint16_t*)out, out_fp32 ? (float*)out : nullptr);
  return sym_host::check_launch("linear_bf16_kernel");
}
