// Device helpers shared by the gfx950 kernels: bf16 bit conversions, wave64 reductions,
// MFMA operand types, and the error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/symbiote_mi355x.h"

namespace sym {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 -> bf16 (the rounding torch uses for .to(torch.bfloat16)), with
// gfx950's v_cvt_pk_bf16_f32 (two values per instruction).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const floatx2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// ---- OCP fp8 e4m3fn (1 sign, 4 exponent bits with bias 7, 3 mantissa bits; no infinities,
// 0x7f / 0xff are NaN; largest finite 448). gfx950's v_cvt_pk_f32_fp8 / v_cvt_pk_fp8_f32 use
// this format. Every e4m3fn value is exact in bf16 and fp32.
constexpr float kFp8Max = 448.0f;

// 4 e4m3fn bytes -> 4 bf16 (two packed words), exact: gfx950's v_cvt_scalef32_pk_bf16_fp8 with
// scale 1 converts two bytes per instruction (checked on the device against v_cvt_pk_f32_fp8 +
// v_cvt_pk_bf16_f32 for every byte value in every byte position: identical bits).
__device__ __forceinline__ uint2 fp8x4_to_bf16x4(uint32_t w) {
  return make_uint2(
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)));
}

// 8 e4m3fn bytes (two words) -> the 8 bf16 of one MFMA operand, exact.
__device__ __forceinline__ uint4 fp8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
  const uint2 a = fp8x4_to_bf16x4(w0), b = fp8x4_to_bf16x4(w1);
  return make_uint4(a.x, a.y, b.x, b.y);
}

// 4 floats -> 4 e4m3fn bytes, round to nearest even. Callers clamp to [-448, 448] first, so
// the result is always finite.
__device__ __forceinline__ uint32_t f32x4_to_fp8x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

__device__ __forceinline__ float clamp_fp8(float x) {
  return fminf(fmaxf(x, -kFp8Max), kFp8Max);
}

// 2^x with the hardware v_exp_f32 alone, for softmax weights. exp2f compiles to a longer
// sequence here (the library keeps results below 2^-126 as denormals: five instructions instead
// of one); a softmax weight that small is 0 for every purpose.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 8 bf16 packed in a uint4 -> 8 floats.
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x);
  f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
  f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z);
  f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(bf16x8, v);
}

// 16 bytes per lane from global memory (base + 32-bit byte offset) into LDS at lds_base + 16 *
// lane (LDS-DMA, global_load_lds_dwordx4; lds_base wave-uniform, in M0). Written as asm so that
// the compiler does not add its own (conservative) waits for these LDS writes: the kernels wait
// for them explicitly (s_waitcnt vmcnt) before the barrier that publishes the data. M0 is written
// here only; no other instruction of the kernels that use this reads M0. On this generation an
// LDS-DMA instruction needs one wait state after an SALU write of M0 (else it may take the
// previous M0, i.e. the previous DMA's destination); the compiler inserts no wait states inside
// inline asm, hence the s_nop.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// base and lds_base are wave-uniform by construction; readfirstlane states it where the
// compiler cannot prove it (values derived from lane shuffles), at no cost where it can.
__device__ __forceinline__ void dma16(const uint16_t* base, uint32_t off,
                                      const uint16_t* lds_base) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_base);
  // (readfirstlane returns int: each half goes through uint32_t, so that the low half is not
  // sign-extended into the high one)
  const uint64_t g = (uint64_t)(uintptr_t)base;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)g);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(g >> 32));
  const uint64_t gu = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off),
               "s"((const uint16_t*)(uintptr_t)gu)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// 8 bytes per lane from LDS, transposed within each group of 16 lanes (gfx950
// ds_read_b64_tr_b16): lane 16G + i receives, as its 16-bit elements j = 0..3, element i % 4 of
// the 8 bytes that lane 16G + 4j + i / 4 addresses. p points into __shared__ memory.
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(p));
  return __builtin_bit_cast(uint2, r);
}

// 16x16x32 bf16 MFMA, fp32 accumulate. Operand layout (wave64):
//   A[16 x 32]: lane l holds A[l % 16][8*(l/16) .. 8*(l/16)+7]
//   B[32 x 16]: lane l holds B[8*(l/16) .. +7][l % 16]
//   D[16 x 16]: lane l holds D[4*(l/16) + i][l % 16], i = 0..3
__device__ __forceinline__ floatx4 mfma16x16x32(const uint4& a, const uint4& b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

typedef float floatx16 __attribute__((ext_vector_type(16)));

// 32x32x16 bf16 MFMA, fp32 accumulate. Operand layout (wave64):
//   A[32 x 16]: lane l holds A[l % 32][8*(l/32) .. 8*(l/32)+7]
//   B[16 x 32]: lane l holds B[8*(l/32) .. +7][l % 32]
//   D[32 x 32]: lane l holds D[8*j + 4*(l/32) + i][l % 32] in element 4j + i, j, i = 0..3
__device__ __forceinline__ floatx16 mfma32x32x16(const uint4& a, const uint4& b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

}  // namespace sym

// ---- host-side error plumbing (one message per calling thread) ----
namespace sym_host {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// compute units of the current device (cached per device; 256 if the query fails)
int cu_count();
}  // namespace sym_host

#define SYM_REQUIRE(cond, code, ...)                         \
  do {                                                       \
    if (!(cond)) return sym_host::set_error((code), __VA_ARGS__); \
  } while (0)
