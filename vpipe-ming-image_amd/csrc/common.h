// Shared device helpers for the MI355X (gfx950) kernels of the DiT
// block-projection path. Wave64 throughout; bf16 values travel as their
// uint16 bit patterns.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ming {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_lo(uint32_t u) {
  return __uint_as_float(u << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t u) {
  return __uint_as_float(u & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float((uint32_t)h << 16);
}

// Round-to-nearest-even f32 -> bf16; NaN stays a quiet NaN (0x7fc0), the
// generator's convention (ming-generator.cc:44-52).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// The same round-to-nearest-even pair conversion by gfx950's
// v_cvt_pk_bf16_f32 (one instruction for two values). Identical to
// pack_bf16x2 for every non-NaN input; a NaN stays a quiet NaN.
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  const bf16x2v v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// silu(g) = g / (1 + exp(-g)) in f32: the SwiGLU gate (ming_ops.metal:97-112).
// One definition for the standalone SwiGLU and the projection epilogue that
// fuses it, so the two give the same bits. The hardware base-2 exponential
// and reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each) replace expf's
// range reduction and the IEEE divide: two transcendental ops per element
// instead of ~30 VALU ops, which matters in the projection epilogue where one
// wave per SIMD leaves nothing to hide them behind. Limits: g -> -inf gives
// e = inf, rcp = 0, silu = -0; g -> +inf gives e = 0, silu = g.
__device__ __forceinline__ float silu_f(float g) {
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// Two bf16 (one u32) -> two fp16 (one u32). Exact for every value inside
// fp16's range, so the rounding mode of the packed conversion is moot.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t u) {
  auto h = __builtin_amdgcn_cvt_pkrtz(bf16_lo(u), bf16_hi(u));
  return __builtin_bit_cast(uint32_t, h);
}

// Two f32 -> two fp16, round to nearest even.
__device__ __forceinline__ uint32_t f32x2_to_f16x2_rne(float a, float b) {
  _Float16 ha = (_Float16)a, hb = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, ha) |
         ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace ming
