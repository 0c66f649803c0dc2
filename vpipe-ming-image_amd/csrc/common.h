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

// Two bf16 (one u32) -> two fp16 (one u32), rounding toward zero. Exact for
// zero and every magnitude in [2^-17, 2^16): bf16's 8 significant bits fit
// fp16's normals, its subnormals down to 2^-17 (a step of 2^-24), and bf16's
// largest value below 2^16, 65280. A finite value of 2^16 or more SATURATES
// to +-65504: the writers of fp16 copies track what they convert with
// range_track and report it with range_report, and the host turns a report
// into MING_ERR_RANGE. Below 2^-17 the low bits are cut to fp16's 2^-24 grid
// and below 2^-24 the value becomes +-0; that loss is NOT tracked (at most
// 2^-24 absolute, against activations of order 1 after the norms).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t u) {
  auto h = __builtin_amdgcn_cvt_pkrtz(bf16_lo(u), bf16_hi(u));
  return __builtin_bit_cast(uint32_t, h);
}

// The largest bf16 magnitude of each 16-bit half seen so far (start from 0):
// one AND and one packed 16-bit max per converted word.
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t range_track(uint32_t seen, uint32_t w) {
  const u16x2_t a = __builtin_bit_cast(u16x2_t, seen);
  const u16x2_t b = __builtin_bit_cast(u16x2_t, w & 0x7fff7fffu);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
}
__device__ __forceinline__ uint32_t range_track4(uint32_t seen, const uint4& v) {
  seen = range_track(seen, v.x);
  seen = range_track(seen, v.y);
  seen = range_track(seen, v.z);
  return range_track(seen, v.w);
}
// Raises *flag (a plain store of 1; concurrent writers store the same value)
// when a tracked magnitude is 2^16 or more, inf or NaN: a value the fp16
// copy does not hold. Only lanes that saw one store.
__device__ __forceinline__ void range_report(int* flag, uint32_t seen) {
  if (flag && ((seen & 0xffffu) >= 0x4780u || (seen >> 16) >= 0x4780u)) *flag = 1;
}

// Two f32 -> two fp16, round to nearest even.
__device__ __forceinline__ uint32_t f32x2_to_f16x2_rne(float a, float b) {
  _Float16 ha = (_Float16)a, hb = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, ha) |
         ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

// Per-head RMSNorm + RoPE of q and k (the qk-norm then the interleaved-pair
// rotation), shared by qk_norm_rope_kernel and the attention kernel's Q
// prologue so both give the same bits. A head's sum of squares is the
// sixteen 8-element chains (eight consecutive elements, fmaf in order)
// added pairwise at group distance 8, 4, 2, 1.
__device__ __forceinline__ float head_ss8(const uint4& v) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = bf16_lo(u[e]), b = bf16_hi(u[e]);
    ss = fmaf(a, a, ss);
    ss = fmaf(b, b, ss);
  }
  return ss;
}
__device__ __forceinline__ float head_rms_inv(float ss, float eps) {
  return 1.0f / sqrtf(ss * (1.0f / 128.0f) + eps);
}
// One interleaved pair (x0, x1): normalized with weight pair w, rounded to
// bf16 (the reference stores the norm), rotated by (c, s) as
// (x0 + i x1)(c + i s), packed to bf16. Every product is rounded before its
// sum (no contraction into an FMA), as the formula is written: the bits then
// follow the source, not the compiler's choice per call site.
__device__ __forceinline__ uint32_t norm_rope_pair(uint32_t u, uint32_t w, float inv, float c,
                                                   float s) {
#pragma clang fp contract(off)
  const uint32_t nb = pack_bf16x2_rne(bf16_lo(u) * inv * bf16_lo(w), bf16_hi(u) * inv * bf16_hi(w));
  const float a = bf16_lo(nb), b = bf16_hi(nb);
  const float re = a * c - b * s;
  const float im = a * s + b * c;
  return pack_bf16x2_rne(re, im);
}

// A 16-byte store with the non-temporal (streaming) hint: the write does not
// allocate in the caches on the way. For an output nothing reads soon (the
// standalone RMSNorm over [4352, 3840]) it measured 16.0 -> 11.1 us (4.2 ->
// 6.0 TB/s) on the MI355X; for one the next kernel reads at once it is slower.
__device__ __forceinline__ void store16_nt(void* p, const uint4& v) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace ming
