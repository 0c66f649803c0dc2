// MFMA throughput ceiling under the board's power limit: back-to-back
// v_mfma_f32_32x32x16_{f16,bf16} on register-resident operands, the
// projection kernels' shape and occupancy (one 256-thread block per CU, each
// wave 16 independent 32x32 accumulators fed by 2 A and 8 B fragments, as
// one k16 step of qproj_fast). Random operands switch the multiplier inputs
// the way real data does; zero operands show what the same instruction
// stream reaches when little switches. A calibration for the bench, not a
// compute path: nothing in the library calls it.
#include <hip/hip_runtime.h>
#include <cstdint>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));

namespace {

__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Two 16-bit values of magnitude in [0.5, 2): random sign and mantissa bits,
// exponent field 14 or 15 for fp16, 126 or 127 for bf16.
__device__ __forceinline__ uint32_t rand_pair(uint32_t h, bool bf16) {
  uint32_t v = 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t r = mix(h + 0x9e3779b9u * (k + 1));
    uint32_t e;
    if (bf16) {
      e = (126u + (r >> 30 & 1u)) << 7;            // bf16 exponent 126/127
      e |= r & 0x7fu;
    } else {
      e = (14u + (r >> 30 & 1u)) << 10;            // fp16 exponent 14/15
      e |= r & 0x3ffu;
    }
    v |= ((r >> 31) << 15 | e) << (16 * k);
  }
  return v;
}

template <bool BF16>
__global__ __launch_bounds__(256, 1) void mfma_ceiling_kernel(uint32_t seed, int iters,
                                                              int zero, float* out) {
  const uint32_t base = mix(seed ^ (blockIdx.x * 256u + threadIdx.x) * 0x85ebca6bu);
  uint4 a[2], b[8];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    uint32_t* p = &a[j].x;
#pragma unroll
    for (int q = 0; q < 4; ++q) p[q] = zero ? 0u : rand_pair(base + 8 * j + q, BF16);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t* p = &b[i].x;
#pragma unroll
    for (int q = 0; q < 4; ++q) p[q] = zero ? 0u : rand_pair(base + 100 + 8 * i + q, BF16);
  }
  floatx16_t acc[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (BF16)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, a[j]), __builtin_bit_cast(bf16x8_t, b[i]),
              acc[j][i], 0, 0, 0);
        else
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              __builtin_bit_cast(half8_t, a[j]), __builtin_bit_cast(half8_t, b[i]),
              acc[j][i], 0, 0, 0);
      }
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[j][i][r];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

// out: blocks * 256 floats. FLOP per launch: blocks * 4 waves * iters *
// 16 MFMAs * 32768.
extern "C" int ming_calib_mfma(int bf16, int blocks, int iters, int zero, uint32_t seed,
                               float* out, void* stream) {
  if (blocks <= 0 || iters <= 0 || !out) return 2;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (bf16)
    hipLaunchKernelGGL(mfma_ceiling_kernel<true>, dim3(blocks), dim3(256), 0, s, seed, iters,
                       zero, out);
  else
    hipLaunchKernelGGL(mfma_ceiling_kernel<false>, dim3(blocks), dim3(256), 0, s, seed, iters,
                       zero, out);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}
