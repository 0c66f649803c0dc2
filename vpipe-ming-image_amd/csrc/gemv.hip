// Projections over a handful of rows: lin() (ming-dit.cc:1763-1771) at
// M <= kGemvMaxM with no live adapter. The forward runs these once per block
// and per forward at M = 1: the adaLN modulation of every modulated block
// (fill_mod, ming-dit.cc:2266-2273; quantized, [4H, adaln_dim]), the timestep
// MLP (2276-2281) and the final layer's adaLN (dense). A 256-row GEMM tile
// would spend 255 of its rows on nothing; this kernel instead streams each
// weight once, HBM-bound, with the rows' activations read wave-uniformly.
//
// Block: 256 threads (4 waves) over 64 output columns; lane l owns column
// 64 * block + l and wave w the 64-wide K groups w, w + 4, w + 8, ... The
// four waves' sums meet in LDS and are added in wave order (the bits do not
// depend on timing). Per group, quantized weights take the reference's
// affine form w = scale * q + bias (the MLX affine convention the reference
// packs follow) as scale * sum(q * x) + bias * sum(x), all in f32; dense
// weights are plain bf16 dot products. The result is rounded to bf16 once.
//
// Weights are read in the resident general layout (kernels.h): codes
// [kt][n][w] with the w4 nibble order {0,2,4,6,1,3,5,7} and w8 bytes in k
// order, sb [kt][n] = bf16 scale | bf16 bias << 16; dense w [n][k].
#include "common.h"
#include "kernels.h"

namespace ming {
namespace {

// The 64 weights of group kt of column n, in k order, as f32 (quantized:
// the integer codes q; dense: the bf16 values).
template <int BITS>
__device__ __forceinline__ void load_group(const GemvArgs& a, int n, int kt, float (&w)[64]) {
  if constexpr (BITS == 4) {
    const uint4* p = reinterpret_cast<const uint4*>(a.codes + ((long long)kt * a.N + n) * 8);
    const uint4 c0 = p[0], c1 = p[1];
    const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // nibble i of word j holds k = 8j + {0,2,4,6,1,3,5,7}[i]
      const uint32_t lo = cw[j] & 0x0F0F0F0Fu;          // nibbles 0,2,4,6: k 0,4,1,5
      const uint32_t hi = (cw[j] >> 4) & 0x0F0F0F0Fu;   // nibbles 1,3,5,7: k 2,6,3,7
      w[8 * j + 0] = (float)(lo & 0xff);
      w[8 * j + 4] = (float)((lo >> 8) & 0xff);
      w[8 * j + 1] = (float)((lo >> 16) & 0xff);
      w[8 * j + 5] = (float)(lo >> 24);
      w[8 * j + 2] = (float)(hi & 0xff);
      w[8 * j + 6] = (float)((hi >> 8) & 0xff);
      w[8 * j + 3] = (float)((hi >> 16) & 0xff);
      w[8 * j + 7] = (float)(hi >> 24);
    }
  } else if constexpr (BITS == 8) {
    const uint4* p = reinterpret_cast<const uint4*>(a.codes + ((long long)kt * a.N + n) * 16);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint4 c = p[v];
      const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) w[16 * v + 4 * j + i] = (float)((cw[j] >> (8 * i)) & 0xff);
    }
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(a.w16 + (long long)n * a.K + 64 * kt);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const uint4 c = p[v];
      const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w[8 * v + 2 * j] = bf16_lo(cw[j]);
        w[8 * v + 2 * j + 1] = bf16_hi(cw[j]);
      }
    }
  }
}

template <int BITS>
__device__ __forceinline__ void gemv_body(const GemvArgs& a) {
  __shared__ float red[4][kGemvMaxM][64];
  const int lane = (int)threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int n = (int)blockIdx.x * 64 + lane;
  const int nc = n < a.N ? n : a.N - 1;     // columns past N compute, never store
  const int KT = a.K / 64;
  float acc[kGemvMaxM];
#pragma unroll
  for (int m = 0; m < kGemvMaxM; ++m) acc[m] = 0.0f;
  for (int kt = wave; kt < KT; kt += 4) {
    float w[64];
    load_group<BITS>(a, nc, kt, w);
    float s = 1.0f, b = 0.0f;
    if constexpr (BITS != 16) {
      const uint32_t sbv = a.sb[(long long)kt * a.N + nc];
      s = bf16_lo(sbv);
      b = bf16_hi(sbv);
    }
#pragma unroll
    for (int m = 0; m < kGemvMaxM; ++m) {
      if (m < a.M) {
        // the row's 64 activations: the same address in every lane
        const uint4* xp = reinterpret_cast<const uint4*>(a.x + (long long)m * a.ldx + 64 * kt);
        float dot = 0.0f, xs = 0.0f;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const uint4 c = xp[v];
          const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float x0 = bf16_lo(cw[j]), x1 = bf16_hi(cw[j]);
            dot = __builtin_fmaf(w[8 * v + 2 * j], x0, dot);
            dot = __builtin_fmaf(w[8 * v + 2 * j + 1], x1, dot);
            xs += x0;
            xs += x1;
          }
        }
        acc[m] += BITS == 16 ? dot : __builtin_fmaf(s, dot, b * xs);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kGemvMaxM; ++m) red[wave][m][lane] = acc[m];
  __syncthreads();
  if (wave == 0 && n < a.N) {
#pragma unroll
    for (int m = 0; m < kGemvMaxM; ++m)
      if (m < a.M) {
        float v = ((red[0][m][lane] + red[1][m][lane]) + red[2][m][lane]) + red[3][m][lane];
        if (a.bias) v += bf16_to_f32(a.bias[n]);
        a.y[(long long)m * a.ldy + n] = (uint16_t)f32_to_bf16_bits(v);
      }
  }
}

template <int BITS>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvArgs a) {
  gemv_body<BITS>(a);
}

template <int BITS>
__global__ __launch_bounds__(256) void gemv_batch_kernel(const GemvBatch b) {
  GemvArgs a = b.base;
  const GemvEntry& e = b.e[blockIdx.y];
  a.codes = e.codes;
  a.sb = e.sb;
  a.w16 = e.w16;
  a.y = e.y;
  gemv_body<BITS>(a);
}

}  // namespace

hipError_t launch_gemv_batch(int bits, const GemvBatch& b, hipStream_t s) {
  const GemvArgs& a = b.base;
  if (b.count <= 0 || a.M <= 0 || a.N <= 0) return hipSuccess;
  if (b.count > kGemvBatch || a.M > kGemvMaxM || a.K % 64 != 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)b.count);
  switch (bits) {
    case 4: hipLaunchKernelGGL(gemv_batch_kernel<4>, grid, dim3(256), 0, s, b); break;
    case 8: hipLaunchKernelGGL(gemv_batch_kernel<8>, grid, dim3(256), 0, s, b); break;
    case 16: hipLaunchKernelGGL(gemv_batch_kernel<16>, grid, dim3(256), 0, s, b); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemv(int bits, const GemvArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.M > kGemvMaxM || a.K % 64 != 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((a.N + 63) / 64));
  switch (bits) {
    case 4: hipLaunchKernelGGL(gemv_kernel<4>, grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL(gemv_kernel<8>, grid, dim3(256), 0, s, a); break;
    case 16: hipLaunchKernelGGL(gemv_kernel<16>, grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t validate_gemv_kernels() {
  hipFuncAttributes fa;
  const void* fns[] = {reinterpret_cast<const void*>(&gemv_kernel<4>),
                       reinterpret_cast<const void*>(&gemv_kernel<8>),
                       reinterpret_cast<const void*>(&gemv_kernel<16>),
                       reinterpret_cast<const void*>(&gemv_batch_kernel<4>),
                       reinterpret_cast<const void*>(&gemv_batch_kernel<8>),
                       reinterpret_cast<const void*>(&gemv_batch_kernel<16>)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&fa, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ming
