// The block glue around the projections, and the pack quantizer.
//
// Elementwise kernels (HBM-bound, 16-byte vector accesses, grid-stride):
//   swiglu          out = bf16(silu(g) * u)             ming_ops.metal:97-112
//   gated_residual  h = bf16(h + tanh(gate[n]) * sub)   ming_ops.metal:59-93
//   residual_add    h = bf16(h + sub)                   ming_ops.metal:43-52
//   fold_gain       nw = bf16(w * (1 + scale))          ming-dit.cc:2266-2273
//   bias_add        y = bf16(y + b[n])                  ming-dit.cc:1773-1779
//   silu            y = bf16(silu(x))                   ming-dit.cc:1788-1794
//   ln_modulate     y = bf16(LN(x) * (1 + scale))       ming-dit.cc:2553-2563
//                   (the final layer's LayerNorm, no affine, eps 1e-6)
//
// quantize: the synthetic pack recipes of the benchmark configs (symmetric
// int8 / affine int4, group 64), one 64-wide group per thread, writing the
// reference's pack layout (codes LSB-first U32, bf16 scales/biases).
#include "common.h"
#include "kernels.h"

namespace ming {
namespace {

__global__ void swiglu_kernel(const uint16_t* g, long long ldg,
                              const uint16_t* u, long long ldu, uint16_t* out,
                              long long ldo, int rows, int n) {
  // blockIdx.x walks the columns, blockIdx.y the rows (grid-stride in both),
  // so no 64-bit division per vector.
  const int n8 = n >> 3;
  for (int r = blockIdx.y; r < rows; r += gridDim.y)
  for (int c8 = blockIdx.x * blockDim.x + threadIdx.x; c8 < n8;
       c8 += gridDim.x * blockDim.x) {
    const int c = c8 * 8;
    const uint4 gv = *reinterpret_cast<const uint4*>(g + r * ldg + c);
    const uint4 uv = *reinterpret_cast<const uint4*>(u + r * ldu + c);
    const uint32_t* gp = &gv.x;
    const uint32_t* up = &uv.x;
    uint4 o;
    uint32_t* op = &o.x;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      op[e] = pack_bf16x2_rne(silu_f(bf16_lo(gp[e])) * bf16_lo(up[e]),
                              silu_f(bf16_hi(gp[e])) * bf16_hi(up[e]));
    *reinterpret_cast<uint4*>(out + r * ldo + c) = o;
  }
}

// t[i] = tanh(gate_msa[i]), t[n + i] = tanh(gate_mlp[i]) from the block's
// adaLN output [scale_msa | gate_msa | scale_mlp | gate_mlp], with tanhf on
// the bf16 value exactly as residual_kernel applies it per element.
__global__ void tanh_gates_kernel(const uint16_t* mods, int n, float* t) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 2 * n) return;
  const int src = i < n ? n + i : 3 * n + (i - n);
  t[i] = tanhf(bf16_to_f32(mods[src]));
}

// A modulated block's adaLN glue in one pass over its n columns (fill_mod,
// ming-dit.cc:2266-2273, with the gain fold): mods = bf16(mods + b) in
// place, the two folded pre-norm gains nw1 = an1 * (1 + scale_msa) and
// nw3 = fn1 * (1 + scale_mlp), and the two f32 residual gates
// t = tanh(gate_msa | gate_mlp). Each value is the expression of
// bias_act_kernel (mode 0), modulate_kernel and tanh_gates_kernel, so the
// bits are theirs.
__device__ __forceinline__ void adaln_glue_body(uint16_t* mods, int n, const uint16_t* b,
                                                const uint16_t* an1, const uint16_t* fn1,
                                                uint16_t* nw1, uint16_t* nw3, float* t) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float m[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = q * n + i;
    const float v = bf16_to_f32(mods[c]);
    const uint16_t r = (uint16_t)f32_to_bf16_bits(v + bf16_to_f32(b[c]));
    m[q] = bf16_to_f32(r);
    mods[c] = (uint16_t)f32_to_bf16_bits(m[q]);
  }
  nw1[i] = (uint16_t)f32_to_bf16_bits(bf16_to_f32(an1[i]) * (1.0f + m[0]) + 0.0f);
  nw3[i] = (uint16_t)f32_to_bf16_bits(bf16_to_f32(fn1[i]) * (1.0f + m[2]) + 0.0f);
  t[i] = tanhf(m[1]);
  t[n + i] = tanhf(m[3]);
}

__global__ void adaln_glue_kernel(uint16_t* mods, int n, const uint16_t* b,
                                  const uint16_t* an1, const uint16_t* fn1, uint16_t* nw1,
                                  uint16_t* nw3, float* t) {
  adaln_glue_body(mods, n, b, an1, fn1, nw1, nw3, t);
}

__global__ void adaln_glue_batch_kernel(const GlueBatch g) {
  const GlueEntry& e = g.e[blockIdx.y];
  adaln_glue_body(e.mods, g.n, e.b, e.an1, e.fn1, e.nw1, e.nw3, e.t);
}

// mode 0: h += tanh(gate[n]) * sub ; mode 1: h += sub
__global__ void residual_kernel(uint16_t* h, long long ldh, const uint16_t* gate,
                                const uint16_t* sub, long long lds, int rows,
                                int n, int mode) {
  const int n8 = n >> 3;
  const long long total = (long long)rows * n8;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long r = i / n8;
    const int c = (int)(i % n8) * 8;
    const uint4 hv = *reinterpret_cast<const uint4*>(h + r * ldh + c);
    const uint4 sv = *reinterpret_cast<const uint4*>(sub + r * lds + c);
    uint4 gv = make_uint4(0, 0, 0, 0);
    if (mode == 0) gv = *reinterpret_cast<const uint4*>(gate + c);
    const uint32_t* hp = &hv.x;
    const uint32_t* sp = &sv.x;
    const uint32_t* gp = &gv.x;
    uint4 o;
    uint32_t* op = &o.x;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
      float s0 = bf16_lo(sp[e]), s1 = bf16_hi(sp[e]);
      if (mode == 0) {
        s0 = tanhf(bf16_lo(gp[e])) * s0;
        s1 = tanhf(bf16_hi(gp[e])) * s1;
      }
      op[e] = pack_bf16x2(bf16_lo(hp[e]) + s0, bf16_hi(hp[e]) + s1);
    }
    *reinterpret_cast<uint4*>(h + r * ldh + c) = o;
  }
}

// y[r][n] = bf16(x[r][n] * (1 + scale[n]) + 0)   (fold_gain when rows == 1)
__global__ void modulate_kernel(const uint16_t* x, long long ldx,
                                const uint16_t* scale, uint16_t* y,
                                long long ldy, int rows, int n) {
  const long long total = (long long)rows * n;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long r = i / n;
    const int c = (int)(i % n);
    const float v = bf16_to_f32(x[r * ldx + c]) * (1.0f + bf16_to_f32(scale[c])) + 0.0f;
    y[r * ldy + c] = (uint16_t)f32_to_bf16_bits(v);
  }
}

// y = bf16(y + b[n]) (mode 0), bf16(silu(y + b[n])) (mode 1),
// bf16(silu(x)) into a second buffer (mode 2, b unused).
__global__ void bias_act_kernel(uint16_t* y, long long ldy, const uint16_t* b,
                                uint16_t* out2, int rows, int n, int mode) {
  const long long total = (long long)rows * n;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long r = i / n;
    const int c = (int)(i % n);
    float v = bf16_to_f32(y[r * ldy + c]);
    if (mode == 2) {
      out2[r * n + c] = (uint16_t)f32_to_bf16_bits(silu_f(v));
      continue;
    }
    v = bf16_to_f32((uint16_t)f32_to_bf16_bits(v + bf16_to_f32(b[c])));
    if (mode == 1) v = silu_f(v);
    y[r * ldy + c] = (uint16_t)f32_to_bf16_bits(v);
  }
}

// Final layer: LayerNorm (no affine, eps) then * (1 + scale[n]); one wave
// per row, stats in f32.
// One wave per row; the row is read once, 16 bytes per load, into registers
// (chunk c = lane + 64 i of 8 elements, D <= 8192), then mean, the centered
// variance and the output are taken from them.
__global__ __launch_bounds__(256) void ln_modulate_kernel(
    const uint16_t* x, long long ldx, const uint16_t* scale, uint16_t* y,
    long long ldy, int rows, int D, float eps) {
  constexpr int CPL = 16;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = D >> 3;
  const uint16_t* xr = x + (long long)row * ldx;
  uint4 v[CPL];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) v[i] = *reinterpret_cast<const uint4*>(xr + 8 * c);
  }
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    if (lane + 64 * i < nch) {
      const uint32_t* u = &v[i].x;
#pragma unroll
      for (int e = 0; e < 4; ++e) s += bf16_lo(u[e]) + bf16_hi(u[e]);
    }
  }
  s = warp_sum(s);
  const float mean = s / (float)D;
  float var = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    if (lane + 64 * i < nch) {
      const uint32_t* u = &v[i].x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d0 = bf16_lo(u[e]) - mean, d1 = bf16_hi(u[e]) - mean;
        var = fmaf(d0, d0, var);
        var = fmaf(d1, d1, var);
      }
    }
  }
  var = warp_sum(var);
  const float inv = 1.0f / sqrtf(var / (float)D + eps);
  uint16_t* yr = y + (long long)row * ldy;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      const uint4 sc = *reinterpret_cast<const uint4*>(scale + 8 * c);
      const uint32_t* u = &v[i].x;
      const uint32_t* su = &sc.x;
      uint4 o;
      uint32_t* ou = &o.x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t nb = pack_bf16x2_rne((bf16_lo(u[e]) - mean) * inv,
                                            (bf16_hi(u[e]) - mean) * inv);
        ou[e] = pack_bf16x2_rne(bf16_lo(nb) * (1.0f + bf16_lo(su[e])),
                                bf16_hi(nb) * (1.0f + bf16_hi(su[e])));
      }
      *reinterpret_cast<uint4*>(yr + 8 * c) = o;
    }
  }
}

__device__ __forceinline__ uint32_t rne_bf16_bits_f(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// One thread per (row, 64-wide group). w f32 [N][K].
__global__ void quantize_kernel(const float* w, int N, int K, int bits,
                                uint32_t* codes, uint16_t* scales,
                                uint16_t* biases) {
  const int G = K / 64;
  const long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x;
  if (idx >= (long long)N * G) return;
  const int n = (int)(idx / G), g = (int)(idx % G);
  const float* wr = w + (long long)n * K + g * 64;
  const int words = K * bits / 32;
  uint32_t* cr = codes + (long long)n * words + g * (64 * bits / 32);
  if (bits == 8) {
    float amax = 0.0f;
    for (int j = 0; j < 64; ++j) amax = fmaxf(amax, fabsf(wr[j]));
    const uint32_t sb = rne_bf16_bits_f(amax / 127.0f);
    const float s = __uint_as_float(sb << 16);
    scales[(long long)n * G + g] = (uint16_t)sb;
    biases[(long long)n * G + g] = (uint16_t)rne_bf16_bits_f(-128.0f * s);
    for (int wd = 0; wd < 16; ++wd) {
      uint32_t o = 0;
      for (int i = 0; i < 4; ++i) {
        float q = s > 0.0f ? rintf(wr[4 * wd + i] / s) : 0.0f;
        q = fminf(fmaxf(q, -127.0f), 127.0f);
        o |= (uint32_t)((int)q + 128) << (8 * i);
      }
      cr[wd] = o;
    }
  } else {
    float mn = wr[0], mx = wr[0];
    for (int j = 1; j < 64; ++j) {
      mn = fminf(mn, wr[j]);
      mx = fmaxf(mx, wr[j]);
    }
    const uint32_t sb = rne_bf16_bits_f((mx - mn) / 15.0f);
    const uint32_t bb = rne_bf16_bits_f(mn);
    const float s = __uint_as_float(sb << 16), b = __uint_as_float(bb << 16);
    scales[(long long)n * G + g] = (uint16_t)sb;
    biases[(long long)n * G + g] = (uint16_t)bb;
    for (int wd = 0; wd < 8; ++wd) {
      uint32_t o = 0;
      for (int i = 0; i < 8; ++i) {
        float q = s > 0.0f ? rintf((wr[8 * wd + i] - b) / s) : 0.0f;
        q = fminf(fmaxf(q, 0.0f), 15.0f);
        o |= (uint32_t)q << (4 * i);
      }
      cr[wd] = o;
    }
  }
}

unsigned grid_for(long long work) {
  long long b = (work + 255) / 256;
  if (b > 4096) b = 4096;
  if (b < 1) b = 1;
  return (unsigned)b;
}

}  // namespace

hipError_t launch_swiglu(const uint16_t* g, long long ldg, const uint16_t* u,
                         long long ldu, uint16_t* out, long long ldo, int rows,
                         int n, hipStream_t s) {
  const unsigned gx = (unsigned)(n / 8 + 255) / 256;
  const unsigned gy = (unsigned)(rows < 1 ? 1 : rows > 65535 ? 65535 : rows);
  hipLaunchKernelGGL(swiglu_kernel, dim3(gx < 1 ? 1 : gx, gy), dim3(256), 0, s,
                     g, ldg, u, ldu, out, ldo, rows, n);
  return hipGetLastError();
}

hipError_t launch_adaln_glue(uint16_t* mods, int n, const uint16_t* b, const uint16_t* an1,
                             const uint16_t* fn1, uint16_t* nw1, uint16_t* nw3, float* t,
                             hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(adaln_glue_kernel, dim3((n + 255) / 256), dim3(256), 0, s, mods, n, b, an1,
                     fn1, nw1, nw3, t);
  return hipGetLastError();
}

hipError_t launch_adaln_glue_batch(const GlueBatch& g, hipStream_t s) {
  if (g.n <= 0 || g.count <= 0) return hipSuccess;
  if (g.count > 32) return hipErrorInvalidValue;
  hipLaunchKernelGGL(adaln_glue_batch_kernel, dim3((g.n + 255) / 256, g.count), dim3(256), 0, s,
                     g);
  return hipGetLastError();
}

hipError_t launch_tanh_gates(const uint16_t* mods, int n, float* t, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(tanh_gates_kernel, dim3((2 * n + 255) / 256), dim3(256), 0, s, mods, n, t);
  return hipGetLastError();
}

hipError_t launch_residual(uint16_t* h, long long ldh, const uint16_t* gate,
                           const uint16_t* sub, long long lds, int rows, int n,
                           int gated, hipStream_t s) {
  hipLaunchKernelGGL(residual_kernel, dim3(grid_for((long long)rows * n / 8)),
                     dim3(256), 0, s, h, ldh, gate, sub, lds, rows, n,
                     gated ? 0 : 1);
  return hipGetLastError();
}

hipError_t launch_modulate(const uint16_t* x, long long ldx,
                           const uint16_t* scale, uint16_t* y, long long ldy,
                           int rows, int n, hipStream_t s) {
  hipLaunchKernelGGL(modulate_kernel, dim3(grid_for((long long)rows * n)),
                     dim3(256), 0, s, x, ldx, scale, y, ldy, rows, n);
  return hipGetLastError();
}

hipError_t launch_bias_act(uint16_t* y, long long ldy, const uint16_t* b,
                           uint16_t* out2, int rows, int n, int mode,
                           hipStream_t s) {
  hipLaunchKernelGGL(bias_act_kernel, dim3(grid_for((long long)rows * n)),
                     dim3(256), 0, s, y, ldy, b, out2, rows, n, mode);
  return hipGetLastError();
}

hipError_t launch_ln_modulate(const uint16_t* x, long long ldx,
                              const uint16_t* scale, uint16_t* y,
                              long long ldy, int rows, int D, float eps,
                              hipStream_t s) {
  hipLaunchKernelGGL(ln_modulate_kernel, dim3((rows + 3) / 4), dim3(256), 0, s,
                     x, ldx, scale, y, ldy, rows, D, eps);
  return hipGetLastError();
}

hipError_t launch_quantize(const float* w, int N, int K, int bits,
                           uint32_t* codes, uint16_t* scales, uint16_t* biases,
                           hipStream_t s) {
  const long long work = (long long)N * (K / 64);
  hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)((work + 255) / 256)),
                     dim3(256), 0, s, w, N, K, bits, codes, scales, biases);
  return hipGetLastError();
}

hipError_t validate_elementwise_kernels() {
  hipFuncAttributes fa;
  const void* fns[] = {reinterpret_cast<const void*>(&adaln_glue_kernel),
                       reinterpret_cast<const void*>(&adaln_glue_batch_kernel),
                       reinterpret_cast<const void*>(&swiglu_kernel),
                       reinterpret_cast<const void*>(&residual_kernel),
                       reinterpret_cast<const void*>(&modulate_kernel),
                       reinterpret_cast<const void*>(&bias_act_kernel),
                       reinterpret_cast<const void*>(&ln_modulate_kernel),
                       reinterpret_cast<const void*>(&quantize_kernel),
                       reinterpret_cast<const void*>(&tanh_gates_kernel)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&fa, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ming
