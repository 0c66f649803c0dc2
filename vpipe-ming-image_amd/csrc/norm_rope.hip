// RMSNorm and fused qk-norm + RoPE, the kernels that feed the projections.
//
// rmsnorm: y = bf16((x * 1/sqrt(mean(x^2) + eps)) * w), statistics in f32
// (the host's rms_norm_fast_f16 as dispatched at ming-dit.cc:1780-1787).
// One pass: each row is read once into registers (16-byte loads), reduced
// across the lanes that own it with DPP/permute shuffles, scaled and
// written back. HBM-bound: 4*D bytes per row (bf16 in + out) plus w.
//
// qk_norm_rope: the per-head RMSNorm of q and k (ming-dit.cc:2083-2084)
// and the interleaved-pair rotation (transpose_rope_pair_ftab_f16,
// ming-dit.cc:1885-1895) in ONE pass, in place on the token-major
// projection output -- the reference reads and writes q and k twice. The
// intermediate bf16 rounding between the two steps is kept, so the result
// is the reference's sequence of roundings. Rows stay token-major (the
// attention reads heads at a column offset), so no transpose pass.
#include "common.h"
#include "kernels.h"

namespace ming {
namespace {

// MODE 0: y = rms(x) * w.
// MODE 1: the same, plus h = fp16(y) (row stride ldh): the fp16 copy the fast
//         projections read, so the projections after the norm skip their own
//         bf16 -> fp16 pass (same bits: fp16 holds every bf16 value in range
//         exactly, converted as bf16_to_f16 converts).
// MODE 2: h = bf16(h + tg[n] * y), y not stored, tg = tanh(gate) in f32
//         computed once per block (tanhf of the bf16 gate, as the residual
//         kernel computes it per element): the post-norm and the gated residual
//         of run_block (ming-dit.cc:2096-2100, 2256-2260) in one pass over the
//         sub-layer output and the stream.
// MODE 3: h = bf16(h + y): the same for the context refiner's plain residual.
// Every mode reduces a row exactly as MODE 0 does and rounds y to bf16 before
// the residual, so each is bit-identical to rmsnorm followed by the separate
// residual / conversion kernel. Roundings to bf16 take v_cvt_pk_bf16_f32
// (round to nearest even; the bit-twiddled rounding's bits for every
// non-NaN value), two VALU per pair fewer than the bit arithmetic.
template <int LPR, int CPL, int MODE>
__global__ __launch_bounds__(256, 5) void rmsnorm_kernel(
    const uint16_t* x, long long ldx, const uint16_t* __restrict__ w,
    uint16_t* y, long long ldy, uint16_t* h, long long ldh,
    const float* __restrict__ tg, int rows, int D, float eps, int* range) {
  constexpr int RPW = 64 / LPR;  // rows per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = (blockIdx.x * 4 + wave) * RPW + lane / LPR;
  const int sub = lane % LPR;
  const int nch = D >> 3;
  const bool live = row < rows;
  const uint16_t* xr = x + (long long)(live ? row : 0) * ldx;
  // Every load of the row is issued before the reduction: the row, and the
  // norm weight (MODE <= 1) or the residual row (MODE >= 2); the weight
  // of the residual modes is read after it, which keeps their registers
  // inside 5 waves per SIMD (4352 rows of 3840 then fit one round).
  uint4 v[CPL], hv[CPL], wv[CPL];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = sub + LPR * i;
    if (live && c < nch) {
      v[i] = *reinterpret_cast<const uint4*>(xr + 8 * c);
      if constexpr (MODE <= 1) wv[i] = *reinterpret_cast<const uint4*>(w + 8 * c);
      else hv[i] = *reinterpret_cast<const uint4*>(h + (long long)row * ldh + 8 * c);
    }
  }
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = sub + LPR * i;
    if (live && c < nch) {
      const uint32_t* u = &v[i].x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = bf16_lo(u[e]), b = bf16_hi(u[e]);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
  }
#pragma unroll
  for (int o = LPR / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  if (!live) return;
  uint32_t seen = 0;   // magnitudes written to the fp16 copy (MODE 1)
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = sub + LPR * i;
    if (c < nch) {
      if constexpr (MODE >= 2) wv[i] = *reinterpret_cast<const uint4*>(w + 8 * c);
      const uint32_t* u = &v[i].x;
      const uint32_t* wu = &wv[i].x;
      uint4 o;
      uint32_t* ou = &o.x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = __fmul_rn(__fmul_rn(bf16_lo(u[e]), inv), bf16_lo(wu[e]));
        const float b = __fmul_rn(__fmul_rn(bf16_hi(u[e]), inv), bf16_hi(wu[e]));
        ou[e] = pack_bf16x2_rne(a, b);
      }
      if (MODE <= 1) {
        // MODE 0 (the standalone op) streams its output past the caches;
        // the block's fused modes keep ordinary stores, whose outputs the
        // next kernels read at once (non-temporal stores there measured
        // 0.35 ms slower per 1024^2 forward)
        if (MODE == 0) store16_nt(y + (long long)row * ldy + 8 * c, o);
        else *reinterpret_cast<uint4*>(y + (long long)row * ldy + 8 * c) = o;
        if (MODE == 1) {
          seen = range_track4(seen, o);
          uint4 f;
          f.x = bf16x2_to_f16x2(o.x);
          f.y = bf16x2_to_f16x2(o.y);
          f.z = bf16x2_to_f16x2(o.z);
          f.w = bf16x2_to_f16x2(o.w);
          *reinterpret_cast<uint4*>(h + (long long)row * ldh + 8 * c) = f;
        }
      } else {
        float t[8];
        if (MODE == 2) {
          const float4 t0 = *reinterpret_cast<const float4*>(tg + 8 * c);
          const float4 t1 = *reinterpret_cast<const float4*>(tg + 8 * c + 4);
          t[0] = t0.x; t[1] = t0.y; t[2] = t0.z; t[3] = t0.w;
          t[4] = t1.x; t[5] = t1.y; t[6] = t1.z; t[7] = t1.w;
        }
        const uint32_t* hp = &hv[i].x;
        uint4 r;
        uint32_t* rp = &r.x;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
          float s0 = bf16_lo(ou[e]), s1 = bf16_hi(ou[e]);
          if (MODE == 2) {
            s0 = t[2 * e] * s0;
            s1 = t[2 * e + 1] * s1;
          }
          rp[e] = pack_bf16x2_rne(bf16_lo(hp[e]) + s0, bf16_hi(hp[e]) + s1);
        }
        *reinterpret_cast<uint4*>(h + (long long)row * ldh + 8 * c) = r;
      }
    }
  }
  if (MODE == 1) range_report(range, seen);
}

// The post-norm + residual of MODE 2 (gated) / 3, then MODE 1 on the new
// stream row, in one pass: h = bf16(h + (tg *) bf16(rms(sub) * wpost)),
// y = bf16(rms(h) * wpre), yh = fp16(y). The new row is normalized from
// registers instead of being read back. Every expression and both
// reductions are rmsnorm_kernel's at the same LPR / CPL, so the result is
// bit-identical to the two launches it replaces.
template <int LPR, int CPL, bool GATED>
__global__ __launch_bounds__(256, 5) void norm_residual_norm_kernel(
    const uint16_t* sub, long long lds, const uint16_t* __restrict__ wpost,
    uint16_t* h, long long ldh, const float* __restrict__ tg,
    const uint16_t* __restrict__ wpre, uint16_t* y, long long ldy, uint16_t* yh,
    long long ldyh, int rows, int D, float eps, int* range) {
  constexpr int RPW = 64 / LPR;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // rows wave-uniform at LPR 64
  const int row = (blockIdx.x * 4 + wave) * RPW + lane / LPR;
  const int sb = lane % LPR;
  const int nch = D >> 3;
  const bool live = row < rows;
  const long long rr = live ? row : 0;
  uint4 v[CPL], hv[CPL];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = sb + LPR * i;
    if (live && c < nch) {
      v[i] = *reinterpret_cast<const uint4*>(sub + rr * lds + 8 * c);
      hv[i] = *reinterpret_cast<const uint4*>(h + rr * ldh + 8 * c);
    }
  }
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = sb + LPR * i;
    if (live && c < nch) {
      const uint32_t* u = &v[i].x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = bf16_lo(u[e]), b = bf16_hi(u[e]);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
  }
#pragma unroll
  for (int o = LPR / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  // the residual: h += (tg *) bf16(rms(sub) * wpost), kept in hv
  float ss2 = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = sb + LPR * i;
    if (live && c < nch) {
      const uint4 wv = *reinterpret_cast<const uint4*>(wpost + 8 * c);
      const uint32_t* u = &v[i].x;
      const uint32_t* wu = &wv.x;
      uint32_t ou[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = __fmul_rn(__fmul_rn(bf16_lo(u[e]), inv), bf16_lo(wu[e]));
        const float b = __fmul_rn(__fmul_rn(bf16_hi(u[e]), inv), bf16_hi(wu[e]));
        ou[e] = pack_bf16x2_rne(a, b);
      }
      float t[8];
      if constexpr (GATED) {
        const float4 t0 = *reinterpret_cast<const float4*>(tg + 8 * c);
        const float4 t1 = *reinterpret_cast<const float4*>(tg + 8 * c + 4);
        t[0] = t0.x; t[1] = t0.y; t[2] = t0.z; t[3] = t0.w;
        t[4] = t1.x; t[5] = t1.y; t[6] = t1.z; t[7] = t1.w;
      }
      uint32_t* hp = &hv[i].x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
        float s0 = bf16_lo(ou[e]), s1 = bf16_hi(ou[e]);
        if constexpr (GATED) {
          s0 = t[2 * e] * s0;
          s1 = t[2 * e + 1] * s1;
        }
        hp[e] = pack_bf16x2_rne(bf16_lo(hp[e]) + s0, bf16_hi(hp[e]) + s1);
      }
      *reinterpret_cast<uint4*>(h + rr * ldh + 8 * c) = hv[i];
      // the next norm's sum of squares, in rmsnorm_kernel's order
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = bf16_lo(hp[e]), b = bf16_hi(hp[e]);
        ss2 = fmaf(a, a, ss2);
        ss2 = fmaf(b, b, ss2);
      }
    }
  }
#pragma unroll
  for (int o = LPR / 2; o >= 1; o >>= 1) ss2 += __shfl_xor(ss2, o, 64);
  const float inv2 = 1.0f / sqrtf(ss2 / (float)D + eps);
  if (!live) return;
  uint32_t seen = 0;   // magnitudes written to the fp16 copy
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = sb + LPR * i;
    if (c < nch) {
      const uint4 wv = *reinterpret_cast<const uint4*>(wpre + 8 * c);
      const uint32_t* u = &hv[i].x;
      const uint32_t* wu = &wv.x;
      uint4 o;
      uint32_t* ou = &o.x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = __fmul_rn(__fmul_rn(bf16_lo(u[e]), inv2), bf16_lo(wu[e]));
        const float b = __fmul_rn(__fmul_rn(bf16_hi(u[e]), inv2), bf16_hi(wu[e]));
        ou[e] = pack_bf16x2_rne(a, b);
      }
      *reinterpret_cast<uint4*>(y + rr * ldy + 8 * c) = o;
      seen = range_track4(seen, o);
      uint4 f;
      f.x = bf16x2_to_f16x2(o.x);
      f.y = bf16x2_to_f16x2(o.y);
      f.z = bf16x2_to_f16x2(o.z);
      f.w = bf16x2_to_f16x2(o.w);
      *reinterpret_cast<uint4*>(yh + rr * ldyh + 8 * c) = f;
    }
  }
  range_report(range, seen);
}

// cos/sin [n][head_dim/2] from three integer positions per row: pairs
// [0, a0/2) on axis 0, then a1/2 on axis 1, then a2/2 on axis 2;
// freq = 1/theta^(2j/d), angle = pos*freq, both f64, stored f32
// (build_rope_, ming-dit.cc:1443-1486).
__global__ void rope_table_kernel(const int32_t* pt, const int32_t* ph,
                                  const int32_t* pw, int n, int a0, int a1,
                                  int a2, int pairs, double theta,
                                  float* cos_t, float* sin_t) {
  const long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x;
  if (idx >= (long long)n * pairs) return;
  const int t = (int)(idx / pairs), p = (int)(idx % pairs);
  int axis, j, d;
  if (p < a0 / 2) {
    axis = 0; j = p; d = a0;
  } else if (p < a0 / 2 + a1 / 2) {
    axis = 1; j = p - a0 / 2; d = a1;
  } else {
    axis = 2; j = p - a0 / 2 - a1 / 2; d = a2;
  }
  const double pos = (double)(axis == 0 ? pt[t] : (axis == 1 ? ph[t] : pw[t]));
  const double freq = 1.0 / pow(theta, (double)(2 * j) / (double)d);
  const double ang = pos * freq;
  cos_t[idx] = (float)cos(ang);
  sin_t[idx] = (float)sin(ang);
}

// A 16-lane group owns the same 8 elements (4 interleaved pairs) of QK_HPL
// heads of a row, so the row's cos / sin load once per QK_HPL heads; block
// (x, y): heads 16 * QK_HPL * x .. of the row's q then k heads, over QK_RPB
// consecutive rows, row groups strided by the grid's y extent (no index
// division). The loads of all QK_RPB rows are issued before the first
// reduction, and both bf16 roundings of a pair take gfx950's
// v_cvt_pk_bf16_f32 (round to nearest even: the bits of the bit-twiddled
// rounding for every non-NaN value). Measured on the MI355X, [4352, 2 x 3840]
// in place: one head a group over 4 rows 31.2 us, two heads over 2 rows
// 29.4 us (the same bits).
constexpr int QK_RPB = 2, QK_HPL = 2;
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    uint16_t* __restrict__ x, long long ld, int q_col, int k_col, int rows,
    int nq, int nk, const uint16_t* __restrict__ wq,
    const uint16_t* __restrict__ wk, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, float eps) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int sub = lane & 15;
  const int grp = (int)blockIdx.x * 16 + (tid >> 4);
  const uint4 wqv = *reinterpret_cast<const uint4*>(wq + 8 * sub);
  const uint4 wkv = *reinterpret_cast<const uint4*>(wk + 8 * sub);
  int col[QK_HPL];
  bool live[QK_HPL], isk[QK_HPL];
#pragma unroll
  for (int h = 0; h < QK_HPL; ++h) {
    const int hh0 = grp * QK_HPL + h;
    live[h] = hh0 < nq + nk;
    const int hh = live[h] ? hh0 : 0;   // a dead slot reads head 0 and stores nothing
    isk[h] = hh >= nq;
    col[h] = (isk[h] ? k_col + (hh - nq) * 128 : q_col + hh * 128) + 8 * sub;
  }
  for (int r0 = (int)blockIdx.y * QK_RPB; r0 < rows; r0 += (int)gridDim.y * QK_RPB) {
    uint4 v[QK_RPB][QK_HPL];
    float4 cv[QK_RPB], sv[QK_RPB];
#pragma unroll
    for (int j = 0; j < QK_RPB; ++j) {
      const int row = r0 + j < rows ? r0 + j : rows - 1;   // the tail re-reads a valid row
#pragma unroll
      for (int h = 0; h < QK_HPL; ++h)
        v[j][h] = *reinterpret_cast<const uint4*>(x + (long long)row * ld + col[h]);
      cv[j] = *reinterpret_cast<const float4*>(cos_t + (long long)row * 64 + 4 * sub);
      sv[j] = *reinterpret_cast<const float4*>(sin_t + (long long)row * 64 + 4 * sub);
    }
#pragma unroll
    for (int j = 0; j < QK_RPB; ++j) {
#pragma unroll
      for (int h = 0; h < QK_HPL; ++h) {
        float ss = head_ss8(v[j][h]);
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        const float inv = head_rms_inv(ss, eps);
        const uint4 wv = isk[h] ? wkv : wqv;
        uint4 o;
        o.x = norm_rope_pair(v[j][h].x, wv.x, inv, cv[j].x, sv[j].x);
        o.y = norm_rope_pair(v[j][h].y, wv.y, inv, cv[j].y, sv[j].y);
        o.z = norm_rope_pair(v[j][h].z, wv.z, inv, cv[j].z, sv[j].z);
        o.w = norm_rope_pair(v[j][h].w, wv.w, inv, cv[j].w, sv[j].w);
        if (live[h] && r0 + j < rows)
          *reinterpret_cast<uint4*>(x + (long long)(r0 + j) * ld + col[h]) = o;
      }
    }
  }
}

// The LLM encoder's fused qk-norm + rotate-half RoPE (LlmOps::qk_norm_rope,
// ming-ops.h:118-122; ming_llm.metal:100-178), in place: heads [0, nq) are
// queries from column 0, heads [nq, nq + nk) keys right after them, 128 wide.
// A 16-lane group owns the same 8 consecutive dims of QK_HPL heads over
// QK_RPB rows a block, loads first, as in qk_norm_rope_kernel (the row's
// tables once per QK_HPL heads). With NORM, each head is RMS-normalized and
// scaled as x * (inv * w). ROT is the rotation's half-width R: element j
// pairs with j + R, which sits R/8 lanes away (lane distance 8 for R = 64, 4
// for R = 32), so each lane takes its partner's 8 raw values with four
// cross-lane moves, normalizes them itself with the partner's weights (the
// same operations the partner applies), and computes its own side:
// x_j c_j - x_{j+R} s_j on the low half, x_{j+R} c_j + x_j s_j on the high.
// R = 32 leaves dims 64..127 unrotated; R = 0 rotates nothing. One bf16
// rounding per element. Measured on the MI355X at [4352, 60 heads] in place,
// against one head a group over one row a block: 41.2 -> 31.9 us (R = 64,
// norm), 37.9 -> 34.0 (R = 32), 32.3 -> 26.0 (norm only), 32.2 -> 26.7
// (rotation only), the same bits.
template <int ROT, bool NORM>
__global__ __launch_bounds__(256) void llm_qk_norm_rope_kernel(
    uint16_t* __restrict__ x, long long ld, int rows, int nq, int nk,
    const uint16_t* __restrict__ wq, const uint16_t* __restrict__ wk,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, float eps) {
  constexpr int PX = ROT == 64 ? 8 : 4;
  const int tid = threadIdx.x, sub = tid & 15;
  const int grp = (int)blockIdx.x * 16 + (tid >> 4);
  const bool rotated = ROT == 64 || (ROT == 32 && sub < 8);
  const bool low = ROT == 64 ? sub < 8 : (sub & 4) == 0;
  constexpr int RM = ROT == 0 ? 1 : ROT;
  const int j0 = (8 * sub) % RM;
  int col[QK_HPL];
  bool live[QK_HPL], isk[QK_HPL];
#pragma unroll
  for (int h = 0; h < QK_HPL; ++h) {
    const int hh0 = grp * QK_HPL + h;
    live[h] = hh0 < nq + nk;
    const int hh = live[h] ? hh0 : 0;
    isk[h] = hh >= nq;
    col[h] = hh * 128 + 8 * sub;
  }
  uint4 wqa = {}, wqb = {}, wka = {}, wkb = {};
  if (NORM) {
    wqa = *reinterpret_cast<const uint4*>(wq + 8 * sub);
    wqb = *reinterpret_cast<const uint4*>(wq + 8 * (sub ^ PX));
    wka = *reinterpret_cast<const uint4*>(wk + 8 * sub);
    wkb = *reinterpret_cast<const uint4*>(wk + 8 * (sub ^ PX));
  }
  for (int r0 = (int)blockIdx.y * QK_RPB; r0 < rows; r0 += (int)gridDim.y * QK_RPB) {
    uint4 v[QK_RPB][QK_HPL];
    float4 c0[QK_RPB], c1[QK_RPB], s0[QK_RPB], s1[QK_RPB];
#pragma unroll
    for (int j = 0; j < QK_RPB; ++j) {
      const int row = r0 + j < rows ? r0 + j : rows - 1;
#pragma unroll
      for (int h = 0; h < QK_HPL; ++h)
        v[j][h] = *reinterpret_cast<const uint4*>(x + (long long)row * ld + col[h]);
      if (ROT != 0 && rotated) {
        const float* cr = cos_t + (long long)row * ROT + j0;
        const float* sr = sin_t + (long long)row * ROT + j0;
        c0[j] = *reinterpret_cast<const float4*>(cr);
        c1[j] = *reinterpret_cast<const float4*>(cr + 4);
        s0[j] = *reinterpret_cast<const float4*>(sr);
        s1[j] = *reinterpret_cast<const float4*>(sr + 4);
      }
    }
#pragma unroll
    for (int j = 0; j < QK_RPB; ++j) {
#pragma unroll
      for (int h = 0; h < QK_HPL; ++h) {
        const uint4 vv = v[j][h];
        float inv = 1.0f;
        if (NORM) {
          float ss = head_ss8(vv);
#pragma unroll
          for (int o = 8; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
          inv = head_rms_inv(ss, eps);
        }
        const uint32_t uv[4] = {vv.x, vv.y, vv.z, vv.w};
        float a[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[2 * e] = bf16_lo(uv[e]);
          a[2 * e + 1] = bf16_hi(uv[e]);
        }
        if (NORM) {
          const uint4 wa = isk[h] ? wka : wqa;
          const uint32_t wu[4] = {wa.x, wa.y, wa.z, wa.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a[2 * e] = __fmul_rn(a[2 * e], __fmul_rn(inv, bf16_lo(wu[e])));
            a[2 * e + 1] = __fmul_rn(a[2 * e + 1], __fmul_rn(inv, bf16_hi(wu[e])));
          }
        }
        if (ROT != 0) {
          const uint32_t pu[4] = {(uint32_t)__shfl_xor((int)vv.x, PX, 64),
                                  (uint32_t)__shfl_xor((int)vv.y, PX, 64),
                                  (uint32_t)__shfl_xor((int)vv.z, PX, 64),
                                  (uint32_t)__shfl_xor((int)vv.w, PX, 64)};
          if (rotated) {
            float b[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              b[2 * e] = bf16_lo(pu[e]);
              b[2 * e + 1] = bf16_hi(pu[e]);
            }
            if (NORM) {
              const uint4 wb = isk[h] ? wkb : wqb;
              const uint32_t wu[4] = {wb.x, wb.y, wb.z, wb.w};
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                b[2 * e] = __fmul_rn(b[2 * e], __fmul_rn(inv, bf16_lo(wu[e])));
                b[2 * e + 1] = __fmul_rn(b[2 * e + 1], __fmul_rn(inv, bf16_hi(wu[e])));
              }
            }
            const float c[8] = {c0[j].x, c0[j].y, c0[j].z, c0[j].w, c1[j].x, c1[j].y, c1[j].z, c1[j].w};
            const float s[8] = {s0[j].x, s0[j].y, s0[j].z, s0[j].w, s1[j].x, s1[j].y, s1[j].z, s1[j].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
#pragma clang fp contract(off)
              a[e] = low ? a[e] * c[e] - b[e] * s[e] : a[e] * c[e] + b[e] * s[e];
            }
          }
        }
        uint4 o;
        o.x = pack_bf16x2_rne(a[0], a[1]);
        o.y = pack_bf16x2_rne(a[2], a[3]);
        o.z = pack_bf16x2_rne(a[4], a[5]);
        o.w = pack_bf16x2_rne(a[6], a[7]);
        if (live[h] && r0 + j < rows)
          *reinterpret_cast<uint4*>(x + (long long)(r0 + j) * ld + col[h]) = o;
      }
    }
  }
}

}  // namespace

hipError_t launch_rmsnorm_ex(int mode, const uint16_t* x, long long ldx, const uint16_t* w,
                             uint16_t* y, long long ldy, uint16_t* h, long long ldh,
                             const float* tg, int rows, int D, float eps,
                             hipStream_t s, int* range) {
  if (rows <= 0) return hipSuccess;
  const int nch = D / 8;
  if (D % 8 != 0 || nch > 64 * 16 || mode < 0 || mode > 3) return hipErrorInvalidValue;
#define MING_RMS_M(LPR, CPL, MODE)                                                \
  hipLaunchKernelGGL((rmsnorm_kernel<LPR, CPL, MODE>), dim3((rows + rpb - 1) / rpb), \
                     dim3(256), 0, s, x, ldx, w, y, ldy, h, ldh, tg, rows, D, eps, range)
#define MING_RMS(LPR, CPL)                                                     \
  do {                                                                         \
    const int rpb = 4 * (64 / (LPR));                                          \
    if (mode == 0) MING_RMS_M(LPR, CPL, 0);                                    \
    else if (mode == 1) MING_RMS_M(LPR, CPL, 1);                               \
    else if (mode == 2) MING_RMS_M(LPR, CPL, 2);                               \
    else MING_RMS_M(LPR, CPL, 3);                                              \
  } while (0)
  if (nch <= 8) MING_RMS(8, 1);
  else if (nch <= 16) MING_RMS(16, 1);
  else if (nch <= 32) MING_RMS(32, 1);
  else if (nch <= 64) MING_RMS(64, 1);
  else if (nch <= 256) MING_RMS(64, 4);
  else if (nch <= 512) MING_RMS(64, 8);
  else MING_RMS(64, 16);
#undef MING_RMS
#undef MING_RMS_M
  return hipGetLastError();
}

hipError_t launch_norm_residual_norm(const uint16_t* sub, long long lds, const uint16_t* wpost,
                                     uint16_t* h, long long ldh, const float* tg,
                                     const uint16_t* wpre, uint16_t* y, long long ldy,
                                     uint16_t* yh, long long ldyh, int rows, int D, float eps,
                                     hipStream_t s, int* range) {
  if (rows <= 0) return hipSuccess;
  const int nch = D / 8;
  if (D % 8 != 0 || nch > 64 * 16) return hipErrorInvalidValue;
#define MING_NRN_G(LPR, CPL, G)                                                          \
  hipLaunchKernelGGL((norm_residual_norm_kernel<LPR, CPL, G>), dim3((rows + rpb - 1) / rpb), \
                     dim3(256), 0, s, sub, lds, wpost, h, ldh, tg, wpre, y, ldy, yh, ldyh,   \
                     rows, D, eps, range)
#define MING_NRN(LPR, CPL)                                                     \
  do {                                                                         \
    const int rpb = 4 * (64 / (LPR));                                          \
    if (tg) MING_NRN_G(LPR, CPL, true);                                        \
    else MING_NRN_G(LPR, CPL, false);                                          \
  } while (0)
  // the (LPR, CPL) choice of launch_rmsnorm_ex: the same reductions
  if (nch <= 8) MING_NRN(8, 1);
  else if (nch <= 16) MING_NRN(16, 1);
  else if (nch <= 32) MING_NRN(32, 1);
  else if (nch <= 64) MING_NRN(64, 1);
  else if (nch <= 256) MING_NRN(64, 4);
  else if (nch <= 512) MING_NRN(64, 8);
  else MING_NRN(64, 16);
#undef MING_NRN
#undef MING_NRN_G
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const uint16_t* x, long long ldx, const uint16_t* w,
                          uint16_t* y, long long ldy, int rows, int D,
                          float eps, hipStream_t s) {
  return launch_rmsnorm_ex(0, x, ldx, w, y, ldy, nullptr, 0, nullptr, rows, D, eps, s);
}

hipError_t launch_rope_table(const int32_t* pt, const int32_t* ph,
                             const int32_t* pw, int n, int a0, int a1, int a2,
                             int head_dim, double theta, float* cos_t,
                             float* sin_t, hipStream_t s) {
  const int pairs = head_dim / 2;
  const long long total = (long long)n * pairs;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((total + 255) / 256)),
                     dim3(256), 0, s, pt, ph, pw, n, a0, a1, a2, pairs, theta,
                     cos_t, sin_t);
  return hipGetLastError();
}

hipError_t launch_qk_norm_rope(uint16_t* x, long long ld, int q_col,
                               int k_col, int rows, int n_heads,
                               const uint16_t* wq, const uint16_t* wk,
                               const float* cos_t, const float* sin_t,
                               float eps, hipStream_t s) {
  if (rows <= 0 || n_heads <= 0) return hipSuccess;
  const int groups = (rows + QK_RPB - 1) / QK_RPB;
  const unsigned gy = (unsigned)(groups < 65535 ? groups : 65535);   // grid y limit; groups stride
  hipLaunchKernelGGL(qk_norm_rope_kernel,
                     dim3((unsigned)((2 * n_heads + 16 * QK_HPL - 1) / (16 * QK_HPL)), gy),
                     dim3(256), 0, s, x, ld, q_col, k_col, rows, n_heads, n_heads, wq,
                     wk, cos_t, sin_t, eps);
  return hipGetLastError();
}

hipError_t launch_k_norm_rope(uint16_t* x, long long ld, int k_col, int rows, int n_heads,
                              const uint16_t* wk, const float* cos_t, const float* sin_t,
                              float eps, hipStream_t s) {
  if (rows <= 0 || n_heads <= 0) return hipSuccess;
  const int groups = (rows + QK_RPB - 1) / QK_RPB;
  const unsigned gy = (unsigned)(groups < 65535 ? groups : 65535);
  hipLaunchKernelGGL(qk_norm_rope_kernel,
                     dim3((unsigned)((n_heads + 16 * QK_HPL - 1) / (16 * QK_HPL)), gy),
                     dim3(256), 0, s, x, ld, k_col, k_col, rows, 0, n_heads, wk, wk,
                     cos_t, sin_t, eps);
  return hipGetLastError();
}

hipError_t launch_llm_qk_norm_rope(uint16_t* x, long long ld, int rows, int nq, int nk,
                                   const uint16_t* wq, const uint16_t* wk, const float* cos_t,
                                   const float* sin_t, int rot_half, float eps, hipStream_t s) {
  if (rows <= 0 || nq + nk <= 0) return hipSuccess;
  const bool norm = wq != nullptr && wk != nullptr;
  const int groups = (rows + QK_RPB - 1) / QK_RPB;
  const dim3 grid((unsigned)((nq + nk + 16 * QK_HPL - 1) / (16 * QK_HPL)),
                  (unsigned)(groups < 65535 ? groups : 65535));
#define MING_LLMQK(R, N)                                                                  \
  hipLaunchKernelGGL((llm_qk_norm_rope_kernel<R, N>), grid, dim3(256), 0, s, x, ld, rows, \
                     nq, nk, wq, wk, cos_t, sin_t, eps)
  if (rot_half == 64) {
    if (norm) MING_LLMQK(64, true); else MING_LLMQK(64, false);
  } else if (rot_half == 32) {
    if (norm) MING_LLMQK(32, true); else MING_LLMQK(32, false);
  } else if (rot_half == 0) {
    if (norm) MING_LLMQK(0, true); else MING_LLMQK(0, false);
  } else {
    return hipErrorInvalidValue;
  }
#undef MING_LLMQK
  return hipGetLastError();
}

}  // namespace ming

namespace ming {
hipError_t validate_norm_kernels() {
  hipFuncAttributes fa;
  const void* fns[] = {
#define MING_RMS_ALL(LPR, CPL)                                      \
  reinterpret_cast<const void*>(&rmsnorm_kernel<LPR, CPL, 0>),      \
      reinterpret_cast<const void*>(&rmsnorm_kernel<LPR, CPL, 1>),  \
      reinterpret_cast<const void*>(&rmsnorm_kernel<LPR, CPL, 2>),  \
      reinterpret_cast<const void*>(&rmsnorm_kernel<LPR, CPL, 3>)
      MING_RMS_ALL(8, 1),  MING_RMS_ALL(16, 1), MING_RMS_ALL(32, 1), MING_RMS_ALL(64, 1),
      MING_RMS_ALL(64, 4), MING_RMS_ALL(64, 8), MING_RMS_ALL(64, 16),
#undef MING_RMS_ALL
#define MING_NRN_ALL(LPR, CPL)                                                  \
  reinterpret_cast<const void*>(&norm_residual_norm_kernel<LPR, CPL, true>),    \
      reinterpret_cast<const void*>(&norm_residual_norm_kernel<LPR, CPL, false>)
      MING_NRN_ALL(8, 1),  MING_NRN_ALL(16, 1), MING_NRN_ALL(32, 1), MING_NRN_ALL(64, 1),
      MING_NRN_ALL(64, 4), MING_NRN_ALL(64, 8), MING_NRN_ALL(64, 16),
#undef MING_NRN_ALL
      reinterpret_cast<const void*>(&rope_table_kernel),
      reinterpret_cast<const void*>(&qk_norm_rope_kernel),
      reinterpret_cast<const void*>(&llm_qk_norm_rope_kernel<64, true>),
      reinterpret_cast<const void*>(&llm_qk_norm_rope_kernel<64, false>),
      reinterpret_cast<const void*>(&llm_qk_norm_rope_kernel<32, true>),
      reinterpret_cast<const void*>(&llm_qk_norm_rope_kernel<32, false>),
      reinterpret_cast<const void*>(&llm_qk_norm_rope_kernel<0, true>),
      reinterpret_cast<const void*>(&llm_qk_norm_rope_kernel<0, false>)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&fa, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}
}  // namespace ming
