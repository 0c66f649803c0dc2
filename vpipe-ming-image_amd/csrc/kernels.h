// Host-side launch interface of the HIP kernels (internal to the library;
// the public boundary is include/ming_dit_amd.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ming {

// ---- quantized / dense projection GEMM with the LoRA tail ------------------
//
// y[m][n] = sum_k x[m][k] W[n][k]  (+ sum_r T[m][seg.t_col0 + r] B[n][r])
//
// W is resident in the tiled layout built by repack_* (K-tile major):
//   bits 4:  codes[kt][n][8]  u32, nibble i of word j holds k = 8j + perm(i)
//            with perm = {0,2,4,6,1,3,5,7}
//   bits 8:  codes[kt][n][16] u32, byte i of word j holds k = 4j + i
//   bits 16: dense bf16 w[n][k] (the checkpoint's own layout)
//   sb[kt][n] = bf16 scale | bf16 bias << 16 (bits 4 and 8)
// T is the LoRA intermediate [M][ldt] bf16 (already scaled), B the
// segment's factors [N_seg][ldb] bf16, gathered per 8-wide rank group by
// `grp` (B column / 8, or -1 for a zero group).
constexpr int kQpBM = 256, kQpBN = 256, kQpBK = 64, kQpThreads = 256;
constexpr int kMaxSeg = 4;
constexpr int kMaxGroups = 512;   // 8-wide rank groups per call (4096 ranks)

struct QprojSeg {
  int n_begin;          // first output column of this segment
  int n_end;
  int t_col0;           // first T column of this segment's live ranks
  int chunks;           // live rank chunks of 32 (0: no adapter)
  int ldb;
  int grp0;             // first entry of this segment in grp[]
  const uint16_t* B;    // row (n - n_begin)
};

struct QprojArgs {
  const uint16_t* x;
  long long ldx;
  const uint32_t* codes;
  const uint32_t* sb;
  const uint16_t* w16;
  uint16_t* y;
  long long ldy;
  int M, N, K;
  const uint16_t* t;
  int ldt;
  int nseg;
  // optional SwiGLU gate: when g != nullptr the output is
  // y = bf16(silu(g) * bf16(x . W^T + LoRA)) (g bf16 [M][ldg], may equal y)
  const uint16_t* g;
  long long ldg;
  // optional fp16 copy of the (final) output, [M][ldyh], 16-byte aligned,
  // ldyh % 8 == 0: the next projection's fast-route input (fast kernel only)
  uint16_t* yh;
  long long ldyh;
  QprojSeg seg[kMaxSeg];
  int16_t grp[kMaxGroups];
  // fast route, split K (kslices > 1): f32 partials [kslices][M][N] in part,
  // summed in slice order by a second launch (N % 4 == 0)
  float* part;
  int kslices;
  // optional: set to 1 when an fp16 conversion of this launch (the general
  // kernel's x tiles, the fast epilogue's yh) met a bf16 value of magnitude
  // >= 2^16, inf or NaN (see range_report)
  int* range;
  // The paired gated launch (launch_qproj_pair): the weight above is the
  // gate projection (one segment, seg[0]) and (codes_u, sb_u, seg_u) the up
  // projection of the same shape, its groups in grp[] from seg_u.grp0, its
  // T columns in the same t; y = bf16(silu(bf16(gate)) * bf16(up)).
  const uint32_t* codes_u;
  const uint32_t* sb_u;
  QprojSeg seg_u;
  // optional bias [N] bf16, added to the f32 result before the output's one
  // bf16 rounding (the general kernel: a dense weight's ming_lin_bias)
  const uint16_t* bias;
};

// wide: bits 4/8 run with bf16 activations and the weight as a bf16 pair
// hi + lo (two passes over K): no fp16 anywhere, any finite input.
hipError_t launch_qproj(int bits, const QprojArgs& a, hipStream_t s, bool wide = false);

// Dense attention, head dim 128: O = softmax(scale * Q K^T) V per head.
// q, k: token-major rows (head h at column 128h); vt: V^T [NH][128][ldv]
// written by the launch from v (token-major), keys zero-padded to ldv (a
// multiple of 64 >= R); o: token-major [R][NH*128]. sl2 = scale * log2(e).
struct AttnArgs {
  const uint16_t* q;
  long long ldq;
  const uint16_t* k;
  long long ldk;
  const uint16_t* vt;
  int ldv;
  uint16_t* o;
  long long ldo;
  // optional per-head RMSNorm + RoPE of q, applied to the Q fragments as
  // they are loaded (launch_qk_norm_rope's arithmetic and bits): weight
  // qw[128], tables [R][64]; q is then the raw projection output
  const uint16_t* qw;
  const float* cos_t;
  const float* sin_t;
  float eps;
  // optional fp16 copy of O (the same bf16 values), [R][NH*128] at ldoh: the
  // fast projection route's input for the o-projection
  uint16_t* oh;
  long long ldoh;
  int* range;           // optional: raised as QprojArgs::range for oh
  int R, NH;
  float sl2;
};
hipError_t launch_attention(const AttnArgs& a, const uint16_t* v, long long ldv_in,
                            hipStream_t s);
hipError_t validate_attention_kernels();

// T[m][c] = bf16(coef[c/16] * sum_k x[m][k] A[row(c)][k]) for c < n_cols,
// row(c) = 16*grp[c/16] + c%16 (grp -1: a zero column). A is [R][K] bf16.
// Up to this many projections share one x.A launch (q, k, v; w1, w3).
constexpr int kMaxXaSources = 4;
struct LoraXaArgs {
  const uint16_t* x;
  long long ldx;
  // A stacks [rows][K]: group entry g reads rows 8 * (g & 4095) + 0..7 of
  // A[g >> 12]; a negative entry is a zero (padding) group
  const uint16_t* A[kMaxXaSources];
  int K;
  int M;
  int n_cols;           // multiple of 64
  uint16_t* t;
  int ldt;
  int16_t grp[kMaxGroups];
  float coef[kMaxGroups];
  // optional (fast kernel only): the fp16 copy of x, [M][ldxh], 16-byte
  // aligned, ldxh % 8 == 0, written by the launch as it stages x (each
  // element once); range as in QprojArgs
  uint16_t* xh;
  long long ldxh;
  int* range;
  // optional (fast kernel only): bias [n_cols] bf16, T = bf16(coef * sum +
  // bias) -- the dense split-K GEMM's ming_lin_bias
  const uint16_t* bias;
};
hipError_t launch_lora_xa(const LoraXaArgs& a, hipStream_t s);

// Repack the reference pack (codes [N][K*bits/32] u32 LSB-first,
// scales/biases bf16 [N][K/64]) into the tiled resident layout.
hipError_t launch_repack(int bits, const uint32_t* codes,
                         const uint16_t* scales, const uint16_t* biases,
                         int N, int K, uint32_t* codes_t, uint32_t* sb,
                         hipStream_t s);

// ---- norms and rotary --------------------------------------------------------
hipError_t launch_rmsnorm(const uint16_t* x, long long ldx, const uint16_t* w,
                          uint16_t* y, long long ldy, int rows, int D,
                          float eps, hipStream_t s);
// mode 0 plain; 1 also h = fp16(y); 2 h = bf16(h + tg * y) with tg = tanh(gate)
// in f32, y unused; 3 h = bf16(h + y) (see rmsnorm_kernel)
// `range` (optional, mode 1): raised as QprojArgs::range for the fp16 copy
hipError_t launch_rmsnorm_ex(int mode, const uint16_t* x, long long ldx, const uint16_t* w,
                             uint16_t* y, long long ldy, uint16_t* h, long long ldh,
                             const float* tg, int rows, int D, float eps,
                             hipStream_t s, int* range = nullptr);
// t[i] = tanhf(bf16 g[i]) for the two gates of a block's adaLN output:
// g = mods + n (gate_msa) and mods + 3n (gate_mlp) -> t[0, n) and t[n, 2n)
hipError_t launch_tanh_gates(const uint16_t* mods, int n, float* t, hipStream_t s);
// mods[4n] = bf16(mods + b) in place; nw1 = bf16(an1 * (1 + mods[0, n))),
// nw3 = bf16(fn1 * (1 + mods[2n, 3n))); t as launch_tanh_gates
// launch_adaln_glue over up to kGemvBatch blocks in one launch (grid y = entry).
struct GlueEntry {
  uint16_t* mods;
  const uint16_t* b;
  const uint16_t* an1;
  const uint16_t* fn1;
  uint16_t* nw1;
  uint16_t* nw3;
  float* t;
};
struct GlueBatch {
  int n;
  int count;
  GlueEntry e[32];
};
hipError_t launch_adaln_glue_batch(const GlueBatch& b, hipStream_t s);
hipError_t launch_adaln_glue(uint16_t* mods, int n, const uint16_t* b, const uint16_t* an1,
                             const uint16_t* fn1, uint16_t* nw1, uint16_t* nw3, float* t,
                             hipStream_t s);
hipError_t launch_rope_table(const int32_t* pt, const int32_t* ph,
                             const int32_t* pw, int n, int a0, int a1, int a2,
                             int head_dim, double theta, float* cos_t,
                             float* sin_t, hipStream_t s);
// h = bf16(h + (tg *) rmsnorm(sub) * wpost) then y = rmsnorm(h) * wpre and
// yh = fp16(y): the residual modes followed by mode 1, bit for bit, in one pass.
hipError_t launch_norm_residual_norm(const uint16_t* sub, long long lds, const uint16_t* wpost,
                                     uint16_t* h, long long ldh, const float* tg,
                                     const uint16_t* wpre, uint16_t* y, long long ldy,
                                     uint16_t* yh, long long ldyh, int rows, int D, float eps,
                                     hipStream_t s, int* range = nullptr);
// The same on k alone (the attention kernel norms q itself).
hipError_t launch_k_norm_rope(uint16_t* x, long long ld, int k_col, int rows, int n_heads,
                              const uint16_t* wk, const float* cos_t, const float* sin_t,
                              float eps, hipStream_t s);
// LlmOps::qk_norm_rope: heads [0, nq) then nk from column 0, norm when both
// weights are given, rotate-half of half-width rot_half (0, 32, 64) by
// tables [rows][rot_half].
hipError_t launch_llm_qk_norm_rope(uint16_t* x, long long ld, int rows, int nq, int nk,
                                   const uint16_t* wq, const uint16_t* wk, const float* cos_t,
                                   const float* sin_t, int rot_half, float eps, hipStream_t s);
hipError_t launch_qk_norm_rope(uint16_t* x, long long ld, int q_col,
                               int k_col, int rows, int n_heads,
                               const uint16_t* wq, const uint16_t* wk,
                               const float* cos_t, const float* sin_t,
                               float eps, hipStream_t s);

// ---- block glue and the pack quantizer (elementwise.hip) ----------------------
hipError_t launch_swiglu(const uint16_t* g, long long ldg, const uint16_t* u,
                         long long ldu, uint16_t* out, long long ldo, int rows,
                         int n, hipStream_t s);
hipError_t launch_residual(uint16_t* h, long long ldh, const uint16_t* gate,
                           const uint16_t* sub, long long lds, int rows, int n,
                           int gated, hipStream_t s);
hipError_t launch_modulate(const uint16_t* x, long long ldx,
                           const uint16_t* scale, uint16_t* y, long long ldy,
                           int rows, int n, hipStream_t s);
hipError_t launch_bias_act(uint16_t* y, long long ldy, const uint16_t* b,
                           uint16_t* out2, int rows, int n, int mode,
                           hipStream_t s);
hipError_t launch_ln_modulate(const uint16_t* x, long long ldx,
                              const uint16_t* scale, uint16_t* y,
                              long long ldy, int rows, int D, float eps,
                              hipStream_t s);
hipError_t launch_quantize(const float* w, int N, int K, int bits,
                           uint32_t* codes, uint16_t* scales, uint16_t* biases,
                           hipStream_t s);

// ---- projections over a handful of rows (gemv.hip) ----------------------------
// y[m][n] = bf16(sum_k x[m][k] W[n][k]) for m < M <= kGemvMaxM, W in the
// resident general layout (codes + sb for bits 4/8, w16 for bits 16).
constexpr int kGemvMaxM = 8;
struct GemvArgs {
  const uint16_t* x;
  long long ldx;
  const uint32_t* codes;
  const uint32_t* sb;
  const uint16_t* w16;
  uint16_t* y;
  long long ldy;
  int M, N, K;
  const uint16_t* bias;   // optional bias [N] bf16, added before the rounding
};
hipError_t launch_gemv(int bits, const GemvArgs& a, hipStream_t s);
// Up to kGemvBatch GEMVs of one shape over one x in one launch (grid y =
// entry): the per-block adaLN projections of a forward, each entry's bits
// those of launch_gemv on it.
constexpr int kGemvBatch = 32;
struct GemvEntry {
  const uint32_t* codes;
  const uint32_t* sb;
  const uint16_t* w16;
  uint16_t* y;
};
struct GemvBatch {
  GemvArgs base;       // x, ldx, ldy, M, N, K (the entry pointers unused)
  int count;
  GemvEntry e[kGemvBatch];
};
hipError_t launch_gemv_batch(int bits, const GemvBatch& b, hipStream_t s);
hipError_t validate_gemv_kernels();

// ---- the fast quantized route (qproj_fast.hip) --------------------------------
// x is fp16 (carrying bf16 values), a.codes / a.sb the fast resident layout.
hipError_t launch_qproj_fast(int bits, const QprojArgs& a, hipStream_t s);
// The gate and up projections of a SwiGLU in one launch (the fields after
// `range` in QprojArgs): each 256 x 256 tile holds 128 columns of each, so
// the gate's output meets the up projection's in LDS and only
// y = bf16(silu(gate) * up) (and its fp16 copy yh) is written. Both weights
// one segment each with the same number of LoRA tail chunks, N % 8 == 0,
// y 16-byte aligned with ldy % 8 == 0; no K split.
hipError_t launch_qproj_pair(int bits, const QprojArgs& a, hipStream_t s);
hipError_t launch_repack_fast(int bits, const uint32_t* codes,
                              const uint16_t* scales, const uint16_t* biases,
                              int N, int K, uint32_t* codes_f, uint32_t* sbf,
                              int* inexact, hipStream_t s);
// x.A_live^T with split-K: `part` holds kslices * M * n_cols f32 (unused
// when kslices == 1).
int lora_xa_fast_slices(int M, int n_cols, int K);
// The same kernel as a plain split-K bf16 GEMM y = x . W^T of a dense W
// [N][K] (identity groups, coefficient 1): its slice count.
int dense_xa_slices(int M, int N, int K);
// Bytes of f32 partials launch_lora_xa_fast needs for kslices > 1 (whole
// 256 x 128 tiles per slice, in the kernel's accumulator order); 0 otherwise.
size_t lora_xa_part_bytes(int M, int n_cols, int kslices);
hipError_t launch_lora_xa_fast(const LoraXaArgs& a, float* part, int kslices,
                               hipStream_t s);
hipError_t launch_bf16_to_f16(const uint16_t* x, long long ldx, uint16_t* y,
                              long long ldy, int rows, int K, hipStream_t s,
                              int* range = nullptr);

hipError_t validate_qproj_kernels();
hipError_t validate_qproj_fast_kernels();
hipError_t validate_norm_kernels();
hipError_t validate_elementwise_kernels();

}  // namespace ming
