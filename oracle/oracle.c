/*
 * oracle.c -- CPU restatement of Ming-Image's DiT block-projection path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or
 * calls this file. It is the checker the GPU kernels are compared with
 * (tests/, __graft_entry__.smoke) and the scalar CPU path that bench.py
 * times beside the GPU as its reported baseline. Plain C11 + pthreads, no
 * intrinsics.
 *
 * Every function names the reference file:line it restates. The reference
 * (tgo-app-dev/vpipe-ming-image) is a Metal plugin whose arithmetic kernels
 * live in the vpipe host at 8ab6c6cb, which is not vendored; where the
 * reference only fixes the MATH (docs/MING-IMAGE.md 2.2, ming-dit.cc
 * call sites), this file states that math and the pinning tests say how it
 * is checked (closed forms, brute force, invariants, known answers).
 *
 * Parity pins (tests/test_oracle.py):
 *   bf16 RNE ........ hand-built bit patterns, torch's own bf16 cast.
 *   torch randn ..... the four known answers of ming-config-test.cc:99-108.
 *   layout .......... every position check of ming-config-test.cc:61-84.
 *   schedule ........ the closed form of ming-config-test.cc:45-59.
 *   pack/quant ...... round trip, hand-built words, exact symmetric w8.
 *   projection ...... numpy float64 matmul (an independent library routine)
 *                     on dequantized weights, LoRA as a dense fused delta.
 *   rmsnorm ......... numpy restatement + invariants (scale invariance).
 *   rope ............ rotation-by-angle closed form, norm preservation,
 *                     position 0 = identity, pair/axis assignment.
 *   rotate-half ..... the complex rotation of the split halves (numpy
 *                     complex128), rot_half 0 = identity / the per-head
 *                     RMSNorm, pass-through dims, zero angle = no rotation.
 *   attention ....... numpy softmax reference, one-key and uniform cases.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_EXPORT __attribute__((visibility("default")))

/* ---- bf16 ------------------------------------------------------------- */

/* Round-to-nearest-even f32 -> bf16, no NaN special case.
 * ming-dit.cc:173-181 (f32_to_bf16_). */
OR_EXPORT uint16_t
or_bf16_rne(float f)
{
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t r = (u >> 16) & 1u;
  u += 0x7fffu + r;
  return (uint16_t)(u >> 16);
}

/* The generator's copy: NaN -> 0x7fc0, else RNE. ming-generator.cc:44-52. */
OR_EXPORT uint16_t
or_bf16_rne_nan(float f)
{
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) { return (uint16_t)0x7fc0; }
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

OR_EXPORT float
or_bf16_to_f32(uint16_t h)
{
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

OR_EXPORT void
or_f32_to_bf16_n(const float* src, uint16_t* dst, size_t n)
{
  for (size_t i = 0; i < n; ++i) { dst[i] = or_bf16_rne(src[i]); }
}

OR_EXPORT void
or_bf16_to_f32_n(const uint16_t* src, float* dst, size_t n)
{
  for (size_t i = 0; i < n; ++i) { dst[i] = or_bf16_to_f32(src[i]); }
}

/* ---- torch's CPU normal sampler ---------------------------------------- */
/* mt19937 (32-bit), seeded from the low 32 bits of the seed, as
 * std::mt19937 / at::mt19937 seed. ming-torch-randn.h:34-38. */
typedef struct {
  uint32_t mt[624];
  int idx;
} or_mt19937;

static void
mt_seed_(or_mt19937* g, uint32_t s)
{
  g->mt[0] = s;
  for (int i = 1; i < 624; ++i) {
    g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) +
               (uint32_t)i;
  }
  g->idx = 624;
}

static uint32_t
mt_next_(or_mt19937* g)
{
  if (g->idx >= 624) {
    for (int i = 0; i < 624; ++i) {
      const uint32_t y = (g->mt[i] & 0x80000000u) |
                         (g->mt[(i + 1) % 624] & 0x7fffffffu);
      uint32_t v = g->mt[(i + 397) % 624] ^ (y >> 1);
      if (y & 1u) { v ^= 0x9908b0dfu; }
      g->mt[i] = v;
    }
    g->idx = 0;
  }
  uint32_t y = g->mt[g->idx++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

/* 24 random bits over 2^24, ming-torch-randn.h:60-65. */
static float
mt_uniform_(or_mt19937* g)
{
  const double x = (double)(mt_next_(g) & 0xffffffu) * (1.0 / 16777216.0);
  return (float)x;
}

/* Sixteen-wide Box-Muller, ming-torch-randn.h:67-80: radius and the
 * trig in float, theta = (float)(2*pi*(double)u2). */
static void
fill16_(float* p)
{
  const double kPi = 3.14159265358979323846;
  for (int j = 0; j < 8; ++j) {
    const float u1 = 1.0f - p[j];
    const float u2 = p[j + 8];
    const float radius = sqrtf(-2.0f * logf(u1));
    const float theta = (float)(2.0 * kPi * (double)u2);
    p[j] = radius * cosf(theta);
    p[j + 8] = radius * sinf(theta);
  }
}

/* torch.Generator("cpu").manual_seed(seed); torch.randn(n) for n >= 16,
 * the tail redrawing the last 16. ming-torch-randn.h:41-55. Returns -1
 * (and writes nothing) below 16 elements, as the reference refuses. */
OR_EXPORT int
or_torch_randn(uint64_t seed, size_t n, float* out)
{
  if (n < 16 || out == NULL) { return -1; }
  or_mt19937* g = (or_mt19937*)malloc(sizeof(or_mt19937));
  if (g == NULL) { return -1; }
  mt_seed_(g, (uint32_t)(seed & 0xffffffffu));
  for (size_t i = 0; i < n; ++i) { out[i] = mt_uniform_(g); }
  for (size_t i = 0; i + 16 <= n; i += 16) { fill16_(out + i); }
  if (n % 16 != 0) {
    float* t = out + n - 16;
    for (int i = 0; i < 16; ++i) { t[i] = mt_uniform_(g); }
    fill16_(t);
  }
  free(g);
  return 0;
}

/* ---- the quant pack ----------------------------------------------------- */
/*
 * The pack the DiT reads (ming-dit.cc:802-831, 1115-1135): per weight
 * `.weight` U32 [N, K*bits/32], `.scales` and `.biases` bf16 [N, K/group],
 * w = scales*q + biases per group of `group` input columns. Codes are
 * unsigned and packed LSB-first within a word (the MLX affine convention
 * the host quantizer follows -- INFERRED, the in-word order is not pinned
 * by anything in the reference; words per row ARE pinned: K/4 for w8 and
 * K/8 for w4, ming-dit.cc:2675).
 *
 * The two quantizers are the synthetic recipes the benchmark configs
 * state (BASELINE configs 1 and 2): symmetric int8 with s = bf16(max|w|/127),
 * q = clamp(rint(w/s), -127, 127), code = q + 128, bias = -128*s (exact);
 * affine int4 with s = bf16((max-min)/15), b = bf16(min),
 * q = clamp(rint((w-b)/s), 0, 15).
 */
static void
put_code_(uint32_t* row, int k, int bits, uint32_t code)
{
  const int per = 32 / bits;
  row[k / per] |= code << ((k % per) * bits);
}

OR_EXPORT uint32_t
or_get_code(const uint32_t* row, int k, int bits)
{
  const int per = 32 / bits;
  return (row[k / per] >> ((k % per) * bits)) & ((1u << bits) - 1u);
}

OR_EXPORT int
or_quant_w8_sym(const float* w, int N, int K, int group, uint32_t* codes,
                uint16_t* scales, uint16_t* biases)
{
  if (N <= 0 || K <= 0 || group <= 0 || K % group != 0) { return -1; }
  const int G = K / group, words = K / 4;
  memset(codes, 0, sizeof(uint32_t) * (size_t)N * (size_t)words);
  for (int n = 0; n < N; ++n) {
    const float* wr = w + (size_t)n * K;
    uint32_t* cr = codes + (size_t)n * words;
    for (int g = 0; g < G; ++g) {
      float amax = 0.0f;
      for (int j = 0; j < group; ++j) {
        const float a = fabsf(wr[g * group + j]);
        if (a > amax) { amax = a; }
      }
      const uint16_t sb = or_bf16_rne(amax / 127.0f);
      const float s = or_bf16_to_f32(sb);
      scales[(size_t)n * G + g] = sb;
      biases[(size_t)n * G + g] = or_bf16_rne(-128.0f * s);
      for (int j = 0; j < group; ++j) {
        float q = s > 0.0f ? rintf(wr[g * group + j] / s) : 0.0f;
        if (q > 127.0f) { q = 127.0f; }
        if (q < -127.0f) { q = -127.0f; }
        put_code_(cr, g * group + j, 8, (uint32_t)((int)q + 128));
      }
    }
  }
  return 0;
}

OR_EXPORT int
or_quant_w4_affine(const float* w, int N, int K, int group, uint32_t* codes,
                   uint16_t* scales, uint16_t* biases)
{
  if (N <= 0 || K <= 0 || group <= 0 || K % group != 0) { return -1; }
  const int G = K / group, words = K / 8;
  memset(codes, 0, sizeof(uint32_t) * (size_t)N * (size_t)words);
  for (int n = 0; n < N; ++n) {
    const float* wr = w + (size_t)n * K;
    uint32_t* cr = codes + (size_t)n * words;
    for (int g = 0; g < G; ++g) {
      float mn = wr[g * group], mx = wr[g * group];
      for (int j = 1; j < group; ++j) {
        const float v = wr[g * group + j];
        if (v < mn) { mn = v; }
        if (v > mx) { mx = v; }
      }
      const uint16_t sb = or_bf16_rne((mx - mn) / 15.0f);
      const uint16_t bb = or_bf16_rne(mn);
      const float s = or_bf16_to_f32(sb), b = or_bf16_to_f32(bb);
      scales[(size_t)n * G + g] = sb;
      biases[(size_t)n * G + g] = bb;
      for (int j = 0; j < group; ++j) {
        float q = s > 0.0f ? rintf((wr[g * group + j] - b) / s) : 0.0f;
        if (q > 15.0f) { q = 15.0f; }
        if (q < 0.0f) { q = 0.0f; }
        put_code_(cr, g * group + j, 4, (uint32_t)q);
      }
    }
  }
  return 0;
}

/* w[n][k] = scales[n][g]*code + biases[n][g] in f32 (the product of a
 * bf16 scale and a <=8-bit code is exact, so this rounds once).
 * The affine dequant of ming-dit.cc:2663-2677 (affine_dequant_w{4,8}). */
OR_EXPORT int
or_dequant(const uint32_t* codes, const uint16_t* scales,
           const uint16_t* biases, int N, int K, int bits, int group,
           float* w)
{
  if ((bits != 4 && bits != 8) || K % group != 0 || K % (32 / bits) != 0) {
    return -1;
  }
  const int G = K / group, words = K * bits / 32;
  for (int n = 0; n < N; ++n) {
    const uint32_t* cr = codes + (size_t)n * words;
    for (int k = 0; k < K; ++k) {
      const float s = or_bf16_to_f32(scales[(size_t)n * G + k / group]);
      const float b = or_bf16_to_f32(biases[(size_t)n * G + k / group]);
      w[(size_t)n * K + k] = s * (float)or_get_code(cr, k, bits) + b;
    }
  }
  return 0;
}

/* ---- the projection: base + runtime LoRA --------------------------------- */
/*
 * y[m][n] = sum_k x[m][k] W[n][k] + sum_live scale_i * fold_i *
 *           sum_r B_i[n][r] (sum_k A_i[r][k] x[m][k])
 *
 * lin = lin_base then the Applier over every live slot
 * (ming-dit.cc:1721-1771); a slot with strength 0 or no factors is not in
 * the stack at all (ming-dit.cc:3007-3022, ming-dit.h:150-154). `fold_i`
 * is the adapter's alpha/rank (A_i holds it folded in the reference's
 * Adapter; the boundary keeps it as a separate f32 factor). Computed with
 * f64 products and sums: a reference more accurate than the fp32 it is
 * named for. W is either the dequantized pack (f32 [N][K]) or computed on
 * the fly from the codes (or_qproj_packed, the CPU baseline's form).
 */
typedef struct {
  const uint16_t* x;
  int M, K, ldx;
  const float* w;            /* dense f32 [N][K] or NULL */
  const uint32_t* codes;     /* packed when w == NULL */
  const uint16_t* scales;
  const uint16_t* biases;
  int bits, group;
  int N;
  int nslots;
  const int* ranks;
  const uint16_t* const* A;  /* [rank][K] bf16 */
  const uint16_t* const* B;  /* [N][rank] bf16 */
  const float* coef;         /* scale_i * fold_i; 0 drops the slot */
  float* y;
  int ldy;
  int m0, m1;
} proj_job_;

static void*
proj_worker_(void* arg)
{
  proj_job_* j = (proj_job_*)arg;
  const int K = j->K, N = j->N;
  double* xr = (double*)malloc(sizeof(double) * (size_t)K);
  double* wr = (double*)malloc(sizeof(double) * (size_t)K);
  int rtot = 0;
  for (int s = 0; s < j->nslots; ++s) { rtot += j->ranks[s]; }
  double* t = (double*)malloc(sizeof(double) * (size_t)(rtot > 0 ? rtot : 1));
  const int G = j->group > 0 ? K / j->group : 0;
  const int words = j->bits > 0 ? K * j->bits / 32 : 0;
  for (int m = j->m0; m < j->m1; ++m) {
    const uint16_t* xm = j->x + (size_t)m * j->ldx;
    for (int k = 0; k < K; ++k) { xr[k] = (double)or_bf16_to_f32(xm[k]); }
    /* LoRA intermediates t_i = A_i x for this row. */
    int ro = 0;
    for (int s = 0; s < j->nslots; ++s) {
      const int r = j->ranks[s];
      if (j->coef[s] != 0.0f && j->A[s] != NULL) {
        for (int q = 0; q < r; ++q) {
          const uint16_t* ar = j->A[s] + (size_t)q * K;
          double acc = 0.0;
          for (int k = 0; k < K; ++k) {
            acc += (double)or_bf16_to_f32(ar[k]) * xr[k];
          }
          t[ro + q] = acc;
        }
      }
      ro += r;
    }
    for (int n = 0; n < N; ++n) {
      const double* wn;
      if (j->w != NULL) {
        const float* src = j->w + (size_t)n * K;
        for (int k = 0; k < K; ++k) { wr[k] = (double)src[k]; }
        wn = wr;
      } else {
        const uint32_t* cr = j->codes + (size_t)n * words;
        for (int g = 0; g < G; ++g) {
          const float sc = or_bf16_to_f32(j->scales[(size_t)n * G + g]);
          const float bi = or_bf16_to_f32(j->biases[(size_t)n * G + g]);
          for (int q = 0; q < j->group; ++q) {
            const int k = g * j->group + q;
            wr[k] = (double)(sc * (float)or_get_code(cr, k, j->bits) + bi);
          }
        }
        wn = wr;
      }
      double acc = 0.0;
      for (int k = 0; k < K; ++k) { acc += xr[k] * wn[k]; }
      ro = 0;
      for (int s = 0; s < j->nslots; ++s) {
        const int r = j->ranks[s];
        if (j->coef[s] != 0.0f && j->B[s] != NULL) {
          const uint16_t* br = j->B[s] + (size_t)n * r;
          double d = 0.0;
          for (int q = 0; q < r; ++q) {
            d += (double)or_bf16_to_f32(br[q]) * t[ro + q];
          }
          acc += (double)j->coef[s] * d;
        }
        ro += r;
      }
      j->y[(size_t)m * j->ldy + n] = (float)acc;
    }
  }
  free(xr);
  free(wr);
  free(t);
  return NULL;
}

static int
proj_run_(proj_job_* base, int nthreads)
{
  if (nthreads < 1) { nthreads = 1; }
  if (nthreads > base->M) { nthreads = base->M > 0 ? base->M : 1; }
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  proj_job_* jobs = (proj_job_*)malloc(sizeof(proj_job_) * (size_t)nthreads);
  if (th == NULL || jobs == NULL) { free(th); free(jobs); return -1; }
  for (int i = 0; i < nthreads; ++i) {
    jobs[i] = *base;
    jobs[i].m0 = (int)((long long)base->M * i / nthreads);
    jobs[i].m1 = (int)((long long)base->M * (i + 1) / nthreads);
    pthread_create(&th[i], NULL, proj_worker_, &jobs[i]);
  }
  for (int i = 0; i < nthreads; ++i) { pthread_join(th[i], NULL); }
  free(th);
  free(jobs);
  return 0;
}

/* Dense-weight form: w is f32 [N][K] (a dequantized pack, or a dense
 * checkpoint's bf16 weights widened). */
OR_EXPORT int
or_proj(const uint16_t* x, int M, int K, int ldx, const float* w, int N,
        int nslots, const int* ranks, const uint16_t* const* A,
        const uint16_t* const* B, const float* coef, float* y, int ldy,
        int nthreads)
{
  proj_job_ j;
  memset(&j, 0, sizeof(j));
  j.x = x; j.M = M; j.K = K; j.ldx = ldx; j.w = w; j.N = N;
  j.nslots = nslots; j.ranks = ranks; j.A = A; j.B = B; j.coef = coef;
  j.y = y; j.ldy = ldy;
  return proj_run_(&j, nthreads);
}

/* Packed form, dequantizing each weight row on the fly: the scalar CPU
 * path of the same op the GPU kernel runs (bench.py's cpu_baseline). */
OR_EXPORT int
or_qproj_packed(const uint16_t* x, int M, int K, int ldx,
                const uint32_t* codes, const uint16_t* scales,
                const uint16_t* biases, int bits, int group, int N,
                int nslots, const int* ranks, const uint16_t* const* A,
                const uint16_t* const* B, const float* coef, float* y,
                int ldy, int nthreads)
{
  if ((bits != 4 && bits != 8) || group <= 0 || K % group != 0) { return -1; }
  proj_job_ j;
  memset(&j, 0, sizeof(j));
  j.x = x; j.M = M; j.K = K; j.ldx = ldx; j.w = NULL; j.codes = codes;
  j.scales = scales; j.biases = biases; j.bits = bits; j.group = group;
  j.N = N; j.nslots = nslots; j.ranks = ranks; j.A = A; j.B = B;
  j.coef = coef; j.y = y; j.ldy = ldy;
  return proj_run_(&j, nthreads);
}

/* ---- RMSNorm -------------------------------------------------------------- */
/* y = bf16((x * 1/sqrt(mean(x^2) + eps)) * w) per row of D, statistics in
 * f32 (the sum taken in f64 here). The host's rms_norm_fast_f16 as
 * dispatched at ming-dit.cc:1780-1787; formula docs/MING-IMAGE.md:434-436
 * and the precision map at :793 ("RMSNorm stats f32"). Rows are read at
 * ldx and written at ldy, so the per-head qk-norm (ming-dit.cc:2083-2084)
 * is this function over rows*NH rows of head_dim with ld = head_dim. */
OR_EXPORT void
or_rmsnorm(const uint16_t* x, int ldx, const uint16_t* w, uint16_t* y,
           int ldy, int rows, int D, float eps)
{
  for (int r = 0; r < rows; ++r) {
    const uint16_t* xr = x + (size_t)r * ldx;
    double ss = 0.0;
    for (int d = 0; d < D; ++d) {
      const double v = (double)or_bf16_to_f32(xr[d]);
      ss += v * v;
    }
    const float inv = 1.0f / sqrtf((float)(ss / (double)D) + eps);
    uint16_t* yr = y + (size_t)r * ldy;
    for (int d = 0; d < D; ++d) {
      const float v = (or_bf16_to_f32(xr[d]) * inv) * or_bf16_to_f32(w[d]);
      yr[d] = or_bf16_rne(v);
    }
  }
}

/* The folded pre-norm gain nw = bf16(norm_w * (1 + scale)): the block's
 * modulation folded into the RMSNorm weight, ming-dit.cc:2266-2273 (the
 * adaln_modulate kernel over one row with a zero shift). */
OR_EXPORT void
or_fold_gain(const uint16_t* norm_w, const uint16_t* scale, uint16_t* out,
             int D)
{
  for (int d = 0; d < D; ++d) {
    const float v = or_bf16_to_f32(norm_w[d]) *
                    (1.0f + or_bf16_to_f32(scale[d])) + 0.0f;
    out[d] = or_bf16_rne(v);
  }
}

/* ---- RoPE ------------------------------------------------------------------ */
/* f32 cos/sin per (row, pair) from three integer positions: pairs
 * [0, axes[0]/2) use axis 0, the next axes[1]/2 axis 1, the rest axis 2;
 * freq = 1/theta^(2j/d) in f64, angle = pos*freq in f64, then f32.
 * ming-dit.cc:1443-1486 (build_rope_, which writes each pair twice; this
 * table holds it once, [n][head_dim/2]). */
OR_EXPORT int
or_rope_table(const int32_t* pos_t, const int32_t* pos_h,
              const int32_t* pos_w, int n, const int* axes, int head_dim,
              double theta, float* cos_out, float* sin_out)
{
  const int pairs = head_dim / 2;
  double freq[512];
  int axis[512];
  if (pairs > 512) { return -1; }
  int pair = 0;
  for (int a = 0; a < 3; ++a) {
    for (int j = 0; j < axes[a] / 2 && pair < pairs; ++j, ++pair) {
      freq[pair] = 1.0 / pow(theta, (double)(2 * j) / (double)axes[a]);
      axis[pair] = a;
    }
  }
  if (pair != pairs) { return -1; }
  for (int t = 0; t < n; ++t) {
    const double pos[3] = {(double)pos_t[t], (double)pos_h[t],
                           (double)pos_w[t]};
    for (int p = 0; p < pairs; ++p) {
      const double ang = pos[axis[p]] * freq[p];
      cos_out[(size_t)t * pairs + p] = (float)cos(ang);
      sin_out[(size_t)t * pairs + p] = (float)sin(ang);
    }
  }
  return 0;
}

/* Interleaved-pair rotation (x[2p] + i x[2p+1]) * (c + i s) in f32,
 * rounded to bf16: transpose_rope_pair_ftab_f16 as dispatched at
 * ming-dit.cc:1885-1895 (without the transpose; the token-major layout is
 * kept), docs/MING-IMAGE.md:446-449. `x` is [rows][ld] holding n_heads
 * heads of head_dim from column col0; table rows start at table_row0. */
OR_EXPORT void
or_rope_apply(uint16_t* x, int ld, int col0, int rows, int n_heads,
              int head_dim, const float* cos_t, const float* sin_t,
              int table_row0)
{
  const int pairs = head_dim / 2;
  for (int r = 0; r < rows; ++r) {
    const float* c = cos_t + (size_t)(table_row0 + r) * pairs;
    const float* s = sin_t + (size_t)(table_row0 + r) * pairs;
    for (int h = 0; h < n_heads; ++h) {
      uint16_t* v = x + (size_t)r * ld + col0 + (size_t)h * head_dim;
      for (int p = 0; p < pairs; ++p) {
        const float a = or_bf16_to_f32(v[2 * p]);
        const float b = or_bf16_to_f32(v[2 * p + 1]);
        v[2 * p] = or_bf16_rne(a * c[p] - b * s[p]);
        v[2 * p + 1] = or_bf16_rne(a * s[p] + b * c[p]);
      }
    }
  }
}

/* qk-norm then RoPE, in place, as run_block sequences them
 * (ming-dit.cc:2083-2086): per-head RMSNorm to bf16, then the rotation
 * of that bf16 to bf16. q heads at column q_col, k heads at k_col. */
OR_EXPORT void
or_qk_norm_rope(uint16_t* x, int ld, int q_col, int k_col, int rows,
                int n_heads, int head_dim, const uint16_t* wq,
                const uint16_t* wk, const float* cos_t, const float* sin_t,
                int table_row0, float eps)
{
  for (int r = 0; r < rows; ++r) {
    uint16_t* row = x + (size_t)r * ld;
    or_rmsnorm(row + q_col, head_dim, wq, row + q_col, head_dim, n_heads,
               head_dim, eps);
    or_rmsnorm(row + k_col, head_dim, wk, row + k_col, head_dim, n_heads,
               head_dim, eps);
  }
  or_rope_apply(x, ld, q_col, rows, n_heads, head_dim, cos_t, sin_t,
                table_row0);
  or_rope_apply(x, ld, k_col, rows, n_heads, head_dim, cos_t, sin_t,
                table_row0);
}

/* The LLM encoder's fused qk-norm + rotate-half RoPE, LlmOps::qk_norm_rope
 * (ming-ops.h:118-122, ming-ops.cc:281-302) as its kernel defines it
 * (ming_llm.metal:100-178). In place on [rows][row_stride] bf16: heads
 * [0, n_q) are queries from column 0, heads [n_q, n_q + n_k) keys right after
 * them, 128 wide each; columns past them (the values) are not touched.
 * With both weights given (ming-ops.cc:287), each head is RMS-normalized (f32
 * statistics, eps) and scaled as x * (inv * w), w = q_w or k_w [128]; then
 * the rotate-half rotation of half-width rot_half by the row's angles,
 * cos/sin [rows][rot_half] f32:
 *   32: pairs (j, j + 32) for j < 32, dims 64..127 pass through;
 *   64: pairs (j, j + 64) for j < 64, the whole head;
 *    0: no rotation;
 * (x_j, x_{j+R}) -> (x_j c_j - x_{j+R} s_j, x_{j+R} c_j + x_j s_j) in f32,
 * and each element is rounded to bf16 once at the end. Returns -1 for
 * another rot_half. */
OR_EXPORT int
or_llm_qk_norm_rope(uint16_t* qkv, int row_stride, const uint16_t* q_w,
                    const uint16_t* k_w, const float* cos_t,
                    const float* sin_t, int rows, int n_q, int n_k,
                    int rot_half, float eps)
{
  if (rot_half != 0 && rot_half != 32 && rot_half != 64) { return -1; }
  const int norm = q_w != NULL && k_w != NULL;
  float v[128];
  for (int r = 0; r < rows; ++r) {
    for (int h = 0; h < n_q + n_k; ++h) {
      uint16_t* p = qkv + (size_t)r * row_stride + (size_t)h * 128;
      for (int d = 0; d < 128; ++d) { v[d] = or_bf16_to_f32(p[d]); }
      if (norm) {
        double ss = 0.0;
        for (int d = 0; d < 128; ++d) { ss += (double)v[d] * (double)v[d]; }
        const float inv = 1.0f / sqrtf((float)(ss / 128.0) + eps);
        const uint16_t* w = h < n_q ? q_w : k_w;
        for (int d = 0; d < 128; ++d) {
          v[d] = v[d] * (inv * or_bf16_to_f32(w[d]));
        }
      }
      if (rot_half > 0) {
        const float* c = cos_t + (size_t)r * rot_half;
        const float* s = sin_t + (size_t)r * rot_half;
        for (int j = 0; j < rot_half; ++j) {
          const float a = v[j], b = v[j + rot_half];
          v[j] = a * c[j] - b * s[j];
          v[j + rot_half] = b * c[j] + a * s[j];
        }
      }
      for (int d = 0; d < 128; ++d) { p[d] = or_bf16_rne(v[d]); }
    }
  }
  return 0;
}

/* ---- sequence layout, schedule, timestep ---------------------------------- */
/* [image | caption] with the pads dropped and the positions keeping the
 * padded caption run: image (roundup32(cap)+1, h, w), caption i
 * (1+i, 0, 0). ming-layout.cc:18-65. info = {img_tokens, cap_len,
 * cap_total, joint_len}. Returns -1 on the reference's refusals. */
OR_EXPORT int
or_build_layout(int grid_h, int grid_w, int query_rows, int text_rows,
                int axis0_len, int32_t* pos_t, int32_t* pos_h,
                int32_t* pos_w, int* info)
{
  if (grid_h <= 0 || grid_w <= 0) { return -1; }
  if (query_rows < 0 || text_rows < 0 || query_rows + text_rows <= 0) {
    return -1;
  }
  const int img = grid_h * grid_w;
  const int cap = query_rows + text_rows;
  const int cap_total = (cap % 32 == 0) ? cap : cap + (32 - cap % 32);
  if (axis0_len > 0 && cap_total + 1 >= axis0_len) { return -1; }
  info[0] = img; info[1] = cap; info[2] = cap_total; info[3] = img + cap;
  if (pos_t == NULL) { return 0; }
  for (int h = 0; h < grid_h; ++h) {
    for (int w = 0; w < grid_w; ++w) {
      const int r = h * grid_w + w;
      pos_t[r] = cap_total + 1;
      pos_h[r] = h;
      pos_w[r] = w;
    }
  }
  for (int i = 0; i < cap; ++i) {
    pos_t[img + i] = i + 1;
    pos_h[img + i] = 0;
    pos_w[img + i] = 0;
  }
  return 0;
}

/* sigma_k = shift*u/(1+(shift-1)*u), u = 1-k/S, in f64 then f32, plus a
 * terminal 0: ming-generator.cc:157-174. `out` holds steps+1 values. */
OR_EXPORT int
or_schedule_sigmas(int steps, float shift, float* out)
{
  if (steps <= 0) { return -1; }
  for (int k = 0; k < steps; ++k) {
    const double u = 1.0 - (double)k / (double)steps;
    const double sig = (double)shift * u / (1.0 + ((double)shift - 1.0) * u);
    out[k] = (float)sig;
  }
  out[steps] = 0.0f;
  return 0;
}

/* Cos-first sinusoid at t = t_scale*(1 - sigma): ming-dit.cc:1422-1437. */
OR_EXPORT void
or_time_proj(float sigma, float t_scale, int D, float* out)
{
  const int half = D / 2;
  const double t = (double)t_scale * (1.0 - (double)sigma);
  for (int i = 0; i < half; ++i) {
    const double f = exp(-log(10000.0) * (double)i / (double)half);
    const double a = t * f;
    out[i] = (float)cos(a);
    out[half + i] = (float)sin(a);
  }
}

/* ---- block glue ------------------------------------------------------------- */
/* h[m][n] = bf16(h + tanh(gate[n]) * sub[m][n]) in f32:
 * gated_residual_tanh_f16, ming_ops.metal:59-74. */
OR_EXPORT void
or_gated_residual(uint16_t* h, int ldh, const uint16_t* gate,
                  const uint16_t* sub, int lds, int rows, int N)
{
  for (int r = 0; r < rows; ++r) {
    for (int n = 0; n < N; ++n) {
      const float v = or_bf16_to_f32(h[(size_t)r * ldh + n]) +
                      tanhf(or_bf16_to_f32(gate[n])) *
                      or_bf16_to_f32(sub[(size_t)r * lds + n]);
      h[(size_t)r * ldh + n] = or_bf16_rne(v);
    }
  }
}

/* out = bf16(g / (1 + exp(-g)) * u): swiglu_v4_f16, ming_ops.metal:97-112. */
OR_EXPORT void
or_swiglu(const uint16_t* g, const uint16_t* u, uint16_t* out, size_t n)
{
  for (size_t i = 0; i < n; ++i) {
    const float gv = or_bf16_to_f32(g[i]);
    const float sg = gv / (1.0f + expf(-gv));
    out[i] = or_bf16_rne(sg * or_bf16_to_f32(u[i]));
  }
}

/* y = bf16(y + b[n]), then bf16(silu(.)) when silu != 0: the bias and
 * silu dispatches of ming-dit.cc:1773-1794 (timestep MLP, adaLN). */
OR_EXPORT void
or_bias_act(uint16_t* y, int ldy, const uint16_t* b, int rows, int N,
            int silu)
{
  for (int r = 0; r < rows; ++r) {
    for (int n = 0; n < N; ++n) {
      float v = or_bf16_to_f32(or_bf16_rne(
          or_bf16_to_f32(y[(size_t)r * ldy + n]) + or_bf16_to_f32(b[n])));
      if (silu) { v = v / (1.0f + expf(-v)); }
      y[(size_t)r * ldy + n] = or_bf16_rne(v);
    }
  }
}

/* The final layer: LayerNorm without affine (eps 1e-6 there), rounded to
 * bf16, then * (1 + scale[n]) (ming-dit.cc:2553-2563; docs/MING-IMAGE.md
 * 2.2 "Final layer"). Mean and variance in f64 here. */
OR_EXPORT void
or_ln_modulate(const uint16_t* x, int ldx, const uint16_t* scale, uint16_t* y,
               int ldy, int rows, int D, float eps)
{
  for (int r = 0; r < rows; ++r) {
    const uint16_t* xr = x + (size_t)r * ldx;
    double s = 0.0;
    for (int d = 0; d < D; ++d) { s += (double)or_bf16_to_f32(xr[d]); }
    const float mean = (float)(s / D);
    double v = 0.0;
    for (int d = 0; d < D; ++d) {
      const double t = (double)(or_bf16_to_f32(xr[d]) - mean);
      v += t * t;
    }
    const float inv = 1.0f / sqrtf((float)(v / D) + eps);
    for (int d = 0; d < D; ++d) {
      const float nrm = or_bf16_to_f32(
          or_bf16_rne((or_bf16_to_f32(xr[d]) - mean) * inv));
      y[(size_t)r * ldy + d] =
          or_bf16_rne(nrm * (1.0f + or_bf16_to_f32(scale[d])));
    }
  }
}

/* Non-causal, maskless softmax(q k^T * scale) v per head, f64 internally,
 * bf16 out: the dense attention run_attn dispatches
 * (ming-dit.cc:1905-2039). q/k/v/o are token-major [rows][ld] with head h
 * at column col + h*head_dim. */
OR_EXPORT void
or_attention(const uint16_t* q, int ldq, const uint16_t* k, int ldk,
             const uint16_t* v, int ldv, uint16_t* o, int ldo, int rows,
             int n_heads, int head_dim, float scale)
{
  double* p = (double*)malloc(sizeof(double) * (size_t)rows);
  double* acc = (double*)malloc(sizeof(double) * (size_t)head_dim);
  for (int h = 0; h < n_heads; ++h) {
    for (int i = 0; i < rows; ++i) {
      const uint16_t* qi = q + (size_t)i * ldq + (size_t)h * head_dim;
      double mx = -1e300;
      for (int j = 0; j < rows; ++j) {
        const uint16_t* kj = k + (size_t)j * ldk + (size_t)h * head_dim;
        double s = 0.0;
        for (int d = 0; d < head_dim; ++d) {
          s += (double)or_bf16_to_f32(qi[d]) * (double)or_bf16_to_f32(kj[d]);
        }
        p[j] = s * (double)scale;
        if (p[j] > mx) { mx = p[j]; }
      }
      double den = 0.0;
      for (int j = 0; j < rows; ++j) { p[j] = exp(p[j] - mx); den += p[j]; }
      for (int d = 0; d < head_dim; ++d) { acc[d] = 0.0; }
      for (int j = 0; j < rows; ++j) {
        const uint16_t* vj = v + (size_t)j * ldv + (size_t)h * head_dim;
        for (int d = 0; d < head_dim; ++d) {
          acc[d] += p[j] * (double)or_bf16_to_f32(vj[d]);
        }
      }
      uint16_t* oi = o + (size_t)i * ldo + (size_t)h * head_dim;
      for (int d = 0; d < head_dim; ++d) {
        oi[d] = or_bf16_rne((float)(acc[d] / den));
      }
    }
  }
  free(p);
  free(acc);
}
