// The DiT's block projections on MI355X: group-64 int4/int8 (or dense bf16)
// weights x bf16 activations, with the runtime-LoRA delta appended along K.
//
// Replaces the reference's lin() = lin_base() + lora::Applier::apply()
// (ming-dit.cc:1721-1771): the host's affine_qmm_steel_w{4,8}g64 /
// dequant->mma route for the base, and one skinny GEMM pair per live slot
// for the adapter. Here one kernel computes
//
//     y = [x | T] . [W_dq | B_live]^T,   T = x . A_live^T * scale (lora_xa)
//
// so the adapter costs no extra pass over y.
//
// Numerics. The base runs on fp16 MFMA: bf16 activations convert to fp16
// exactly (inside fp16's range) and each weight dequantizes as
// fma(code, scale, bias) in f32, rounded once to fp16 -- an error ~8x below
// a bf16 weight tile's, which keeps the output at the bf16-output floor
// (rel-L2 ~1.66e-3 against fp32) where bf16 weight tiles land at ~2.3e-3.
// Dense bf16 weights and the LoRA tail run on bf16 MFMA (both operands
// exact). Accumulation is fp32 throughout; the output rounds once to bf16.
//
// Geometry. 256 threads = 4 wave64s, block tile 256(M) x 256(N) x 64(K),
// each wave a 128 x 128 quadrant of 4 x 4 v_mfma_f32_32x32x16 tiles.
// Double-buffered LDS (2 x 64 KB): x tile [256][64] and w tile [256][64]
// as 16-byte chunks XOR-swizzled by row so both the stores and the
// fragment reads are bank-conflict free. Blocks are remapped so each XCD
// works a contiguous range of the tile grid (its own L2 sees the reuse).
#include "common.h"
#include "kernels.h"

namespace ming {
namespace {

constexpr int BM = kQpBM, BN = kQpBN, BK = kQpBK, NT = kQpThreads;
constexpr int CH = BK / 8;  // 16-byte chunks per tile row

// 16-byte chunks XOR-swizzled by (row >> 1) & 7: a ds_read_b128 serves 16
// lanes per cycle on gfx950's 64 banks, and 128-B rows pair up per bank line.
__device__ __forceinline__ int swz(int row, int c) {
  return row * CH + (c ^ ((row >> 1) & 7));
}

// Logical tile for this block: XCD-contiguous ranges, then grouped raster
// (GM tile-rows per group) inside each range.
__device__ __forceinline__ void tile_of_block(int b, int tiles_m, int tiles_n,
                                              int* tm, int* tn) {
  const int nb = tiles_m * tiles_n;
  const int q = nb / 8, rem = nb % 8;
  const int xcd = b % 8, local = b / 8;
  const int v = xcd * q + (xcd < rem ? xcd : rem) + local;
  constexpr int GM = 4;
  const int gsz = GM * tiles_n;
  const int g = v / gsz;
  const int first = g * GM;
  const int gm = (tiles_m - first) < GM ? (tiles_m - first) : GM;
  const int r = v - g * gsz;
  *tm = first + r % gm;
  *tn = r / gm;
}

// w4 word (8 codes, permuted nibbles) -> 8 fp16 at natural k order.
__device__ __forceinline__ uint4 dequant8_w4(uint32_t w, float s, float b) {
  // nibble i holds k = perm[i], perm = {0,2,4,6,1,3,5,7}
  uint4 o;
  uint32_t* op = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float c0 = (float)((w >> (4 * p)) & 15u);
    const float c1 = (float)((w >> (4 * p + 16)) & 15u);
    op[p] = f32x2_to_f16x2_rne(fmaf(c0, s, b), fmaf(c1, s, b));
  }
  return o;
}

// two w8 words (8 codes, byte i of word j = k 4j+i) -> 8 fp16.
__device__ __forceinline__ uint4 dequant8_w8(uint32_t w0, uint32_t w1,
                                             float s, float b) {
  uint4 o;
  o.x = f32x2_to_f16x2_rne(fmaf((float)(w0 & 255u), s, b),
                           fmaf((float)((w0 >> 8) & 255u), s, b));
  o.y = f32x2_to_f16x2_rne(fmaf((float)((w0 >> 16) & 255u), s, b),
                           fmaf((float)(w0 >> 24), s, b));
  o.z = f32x2_to_f16x2_rne(fmaf((float)(w1 & 255u), s, b),
                           fmaf((float)((w1 >> 8) & 255u), s, b));
  o.w = f32x2_to_f16x2_rne(fmaf((float)((w1 >> 16) & 255u), s, b),
                           fmaf((float)(w1 >> 24), s, b));
  return o;
}

// The wide route's weights: w = fma(code, s, b) in f32 as a pair of bf16
// hi = bf16(w), lo = bf16(w - hi) (the difference is exact in f32), so
// hi + lo carries w to ~2^-17 relative; `lo` picks the member a tile holds.
__device__ __forceinline__ uint32_t wide_pair(float v0, float v1, bool lo) {
  const uint32_t hi = pack_bf16x2_rne(v0, v1);
  if (!lo) return hi;
  return pack_bf16x2_rne(v0 - bf16_lo(hi), v1 - bf16_hi(hi));
}

__device__ __forceinline__ uint4 dequant8_w4_wide(uint32_t w, float s, float b, bool lo) {
  uint4 o;
  uint32_t* op = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float c0 = (float)((w >> (4 * p)) & 15u);
    const float c1 = (float)((w >> (4 * p + 16)) & 15u);
    op[p] = wide_pair(fmaf(c0, s, b), fmaf(c1, s, b), lo);
  }
  return o;
}

__device__ __forceinline__ uint4 dequant8_w8_wide(uint32_t w0, uint32_t w1, float s, float b,
                                                  bool lo) {
  uint4 o;
  o.x = wide_pair(fmaf((float)(w0 & 255u), s, b), fmaf((float)((w0 >> 8) & 255u), s, b), lo);
  o.y = wide_pair(fmaf((float)((w0 >> 16) & 255u), s, b), fmaf((float)(w0 >> 24), s, b), lo);
  o.z = wide_pair(fmaf((float)(w1 & 255u), s, b), fmaf((float)((w1 >> 8) & 255u), s, b), lo);
  o.w = wide_pair(fmaf((float)((w1 >> 16) & 255u), s, b), fmaf((float)(w1 >> 24), s, b), lo);
  return o;
}

__device__ __forceinline__ uint4 bf16x8_to_f16x8(uint4 v) {
  uint4 o;
  o.x = bf16x2_to_f16x2(v.x);
  o.y = bf16x2_to_f16x2(v.y);
  o.z = bf16x2_to_f16x2(v.z);
  o.w = bf16x2_to_f16x2(v.w);
  return o;
}

// WIDE (bits 4/8): x stays bf16 and each weight tile is the hi or the lo
// member of its bf16 pair; K is walked twice (hi, then lo) into the same
// accumulators on bf16 MFMA, so no value passes through fp16.
template <int BITS, bool WIDE>
__global__ __launch_bounds__(NT, 1) void qproj_kernel(const QprojArgs a) {
  constexpr bool F16 = BITS != 16 && !WIDE;   // fp16 x tiles and weights
  __shared__ uint4 lds[2][2][BM * CH];  // [buf][0: x, 1: w][row*8+chunk]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int tiles_m = (a.M + BM - 1) / BM;
  const int tiles_n = (a.N + BN - 1) / BN;
  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;

  // The segment this N tile belongs to (segments are BN-aligned).
  int sg = 0;
  for (int i = 1; i < a.nseg; ++i)
    if (n0 >= a.seg[i].n_begin) sg = i;
  const int t_col0 = a.seg[sg].t_col0;
  // the tail runs in 64-rank steps; an odd count of 32-rank chunks leaves
  // the upper half of the last step as zeros (T and B both)
  const int chunks32 = a.seg[sg].chunks;
  const int chunks = (chunks32 + 1) / 2;
  const int ldb = a.seg[sg].ldb;
  const int grp0 = a.seg[sg].grp0;
  const int seg_nb = a.seg[sg].n_begin, seg_ne = a.seg[sg].n_end;
  const uint16_t* __restrict__ Bp = a.seg[sg].B;

  const int KT = a.K / BK;

  // Per-thread load roles. "row pattern": rows pr + 32 i, chunk pc (x, T,
  // B and dense-weight tiles). Quantized weights: one full 64-wide
  // row-group per thread (row = tid).
  const int pr = tid >> 3, pc = tid & 7;
  // Row clamps: loads past M / N re-read the last row (stores are masked).
  const int mlast = a.M - 1;
  int wrow = n0 + tid;
  wrow = wrow < a.N ? wrow : a.N - 1;

  uint4 xr[8];
  uint4 wr[8];
  uint32_t sbr = 0;
  uint32_t seen = 0;   // magnitudes converted to fp16 (range_report)

  const int fr = lane & 31, fk = lane >> 5;
  floatx16_t acc[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;

  // ---- base stage: x tile + weight tile at k-tile kt ----
  auto load_base = [&](int kt) {
    const int k0 = kt * BK + pc * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int m = m0 + pr + 32 * i;
      m = m < mlast ? m : mlast;
      xr[i] = *reinterpret_cast<const uint4*>(a.x + (long long)m * a.ldx + k0);
    }
    if constexpr (BITS == 16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int n = n0 + pr + 32 * i;
        n = n < a.N ? n : a.N - 1;
        wr[i] = *reinterpret_cast<const uint4*>(a.w16 + (long long)n * a.K + k0);
      }
    } else {
      constexpr int WPR = BITS == 4 ? 8 : 16;
      const uint4* src = reinterpret_cast<const uint4*>(
          a.codes + ((long long)kt * a.N + wrow) * WPR);
#pragma unroll
      for (int i = 0; i < WPR / 4; ++i) wr[i] = src[i];
      sbr = a.sb[(long long)kt * a.N + wrow];
    }
  };
  auto store_base = [&](int buf, bool lo) {
    uint4* lx = lds[buf][0];
    uint4* lw = lds[buf][1];
    if constexpr (BITS == 16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        lx[swz(pr + 32 * i, pc)] = xr[i];
        lw[swz(pr + 32 * i, pc)] = wr[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (F16) {
          seen = range_track4(seen, xr[i]);
          lx[swz(pr + 32 * i, pc)] = bf16x8_to_f16x8(xr[i]);
        } else {
          lx[swz(pr + 32 * i, pc)] = xr[i];
        }
      }
      const float s = bf16_lo(sbr), b = bf16_hi(sbr);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint4 d;
        if constexpr (BITS == 4) {
          const uint32_t w = j < 4 ? (&wr[0].x)[j] : (&wr[1].x)[j - 4];
          d = F16 ? dequant8_w4(w, s, b) : dequant8_w4_wide(w, s, b, lo);
        } else {
          const uint4 q = wr[j >> 1];
          if constexpr (F16)
            d = (j & 1) ? dequant8_w8(q.z, q.w, s, b) : dequant8_w8(q.x, q.y, s, b);
          else
            d = (j & 1) ? dequant8_w8_wide(q.z, q.w, s, b, lo)
                        : dequant8_w8_wide(q.x, q.y, s, b, lo);
        }
        lw[swz(tid, j)] = d;
      }
    }
  };
  // ---- tail stage: T chunk + gathered B chunk ----
  auto load_tail = [&](int ch) {
    const int tc = t_col0 + ch * 64 + pc * 8;
    const bool in = ch * 64 + pc * 8 < 32 * chunks32;   // inside the segment's ranks
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int m = m0 + pr + 32 * i;
      m = m < mlast ? m : mlast;
      xr[i] = in ? *reinterpret_cast<const uint4*>(a.t + (long long)m * a.ldt + tc)
                 : make_uint4(0, 0, 0, 0);
    }
    const int g = in ? a.grp[grp0 + ch * 8 + pc] : -1;
    const int bc = g < 0 ? 0 : g * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int n = n0 + pr + 32 * i;
      n = n < seg_ne ? n : seg_ne - 1;
      uint4 v = *reinterpret_cast<const uint4*>(Bp + (long long)(n - seg_nb) * ldb + bc);
      wr[i] = g < 0 ? make_uint4(0, 0, 0, 0) : v;
    }
  };
  auto store_tail = [&](int buf) {
    uint4* lx = lds[buf][0];
    uint4* lw = lds[buf][1];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lx[swz(pr + 32 * i, pc)] = xr[i];
      lw[swz(pr + 32 * i, pc)] = wr[i];
    }
  };

  auto compute_f16 = [&](int buf) {
    const uint4* lx = lds[buf][0];
    const uint4* lw = lds[buf][1];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = 2 * kk + fk;
      uint4 wa[4], xb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) wa[j] = lw[swz(128 * wn + 32 * j + fr, c)];
#pragma unroll
      for (int i = 0; i < 4; ++i) xb[i] = lx[swz(128 * wm + 32 * i + fr, c)];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              __builtin_bit_cast(half8_t, wa[j]),
              __builtin_bit_cast(half8_t, xb[i]), acc[j][i], 0, 0, 0);
    }
  };
  auto compute_bf16 = [&](int buf) {
    const uint4* lx = lds[buf][0];
    const uint4* lw = lds[buf][1];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = 2 * kk + fk;
      uint4 wa[4], xb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) wa[j] = lw[swz(128 * wn + 32 * j + fr, c)];
#pragma unroll
      for (int i = 0; i < 4; ++i) xb[i] = lx[swz(128 * wm + 32 * i + fr, c)];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, wa[j]),
              __builtin_bit_cast(bf16x8_t, xb[i]), acc[j][i], 0, 0, 0);
    }
  };

  // Base K loop: one barrier per stage; stage s+1 is fetched into
  // registers before stage s's MFMAs and stored to the other buffer after
  // them. The wide route's stages KT..2KT-1 walk K again with the lo weights.
  constexpr int PASSES = (WIDE && BITS != 16) ? 2 : 1;
  const int KS = KT * PASSES;
  load_base(0);
  store_base(0, false);
  __syncthreads();
  for (int st = 0; st < KS; ++st) {
    const int cur = st & 1;
    const bool more = st + 1 < KS;
    const bool next_lo = st + 1 >= KT;
    if (more) load_base(next_lo ? st + 1 - KT : st + 1);
    else if (chunks > 0) load_tail(0);
    if constexpr (F16) compute_f16(cur);
    else compute_bf16(cur);
    if (more) store_base(cur ^ 1, next_lo);
    else if (chunks > 0) store_tail(cur ^ 1);
    __syncthreads();
  }
  if constexpr (F16) range_report(a.range, seen);
  // LoRA tail: the live ranks, appended along K.
  for (int ch = 0; ch < chunks; ++ch) {
    const int cur = (KS + ch) & 1;
    const bool more = ch + 1 < chunks;
    if (more) load_tail(ch + 1);
    compute_bf16(cur);
    if (more) store_tail(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: D[n][m] per tile; lane owns column m, four consecutive n per
  // register quad -> one 8-byte store of 4 bf16.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 128 * wm + 32 * i + fr;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + 128 * wn + 32 * j + 8 * q + 4 * fk;
        if (m < a.M && n < a.N) {
          float r[4] = {acc[j][i][4 * q + 0], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2],
                        acc[j][i][4 * q + 3]};
          if (a.bias) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < a.N) r[e] += bf16_to_f32(a.bias[n + e]);
          }
          uint2 v;
          v.x = pack_bf16x2_rne(r[0], r[1]);
          v.y = pack_bf16x2_rne(r[2], r[3]);
          *reinterpret_cast<uint2*>(a.y + (long long)m * a.ldy + n) = v;
        }
      }
    }
  }
}

// ---- T = x . A_live^T * coef (the adapters' stacked down-projection) -----
constexpr int XA_BM = 128, XA_BN = 64;

__global__ __launch_bounds__(256, 2) void lora_xa_kernel(const LoraXaArgs a) {
  __shared__ uint4 lx[2][XA_BM * CH];
  __shared__ uint4 la[2][XA_BN * CH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.x * XA_BM, c0 = blockIdx.y * XA_BN;
  const int pr = tid >> 3, pc = tid & 7;
  const int KT = a.K / BK;

  const uint16_t* xrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int m = m0 + pr + 32 * i;
    m = m < a.M ? m : a.M - 1;
    xrow[i] = a.x + (long long)m * a.ldx + pc * 8;
  }
  const uint16_t* arow[2];
  bool azero[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = c0 + pr + 32 * i;
    const int g = a.grp[c >> 3];
    azero[i] = g < 0;
    // a padding group reads (and zeroes) rows of the first live group's stack
    const int gs = g < 0 ? a.grp[0] : g;
    arow[i] = a.A[gs >> 12] + (long long)(g < 0 ? 0 : (8 * (g & 4095) + (c & 7))) * a.K +
              pc * 8;
  }
  uint4 xr[4], ar[2];
  auto load = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i) xr[i] = *reinterpret_cast<const uint4*>(xrow[i] + k0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      ar[i] = azero[i] ? make_uint4(0, 0, 0, 0)
                       : *reinterpret_cast<const uint4*>(arow[i] + k0);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) lx[buf][swz(pr + 32 * i, pc)] = xr[i];
#pragma unroll
    for (int i = 0; i < 2; ++i) la[buf][swz(pr + 32 * i, pc)] = ar[i];
  };
  floatx16_t acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  const int fr = lane & 31, fk = lane >> 5;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load(kt + 1);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = 2 * kk + fk;
      const uint4 xb = lx[cur][swz(32 * wave + fr, c)];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint4 aa = la[cur][swz(32 * j + fr, c)];
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, aa), __builtin_bit_cast(bf16x8_t, xb),
            acc[j], 0, 0, 0);
      }
    }
    if (kt + 1 < KT) store(cur ^ 1);
    __syncthreads();
  }
  const int m = m0 + 32 * wave + fr;
  if (m >= a.M) return;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = c0 + 32 * j + 8 * q + 4 * fk;
      const float f = a.coef[c >> 3];
      uint2 v;
      v.x = pack_bf16x2_rne(f * acc[j][4 * q + 0], f * acc[j][4 * q + 1]);
      v.y = pack_bf16x2_rne(f * acc[j][4 * q + 2], f * acc[j][4 * q + 3]);
      *reinterpret_cast<uint2*>(a.t + (long long)m * a.ldt + c) = v;
    }
  }
}

// ---- pack -> resident tiled layout ------------------------------------------
__global__ void repack_codes_kernel(int bits, const uint32_t* codes, int N,
                                    int K, uint32_t* codes_t) {
  const int wpr = bits == 4 ? 8 : 16;
  const long long total = (long long)(K / 64) * N * wpr;
  for (long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x;
       idx < total; idx += (long long)gridDim.x * blockDim.x) {
    const int j = (int)(idx % wpr);
    const long long rest = idx / wpr;
    const int n = (int)(rest % N);
    const int kt = (int)(rest / N);
    const long long words_row = (long long)K * bits / 32;
    const uint32_t w = codes[(long long)n * words_row + (long long)kt * wpr + j];
    uint32_t o = w;
    if (bits == 4) {
      // new nibble i <- old nibble perm[i], perm = {0,2,4,6,1,3,5,7}
      o = 0;
      const int perm[8] = {0, 2, 4, 6, 1, 3, 5, 7};
#pragma unroll
      for (int i = 0; i < 8; ++i) o |= ((w >> (4 * perm[i])) & 15u) << (4 * i);
    }
    codes_t[idx] = o;
  }
}

__global__ void repack_sb_kernel(const uint16_t* scales, const uint16_t* biases,
                                 int N, int G, uint32_t* sb) {
  const long long total = (long long)G * N;
  for (long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x;
       idx < total; idx += (long long)gridDim.x * blockDim.x) {
    const int n = (int)(idx % N);
    const int g = (int)(idx / N);
    sb[idx] = (uint32_t)scales[(long long)n * G + g] |
              ((uint32_t)biases[(long long)n * G + g] << 16);
  }
}

}  // namespace

hipError_t launch_qproj(int bits, const QprojArgs& a, hipStream_t s, bool wide) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (tiles <= 0) return hipSuccess;
  const dim3 g(tiles), b(NT);
  switch (bits) {
    case 4:
      if (wide) hipLaunchKernelGGL((qproj_kernel<4, true>), g, b, 0, s, a);
      else hipLaunchKernelGGL((qproj_kernel<4, false>), g, b, 0, s, a);
      break;
    case 8:
      if (wide) hipLaunchKernelGGL((qproj_kernel<8, true>), g, b, 0, s, a);
      else hipLaunchKernelGGL((qproj_kernel<8, false>), g, b, 0, s, a);
      break;
    case 16: hipLaunchKernelGGL((qproj_kernel<16, false>), g, b, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_lora_xa(const LoraXaArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.n_cols <= 0) return hipSuccess;
  dim3 grid((a.M + XA_BM - 1) / XA_BM, a.n_cols / XA_BN);
  hipLaunchKernelGGL(lora_xa_kernel, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_repack(int bits, const uint32_t* codes,
                         const uint16_t* scales, const uint16_t* biases, int N,
                         int K, uint32_t* codes_t, uint32_t* sb,
                         hipStream_t s) {
  hipLaunchKernelGGL(repack_codes_kernel, dim3(1024), dim3(256), 0, s, bits,
                     codes, N, K, codes_t);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(repack_sb_kernel, dim3(256), dim3(256), 0, s, scales,
                     biases, N, K / 64, sb);
  return hipGetLastError();
}

}  // namespace ming

namespace ming {
// Every kernel of this unit must have code for the current device.
hipError_t validate_qproj_kernels() {
  hipFuncAttributes fa;
  const void* fns[] = {
      reinterpret_cast<const void*>(&qproj_kernel<4, false>),
      reinterpret_cast<const void*>(&qproj_kernel<8, false>),
      reinterpret_cast<const void*>(&qproj_kernel<16, false>),
      reinterpret_cast<const void*>(&qproj_kernel<4, true>),
      reinterpret_cast<const void*>(&qproj_kernel<8, true>),
      reinterpret_cast<const void*>(&lora_xa_kernel),
      reinterpret_cast<const void*>(&repack_codes_kernel),
      reinterpret_cast<const void*>(&repack_sb_kernel)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&fa, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}
}  // namespace ming
