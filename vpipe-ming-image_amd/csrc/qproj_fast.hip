// The quantized projection's fast route on MI355X (gfx950): a three-stage
// LDS ring filled by direct global->LDS DMA (global_load_lds_dwordx4), raw
// int codes dequantized per MFMA fragment with packed-fp16 arithmetic,
// and the LoRA tail through the same ring.
//
// Same contract as qproj_kernel (y = [x | T] . [W_dq | B_live]^T, see
// qproj.hip), with two preconditions the host checks:
//   * x arrives as fp16 carrying bf16 values (exact inside fp16's range);
//   * every scale and bias of the weight is exact in fp16, so the weight
//     is dequantized as fp16(fma(code, s, b)) with ONE rounding by
//     v_pk_fma_f16 on the exact integer code (built with the 0x6400 magic:
//     (0x6400 | c) is 1024 + c in fp16, and 1024 is subtracted exactly).
//
// Per block: 256 threads (4 wave64s), tile 256(M) x 256(N) x 64(K); the
// waves split N, each owning 64 columns x 256 rows (2 x 8 tiles of
// v_mfma_f32_32x32x16_f16), so each weight is dequantized once. Per stage
// the DMA moves the fp16 x tile (32 KB), the code tile (8 KB w4 / 16 KB
// w8) and 256 fp16 (scale, bias) pairs. No VGPR round trip, and each wave
// waits on its own vmcnt for the stage two behind the one in flight.
// Every stage buffer is its own __shared__ object so the compiler's LDS-DMA
// tracking sees that reads of one stage do not alias the DMA into another.
//
// Resident code layout this kernel reads (built by repack_*_fast):
//   w4: codes[kt][n][fk][kk]   one u32 = the 8 codes of k = 16kk + 8fk + 0..7,
//       nibbles ordered {k0,k4,k1,k5,k2,k6,k3,k7} so w & 0x0F0F0F0F holds
//       k0..k3 one per byte and (w >> 4) & 0x0F0F0F0F holds k4..k7
//   w8: codes[kt][n][fk][kk][2] two u32 = those 8 codes, bytes in k order
//   sbf[kt][n] = fp16 scale | fp16 bias << 16
#include "common.h"
#include "kernels.h"

namespace ming {
namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BN = 256, BK = 64;

// LDS swizzles for gfx950's 64 x 4-byte banks: a ds_read_b128 serves 16
// lanes (256 B) per cycle, and a fragment read has those 16 lanes on 16
// consecutive rows at one logical chunk. Rows of 128 B (8 chunks) pair up
// per 256-B bank line, so the chunk is XORed with (row >> 1) & 7; rows of
// 64 B (4 chunks) fill a line four at a time: XOR with (row >> 2) & 3.
__device__ __forceinline__ int swz8(int row, int c) { return row * 8 + (c ^ ((row >> 1) & 7)); }
__device__ __forceinline__ int swz4(int row, int c) { return row * 4 + (c ^ ((row >> 2) & 3)); }

// Workgroup barrier for the DMA ring: this wave's LDS reads are complete
// (so another wave may DMA over them) and, being an asm with a memory
// clobber, no LDS access or DMA issue moves across it -- without the
// vmcnt(0) a __syncthreads() would add, which would drain the ring.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// s_waitcnt immediate for "vmcnt <= v" (gfx9 encoding: vmcnt[3:0] and
// vmcnt[5:4] at bits 15:14; expcnt and lgkmcnt left at no-wait).
constexpr unsigned vm_wait(unsigned v) {
  return (v & 0xFu) | ((v >> 4) << 14) | (0x7u << 4) | (0xFu << 8);
}

__device__ __forceinline__ void dma16(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, lds_wave_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, lds_wave_base, 4, 0, 0);
}

// 8 codes (one w4 word) -> 8 fp16 dequantized values. The word's nibbles
// are ordered {k0,k4,k1,k5,k2,k6,k3,k7}, so lo = w & 0x0F0F0F0F holds
// k0..k3 one per byte and hi = (w >> 4) & 0x0F0F0F0F holds k4..k7; one
// v_perm per pair then lays a code under the 0x64 magic byte.
__device__ __forceinline__ uint4 deq_w4(uint32_t w, half2v s2, half2v b2) {
  const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  const uint32_t lo = w & 0x0F0F0F0Fu;
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
  uint32_t v[4];
  v[0] = __builtin_amdgcn_perm(0x64646464u, lo, 0x05010400u);
  v[1] = __builtin_amdgcn_perm(0x64646464u, lo, 0x05030402u);
  v[2] = __builtin_amdgcn_perm(0x64646464u, hi, 0x05010400u);
  v[3] = __builtin_amdgcn_perm(0x64646464u, hi, 0x05030402u);
  uint4 o;
  uint32_t* op = &o.x;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const half2v c = __builtin_bit_cast(half2v, v[p]) - k1024;
    op[p] = __builtin_bit_cast(uint32_t, c * s2 + b2);
  }
  return o;
}

// 8 codes (two w8 words, bytes in k order) -> 8 fp16.
__device__ __forceinline__ uint4 deq_w8(uint32_t w0, uint32_t w1, half2v s2,
                                        half2v b2) {
  const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  uint32_t v[4];
  v[0] = __builtin_amdgcn_perm(0x64646464u, w0, 0x05010400u);
  v[1] = __builtin_amdgcn_perm(0x64646464u, w0, 0x05030402u);
  v[2] = __builtin_amdgcn_perm(0x64646464u, w1, 0x05010400u);
  v[3] = __builtin_amdgcn_perm(0x64646464u, w1, 0x05030402u);
  uint4 o;
  uint32_t* op = &o.x;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const half2v c = __builtin_bit_cast(half2v, v[p]) - k1024;
    op[p] = __builtin_bit_cast(uint32_t, c * s2 + b2);
  }
  return o;
}

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

// Code-chunk swizzle inside a row group: chunk h of row n sits at
// n*CPR + (h ^ sw(n)), so the 16 rows a fragment read serves per LDS cycle
// land on distinct banks (rows are 32 B (w4) / 64 B (w8) apart).
template <int CPR>
__device__ __forceinline__ int wswz(int n) {
  return CPR == 2 ? ((n >> 3) & 1) : ((n >> 2) & 3);
}
template <int CPR>
__device__ __forceinline__ int wchunk(int n, int h) {
  return n * CPR + (h ^ wswz<CPR>(n));
}

template <int BITS>
__global__ __launch_bounds__(256, 1) void qproj_fast_kernel(const QprojArgs a) {
  constexpr int WCH = BITS == 4 ? 512 : 1024;    // 16-B code chunks per stage
  constexpr int CPR = BITS == 4 ? 2 : 4;         // code chunks per row
  constexpr int WDMA = WCH / 256;                // code DMAs per wave per stage
  constexpr int PER = 8 + WDMA + 1;              // DMAs per wave per base stage
  // One __shared__ object per stage ([x 32 KB | codes | (s, b)]): the
  // compiler tracks LDS DMA per object, and three objects stay within
  // what it tracks, so a read of one stage never waits on another's DMA.
  constexpr int STG = BM * 8 + WCH + BN / 4;
  __shared__ uint4 st0[STG], st1[STG], st2[STG];
  uint4* const sX0 = st0;
  uint4* const sX1 = st1;
  uint4* const sX2 = st2;
  uint4* const sW0 = st0 + BM * 8;
  uint4* const sW1 = st1 + BM * 8;
  uint4* const sW2 = st2 + BM * 8;
  uint32_t* const sS0 = reinterpret_cast<uint32_t*>(st0 + BM * 8 + WCH);
  uint32_t* const sS1 = reinterpret_cast<uint32_t*>(st1 + BM * 8 + WCH);
  uint32_t* const sS2 = reinterpret_cast<uint32_t*>(st2 + BM * 8 + WCH);

  // Waves split N only: wave w owns output columns [64w, 64w+64) for all
  // 256 rows (2 x 8 tiles of 32x32), so every weight fragment is
  // dequantized by exactly one wave.
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fk = lane >> 5;

  const int tiles_m = (a.M + BM - 1) / BM;
  const int tiles_n = (a.N + BN - 1) / BN;
  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT = a.K / BK;
  const int mlast = a.M - 1, nlast = a.N - 1;

  const _Float16* __restrict__ x16 = reinterpret_cast<const _Float16*>(a.x);
  const uint4* __restrict__ codes = reinterpret_cast<const uint4*>(a.codes);

  // DMA sources for this lane, per stage (advance by k).
  // x tile: wave issues chunks q = 8*wave + i; lane p = 64q + lane.
  long long xoff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int p = 64 * (8 * wave + i) + lane;
    const int row = p >> 3;
    const int c = (p & 7) ^ ((row >> 1) & 7);
    int m = m0 + row;
    m = m < mlast ? m : mlast;
    xoff[i] = (long long)m * a.ldx + 8 * c;
  }
  // code tile: LDS chunk p holds row p / CPR, logical chunk (p % CPR) ^ sw
  long long woff[WDMA];
#pragma unroll
  for (int i = 0; i < WDMA; ++i) {
    const int p = 64 * (WDMA * wave + i) + lane;
    const int r = p / CPR;
    const int h = (p % CPR) ^ wswz<CPR>(r);
    int n = n0 + r;
    n = n < nlast ? n : nlast;
    woff[i] = (long long)n * CPR + h;
  }
  int sn = n0 + 64 * wave + lane;
  sn = sn < nlast ? sn : nlast;

  auto issue = [&](int kt, uint4* X, uint4* W, uint32_t* S) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dma16(x16 + xoff[i] + kt * BK, X + 64 * (8 * wave + i));
#pragma unroll
    for (int i = 0; i < WDMA; ++i)
      dma16(codes + (long long)kt * a.N * CPR + woff[i], W + 64 * (WDMA * wave + i));
    dma4(a.sb + (long long)kt * a.N + sn, S + 64 * wave);
  };

  floatx16_t acc[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;

  // One stage of MFMA work: code words + (s, b) for the wave's 2 n-tiles,
  // then 4 k16 steps, each reading and dequantizing the next step's
  // fragments beside this step's 16 MFMAs. The interleave is pinned with
  // scheduling-group barriers: left alone, the scheduler (at the VGPR
  // limit) sinks each fragment read next to its MFMA and exposes the LDS
  // latency every few MFMAs. `pre` runs inside step 0 (the ring's DMA
  // issue), interleaved with its MFMAs.
  auto compute = [&](const uint4* X, const uint4* W, const uint32_t* S, auto&& pre) {
    uint4 wc[2][CPR / 2];
    half2v s2[2], b2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = 64 * wave + 32 * j + fr;
#pragma unroll
      for (int h = 0; h < CPR / 2; ++h)
        wc[j][h] = W[wchunk<CPR>(n, fk * (CPR / 2) + h)];
      const uint32_t sb = S[n];
      s2[j] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(sb, sb, 0x01000100u));
      b2[j] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(sb, sb, 0x03020302u));
    }
    auto deq = [&](int j, int kk) -> uint4 {
      if constexpr (BITS == 4) {
        return deq_w4((&wc[j][0].x)[kk], s2[j], b2[j]);
      } else {
        const uint32_t* w = &wc[j][kk >> 1].x;
        return deq_w8(w[(kk & 1) * 2], w[(kk & 1) * 2 + 1], s2[j], b2[j]);
      }
    };
    uint4 wa[2], xb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xb[i] = X[swz8(32 * i + fr, fk)];
#pragma unroll
    for (int j = 0; j < 2; ++j) wa[j] = deq(j, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4 wn_[2], xn_[8];
      if (kk == 0) pre();
      if (kk < 3) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xn_[i] = X[swz8(32 * i + fr, 2 * (kk + 1) + fk)];
#pragma unroll
        for (int j = 0; j < 2; ++j) wn_[j] = deq(j, kk + 1);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              __builtin_bit_cast(half8_t, wa[j]), __builtin_bit_cast(half8_t, xb[i]),
              acc[j][i], 0, 0, 0);
      if (kk == 0) {
        // the ring's DMAs (with their address and M0 setup), one per MFMA
#pragma unroll
        for (int g = 0; g < PER; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        }
      }
      if (kk < 3) {
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // 4 VALU
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (kk < 3) {
#pragma unroll
        for (int j = 0; j < 2; ++j) wa[j] = wn_[j];
#pragma unroll
        for (int i = 0; i < 8; ++i) xb[i] = xn_[i];
      }
    }
  };

  // ---- base ring: stage kt lives in buffer kt % 3 ----
  // Iteration kt: wait for stage kt (this wave's DMAs; stage kt+1 stays in
  // flight), barrier (every wave's stage kt landed AND every wave is done
  // reading buffer (kt+2)%3 from iteration kt-1), issue stage kt+2 beside
  // stage kt's first MFMAs, compute stage kt. Every iteration issues and
  // waits the same way -- past the end the "next" stage re-reads stage
  // KT-1 into a buffer nothing reads -- so the waits are one static vmcnt
  // and the compiler adds no drain of its own.
  auto step = [&](int kt, uint4* Xc, uint4* Wc, uint32_t* Sc, uint4* Xn,
                  uint4* Wn, uint32_t* Sn) {
    __builtin_amdgcn_s_waitcnt(vm_wait(PER));   // stage kt done
    ring_barrier();
    const int nk = kt + 2 < KT ? kt + 2 : KT - 1;
    if (kt < KT) {
      compute(Xc, Wc, Sc, [&] { issue(nk, Xn, Wn, Sn); });
    } else {
      issue(nk, Xn, Wn, Sn);
    }
  };

  issue(0, sX0, sW0, sS0);
  issue(KT > 1 ? 1 : 0, sX1, sW1, sS1);
  // Three steps per trip, all issuing and waiting (a step past KT only
  // skips its MFMA work), so no path through the loop leaves a different
  // set of DMAs in flight.
  for (int kt = 0; kt < KT; kt += 3) {
    step(kt, sX0, sW0, sS0, sX2, sW2, sS2);
    step(kt + 1, sX1, sW1, sS1, sX0, sW0, sS0);
    step(kt + 2, sX2, sW2, sS2, sX1, sW1, sS1);
  }
  __builtin_amdgcn_s_waitcnt(vm_wait(0));       // drain the ring

  // ---- LoRA tail: T and gathered B chunks of 32 ranks, same ring ----
  int sg = 0;
  for (int i = 1; i < a.nseg; ++i)
    if (n0 >= a.seg[i].n_begin) sg = i;
  const int chunks32 = 2 * a.seg[sg].chunks;
  if (chunks32 > 0) {
    const int t_col0 = a.seg[sg].t_col0;
    const int ldb = a.seg[sg].ldb;
    const int grp0 = a.seg[sg].grp0;
    const int seg_nb = a.seg[sg].n_begin, seg_ne = a.seg[sg].n_end;
    const uint16_t* __restrict__ Bp = a.seg[sg].B;
    // the first live group of the segment: a finite source for padding
    // groups (their T columns are exactly 0)
    const int g_safe = a.grp[grp0];
    long long toff[4];
    long long boff[4];
    int bc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 64 * (4 * wave + i) + lane;
      const int row = p >> 2;
      const int c = (p & 3) ^ ((row >> 2) & 3);
      int m = m0 + row;
      m = m < mlast ? m : mlast;
      toff[i] = (long long)m * a.ldt + t_col0 + 8 * c;
      int n = n0 + row;
      n = n < seg_ne - 1 ? n : seg_ne - 1;
      boff[i] = (long long)(n - seg_nb) * ldb;
      bc[i] = c;
    }
    // T region = first 16 KB of the stage's x slot, B region = second.
    auto issue_t = [&](int ch, uint4* X) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dma16(a.t + toff[i] + 32 * ch, X + 64 * (4 * wave + i));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int g = a.grp[grp0 + 2 * ch + (bc[i] >> 1)];
        g = g < 0 ? g_safe : g;
        dma16(Bp + boff[i] + 16 * g + 8 * (bc[i] & 1), X + 1024 + 64 * (4 * wave + i));
      }
    };
    auto compute_t = [&](const uint4* X) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int c = 2 * kk + fk;
        uint4 wa[2], xb[8];
#pragma unroll
        for (int j = 0; j < 2; ++j) wa[j] = X[1024 + swz4(64 * wave + 32 * j + fr, c)];
#pragma unroll
        for (int i = 0; i < 8; ++i) xb[i] = X[swz4(32 * i + fr, c)];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8_t, wa[j]), __builtin_bit_cast(bf16x8_t, xb[i]),
                acc[j][i], 0, 0, 0);
      }
    };
    auto step_t = [&](int ch, uint4* Xc, uint4* Xn) {
      __builtin_amdgcn_s_waitcnt(vm_wait(8));   // chunk ch done
      ring_barrier();
      issue_t(ch + 2 < chunks32 ? ch + 2 : chunks32 - 1, Xn);
      if (ch < chunks32) compute_t(Xc);
    };
    // every wave is past its last base-stage read before the ring is reused
    ring_barrier();
    issue_t(0, sX0);
    issue_t(chunks32 > 1 ? 1 : 0, sX1);
    for (int ch = 0; ch < chunks32; ch += 3) {
      step_t(ch, sX0, sX2);
      step_t(ch + 1, sX1, sX0);
      step_t(ch + 2, sX2, sX1);
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
  }

  // Epilogue: D[n][m] per tile -> 4 consecutive n per register quad.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int m = m0 + 32 * i + fr;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + 64 * wave + 32 * j + 8 * q + 4 * fk;
        if (m < a.M && n < a.N) {
          uint2 v;
          v.x = pack_bf16x2(acc[j][i][4 * q + 0], acc[j][i][4 * q + 1]);
          v.y = pack_bf16x2(acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]);
          *reinterpret_cast<uint2*>(a.y + (long long)m * a.ldy + n) = v;
        }
      }
    }
  }
}

// ---- T = x . A_live^T * coef: the adapters' stacked down-projection --------
// Block tile 256 rows x 64 ranks, 4 waves x (64 rows x 64 ranks) of
// v_mfma_f32_32x32x16_bf16, the same three-stage DMA ring, and split-K so
// even a 320-rank stack over 4352 rows fills the chip: slice s writes f32
// partials P[s] and xa_reduce sums the slices in a fixed order (no atomics,
// so the bits do not depend on timing).
__global__ __launch_bounds__(256, 1) void lora_xa_fast_kernel(const LoraXaArgs a,
                                                              float* part,
                                                              int kslices) {
  constexpr int STG = 256 * 8 + 64 * 8;          // x tile + A tile, 16-B chunks
  constexpr int PER = 8 + 2;
  __shared__ uint4 st0[STG], st1[STG], st2[STG];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fk = lane >> 5;
  const int m0 = blockIdx.x * 256, c0 = blockIdx.y * 64, ks = blockIdx.z;
  const int KT = a.K / 64;
  const int kt0 = (int)((long long)KT * ks / kslices);
  const int kt1 = (int)((long long)KT * (ks + 1) / kslices);
  const int NT = kt1 - kt0;
  const int mlast = a.M - 1;

  long long xoff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int p = 64 * (8 * wave + i) + lane;
    const int row = p >> 3;
    const int c = (p & 7) ^ ((row >> 1) & 7);
    int m = m0 + row;
    m = m < mlast ? m : mlast;
    xoff[i] = (long long)m * a.ldx + 8 * c;
  }
  // the first live group: a finite row for padding columns (their coef is 0)
  const int g_safe = a.grp[0];
  long long aoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = 64 * (2 * wave + i) + lane;
    const int r = p >> 3;
    const int c = (p & 7) ^ ((r >> 1) & 7);
    const int col = c0 + r;
    int g = a.grp[col >> 4];
    const int row = g < 0 ? 16 * g_safe : 16 * g + (col & 15);
    aoff[i] = (long long)row * a.K + 8 * c;
  }
  auto issue = [&](int kt, uint4* S) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dma16(a.x + xoff[i] + kt * 64, S + 64 * (8 * wave + i));
#pragma unroll
    for (int i = 0; i < 2; ++i)
      dma16(a.A + aoff[i] + kt * 64, S + 2048 + 64 * (2 * wave + i));
  };
  floatx16_t acc[2][2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;
  auto compute = [&](const uint4* S) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = 2 * kk + fk;
      uint4 av[2], xv[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) av[j] = S[2048 + swz8(32 * j + fr, c)];
#pragma unroll
      for (int i = 0; i < 2; ++i) xv[i] = S[swz8(64 * wave + 32 * i + fr, c)];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, av[j]), __builtin_bit_cast(bf16x8_t, xv[i]),
              acc[j][i], 0, 0, 0);
    }
  };
  auto step = [&](int t, uint4* Sc, uint4* Sn) {
    __builtin_amdgcn_s_waitcnt(vm_wait(PER));
    ring_barrier();
    issue(kt0 + (t + 2 < NT ? t + 2 : NT - 1), Sn);
    if (t < NT) compute(Sc);
  };
  issue(kt0, st0);
  issue(kt0 + (NT > 1 ? 1 : 0), st1);
  for (int t = 0; t < NT; t += 3) {
    step(t, st0, st2);
    step(t + 1, st1, st0);
    step(t + 2, st2, st1);
  }
  __builtin_amdgcn_s_waitcnt(vm_wait(0));

  // D[c][m]: lane owns row m, four consecutive ranks per register quad.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + 64 * wave + 32 * i + fr;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = c0 + 32 * j + 8 * q + 4 * fk;
        if (kslices == 1) {
          const float f = a.coef[c >> 4];
          uint2 v;
          if (f == 0.0f) {
            v = make_uint2(0, 0);
          } else {
            v.x = pack_bf16x2(f * acc[j][i][4 * q + 0], f * acc[j][i][4 * q + 1]);
            v.y = pack_bf16x2(f * acc[j][i][4 * q + 2], f * acc[j][i][4 * q + 3]);
          }
          *reinterpret_cast<uint2*>(a.t + (long long)m * a.ldt + c) = v;
        } else {
          float4 v = make_float4(acc[j][i][4 * q + 0], acc[j][i][4 * q + 1],
                                 acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]);
          *reinterpret_cast<float4*>(
              part + ((long long)ks * a.M + m) * a.n_cols + c) = v;
        }
      }
    }
  }
}

// T[m][c] = bf16(coef * sum_s P[s][m][c]), slices summed in order 0..S-1.
__global__ void lora_xa_reduce_kernel(const float* part, int kslices, int M,
                                      int n_cols, const LoraXaArgs a) {
  const int c4 = n_cols >> 2;
  const long long total = (long long)M * c4;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long m = i / c4;
    const int c = (int)(i % c4) * 4;
    float4 s = *reinterpret_cast<const float4*>(part + m * n_cols + c);
    for (int k = 1; k < kslices; ++k) {
      const float4 v = *reinterpret_cast<const float4*>(
          part + ((long long)k * M + m) * n_cols + c);
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    const float f = a.coef[c >> 4];
    uint2 o;
    if (f == 0.0f) {
      o = make_uint2(0, 0);
    } else {
      o.x = pack_bf16x2(f * s.x, f * s.y);
      o.y = pack_bf16x2(f * s.z, f * s.w);
    }
    *reinterpret_cast<uint2*>(a.t + m * a.ldt + c) = o;
  }
}

// ---- resident layout for the fast route ------------------------------------
// codes: from the reference pack (LSB-first, [N][K*bits/32]) into
// [kt][n][fk][kk](w4) / [kt][n][fk][kk][2](w8); sbf: fp16 (s, b) pairs and
// a flag raised when any scale or bias is not exact in fp16.
__global__ void repack_fast_kernel(int bits, const uint32_t* codes, int N, int K,
                                   uint32_t* out) {
  const int wpr = bits == 4 ? 8 : 16;
  const long long total = (long long)(K / 64) * N * wpr;
  const long long words_row = (long long)K * bits / 32;
  for (long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x;
       idx < total; idx += (long long)gridDim.x * blockDim.x) {
    const int slot = (int)(idx % wpr);
    const long long rest = idx / wpr;
    const int n = (int)(rest % N);
    const int kt = (int)(rest / N);
    uint32_t o;
    if (bits == 4) {
      // slot = fk*4 + kk -> source word j = 2kk + fk (k = 8j .. 8j+7)
      const int fk = slot >> 2, kk = slot & 3;
      const uint32_t w = codes[(long long)n * words_row + (long long)kt * 8 + 2 * kk + fk];
      // new nibble i holds old nibble perm[i]: {k0,k4,k1,k5,k2,k6,k3,k7}
      const int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
      o = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) o |= ((w >> (4 * perm[i])) & 15u) << (4 * i);
    } else {
      // slot = fk*8 + kk*2 + h -> k = 16kk + 8fk + 4h: source word (16kk+8fk+4h)/4
      const int fk = slot >> 3, kk = (slot >> 1) & 3, h = slot & 1;
      o = codes[(long long)n * words_row + (long long)kt * 16 + 4 * kk + 2 * fk + h];
    }
    out[idx] = o;
  }
}

__device__ __forceinline__ uint32_t bf16_to_f16_bits(uint16_t h, bool* exact) {
  const float f = __uint_as_float((uint32_t)h << 16);
  const _Float16 x = (_Float16)f;
  if ((float)x != f) *exact = false;
  return (uint32_t)__builtin_bit_cast(uint16_t, x);
}

__global__ void repack_sbf_kernel(const uint16_t* scales, const uint16_t* biases,
                                  int N, int G, uint32_t* sbf, int* inexact) {
  const long long total = (long long)G * N;
  bool exact = true;
  for (long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x;
       idx < total; idx += (long long)gridDim.x * blockDim.x) {
    const int n = (int)(idx % N);
    const int g = (int)(idx / N);
    const uint32_t s = bf16_to_f16_bits(scales[(long long)n * G + g], &exact);
    const uint32_t b = bf16_to_f16_bits(biases[(long long)n * G + g], &exact);
    sbf[idx] = s | (b << 16);
  }
  if (!exact) atomicOr(inexact, 1);
}

__global__ void bf16_to_f16_kernel(const uint16_t* x, long long ldx, uint16_t* y,
                                   long long ldy, int rows, int K) {
  const int k8 = K >> 3;
  const long long total = (long long)rows * k8;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long r = i / k8;
    const int c = (int)(i % k8) * 8;
    const uint4 v = *reinterpret_cast<const uint4*>(x + r * ldx + c);
    uint4 o;
    o.x = bf16x2_to_f16x2(v.x);
    o.y = bf16x2_to_f16x2(v.y);
    o.z = bf16x2_to_f16x2(v.z);
    o.w = bf16x2_to_f16x2(v.w);
    *reinterpret_cast<uint4*>(y + r * ldy + c) = o;
  }
}

}  // namespace

hipError_t launch_qproj_fast(int bits, const QprojArgs& a, hipStream_t s) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (tiles <= 0) return hipSuccess;
  if (bits == 4)
    hipLaunchKernelGGL(qproj_fast_kernel<4>, dim3(tiles), dim3(256), 0, s, a);
  else if (bits == 8)
    hipLaunchKernelGGL(qproj_fast_kernel<8>, dim3(tiles), dim3(256), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

int lora_xa_fast_slices(int M, int n_cols, int K) {
  const int tiles = ((M + 255) / 256) * (n_cols / 64);
  const int KT = K / 64;
  int ks = (512 + tiles - 1) / tiles;          // aim at ~2 blocks per CU
  const int kmax = KT / 6 > 1 ? KT / 6 : 1;     // keep >= 6 K steps per slice
  if (ks > kmax) ks = kmax;
  return ks < 1 ? 1 : ks;
}

hipError_t launch_lora_xa_fast(const LoraXaArgs& a, float* part, int kslices,
                               hipStream_t s) {
  if (a.M <= 0 || a.n_cols <= 0) return hipSuccess;
  dim3 grid((a.M + 255) / 256, a.n_cols / 64, kslices);
  hipLaunchKernelGGL(lora_xa_fast_kernel, grid, dim3(256), 0, s, a, part, kslices);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || kslices == 1) return e;
  long long work = (long long)a.M * (a.n_cols / 4);
  long long blocks = (work + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(lora_xa_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                     part, kslices, a.M, a.n_cols, a);
  return hipGetLastError();
}

hipError_t launch_repack_fast(int bits, const uint32_t* codes,
                              const uint16_t* scales, const uint16_t* biases,
                              int N, int K, uint32_t* codes_f, uint32_t* sbf,
                              int* inexact, hipStream_t s) {
  hipLaunchKernelGGL(repack_fast_kernel, dim3(1024), dim3(256), 0, s, bits,
                     codes, N, K, codes_f);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(repack_sbf_kernel, dim3(256), dim3(256), 0, s, scales,
                     biases, N, K / 64, sbf, inexact);
  return hipGetLastError();
}

hipError_t launch_bf16_to_f16(const uint16_t* x, long long ldx, uint16_t* y,
                              long long ldy, int rows, int K, hipStream_t s) {
  long long work = (long long)rows * (K / 8);
  long long blocks = (work + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(bf16_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     s, x, ldx, y, ldy, rows, K);
  return hipGetLastError();
}

hipError_t validate_qproj_fast_kernels() {
  hipFuncAttributes fa;
  const void* fns[] = {reinterpret_cast<const void*>(&qproj_fast_kernel<4>),
                       reinterpret_cast<const void*>(&qproj_fast_kernel<8>),
                       reinterpret_cast<const void*>(&repack_fast_kernel),
                       reinterpret_cast<const void*>(&repack_sbf_kernel),
                       reinterpret_cast<const void*>(&bf16_to_f16_kernel),
                       reinterpret_cast<const void*>(&lora_xa_fast_kernel),
                       reinterpret_cast<const void*>(&lora_xa_reduce_kernel)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&fa, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ming
