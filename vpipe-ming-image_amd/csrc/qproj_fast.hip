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
// The same body also runs as qproj_pair_kernel (a SwiGLU's gate and up
// projections in one tile, 128 columns of each) and, for the last tile row
// of a paired grid whose last round would hold only that row, with 128-row
// tiles (4 row fragments a wave instead of 8).
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

// The DMA written as inline asm, for rings whose waits are all
// explicit: the compiler then sees no LDS store it must order reads
// against, so it cannot add a drain of its own (its alias tracking of LDS
// DMA gives up at loop joins and would wait for vmcnt(0)). M0 carries the
// wave's LDS byte address; the s_nop covers the M0 -> LDS-DMA hazard.
// Correctness rests on the ring's own waits: ring_wait<N>() below, which
// also orders every LDS access against the DMAs through its memory clobber.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// Scalar-base form: address = 64-bit wave-uniform base (SGPRs) + 32-bit
// per-lane byte offset, so advancing a stage is a scalar add and the issue
// needs no VALU address arithmetic.
__device__ __forceinline__ void dma16_sb(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(off), "s"(base), "s"(lds) : "m0");
}
__device__ __forceinline__ void dma4_sb(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(off), "s"(base), "s"(lds) : "m0");
}
#pragma clang diagnostic pop

// LDS byte address of a __shared__ object: the low half of its generic
// address is the offset inside the workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Ring barrier with its vmcnt: this wave's DMAs except the newest N have
// landed, its LDS reads are complete, then the workgroup barrier. After it
// every wave's older DMAs are visible and every wave is done reading.
template <int N>
__device__ __forceinline__ void ring_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(N) : "memory");
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

// SPLIT (a.kslices > 1, a projection of few tiles): block b is slice
// b / tiles of tile b % tiles. The slice runs its share of K (the last one
// also the LoRA tail) and writes f32 partials to a.part; the split reduce
// then sums the slices in order and finishes as the epilogue does.
//
// PAIR (launch_qproj_pair): the tile's 256 weight rows are 128 rows of the
// gate weight (waves 0-1) and the same 128 rows of the up weight (waves
// 2-3); the tail stages the gate's and the up projection's T chunks side by
// side; the epilogue meets the two in LDS and writes only the SwiGLU.
template <int BITS, bool SPLIT, bool PAIR, int RF>
__device__ __forceinline__ void qproj_fast_body(const QprojArgs& a) {
  constexpr int WCH = BITS == 4 ? 512 : 1024;    // 16-B code chunks per stage
  constexpr int CPR = BITS == 4 ? 2 : 4;         // code chunks per row
  constexpr int WDMA = WCH / 256;                // code DMAs per wave per stage
  constexpr int BMT = 32 * RF;                   // rows per tile: RF fragments of 32
  constexpr int XD = RF;                         // x DMAs per wave per stage
  constexpr int TD = RF / 2;                     // T DMAs per wave per tail chunk
  constexpr int PER = XD + WDMA + 1;             // DMAs per wave per base stage
  constexpr int TPER = (PAIR ? 2 : 1) * TD + 4;  // DMAs per wave per tail chunk
  constexpr int BNT = PAIR ? BN / 2 : BN;        // output columns per tile
  // One __shared__ object per stage: [x 32 KB | codes | (s, b)]; a tail
  // chunk is [T 16 KB | B 16 KB (| the up projection's T 16 KB)].
  constexpr int STG0 = BMT * 8 + WCH + BN / 4;
  constexpr int STG = PAIR && STG0 < 3072 ? 3072 : STG0;
  __shared__ uint4 st0[STG], st1[STG], st2[STG];

  // Waves split N only: wave w owns output columns [64w, 64w+64) for all
  // 256 rows (2 x 8 tiles of 32x32), so every weight fragment is
  // dequantized by exactly one wave.
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fk = lane >> 5;
  // PAIR: waves 2-3 read the up weight; their columns are the gate's again
  const bool upw = PAIR && wave >= 2;
  const int wcol = PAIR ? 64 * (wave & 1) : 64 * wave;

  const int tiles_m = (a.M + BMT - 1) / BMT;
  const int tiles_n = (a.N + BNT - 1) / BNT;
  int tm, tn, blk = (int)blockIdx.x, ks = 0, kt0 = 0;
  int KT = a.K / BK;
  if constexpr (SPLIT) {
    ks = blk / (tiles_m * tiles_n);
    blk -= ks * (tiles_m * tiles_n);
    kt0 = KT * ks / a.kslices;
    KT = KT * (ks + 1) / a.kslices - kt0;
  }
  tile_of_block(blk, tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * BMT, n0 = tn * BNT;
  const int mlast = a.M - 1, nlast = a.N - 1;

  // stage 0 of this block's K range
  const _Float16* __restrict__ x16 = reinterpret_cast<const _Float16*>(a.x) + (long long)kt0 * BK;
  const uint4* __restrict__ codes =
      reinterpret_cast<const uint4*>(upw ? a.codes_u : a.codes) + (long long)kt0 * a.N * CPR;
  const uint32_t* __restrict__ sbp = (upw ? a.sb_u : a.sb) + (long long)kt0 * a.N;

  // DMA sources for this lane, per stage (advance by k).
  // x tile: wave issues chunks q = 8*wave + i; lane p = 64q + lane.
  // Byte offsets from the stage's base (the host keeps every operand
  // within 2 GiB of its base, so they fit 31 bits whether the hardware reads
  // the offset as signed or unsigned).
  uint32_t xoff[XD];
#pragma unroll
  for (int i = 0; i < XD; ++i) {
    const int p = 64 * (XD * wave + i) + lane;
    const int row = p >> 3;
    const int c = (p & 7) ^ ((row >> 1) & 7);
    int m = m0 + row;
    m = m < mlast ? m : mlast;
    xoff[i] = (uint32_t)(((long long)m * a.ldx + 8 * c) * 2);
  }
  // code tile: LDS chunk p holds row p / CPR, logical chunk (p % CPR) ^ sw
  uint32_t woff[WDMA];
#pragma unroll
  for (int i = 0; i < WDMA; ++i) {
    const int p = 64 * (WDMA * wave + i) + lane;
    const int r = p / CPR;
    const int h = (p % CPR) ^ wswz<CPR>(r);
    int n = n0 + (PAIR ? (r & 127) : r);
    n = n < nlast ? n : nlast;
    woff[i] = (uint32_t)((n * CPR + h) * 16);
  }
  int sn = n0 + wcol + lane;
  sn = sn < nlast ? sn : nlast;
  const uint32_t soff = (uint32_t)sn * 4u;

  // The stage's DMAs in three groups (x rows 0-127, x rows 128-255, codes +
  // (s, b)), issued one group per k16 step of the stage before.
  auto issue_grp = [&](int g, int kt, const uint4* B) {
    if (g < 2) {
      const void* base = x16 + (long long)kt * BK;
#pragma unroll
      for (int i = (XD / 2) * g; i < (XD / 2) * (g + 1); ++i)
        dma16_sb(base, xoff[i], lds_addr(B + 64 * (XD * wave + i)));
    } else {
      const void* wbase = codes + (long long)kt * a.N * CPR;
#pragma unroll
      for (int i = 0; i < WDMA; ++i)
        dma16_sb(wbase, woff[i], lds_addr(B + BMT * 8 + 64 * (WDMA * wave + i)));
      dma4_sb(sbp + (long long)kt * a.N, soff,
              lds_addr(reinterpret_cast<const uint32_t*>(B + BMT * 8 + WCH) + 64 * wave));
    }
  };

  floatx16_t acc[2][RF];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < RF; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;

  // Stage state in registers: the code words and (s, b) of the wave's two
  // n-tiles, and the current k16 step's operands.
  uint4 wc[2][CPR / 2];
  half2v s2[2], b2[2];
  uint4 wa[2], xb[RF];

  auto load_ws = [&](const uint4* B, uint4 (&wcv)[2][CPR / 2], half2v (&s2v)[2],
                     half2v (&b2v)[2]) {
    const uint4* W = B + BMT * 8;
    const uint32_t* S = reinterpret_cast<const uint32_t*>(B + BMT * 8 + WCH);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = 64 * wave + 32 * j + fr;
#pragma unroll
      for (int h = 0; h < CPR / 2; ++h)
        wcv[j][h] = W[wchunk<CPR>(n, fk * (CPR / 2) + h)];
      const uint32_t sb = S[n];
      s2v[j] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(sb, sb, 0x01000100u));
      b2v[j] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(sb, sb, 0x03020302u));
    }
  };
  auto deq = [&](const uint4 (&wcv)[2][CPR / 2], const half2v (&s2v)[2],
                 const half2v (&b2v)[2], int j, int kk) -> uint4 {
    if constexpr (BITS == 4) {
      return deq_w4((&wcv[j][0].x)[kk], s2v[j], b2v[j]);
    } else {
      const uint32_t* w = &wcv[j][kk >> 1].x;
      return deq_w8(w[(kk & 1) * 2], w[(kk & 1) * 2 + 1], s2v[j], b2v[j]);
    }
  };

  // One stage, software-pipelined across the stage boundary. Steps 0-2
  // read and dequantize the next step's fragments beside the current
  // step's 16 MFMAs and issue one DMA group of stage kt+2 into Pv (the
  // buffer stage kt-1 left). Between steps 2 and 3 the wave waits for its
  // stage kt+1 DMAs and the workgroup meets at the barrier: stage kt+1 is
  // in LDS and nobody reads stage kt's buffer again. Step 3's MFMAs then
  // carry the next stage's code / (s, b) reads, its first x fragments and
  // their dequantization, so no stage starts with an LDS round trip.
  // Interleave pinned with scheduling-group barriers (0x008 MFMA, 0x100 DS
  // read, 0x002 VALU). Past the last stage the DMA re-reads stage KT-1 into
  // a buffer nothing reads, so every stage issues and waits alike.
  auto body = [&](int kt, const uint4* C, const uint4* Nx, const uint4* Pv) {
    const int nk = kt + 2 < KT ? kt + 2 : KT - 1;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4 wn_[2], xn_[RF];
      uint4 wcn[2][CPR / 2];
      half2v s2n[2], b2n[2];
      if (kk < 3) {
        issue_grp(kk, nk, Pv);
#pragma unroll
        for (int i = 0; i < RF; ++i) xn_[i] = C[swz8(32 * i + fr, 2 * (kk + 1) + fk)];
#pragma unroll
        for (int j = 0; j < 2; ++j) wn_[j] = deq(wc, s2, b2, j, kk + 1);
      } else {
        load_ws(Nx, wcn, s2n, b2n);
#pragma unroll
        for (int i = 0; i < RF; ++i) xn_[i] = Nx[swz8(32 * i + fr, fk)];
#pragma unroll
        for (int j = 0; j < 2; ++j) wn_[j] = deq(wcn, s2n, b2n, j, 0);
      }
#pragma unroll
      for (int i = 0; i < RF; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              __builtin_bit_cast(half8_t, wa[j]), __builtin_bit_cast(half8_t, xb[i]),
              acc[j][i], 0, 0, 0);
      if (kk < 3) {
#pragma unroll
        for (int g = 0; g < RF; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        }
#pragma unroll
        for (int g = 0; g < RF; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x002, 32 / RF, 0);   // VALU
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         // MFMA
        }
      } else {
        // step 3: NDS reads over the DSM MFMAs left after the VG that carry
        // the next stage's first dequantization (w4 at 256 rows: spread
        // over 10 MFMAs, 4 VALU each, which measured ~0.5% faster launches
        // than 6 MFMAs of 6; the reads then go two per MFMA)
        constexpr int NDS = RF + 2 * (CPR / 2) + 2;
        constexpr int VG = RF == 8 && CPR == 2 ? RF + 2 : 3 * RF / 4;
        constexpr int VPG = RF == 8 && CPR == 2 ? 4 : 6;   // VALU per group
        constexpr int DSM = 2 * RF - VG;
        static_assert(NDS >= DSM && NDS <= 2 * DSM, "step-3 DS reads per MFMA pin");
#pragma unroll
        for (int g = 0; g < NDS - DSM; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
#pragma unroll
        for (int g = NDS - DSM; g < DSM; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
#pragma unroll
        for (int g = 0; g < VG; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x002, VPG, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (kk == 2) {
        ring_wait<PER>();                      // stage kt+1 landed, kt done
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) wa[j] = wn_[j];
#pragma unroll
      for (int i = 0; i < RF; ++i) xb[i] = xn_[i];
      if (kk == 3) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
          for (int h = 0; h < CPR / 2; ++h) wc[j][h] = wcn[j][h];
          s2[j] = s2n[j];
          b2[j] = b2n[j];
        }
      }
    }
  };

  // Prologue: stages 0 and 1 in flight, wait for stage 0, load its state.
#pragma unroll
  for (int g = 0; g < 3; ++g) issue_grp(g, 0, st0);
#pragma unroll
  for (int g = 0; g < 3; ++g) issue_grp(g, KT > 1 ? 1 : 0, st1);
  ring_wait<PER>();
  load_ws(st0, wc, s2, b2);
#pragma unroll
  for (int i = 0; i < RF; ++i) xb[i] = st0[swz8(32 * i + fr, fk)];
#pragma unroll
  for (int j = 0; j < 2; ++j) wa[j] = deq(wc, s2, b2, j, 0);

  // Stage kt lives in buffer kt % 3; three stages per trip, the remainder
  // (KT % 3) after the loop, so the loop body has no branch.
  int kt = 0;
  for (; kt + 3 <= KT; kt += 3) {
    body(kt, st0, st1, st2);
    body(kt + 1, st1, st2, st0);
    body(kt + 2, st2, st0, st1);
  }
  if (KT - kt >= 1) body(kt, st0, st1, st2);
  if (KT - kt == 2) body(kt + 1, st1, st2, st0);
  ring_wait<0>();                               // drained; LDS free

  // ---- LoRA tail: T and gathered B chunks of 32 ranks, same ring ----
  int sg = 0;
  for (int i = 1; i < a.nseg; ++i)
    if (n0 >= a.seg[i].n_begin) sg = i;
  const int chunks32 = (!SPLIT || ks == a.kslices - 1) ? a.seg[sg].chunks : 0;
  if (chunks32 > 0) {
    // PAIR: waves 2-3 gather the up projection's B (its segment, its
    // groups); both T chunks are staged for every wave
    const QprojSeg& sw = upw ? a.seg_u : a.seg[sg];
    const int t_col0 = a.seg[sg].t_col0;
    const int ldb = sw.ldb;
    const int grp0 = sw.grp0;
    const int seg_nb = sw.n_begin, seg_ne = sw.n_end;
    const uint16_t* __restrict__ Bp = sw.B;
    const uint16_t* const tu = a.t + (PAIR ? a.seg_u.t_col0 - t_col0 : 0);
    // the first live group of the segment: a finite source for padding
    // groups (their T columns are exactly 0)
    const int g_safe = a.grp[grp0];
    // T: BMT rows x 4 chunks (TD DMAs a wave); B: 256 rows x 4 chunks (4)
    uint32_t toff[TD];
    uint32_t boff[4];
    int bc[4];
    if constexpr (TD == 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = 64 * (4 * wave + i) + lane;
        const int row = p >> 2;
        const int c = (p & 3) ^ ((row >> 2) & 3);
        int m = m0 + row;
        m = m < mlast ? m : mlast;
        toff[i] = (uint32_t)(((long long)m * a.ldt + t_col0 + 8 * c) * 2);
        int n = n0 + (PAIR ? (row & 127) : row);
        n = n < seg_ne - 1 ? n : seg_ne - 1;
        boff[i] = (uint32_t)((long long)(n - seg_nb) * ldb * 2);
        bc[i] = c;
      }
    } else {
#pragma unroll
      for (int i = 0; i < TD; ++i) {
        const int p = 64 * (TD * wave + i) + lane;
        const int row = p >> 2;
        const int c = (p & 3) ^ ((row >> 2) & 3);
        int m = m0 + row;
        m = m < mlast ? m : mlast;
        toff[i] = (uint32_t)(((long long)m * a.ldt + t_col0 + 8 * c) * 2);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = 64 * (4 * wave + i) + lane;
        const int row = p >> 2;
        const int c = (p & 3) ^ ((row >> 2) & 3);
        int n = n0 + (PAIR ? (row & 127) : row);
        n = n < seg_ne - 1 ? n : seg_ne - 1;
        boff[i] = (uint32_t)((long long)(n - seg_nb) * ldb * 2);
        bc[i] = c;
      }
    }
    // T region = first 16 KB of the stage buffer, B region = second. A
    // lane's 16 bytes are the 8 ranks of one group; the chunk's four groups
    // are wave-uniform (scalar loads).
    auto grp_word = [&](int ch) -> uint2 {
      const int gi = __builtin_amdgcn_readfirstlane(grp0 + 4 * ch);
      return reinterpret_cast<const uint2*>(a.grp)[gi >> 2];
    };
    uint2 gw_next = grp_word(0);
    auto issue_t = [&](int ch, const uint4* X) {
#pragma unroll
      for (int i = 0; i < TD; ++i)
        dma16_sb(a.t + 32 * ch, toff[i], lds_addr(X + 64 * (TD * wave + i)));
      if constexpr (PAIR) {
#pragma unroll
        for (int i = 0; i < TD; ++i)
          dma16_sb(tu + 32 * ch, toff[i], lds_addr(X + 2048 + 64 * (TD * wave + i)));
      }
      // The chunk's four groups are one aligned 8-byte word of the table (a
      // segment's groups start at a multiple of 4), read by a wave-uniform
      // scalar load one issue ahead, so no issue waits on it. A lane picks
      // its group's 16 bits with a select and a shift (no branch).
      const uint2 gw = gw_next;
      const int nx = ch + 1 < chunks32 ? ch + 1 : chunks32 - 1;
      gw_next = grp_word(nx);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = (bc[i] & 2) ? gw.y : gw.x;
        int g = (int16_t)(w >> ((bc[i] & 1) << 4));
        g = g < 0 ? g_safe : g;
        dma16_sb(Bp, boff[i] + (uint32_t)g * 16u, lds_addr(X + 1024 + 64 * (4 * wave + i)));
      }
    };
    uint4 ta[2], tb[RF];
    auto read_t = [&](const uint4* X, int kk, uint4 (&av)[2], uint4 (&bv)[RF]) {
      const int c = 2 * kk + fk;
#pragma unroll
      for (int j = 0; j < 2; ++j) av[j] = X[1024 + swz4(64 * wave + 32 * j + fr, c)];
      const uint4* const XT = upw ? X + 2048 : X;
#pragma unroll
      for (int i = 0; i < RF; ++i) bv[i] = XT[swz4(32 * i + fr, c)];
    };
    // Chunk ch: step 0 reads step 1's fragments and issues chunk ch+2 into
    // Pv; the wait + barrier sit between the steps; step 1 reads the next
    // chunk's step-0 fragments.
    auto body_t = [&](int ch, const uint4* C, const uint4* Nx, const uint4* Pv) {
      const int nc = ch + 2 < chunks32 ? ch + 2 : chunks32 - 1;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        uint4 an[2], bn[RF];
        if (kk == 0) {
          issue_t(nc, Pv);
          read_t(C, 1, an, bn);
        } else {
          read_t(Nx, 0, an, bn);
        }
#pragma unroll
        for (int i = 0; i < RF; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8_t, ta[j]), __builtin_bit_cast(bf16x8_t, tb[i]),
                acc[j][i], 0, 0, 0);
#pragma unroll
        for (int g = 0; g < 2 + RF; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kk == 0) {
          ring_wait<TPER>();                       // chunk ch+1 landed, ch done
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) ta[j] = an[j];
#pragma unroll
        for (int i = 0; i < RF; ++i) tb[i] = bn[i];
      }
    };
    issue_t(0, st0);
    issue_t(chunks32 > 1 ? 1 : 0, st1);
    ring_wait<TPER>();
    read_t(st0, 0, ta, tb);
    int ch = 0;
    for (; ch + 3 <= chunks32; ch += 3) {
      body_t(ch, st0, st1, st2);
      body_t(ch + 1, st1, st2, st0);
      body_t(ch + 2, st2, st0, st1);
    }
    if (chunks32 - ch >= 1) body_t(ch, st0, st1, st2);
    if (chunks32 - ch == 2) body_t(ch + 1, st1, st2, st0);
    ring_wait<0>();
  }

  if constexpr (SPLIT) {
    // f32 partials P[ks][m][n]: lane row 32i + fr, four columns per quad
#pragma unroll
    for (int i = 0; i < RF; ++i) {
      const int m = m0 + 32 * i + fr;
      if (m >= a.M) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + 64 * wave + 32 * j + 8 * q + 4 * fk;
          if (n < a.N)
            *reinterpret_cast<float4*>(a.part + ((long long)ks * a.M + m) * a.N + n) =
                make_float4(acc[j][i][4 * q + 0], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2],
                            acc[j][i][4 * q + 3]);
        }
    }
    return;
  }

  if constexpr (PAIR) {
    // The gate's and the up projection's bf16 outputs meet in LDS, 128 rows
    // at a time: wave w writes its 64 columns to region w (as below), and
    // after the barrier wave w reads column half c = w & 1 of rows
    // [64 (w >> 1), +64) from the gate's region c and the up projection's
    // region 2 + c, and writes y = bf16(silu(g) * u) and its fp16 copy: the
    // bits of the gate's own epilogue followed by the gated one.
    uint2* const Ew = reinterpret_cast<uint2*>((wave < 2 ? st0 : st1) + 1024 * (wave & 1));
    const uint4* const Eg = st0 + 1024 * (wave & 1);
    const uint4* const Eu = st1 + 1024 * (wave & 1);
    const int cl = lane & 7;
    const int n = n0 + wcol + 8 * cl;
    uint32_t seen = 0;
#pragma unroll
    for (int h = 0; h < RF / 4; ++h) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * h + ii;
        const int ml = 32 * ii + fr;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int c = 4 * j + q;
            uint2 v;
            v.x = pack_bf16x2_rne(acc[j][i][4 * q + 0], acc[j][i][4 * q + 1]);
            v.y = pack_bf16x2_rne(acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]);
            Ew[ml * 16 + 2 * (c ^ ((ml >> 1) & 7)) + fk] = v;
          }
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int ml = 64 * (wave >> 1) + 8 * r + (lane >> 3);
        const int e = ml * 8 + (cl ^ ((ml >> 1) & 7));
        const uint4 gv = Eg[e];
        uint4 v = Eu[e];
        const int m = m0 + 128 * h + ml;
        if (m < a.M && n < a.N) {
          const uint32_t* gp = &gv.x;
          uint32_t* vp = &v.x;
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2)
            vp[e2] = pack_bf16x2_rne(silu_f(bf16_lo(gp[e2])) * bf16_lo(vp[e2]),
                                     silu_f(bf16_hi(gp[e2])) * bf16_hi(vp[e2]));
          *reinterpret_cast<uint4*>(a.y + (long long)m * a.ldy + n) = v;
          if (a.yh) {
            seen = range_track4(seen, v);
            uint4 f;
            f.x = bf16x2_to_f16x2(v.x);
            f.y = bf16x2_to_f16x2(v.y);
            f.z = bf16x2_to_f16x2(v.z);
            f.w = bf16x2_to_f16x2(v.w);
            *reinterpret_cast<uint4*>(a.yh + (long long)m * a.ldyh + n) = f;
          }
        }
      }
      __syncthreads();   // the next half rewrites the regions
    }
    if (a.yh) range_report(a.range, seen);
    return;
  }

  // Epilogue through LDS: each wave converts its 64 columns x 128 rows at a
  // time to bf16 in its own 16 KB region (rows of 128 B, chunks swizzled by
  // (row >> 1) & 7 so both the 8-B writes and the 16-B reads are
  // conflict-free), then stores whole 128-B row segments, 8 rows per
  // instruction. Only the wave itself touches its region, and LDS accesses
  // of one wave complete in order, so no barrier is needed inside.
  uint4* const E = (wave < 2 ? st0 : st1) + 1024 * (wave & 1);
  const bool st16 = (a.ldy & 7) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0;
  const int cl = lane & 7;
  const int n = n0 + 64 * wave + 8 * cl;
  uint32_t seen = 0;   // magnitudes written to the fp16 copy (range_report)
#pragma unroll
  for (int h = 0; h < RF / 4; ++h) {
    // Fused SwiGLU: this half's gate rows are loaded first, so their memory
    // latency overlaps the conversion below instead of stalling each store.
    uint4 gv[16];
    if (a.g) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int m = m0 + 128 * h + 8 * r + (lane >> 3);
        m = m < a.M ? m : a.M - 1;
        const int nn = n < a.N ? n : a.N - 8;
        gv[r] = *reinterpret_cast<const uint4*>(a.g + (long long)m * a.ldg + nn);
      }
    }
    uint2* const E2 = reinterpret_cast<uint2*>(E);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int i = 4 * h + ii;
      const int ml = 32 * ii + fr;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = 4 * j + q;
          uint2 v;
          v.x = pack_bf16x2_rne(acc[j][i][4 * q + 0], acc[j][i][4 * q + 1]);
          v.y = pack_bf16x2_rne(acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]);
          E2[ml * 16 + 2 * (c ^ ((ml >> 1) & 7)) + fk] = v;
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ml = 8 * r + (lane >> 3);
      uint4 v = E[ml * 8 + (cl ^ ((ml >> 1) & 7))];
      const int m = m0 + 128 * h + ml;
      if (m < a.M && n < a.N) {
        if (a.g) {
          // the bf16 projection output is the "up" operand
          const uint32_t* gp = &gv[r].x;
          uint32_t* vp = &v.x;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            vp[e] = pack_bf16x2_rne(silu_f(bf16_lo(gp[e])) * bf16_lo(vp[e]),
                                    silu_f(bf16_hi(gp[e])) * bf16_hi(vp[e]));
        }
        uint16_t* yp = a.y + (long long)m * a.ldy + n;
        if (st16) {
          *reinterpret_cast<uint4*>(yp) = v;
        } else {
          reinterpret_cast<uint2*>(yp)[0] = make_uint2(v.x, v.y);
          reinterpret_cast<uint2*>(yp)[1] = make_uint2(v.z, v.w);
        }
        if (a.yh) {
          seen = range_track4(seen, v);
          uint4 f;
          f.x = bf16x2_to_f16x2(v.x);
          f.y = bf16x2_to_f16x2(v.y);
          f.z = bf16x2_to_f16x2(v.z);
          f.w = bf16x2_to_f16x2(v.w);
          *reinterpret_cast<uint4*>(a.yh + (long long)m * a.ldyh + n) = f;
        }
      }
    }
  }
  if (a.yh) range_report(a.range, seen);
}

template <int BITS, bool SPLIT>
__global__ __launch_bounds__(256, 1) void qproj_fast_kernel(const QprojArgs a) {
  qproj_fast_body<BITS, SPLIT, false, 8>(a);
}

// RF = 8: 256-row tiles; RF = 4: 128-row tiles (the rows of a grid's last,
// mostly empty round, see launch_qproj_pair)
template <int BITS, int RF>
__global__ __launch_bounds__(256, 1) void qproj_pair_kernel(const QprojArgs a) {
  qproj_fast_body<BITS, false, true, RF>(a);
}

// The split projection's end: y = bf16(sum of the slices in order), then as
// the epilogue: the fused SwiGLU bf16(silu(g) * y) and the fp16 copy.
// 32-bit indices: the host keeps M * N / 4 below 2^31.
__global__ void qproj_split_reduce_kernel(const QprojArgs a) {
  const unsigned n4 = (unsigned)a.N >> 2;
  const unsigned total = (unsigned)a.M * n4;
  const size_t plane = (size_t)a.M * (size_t)a.N;
  uint32_t seen = 0;
  for (unsigned i = blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += gridDim.x * blockDim.x) {
    const unsigned m = i / n4;
    const unsigned n = (i - m * n4) * 4;
    const float* p = a.part + (size_t)m * a.N + n;
    float4 sum = *reinterpret_cast<const float4*>(p);
    for (int k = 1; k < a.kslices; ++k) {
      p += plane;
      const float4 v = *reinterpret_cast<const float4*>(p);
      sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
    }
    uint32_t vp[2] = {pack_bf16x2_rne(sum.x, sum.y), pack_bf16x2_rne(sum.z, sum.w)};
    if (a.g) {
      const uint2 gv = *reinterpret_cast<const uint2*>(a.g + (size_t)m * a.ldg + n);
      const uint32_t gp[2] = {gv.x, gv.y};
#pragma unroll
      for (int e = 0; e < 2; ++e)
        vp[e] = pack_bf16x2_rne(silu_f(bf16_lo(gp[e])) * bf16_lo(vp[e]),
                                silu_f(bf16_hi(gp[e])) * bf16_hi(vp[e]));
    }
    *reinterpret_cast<uint2*>(a.y + (size_t)m * a.ldy + n) = make_uint2(vp[0], vp[1]);
    if (a.yh) {
      seen = range_track(range_track(seen, vp[0]), vp[1]);
      *reinterpret_cast<uint2*>(a.yh + (size_t)m * a.ldyh + n) =
          make_uint2(bf16x2_to_f16x2(vp[0]), bf16x2_to_f16x2(vp[1]));
    }
  }
  range_report(a.range, seen);
}

// ---- T = x . A_live^T * coef: the adapters' stacked down-projection --------
// Block tile 256 rows x 128 stacked ranks. Four MFMA waves in 2 x 2, each
// 128 rows x 64 ranks (4 x 2 tiles of v_mfma_f32_32x32x16_bf16, D[rank][row],
// so a lane owns one row and 4 consecutive ranks per register quad), and a
// DMA-only wave beside each on its SIMD: a global_load_lds holds the wave
// that issues it for ~16 cycles its MFMAs do not hide, so no MFMA wave
// issues one. Split-K over kslices so the grid is about one round of the
// chip; slice s writes f32 partials P[s] and lora_xa_reduce_kernel sums the
// slices in a fixed order (no atomics: the bits do not depend on timing).
// With one slice the block writes T directly. A three-stage ring of [x 32 KB
// | A 16 KB] filled by inline-asm DMA, one barrier a stage, which every wave
// passes once: before it the DMA waves issue stage t + 2 into the buffer
// stage t - 1 left and wait until stage t + 1 has landed; the MFMA waves
// have then finished every read of stage t (steps 0-2 read it; step 3,
// after the barrier, reads stage t + 1's first fragments).
__global__ __launch_bounds__(512, 1) void lora_xa_fast_kernel(const LoraXaArgs a, float* part,
                                                              int kslices) {
  constexpr int STG = 256 * 8 + 128 * 8;         // x tile + A tile, 16-B chunks
  constexpr int PER = 12;                        // 8 x + 4 A DMAs per DMA wave
  __shared__ uint4 st0[STG], st1[STG], st2[STG];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool dma_wave = wave >= 4;
  const int rw = wave & 3;                       // the role's wave index
  const int fr = lane & 31, fk = lane >> 5;
  const int wm = rw & 1, wc = rw >> 1;
  int m0, c0, ks;
  {
    const int tiles_m = (a.M + 255) / 256, tiles_c = (a.n_cols + 127) / 128;
    const int nb = (int)gridDim.x;
    const int q = nb / 8, rem = nb % 8;
    const int xcd = (int)blockIdx.x % 8, local = (int)blockIdx.x / 8;
    const int v = xcd * q + (xcd < rem ? xcd : rem) + local;
    const int tc = v % tiles_c, rest = v / tiles_c;
    m0 = (rest % tiles_m) * 256;
    c0 = tc * 128;
    ks = rest / tiles_m;
  }
  const int KT = a.K / 64;
  const int kt0 = (int)((long long)KT * ks / kslices);
  const int kt1 = (int)((long long)KT * (ks + 1) / kslices);
  const int NT = kt1 - kt0;
  const int mlast = a.M - 1;

  if (dma_wave) {
    uint32_t xoff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int p = 64 * (8 * rw + i) + lane;
      const int row = p >> 3;
      const int c = (p & 7) ^ ((row >> 1) & 7);
      int m = m0 + row;
      m = m < mlast ? m : mlast;
      xoff[i] = (uint32_t)(((long long)m * a.ldx + 8 * c) * 2);
    }
    const int g_safe = a.grp[0];
    uint32_t aoff[4];
    int asrc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 64 * (4 * rw + i) + lane;
      const int r = p >> 3;
      const int c = (p & 7) ^ ((r >> 1) & 7);
      const int col = c0 + r;
      const int g = col < a.n_cols ? a.grp[col >> 3] : -1;
      const int gs = g < 0 ? g_safe : g;
      const int row = 8 * (gs & 4095) + (g < 0 ? 0 : (col & 7));
      aoff[i] = (uint32_t)(((long long)row * a.K + 8 * c) * 2);
      asrc[i] = __builtin_amdgcn_readfirstlane(gs >> 12);
    }
    auto issue = [&](int kt, const uint4* S) {
      const void* base = a.x + (long long)kt * 64;
#pragma unroll
      for (int i = 0; i < 8; ++i) dma16_sb(base, xoff[i], lds_addr(S + 64 * (8 * rw + i)));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dma16_sb(a.A[asrc[i]] + (long long)kt * 64, aoff[i],
                 lds_addr(S + 2048 + 64 * (4 * rw + i)));
    };
    // The fp16 copy of x (a.xh): the column blocks of one row tile and K
    // slice split its 256 rows, so each element is converted once. Stage t
    // is converted while it is in LDS (landed at the previous wait, its
    // buffer rewritten only after the next barrier): lane q takes chunk
    // q & 7 of rows r0 + q / 8 + 32 j.
    const int tiles_c = (a.n_cols + 127) / 128, tc = c0 / 128;
    const int r0 = 256 * tc / tiles_c, r1 = 256 * (tc + 1) / tiles_c;
    const int q = 64 * rw + lane, qc = q & 7;
    uint32_t seen = 0;
    auto convert = [&](int t, const uint4* S) {
      if (!a.xh) return;
#pragma unroll 1
      for (int r = r0 + (q >> 3); r < r1; r += 32) {
        const uint4 v = S[r * 8 + (qc ^ ((r >> 1) & 7))];
        if (m0 + r < a.M) {
          seen = range_track4(seen, v);
          uint4 f;
          f.x = bf16x2_to_f16x2(v.x);
          f.y = bf16x2_to_f16x2(v.y);
          f.z = bf16x2_to_f16x2(v.z);
          f.w = bf16x2_to_f16x2(v.w);
          *reinterpret_cast<uint4*>(a.xh + (long long)(m0 + r) * a.ldxh +
                                    (long long)(kt0 + t) * 64 + 8 * qc) = f;
        }
      }
    };
    issue(kt0, st0);
    issue(kt0 + (NT > 1 ? 1 : 0), st1);
    ring_wait<PER>();                             // stage 0 landed
    // stage t: the copy of stage t, stage t + 2 (a re-read of the last past
    // the end) into the buffer of stage t - 1, then stage t + 1 landed, then
    // the barrier. The copy's stores go before the DMAs: vmcnt counts both
    // in issue order, so the wait for all but the newest PER (stage t + 2)
    // also covers the stores, whose latency the MFMA waves' stage hides.
    auto step = [&](int t, const uint4* C, const uint4* Pv) {
      convert(t, C);
      issue(kt0 + (t + 2 < NT ? t + 2 : NT - 1), Pv);
      ring_wait<PER>();
    };
    int t = 0;
    for (; t + 3 <= NT; t += 3) {
      step(t, st0, st2);
      step(t + 1, st1, st0);
      step(t + 2, st2, st1);
    }
    if (NT - t >= 1) step(t, st0, st2);
    if (NT - t == 2) step(t + 1, st1, st0);
    // no DMA outlives the block; no barrier: the MFMA waves meet no more
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (a.xh) range_report(a.range, seen);
    return;
  }

  floatx16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  const bool live = c0 + 64 * wc < a.n_cols;
  uint4 xb[4], ab[2];
  auto read_frags = [&](const uint4* S, int kk, uint4 (&xv)[4], uint4 (&av)[2]) {
    const int c = 2 * kk + fk;
#pragma unroll
    for (int i = 0; i < 4; ++i) xv[i] = S[swz8(128 * wm + 32 * i + fr, c)];
#pragma unroll
    for (int j = 0; j < 2; ++j) av[j] = S[2048 + swz8(64 * wc + 32 * j + fr, c)];
  };
  auto body = [&](const uint4* C, const uint4* Nx) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4 xn[4], an[2];
      if (kk < 3) read_frags(C, kk + 1, xn, an);
      else read_frags(Nx, 0, xn, an);
      if (live) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8_t, ab[j]), __builtin_bit_cast(bf16x8_t, xb[i]),
                acc[i][j], 0, 0, 0);
      }
#pragma unroll
      for (int g = 0; g < 6; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
      }
      __builtin_amdgcn_sched_barrier(0);
      if (kk == 2) {
        ring_wait<0>();                          // (no DMAs of its own) reads done + barrier
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) xb[i] = xn[i];
#pragma unroll
      for (int j = 0; j < 2; ++j) ab[j] = an[j];
    }
  };
  ring_wait<0>();                                // stage 0 landed (the DMA waves' wait)
  read_frags(st0, 0, xb, ab);
  int t = 0;
  for (; t + 3 <= NT; t += 3) {
    body(st0, st1);
    body(st1, st2);
    body(st2, st0);
  }
  if (NT - t >= 1) body(st0, st1);
  if (NT - t == 2) body(st1, st2);

  if (!live) return;
  if (kslices > 1) {
    // The partials in the accumulators' own order: slice ks, tile (row tile,
    // column block), MFMA wave, fragment f = 8i + 4j + q, lane -- each store
    // instruction writes 64 lanes x 16 B contiguous (the row-major layout
    // scattered every instruction over 32 rows). lora_xa_reduce_kernel reads
    // the same order.
    const int tiles_c = (a.n_cols + 127) / 128;
    const long long tile = (long long)(m0 / 256) * tiles_c + c0 / 128;
    const long long ntiles = (long long)((a.M + 255) / 256) * tiles_c;
    float4* pw = reinterpret_cast<float4*>(part) + (((ks * ntiles + tile) * 4 + rw) * 32) * 64 + lane;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          pw[(8 * i + 4 * j + q) * 64] =
              make_float4(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                          acc[i][j][4 * q + 3]);
    return;
  }
  // D[c][m]: lane owns row m, four consecutive ranks per register quad.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + 128 * wm + 32 * i + fr;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = c0 + 64 * wc + 32 * j + 8 * q + 4 * fk;
        const float f = a.coef[c >> 3];
        uint2 v;
        if (f == 0.0f) {
          v = make_uint2(0, 0);
        } else if (a.bias) {
          // the dense split-K GEMM with a bias (coef 1): one rounding
          float r[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) r[e] = f * acc[i][j][4 * q + e] + bf16_to_f32(a.bias[c + e]);
          v.x = pack_bf16x2_rne(r[0], r[1]);
          v.y = pack_bf16x2_rne(r[2], r[3]);
        } else {
          v.x = pack_bf16x2_rne(f * acc[i][j][4 * q + 0], f * acc[i][j][4 * q + 1]);
          v.y = pack_bf16x2_rne(f * acc[i][j][4 * q + 2], f * acc[i][j][4 * q + 3]);
        }
        *reinterpret_cast<uint2*>(a.t + (long long)m * a.ldt + c) = v;
      }
    }
  }
}

// T[m][c] = bf16(coef * sum_s P[s][m][c]), slices summed in order 0..S-1,
// over the partials in the order lora_xa_fast_kernel writes them. One thread
// per row and 8 consecutive ranks: the float4s of accumulator lanes fr and
// fr + 32 (ranks 8q + 0..3 and 8q + 4..7 of one row), read from every slice
// at the same positions (32 threads cover each 1-KB run, every load
// coalesced), one 16-byte store of T. Positions of row tiles past M or
// column blocks past n_cols are skipped. 32-bit indices (the host keeps a
// slice's float4 count below 2^31).
__global__ void lora_xa_reduce_kernel(const float* part, int kslices, int M,
                                      int n_cols, const LoraXaArgs a) {
  const unsigned tiles_c = ((unsigned)n_cols + 127) / 128;
  const unsigned ntiles = (((unsigned)M + 255) / 256) * tiles_c;
  const unsigned total = ntiles * 8192u;             // float4s per slice
  const bool st16 = (reinterpret_cast<uintptr_t>(a.t) & 15) == 0 && (a.ldt & 7) == 0;
  const float4* p4 = reinterpret_cast<const float4*>(part);
  for (unsigned t = blockIdx.x * blockDim.x + threadIdx.x; t < total / 2;
       t += gridDim.x * blockDim.x) {
    // the float4 of accumulator lane fr: ((tile * 4 + wave) * 32 + f) * 64 + fr,
    // f = 8 fi + 4 fj + fq; lane fr + 32 is 32 float4s on
    const unsigned fr = t & 31, g = t >> 5;
    const unsigned i = g * 64 + fr;
    const unsigned f = g & 31, wave = (g >> 5) & 3, tile = g >> 7;
    const unsigned fi = f >> 3, fj = (f >> 2) & 1, fq = f & 3;
    const unsigned tm = tile / tiles_c, tc = tile - tm * tiles_c;
    const unsigned m = 256 * tm + 128 * (wave & 1) + 32 * fi + fr;
    const unsigned c = 128 * tc + 64 * (wave >> 1) + 32 * fj + 8 * fq;
    if (m >= (unsigned)M || c >= (unsigned)n_cols) continue;
    float4 s0 = p4[i], s1 = p4[i + 32];
    for (int k = 1; k < kslices; ++k) {
      const float4 v0 = p4[(size_t)k * total + i];
      const float4 v1 = p4[(size_t)k * total + i + 32];
      s0.x += v0.x; s0.y += v0.y; s0.z += v0.z; s0.w += v0.w;
      s1.x += v1.x; s1.y += v1.y; s1.z += v1.z; s1.w += v1.w;
    }
    const float co = a.coef[c >> 3];
    uint4 o = make_uint4(0, 0, 0, 0);
    if (co != 0.0f && a.bias) {
      // the dense split-K GEMM with a bias (coef 1): one rounding
      float r[8] = {co * s0.x, co * s0.y, co * s0.z, co * s0.w,
                    co * s1.x, co * s1.y, co * s1.z, co * s1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] += bf16_to_f32(a.bias[c + e]);
      o.x = pack_bf16x2_rne(r[0], r[1]);
      o.y = pack_bf16x2_rne(r[2], r[3]);
      o.z = pack_bf16x2_rne(r[4], r[5]);
      o.w = pack_bf16x2_rne(r[6], r[7]);
    } else if (co != 0.0f) {
      o.x = pack_bf16x2_rne(co * s0.x, co * s0.y);
      o.y = pack_bf16x2_rne(co * s0.z, co * s0.w);
      o.z = pack_bf16x2_rne(co * s1.x, co * s1.y);
      o.w = pack_bf16x2_rne(co * s1.z, co * s1.w);
    }
    uint16_t* const tp = a.t + (size_t)m * a.ldt + c;
    if (st16) {
      *reinterpret_cast<uint4*>(tp) = o;
    } else {
      reinterpret_cast<uint2*>(tp)[0] = make_uint2(o.x, o.y);
      reinterpret_cast<uint2*>(tp)[1] = make_uint2(o.z, o.w);
    }
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
                                   long long ldy, int rows, int K, int* range) {
  const int k8 = K >> 3;
  const long long total = (long long)rows * k8;
  uint32_t seen = 0;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long r = i / k8;
    const int c = (int)(i % k8) * 8;
    const uint4 v = *reinterpret_cast<const uint4*>(x + r * ldx + c);
    seen = range_track4(seen, v);
    uint4 o;
    o.x = bf16x2_to_f16x2(v.x);
    o.y = bf16x2_to_f16x2(v.y);
    o.z = bf16x2_to_f16x2(v.z);
    o.w = bf16x2_to_f16x2(v.w);
    *reinterpret_cast<uint4*>(y + r * ldy + c) = o;
  }
  range_report(range, seen);
}

}  // namespace

hipError_t launch_qproj_fast(int bits, const QprojArgs& a, hipStream_t s) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (tiles <= 0) return hipSuccess;
  if (a.kslices > 1) {
    if (!a.part || a.N % 4 != 0 || (long long)a.M * (a.N / 4) >= (1ll << 31))
      return hipErrorInvalidValue;
    const dim3 grid((unsigned)(tiles * a.kslices));
    if (bits == 4)
      hipLaunchKernelGGL((qproj_fast_kernel<4, true>), grid, dim3(256), 0, s, a);
    else if (bits == 8)
      hipLaunchKernelGGL((qproj_fast_kernel<8, true>), grid, dim3(256), 0, s, a);
    else
      return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    long long blocks = ((long long)a.M * (a.N / 4) + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(qproj_split_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  if (bits == 4)
    hipLaunchKernelGGL((qproj_fast_kernel<4, false>), dim3(tiles), dim3(256), 0, s, a);
  else if (bits == 8)
    hipLaunchKernelGGL((qproj_fast_kernel<8, false>), dim3(tiles), dim3(256), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// CUs of the current device (the launch rounds are counted against it).
static int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// A grid whose last round of the chip's CUs is mostly empty (4352 rows: 1360
// tiles, 80 in a sixth round on 256 CUs) runs its last tile row as 128-row
// tiles in a second launch over the same arguments shifted down: twice the
// blocks at about half the time each. Each output element
// is computed by the same MFMA sequence either way, so the bits do not
// depend on the split.
hipError_t launch_qproj_pair(int bits, const QprojArgs& a, hipStream_t s) {
  const int tiles_n = (a.N + BN / 2 - 1) / (BN / 2);
  const int tiles_m = (a.M + BM - 1) / BM;
  const int tiles = tiles_m * tiles_n;
  if (tiles <= 0) return hipSuccess;
  if (a.kslices > 1 || a.g || !a.codes_u || !a.sb_u || a.nseg != 1 ||
      a.seg[0].chunks != a.seg_u.chunks || a.N % 8 != 0 || a.ldy % 8 != 0 ||
      (reinterpret_cast<uintptr_t>(a.y) & 15) != 0 || (bits != 4 && bits != 8))
    return hipErrorInvalidValue;
  // Rounds of the chip, one 256-row tile a CU: the whole grid against the
  // grid without its last tile row plus that row as 128-row tiles (about
  // 0.55 of a round each, measured); split when that saves a fifth of a
  // round or more.
  const int cus = device_cus();
  const int main_tiles = tiles - tiles_n;
  const int half_blocks = ((a.M - (tiles_m - 1) * BM + BM / 2 - 1) / (BM / 2)) * tiles_n;
  const double rounds_whole = (double)((tiles + cus - 1) / cus);
  const double rounds_split =
      (double)((main_tiles + cus - 1) / cus) + 0.55 * (double)((half_blocks + cus - 1) / cus);
  const int rows_main =
      (tiles_m >= 2 && rounds_split + 0.2 <= rounds_whole) ? (tiles_m - 1) * BM : a.M;
  {
    QprojArgs m = a;
    m.M = rows_main;
    const dim3 grid((unsigned)(tiles_m - (rows_main < a.M ? 1 : 0)) * tiles_n);
    if (bits == 4)
      hipLaunchKernelGGL((qproj_pair_kernel<4, 8>), grid, dim3(256), 0, s, m);
    else
      hipLaunchKernelGGL((qproj_pair_kernel<8, 8>), grid, dim3(256), 0, s, m);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || rows_main == a.M) return e;
  }
  QprojArgs h = a;
  h.M = a.M - rows_main;
  h.x = a.x + (long long)rows_main * a.ldx;
  h.y = a.y + (long long)rows_main * a.ldy;
  if (a.yh) h.yh = a.yh + (long long)rows_main * a.ldyh;
  if (a.t) h.t = a.t + (long long)rows_main * a.ldt;
  const dim3 grid((unsigned)(((h.M + BM / 2 - 1) / (BM / 2)) * tiles_n));
  if (bits == 4)
    hipLaunchKernelGGL((qproj_pair_kernel<4, 4>), grid, dim3(256), 0, s, h);
  else
    hipLaunchKernelGGL((qproj_pair_kernel<8, 4>), grid, dim3(256), 0, s, h);
  return hipGetLastError();
}

// The K split depends on M and K only, never on how many columns are
// stacked: each T column is then summed in the same order, and so has the
// same bits, whether its projection's x.A runs alone or stacked with others
// over the same x. It is sized for an assumed number of 128-wide column
// blocks per launch, by K:
//  - K <= 4096 (the hidden-width inputs: q|k|v, o, w1|w3): 5 blocks, between
//    one projection's 2.5 and q|k|v's 7.5 at the config-2 adapter set. At
//    4352 rows that is 3 slices, measured best of 1, 2, 3, 5 and 8 over the
//    1024^2 forward's 136 launches (6.59 ms against 6.91 ms for 5).
//  - K > 4096 (the FFN-width input of w2, whose x.A always runs alone): 2
//    blocks (the config-2 set's 256 packed ranks), i.e. 7 slices at 4352
//    rows, one round of 238 blocks: w2's x.A 3.7 us faster than with 5
//    slices (3 blocks, 255 blocks of 32 K steps each).
int lora_xa_fast_slices(int M, int n_cols, int K) {
  (void)n_cols;
  const int tiles = ((M + 255) / 256) * (K > 4096 ? 2 : 5);
  const int KT = K / 64;
  int ks = 256 / (tiles > 0 ? tiles : 1);       // about one round of the chip
  const int kmax = KT / 8 > 1 ? KT / 8 : 1;      // keep >= 8 K steps per slice
  if (ks > kmax) ks = kmax;
  return ks < 1 ? 1 : ks;
}

// A dense projection through the x.A kernel: as many slices as fill about
// one round of the chip, at least 8 K steps each.
int dense_xa_slices(int M, int N, int K) {
  const int tiles = ((M + 255) / 256) * ((N + 127) / 128);
  const int KT = K / 64;
  int ks = 256 / (tiles > 0 ? tiles : 1);
  const int kmax = KT / 8 > 1 ? KT / 8 : 1;
  if (ks > kmax) ks = kmax;
  return ks < 1 ? 1 : ks;
}

size_t lora_xa_part_bytes(int M, int n_cols, int kslices) {
  if (kslices <= 1) return 0;
  return (size_t)kslices * (size_t)((M + 255) / 256) * (size_t)((n_cols + 127) / 128) *
         (256 * 128 * 4);
}

hipError_t launch_lora_xa_fast(const LoraXaArgs& a, float* part, int kslices,
                               hipStream_t s) {
  if (a.M <= 0 || a.n_cols <= 0) return hipSuccess;
  // the reduce's 32-bit indexing: one thread per float4 of a slice
  const long long work = (long long)((a.M + 255) / 256) * ((a.n_cols + 127) / 128) * 8192;
  if (kslices > 1 && (a.n_cols % 8 != 0 || work >= (1ll << 31))) return hipErrorInvalidValue;
  const unsigned nblk = (unsigned)(((a.M + 255) / 256) * ((a.n_cols + 127) / 128) * kslices);
  hipLaunchKernelGGL(lora_xa_fast_kernel, dim3(nblk), dim3(512), 0, s, a, part, kslices);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || kslices == 1) return e;
  long long blocks = (work / 2 + 255) / 256;
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
                              long long ldy, int rows, int K, hipStream_t s, int* range) {
  long long work = (long long)rows * (K / 8);
  long long blocks = (work + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(bf16_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     s, x, ldx, y, ldy, rows, K, range);
  return hipGetLastError();
}

hipError_t validate_qproj_fast_kernels() {
  hipFuncAttributes fa;
  const void* fns[] = {reinterpret_cast<const void*>(&qproj_fast_kernel<4, false>),
                       reinterpret_cast<const void*>(&qproj_fast_kernel<8, false>),
                       reinterpret_cast<const void*>(&qproj_fast_kernel<4, true>),
                       reinterpret_cast<const void*>(&qproj_fast_kernel<8, true>),
                       reinterpret_cast<const void*>(&qproj_split_reduce_kernel),
                       reinterpret_cast<const void*>(&repack_fast_kernel),
                       reinterpret_cast<const void*>(&repack_sbf_kernel),
                       reinterpret_cast<const void*>(&bf16_to_f16_kernel),
                       reinterpret_cast<const void*>(&qproj_pair_kernel<4, 8>),
                       reinterpret_cast<const void*>(&qproj_pair_kernel<8, 8>),
                       reinterpret_cast<const void*>(&qproj_pair_kernel<4, 4>),
                       reinterpret_cast<const void*>(&qproj_pair_kernel<8, 4>),
                       reinterpret_cast<const void*>(&lora_xa_fast_kernel),
                       reinterpret_cast<const void*>(&lora_xa_reduce_kernel)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&fa, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ming
