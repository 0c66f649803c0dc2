// Dense bidirectional attention for the DiT blocks on MI355X (gfx950):
// head dim 128, no mask, any sequence length (the ragged last key block is
// masked out of the softmax, as the reference's unaligned specialization
// does, ming-dit.cc:1905-1915).
//
// Operands stay where the block's projections put them: Q and K are read
// token-major straight from the fused qkv output (head h at column +128h),
// and the output is written token-major, so no head-major transpose of Q,
// K or O exists. Only V is transposed (vt_transpose_kernel) into
// V^T [head][d][key], keys contiguous and zero-padded to a multiple of 64.
//
// Per block: 4 waves x 32 queries = 128 queries of one head; keys in steps
// of 64 through a two-stage LDS ring filled by direct global->LDS DMA.
// Per step and wave:
//   S^T = K . Q^T   2 key tiles x 8 d-slices of v_mfma_f32_32x32x16_bf16.
//                   Each lane owns ONE query (the MFMA's column), so the
//                   softmax row reductions are in-lane plus one exchange
//                   with the other lane half. The K rows of every 16-key
//                   slice are fed in the order {0-3, 8-11, 4-7, 12-15}
//                   (bits 2 and 3 of the row swapped), which leaves lane
//                   half h holding keys 8h..8h+7 of each slice in
//                   consecutive registers -- exactly the B operand layout
//                   of the P.V MFMA, so P never leaves registers.
//   online softmax  exp2 domain (scale*log2 e folded into the exp2
//                   argument), a lazily moved reference max exchanged
//                   across lane halves, running sums kept per lane half
//                   and combined at the end.
//   O^T += V^T.P^T  4 d-tiles x 4 key slices, P rounded to bf16 (the
//                   reference's steel kernel also feeds P as the input
//                   type to its second GEMM). V^T rows are fed in the same
//                   swapped order, so each lane ends holding 8 consecutive
//                   d of its query: 16-byte token-major stores.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace ming {
namespace {

constexpr int ABQ = 128, ABK = 64, AHD = 128;

__device__ __forceinline__ int swap23(int i) {
  return (i & ~12) | ((i >> 2) & 1) << 3 | ((i >> 3) & 1) << 2;
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void adma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(off), "s"(base), "s"(lds) : "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t alds(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// vmcnt(0) + LDS reads done + workgroup barrier (the DMAs are inline asm,
// so every wait on them is explicit).
__device__ __forceinline__ void attn_sync() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A value and its twin in the other lane half (lane ^ 32) combined by gfx950's
// v_permlane32_swap: after the swap the two results hold, in every lane, the
// lane-half-0 and lane-half-1 values of the pair, so their sum or max is the
// pair's in either order (no LDS round trip, as a bpermute takes).
__device__ __forceinline__ void halves(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum32(float v) {
  float a, b;
  halves(v, a, b);
  return a + b;
}
__device__ __forceinline__ float max32(float v) {
  float a, b;
  halves(v, a, b);
  return fmaxf(a, b);
}

__global__ __launch_bounds__(256, 2) void attention_kernel(const AttnArgs a) {
  // stage = K tile [64 keys][128 d] (16-B chunk c of row r at
  // 16r + (c ^ (r & 15))) + V^T tile [128 d][64 keys] (swz8 rows of 128 B)
  __shared__ uint4 sk0[1024], sv0[1024], sk1[1024], sv1[1024];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  const int q0 = blockIdx.x * ABQ;
  const int head = blockIdx.y;
  const int R = a.R;
  const int NKB = (R + ABK - 1) / ABK;

  // Q^T fragments (B operand): lane = query fr, d = 16s + 8fh + 0..7
  int qr = q0 + 32 * wave + fr;
  qr = qr < R ? qr : R - 1;
  uint4 qf[8];
  {
    const uint16_t* qp = a.q + (long long)qr * a.ldq + head * AHD + 8 * fh;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *reinterpret_cast<const uint4*>(qp + 16 * s);
  }
  // With a.qw, q is the raw projection output: its per-head RMSNorm + RoPE
  // (launch_qk_norm_rope's arithmetic) is applied here. The lane holds the
  // 8-column groups 2s + fh of its query; the head's reduction tree (groups
  // at distance 8, 4, 2, 1) is s ^ 4, s ^ 2, s ^ 1 in registers, then the
  // other lane half. Weights and table rows load beside q.
  uint4 qwv[8];
  float4 qcs[8], qsn[8];
  if (a.qw) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      qwv[s] = *reinterpret_cast<const uint4*>(a.qw + 16 * s + 8 * fh);
      qcs[s] = *reinterpret_cast<const float4*>(a.cos_t + (long long)qr * 64 + 8 * s + 4 * fh);
      qsn[s] = *reinterpret_cast<const float4*>(a.sin_t + (long long)qr * 64 + 8 * s + 4 * fh);
    }
  }
  // Wait for them here (vmcnt(0); expcnt, lgkmcnt open): the compiler then
  // puts no wait for them into the key loop, where a vmcnt wait would also
  // wait for the ring's DMA of the next tile, every step.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  if (a.qw) {
    float t8[8], t4[8], t2[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) t8[s] = head_ss8(qf[s]);
#pragma unroll
    for (int s = 0; s < 8; ++s) t4[s] = t8[s] + t8[s ^ 4];
#pragma unroll
    for (int s = 0; s < 8; ++s) t2[s] = t4[s] + t4[s ^ 2];
    const float t1 = t2[0] + t2[1];
    const float inv = head_rms_inv(sum32(t1), a.eps);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      qf[s].x = norm_rope_pair(qf[s].x, qwv[s].x, inv, qcs[s].x, qsn[s].x);
      qf[s].y = norm_rope_pair(qf[s].y, qwv[s].y, inv, qcs[s].y, qsn[s].y);
      qf[s].z = norm_rope_pair(qf[s].z, qwv[s].z, inv, qcs[s].z, qsn[s].z);
      qf[s].w = norm_rope_pair(qf[s].w, qwv[s].w, inv, qcs[s].w, qsn[s].w);
    }
  }

  // DMA offsets (bytes from the step's base). K: chunk p -> row p >> 4,
  // logical chunk (p & 15) ^ (row & 15). V^T: chunk p -> row p >> 3,
  // logical chunk (p & 7) ^ ((row >> 1) & 7).
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = 64 * (4 * wave + i) + lane;
    const int kr = p >> 4;
    const int kc = (p & 15) ^ (kr & 15);
    // R < 64: one block, loaded from row 0; rows past R re-read row R-1
    const int krow = R < ABK ? (kr < R ? kr : R - 1) : kr;
    koff[i] = (uint32_t)(krow * a.ldk * 2 + kc * 16);
    const int vr = p >> 3;
    const int vc = (p & 7) ^ ((vr >> 1) & 7);
    voff[i] = (uint32_t)(vr * a.ldv * 2 + vc * 16);
  }
  const uint16_t* kbase0 = a.k + head * AHD;
  const uint16_t* vbase0 = a.vt + (long long)head * AHD * a.ldv;
  // The last key block reads rows up to 63 past its start: clamp the block
  // start so K rows stay inside [0, R) (the masked keys re-read valid rows).
  auto issue = [&](int kb, uint4* SK, uint4* SV) {
    int kstart = kb * ABK;
    const int kmax = R - ABK;
    const int kclamp = kstart < kmax ? kstart : (kmax > 0 ? kmax : 0);
    const uint16_t* kb_base = kbase0 + (long long)kclamp * a.ldk;
    const uint16_t* vb_base = vbase0 + kstart;
#pragma unroll
    for (int i = 0; i < 4; ++i) adma16(kb_base, koff[i], alds(SK + 64 * (4 * wave + i)));
#pragma unroll
    for (int i = 0; i < 4; ++i) adma16(vb_base, voff[i], alds(SV + 64 * (4 * wave + i)));
  };

  floatx16_t oacc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[u][r] = 0.0f;
  // Lazy online softmax (exp2 domain): P = exp2(sl2 * s - mref) against a
  // reference max mref that moves only when some query's max rises more
  // than kLazy above it, so P <= 2^kLazy and O and l are rescaled only then
  // (a wave-uniform branch), not at every key block.
  constexpr float kLazy = 8.0f;
  float mref = -INFINITY, lrun = 0.0f;
  const float sl2 = a.sl2;

  // MASK: the last key block, which may be shifted back to stay inside
  // [0, R) and may hold keys past R; every other block runs unmasked.
  auto step = [&](auto mask_tag, int kb, const uint4* SK, const uint4* SV) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int kstart = kb * ABK;
    int shift = 0;
    if constexpr (MASK) {
      // When R < 64 the (single) block was loaded from row 0; otherwise the
      // last block was shifted back to R - 64: keys are then offset.
      const int kmax = R - ABK;
      const int kload = kstart < kmax ? kstart : (kmax > 0 ? kmax : 0);
      shift = kstart - kload;
    }
    floatx16_t sacc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[t][r] = 0.0f;
    // the two key tiles alternate, so consecutive MFMAs never chain on one
    // accumulator
    int rr[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      rr[t] = 32 * t + swap23(fr);                    // K row in the loaded tile
      if constexpr (MASK) {
        rr[t] += shift;
        rr[t] = rr[t] < ABK ? rr[t] : ABK - 1;
      }
    }
    // The 16 K fragments of the step, read 4 ahead of their MFMAs (pinned;
    // the scheduler alone keeps about 2 in flight).
    uint4 kfa[16];
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        kfa[2 * s + t] = SK[16 * rr[t] + ((2 * s + fh) ^ (rr[t] & 15))];
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        sacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, kfa[2 * s + t]), __builtin_bit_cast(bf16x8_t, qf[s]),
            sacc[t], 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 4; ++g) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int g = 0; g < 16 - 4; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_barrier(0);
    // register r of tile t holds key 32t + 16(r/8) + 8fh + (r%8)
    if constexpr (MASK) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kstart + 32 * t + 16 * (r >> 3) + 8 * fh + (r & 7);
          sacc[t][r] = key < R ? sacc[t][r] : -INFINITY;
        }
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, sacc[t][r]);
    mloc = max32(mloc) * sl2;                         // sl2 > 0: max commutes
    if (__any(mloc > mref + kLazy)) {
      const float mnew = fmaxf(mref, mloc);
      const float alpha = __builtin_amdgcn_exp2f(mref - mnew);
      mref = mnew;
      lrun *= alpha;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[u][r] *= alpha;
    }
    const float nm = -mref;
    float psum = 0.0f;
    uint4 pf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = j >> 1, r0 = 8 * (j & 1);
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[t][r0 + e], sl2, nm));
        psum += p[e];
      }
      pf[j].x = pack_bf16x2_rne(p[0], p[1]);
      pf[j].y = pack_bf16x2_rne(p[2], p[3]);
      pf[j].z = pack_bf16x2_rne(p[4], p[5]);
      pf[j].w = pack_bf16x2_rne(p[6], p[7]);
    }
    lrun += psum;
    // O^T[d][q] += V^T[d][k] P^T[k][q]; V^T row fed for output row i is
    // d = 32u + swap23(i). The four d-tiles alternate (no accumulator chain).
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int vrow = 32 * u + swap23(fr);
        const uint4 vf = SV[vrow * 8 + ((2 * j + fh) ^ ((vrow >> 1) & 7))];
        oacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, vf), __builtin_bit_cast(bf16x8_t, pf[j]),
            oacc[u], 0, 0, 0);
      }
  };
  const std::integral_constant<bool, false> whole{};
  const std::integral_constant<bool, true> last{};

  // Steady state: pairs of unmasked steps with no branch between them (a
  // step that may be the last one inside the loop made the compiler copy the
  // loop-carried accumulators at every step); then the one or two steps left,
  // the last one masked.
  issue(0, sk0, sv0);
  int kb = 0;
  for (; kb + 2 < NKB; kb += 2) {
    attn_sync();                                   // stage kb landed; sk1/sv1 free
    issue(kb + 1, sk1, sv1);
    step(whole, kb, sk0, sv0);
    attn_sync();
    issue(kb + 2, sk0, sv0);
    step(whole, kb + 1, sk1, sv1);
  }
  attn_sync();                                     // stage kb landed
  if (kb + 1 < NKB) {
    issue(kb + 1, sk1, sv1);
    step(whole, kb, sk0, sv0);
    attn_sync();
    step(last, kb + 1, sk1, sv1);
  } else {
    step(last, kb, sk0, sv0);
  }
  attn_sync();                                     // no DMA outlives the block

  const float ltot = sum32(lrun);
  const float inv = 1.0f / ltot;
  const int q = q0 + 32 * wave + fr;
  if (q < R) {
    uint16_t* op = a.o + (long long)q * a.ldo + head * AHD + 8 * fh;
    uint32_t seen = 0;   // magnitudes written to the fp16 copy
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        uint4 v;
        v.x = pack_bf16x2_rne(oacc[u][8 * hh + 0] * inv, oacc[u][8 * hh + 1] * inv);
        v.y = pack_bf16x2_rne(oacc[u][8 * hh + 2] * inv, oacc[u][8 * hh + 3] * inv);
        v.z = pack_bf16x2_rne(oacc[u][8 * hh + 4] * inv, oacc[u][8 * hh + 5] * inv);
        v.w = pack_bf16x2_rne(oacc[u][8 * hh + 6] * inv, oacc[u][8 * hh + 7] * inv);
        *reinterpret_cast<uint4*>(op + 32 * u + 16 * hh) = v;
        if (a.oh) {
          seen = range_track4(seen, v);
          uint4 f;
          f.x = bf16x2_to_f16x2(v.x);
          f.y = bf16x2_to_f16x2(v.y);
          f.z = bf16x2_to_f16x2(v.z);
          f.w = bf16x2_to_f16x2(v.w);
          *reinterpret_cast<uint4*>(a.oh + (long long)q * a.ldoh + head * AHD + 8 * fh +
                                    32 * u + 16 * hh) = f;
        }
      }
    if (a.oh) range_report(a.range, seen);
  }
}

// V [R][head*128 + d] (token-major) -> V^T [head][d][key], keys padded with
// zeros to ldv. One block transposes 64 keys x 64 d through LDS.
__global__ __launch_bounds__(256) void vt_transpose_kernel(const uint16_t* v, long long ldv_in,
                                                           uint16_t* vt, int ldv, int R) {
  __shared__ uint16_t t[64][64 + 2];
  const int k0 = blockIdx.x * 64;
  const int head = blockIdx.y >> 1, d0 = (blockIdx.y & 1) * 64;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i;          // 512 chunks of 8 d
    const int key = c >> 3, dc = (c & 7) * 8;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (k0 + key < R)
      val = *reinterpret_cast<const uint4*>(v + (long long)(k0 + key) * ldv_in + head * AHD + d0 + dc);
    const uint16_t* e = reinterpret_cast<const uint16_t*>(&val);
#pragma unroll
    for (int j = 0; j < 8; ++j) t[dc + j][key] = e[j];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i;          // 512 chunks of 8 keys
    const int d = c >> 3, kc = (c & 7) * 8;
    uint16_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = t[d][kc + j];
    uint4 val;
    val.x = e[0] | ((uint32_t)e[1] << 16);
    val.y = e[2] | ((uint32_t)e[3] << 16);
    val.z = e[4] | ((uint32_t)e[5] << 16);
    val.w = e[6] | ((uint32_t)e[7] << 16);
    *reinterpret_cast<uint4*>(vt + ((long long)head * AHD + d0 + d) * ldv + k0 + kc) = val;
  }
}

}  // namespace

hipError_t launch_attention(const AttnArgs& a, const uint16_t* v, long long ldv_in,
                            hipStream_t s) {
  if (a.R <= 0 || a.NH <= 0) return hipSuccess;
  const int kblocks = a.ldv / 64;
  hipLaunchKernelGGL(vt_transpose_kernel, dim3(kblocks, 2 * a.NH), dim3(256), 0, s, v,
                     ldv_in, const_cast<uint16_t*>(a.vt), a.ldv, a.R);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attention_kernel, dim3((a.R + ABQ - 1) / ABQ, a.NH), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t validate_attention_kernels() {
  hipFuncAttributes fa;
  const void* fns[] = {reinterpret_cast<const void*>(&attention_kernel),
                       reinterpret_cast<const void*>(&vt_transpose_kernel)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&fa, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ming
