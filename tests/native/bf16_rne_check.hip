// TEST INFRASTRUCTURE ONLY: checks, over all 2^32 f32 bit patterns on the
// device, that the pair conversion every kernel of the library rounds with
// (ming::pack_bf16x2_rne in csrc/common.h: gfx950's v_cvt_pk_bf16_f32) is
// round-to-nearest-even as the reference defines it for bf16
// (ming-dit.cc:173-181): the bit arithmetic u + 0x7fff + ((u >> 16) & 1),
// upper half. Built with the library's own flags (tests/native/Makefile).
#include <hip/hip_runtime.h>

#include "../../vpipe-ming-image_amd/csrc/common.h"

namespace {

// counts[0]: non-NaN patterns whose result differs from the bit arithmetic;
// counts[1]: NaN patterns whose result is not a NaN; counts[2]: NaN patterns
// whose result is not the canonical quiet NaN 0x7fc0 / 0xffc0 (the hardware
// keeps payload bits; informational).
__global__ __launch_bounds__(256) void rne_check_kernel(unsigned long long* counts) {
  const uint32_t base = (blockIdx.x * 256u + threadIdx.x) * 1024u;
  uint32_t bad = 0, nan_bad = 0, nan_payload = 0;
  for (uint32_t i = 0; i < 1024u; i += 2) {
    const uint32_t u[2] = {base + i, base + i + 1};
    const uint32_t hw = ming::pack_bf16x2_rne(__uint_as_float(u[0]), __uint_as_float(u[1]));
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t h = e ? hw >> 16 : hw & 0xffffu;
      if ((u[e] & 0x7fffffffu) > 0x7f800000u) {
        nan_bad += ((h & 0x7f80u) != 0x7f80u || (h & 0x7fu) == 0u) ? 1u : 0u;
        nan_payload += (h & 0x7fffu) != 0x7fc0u ? 1u : 0u;
      } else {
        const uint32_t want = (u[e] + 0x7fffu + ((u[e] >> 16) & 1u)) >> 16;
        bad += h != want ? 1u : 0u;
      }
    }
  }
  // one atomic per wave and count
  for (int o = 32; o >= 1; o >>= 1) {
    bad += __shfl_xor(bad, o, 64);
    nan_bad += __shfl_xor(nan_bad, o, 64);
    nan_payload += __shfl_xor(nan_payload, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&counts[0], (unsigned long long)bad);
    atomicAdd(&counts[1], (unsigned long long)nan_bad);
    atomicAdd(&counts[2], (unsigned long long)nan_payload);
  }
}

}  // namespace

// Runs the check on the current device; out[3] receives the counts. 0 on
// success, else the HIP error code.
extern "C" int bf16_rne_check(unsigned long long* out) {
  unsigned long long* d = nullptr;
  hipError_t e = hipMalloc(&d, 3 * sizeof(unsigned long long));
  if (e != hipSuccess) return (int)e;
  e = hipMemset(d, 0, 3 * sizeof(unsigned long long));
  if (e == hipSuccess) {
    hipLaunchKernelGGL(rne_check_kernel, dim3(16384), dim3(256), 0, 0, d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess)
    e = hipMemcpy(out, d, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  return (int)e;
}
