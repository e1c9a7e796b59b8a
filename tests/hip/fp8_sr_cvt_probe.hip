// Test program: comparison of the hardware stochastic fp8 convert
// (v_cvt_sr_fp8_f32, which the quantizers' stochastic-rounding tile paths
// use) with the software rule e4m3_sr (20 bits below the e4m3 spacing plus
// r >> 12 carry into the code), over every fp32 bit pattern with |v| <= 448,
// each with four random words: a hash of the pattern, its complement, and
// for normal |v| the word that puts frac20 + (r >> 12) exactly at 2^20 and the
// one just below.  Exit status 0 iff every pair agrees.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include "../../nano-train_amd/csrc/ntlb_device.h"
__device__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16; x *= 0x7feb352dU; x ^= x >> 15; x *= 0x846ca68bU; x ^= x >> 16;
  return x;
}
__global__ void cmp(unsigned long long* bad, unsigned* first, unsigned long long* checked) {
  unsigned long long nb = 0, nc = 0;
  const uint32_t total_threads = gridDim.x * blockDim.x;
  for (uint64_t u = blockIdx.x * blockDim.x + threadIdx.x; u < (1ull << 32); u += total_threads) {
    const uint32_t ab = (uint32_t)u & 0x7FFFFFFFu;
    if (ab > 0x43E00000u) continue;  // |v| <= 448 only (the tile paths clamp first; NaN excluded)
    const float v = __uint_as_float((uint32_t)u);
    const uint32_t h = mix32((uint32_t)u * 2654435761u + 0x9e3779b9u);
    const uint32_t at = ((0x100000u - (ab & 0xFFFFFu)) & 0xFFFFFu) << 12;
    const uint32_t rs[4] = {h, ~h, at, at - 4096u};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t hw = (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(v, (int)rs[k], 0, 0) & 0xFFu;
      const uint32_t sw = ntlb::e4m3_sr(v, rs[k]);
      ++nc;
      if (hw != sw) {
        ++nb;
        const unsigned idx = atomicAdd(first, 1u);
        if (idx < 12) first[1 + 3 * idx] = (uint32_t)u, first[2 + 3 * idx] = rs[k], first[3 + 3 * idx] = (hw << 8) | sw;
      }
    }
  }
  atomicAdd(bad, nb); atomicAdd(checked, nc);
}
int main() {
  unsigned long long *bad, *checked; unsigned* first;
  (void)hipMalloc(&bad, 8); (void)hipMalloc(&checked, 8); (void)hipMalloc(&first, 160);
  (void)hipMemset(bad, 0, 8); (void)hipMemset(checked, 0, 8); (void)hipMemset(first, 0, 160);
  cmp<<<8192, 256>>>(bad, first, checked);
  hipError_t e = hipDeviceSynchronize();
  unsigned long long hb = 0, hc = 0; unsigned hf[40];
  (void)hipMemcpy(&hb, bad, 8, hipMemcpyDeviceToHost); (void)hipMemcpy(&hc, checked, 8, hipMemcpyDeviceToHost);
  (void)hipMemcpy(hf, first, 160, hipMemcpyDeviceToHost);
  printf("status=%s checked=%llu mismatches=%llu\n", hipGetErrorString(e), hc, hb);
  for (unsigned i = 0; i < hf[0] && i < 12; ++i)
    printf("  v=0x%08x r=0x%08x hw=0x%02x sw=0x%02x\n", hf[1 + 3 * i], hf[2 + 3 * i], hf[3 + 3 * i] >> 8, hf[3 + 3 * i] & 0xFF);
  return (e != hipSuccess || hb != 0) ? 1 : 0;
}
