// Test program: exhaustive comparison of the hardware bf16 pack-convert
// (v_cvt_pk_bf16_f32, what a (__bf16) cast compiles to on gfx950) with the
// software round-to-nearest-even f32_to_bf16_bits, over every fp32 bit
// pattern.  Non-NaN inputs must give identical bits; NaN inputs must give a
// NaN.  Exit status 0 iff both hold.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include "../../nano-train_amd/csrc/ntlb_device.h"
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__global__ void cmp(unsigned long long* bad, unsigned* first, unsigned long long* checked,
                    unsigned long long* bad_nan) {
  unsigned long long nb = 0, nc = 0, nn = 0;
  const uint32_t total_threads = gridDim.x * blockDim.x;
  for (uint64_t u = blockIdx.x * blockDim.x + threadIdx.x; u < (1ull << 32); u += total_threads) {
    const float v = __uint_as_float((uint32_t)u);
    const bool nan = ((uint32_t)u & 0x7FFFFFFFu) > 0x7F800000u;
    const v2bf p = {(__bf16)v, (__bf16)v};
    const uint32_t hw = __builtin_bit_cast(uint32_t, p) & 0xFFFFu;
    const uint32_t sw = ntlb::f32_to_bf16_bits(v);
    ++nc;
    if (nan) {
      if ((hw & 0x7FFFu) <= 0x7F80u) ++nn;
    } else if (hw != sw) {
      ++nb;
      const unsigned idx = atomicAdd(first, 1u);
      if (idx < 16) first[1 + 2 * idx] = (uint32_t)u, first[2 + 2 * idx] = (hw << 16) | sw;
    }
  }
  atomicAdd(bad, nb); atomicAdd(checked, nc); atomicAdd(bad_nan, nn);
}
int main() {
  unsigned long long *bad, *checked, *bad_nan; unsigned* first;
  if (hipMalloc(&bad, 8) || hipMalloc(&checked, 8) || hipMalloc(&bad_nan, 8) || hipMalloc(&first, 4 * 40)) return 2;
  (void)hipMemset(bad, 0, 8); (void)hipMemset(checked, 0, 8); (void)hipMemset(bad_nan, 0, 8);
  (void)hipMemset(first, 0, 160);
  cmp<<<8192, 256>>>(bad, first, checked, bad_nan);
  hipError_t e = hipDeviceSynchronize();
  unsigned long long hb = 0, hc = 0, hn = 0; unsigned hf[40];
  (void)hipMemcpy(&hb, bad, 8, hipMemcpyDeviceToHost); (void)hipMemcpy(&hc, checked, 8, hipMemcpyDeviceToHost);
  (void)hipMemcpy(&hn, bad_nan, 8, hipMemcpyDeviceToHost); (void)hipMemcpy(hf, first, 160, hipMemcpyDeviceToHost);
  printf("status=%s checked=%llu non_nan_mismatches=%llu nan_not_nan=%llu\n", hipGetErrorString(e), hc, hb, hn);
  for (unsigned i = 0; i < hf[0] && i < 16; ++i) printf("  u=0x%08x hw=0x%04x sw=0x%04x\n", hf[1+2*i], hf[2+2*i] >> 16, hf[2+2*i] & 0xFFFF);
  return (e != hipSuccess || hb != 0 || hn != 0) ? 1 : 0;
}
