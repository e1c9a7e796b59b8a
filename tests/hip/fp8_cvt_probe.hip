// Test program: exhaustive comparison of the hardware fp8 pack-convert
// (v_cvt_pk_fp8_f32) with the software e4m3 round-to-nearest-even of the
// quantizers, over every fp32 bit pattern with |v| <= 448 or NaN.  Prints the
// mismatch count split into NaN and non-NaN inputs; exit status 0 iff every
// non-NaN input agrees (NaN tiles never reach the hardware conversion).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include "../../nano-train_amd/csrc/ntlb_device.h"
__global__ void cmp(unsigned long long* bad, unsigned* first, unsigned long long* checked,
                    unsigned long long* bad_finite) {
  unsigned long long nb = 0, nc = 0, nf = 0;
  const uint32_t total_threads = gridDim.x * blockDim.x;
  for (uint64_t u = blockIdx.x * blockDim.x + threadIdx.x; u < (1ull << 32); u += total_threads) {
    float v = __uint_as_float((uint32_t)u);
    uint32_t ab = (uint32_t)u & 0x7FFFFFFFu;
    bool nan = ab > 0x7F800000u;
    if (!nan && __uint_as_float(ab) > 448.0f) continue;
    uint32_t hw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false) & 0xFFu;
    uint32_t sw = ntlb::e4m3_rne(v);
    ++nc;
    if (hw != sw && !nan) ++nf;
    if (hw != sw) { ++nb; unsigned idx = atomicAdd(first, 1u); if (idx < 16) first[1 + 2*idx] = (uint32_t)u, first[2 + 2*idx] = (hw << 8) | sw; }
  }
  atomicAdd(bad, nb); atomicAdd(checked, nc); atomicAdd(bad_finite, nf);
}
int main() {
  unsigned long long *bad, *checked, *bad_finite; unsigned* first;
  if (hipMalloc(&bad, 8) || hipMalloc(&checked, 8) || hipMalloc(&bad_finite, 8) || hipMalloc(&first, 4 * 40)) return 2;
  (void)hipMemset(bad, 0, 8); (void)hipMemset(checked, 0, 8); (void)hipMemset(bad_finite, 0, 8);
  (void)hipMemset(first, 0, 160);
  cmp<<<8192, 256>>>(bad, first, checked, bad_finite);
  hipError_t e = hipDeviceSynchronize();
  unsigned long long hb = 0, hc = 0, hnf = 0; unsigned hf[40];
  (void)hipMemcpy(&hb, bad, 8, hipMemcpyDeviceToHost); (void)hipMemcpy(&hc, checked, 8, hipMemcpyDeviceToHost);
  (void)hipMemcpy(&hnf, bad_finite, 8, hipMemcpyDeviceToHost); (void)hipMemcpy(hf, first, 160, hipMemcpyDeviceToHost);
  printf("status=%s checked=%llu mismatches=%llu non_nan_mismatches=%llu\n", hipGetErrorString(e), hc, hb, hnf);
  for (unsigned i = 0; i < hf[0] && i < 16; ++i) printf("  u=0x%08x hw=0x%02x sw=0x%02x\n", hf[1+2*i], hf[2+2*i] >> 8, hf[2+2*i] & 0xFF);
  return (e != hipSuccess || hnf != 0) ? 1 : 0;
}
