// The straight-through operand of te_backend.py:250-251:
//   out = t + (t_dq - t)
// evaluated elementwise in t's dtype as torch evaluates it: each binary op
// in fp32 on the widened operands, its result rounded to the dtype (round to
// nearest even) before the next op.  Under round to nearest the result is
// t_dq itself (t_dq and t lie within a factor of two, so the difference is
// exact); under stochastic rounding a code can land far from t / s, the
// difference is then rounded, and the sum can differ from t_dq.  The
// low-bit layers take this operand wherever they multiply the reference's
// dequantized values under stochastic rounding.
//
// HBM-bound: 2 x dtype bytes in, dtype bytes out per element; 16-byte
// vectors per thread over a grid-stride loop.
#include <hip/hip_runtime.h>

#include "ntlb_device.h"
#include "ntlb_host.h"

namespace ntlb {

template <int DT>
__device__ __forceinline__ float ste_one(float t, float dq) {
  const float d = round_to_dtype(dq - t, DT);
  return round_to_dtype(t + d, DT);
}

// 16 bytes of each operand per step: 8 bf16 / f16 or 4 fp32 elements
template <int DT>
__global__ void __launch_bounds__(256) ste_value_vec_kernel(const uint4* __restrict__ t, const uint4* __restrict__ dq,
                                                            uint4* __restrict__ out, int64_t nvec) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    const uint4 a = t[i], b = dq[i];
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
    uint32_t ow[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if constexpr (DT == DT_F32) {
        ow[w] = __float_as_uint(ste_one<DT>(__uint_as_float(aw[w]), __uint_as_float(bw[w])));
      } else {
        uint32_t r = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint16_t ab = (uint16_t)(aw[w] >> (16 * h)), bb = (uint16_t)(bw[w] >> (16 * h));
          float tv, dv;
          if constexpr (DT == DT_BF16) {
            tv = bf16_bits_to_f32(ab);
            dv = bf16_bits_to_f32(bb);
          } else {
            tv = __half2float(__ushort_as_half(ab));
            dv = __half2float(__ushort_as_half(bb));
          }
          const float o = ste_one<DT>(tv, dv);
          const uint32_t ob = DT == DT_BF16 ? (uint32_t)f32_to_bf16_bits(o) : (uint32_t)__half_as_ushort(f32_to_f16(o));
          r |= ob << (16 * h);
        }
        ow[w] = r;
      }
    }
    out[i] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
}

// any alignment: one element per step
template <int DT>
__global__ void __launch_bounds__(256) ste_value_elem_kernel(const void* t, const void* dq, void* out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    store_elem(out, DT, i, ste_one<DT>(load_elem(t, DT, i), load_elem(dq, DT, i)));
}

template <int DT>
static void launch_ste(const void* t, const void* dq, void* out, int64_t n, hipStream_t st) {
  const int esz = DT == DT_F32 ? 4 : 2;
  const int64_t per_vec = 16 / esz;
  const bool vec = aligned(t, 16) && aligned(dq, 16) && aligned(out, 16);
  int64_t done = 0;
  if (vec && n >= per_vec) {
    const int64_t nvec = n / per_vec;
    ste_value_vec_kernel<DT><<<grid_for(nvec, 256), 256, 0, st>>>(
        reinterpret_cast<const uint4*>(t), reinterpret_cast<const uint4*>(dq), reinterpret_cast<uint4*>(out), nvec);
    done = nvec * per_vec;
  }
  if (done < n) {
    const int64_t off = done * esz;
    ste_value_elem_kernel<DT><<<grid_for(n - done, 256), 256, 0, st>>>(
        static_cast<const char*>(t) + off, static_cast<const char*>(dq) + off, static_cast<char*>(out) + off,
        n - done);
  }
}

}  // namespace ntlb

using namespace ntlb;

extern "C" int ntlb_ste_value(int dtype, const void* t, const void* t_dq, void* out, int64_t n, void* stream) {
  const char* fn = "ntlb_ste_value";
  if (!valid_dtype(dtype)) return fail(NTLB_EINVAL, "%s: bad dtype %d", fn, dtype);
  if (n < 0) return fail(NTLB_EINVAL, "%s: negative element count", fn);
  if (n == 0) return NTLB_OK;
  if (!t || !t_dq || !out) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  hipStream_t st = as_stream(stream);
  if (dtype == NTLB_BF16)
    launch_ste<DT_BF16>(t, t_dq, out, n, st);
  else if (dtype == NTLB_F16)
    launch_ste<DT_F16>(t, t_dq, out, n, st);
  else
    launch_ste<DT_F32>(t, t_dq, out, n, st);
  return check_launch(fn);
}
