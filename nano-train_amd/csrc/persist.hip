// Persistent low-bit weights for gfx950: NF4 (src/layers.py:60-184) and
// MXFP4 (OCP MX v1.0 e2m1 + e8m0; no reference function), their refresh
// (quantize) and dequantize kernels, and the GEMM with the dequantization
// fused into the B-tile prologue on bf16 MFMA.
//
// NF4: one fp32 scale per run of `block` consecutive elements of the flat
// weight (block = K per output row for per_channel, numel for per_tensor, 64
// for the 64-element recipe): scale = amax, non-finite or <= 0 -> 1
// (layers.py:86-101); code = argmin_i |clamp(w/s, -1, 1) - cb_i| with the
// first minimum winning (layers.py:165-166); two codes per byte, the even
// element in the low nibble (layers.py:130-139).  Dequantized value:
// bf16/fp32 of cb[code] * scale (layers.py:172-184).
//
// MXFP4: 32-element blocks, shared scale X = 2^(floor(log2 amax) - 2) stored
// as e8m0 (exponent clamped to [-127, 127]; 0xFF = NaN when the block holds a
// NaN or inf), elements rounded to nearest even onto e2m1 with saturation.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "ntlb_device.h"
#include "ntlb_host.h"
#include "ntlb_quant8.h"
#include "ntlb_splitk.h"

#pragma clang fp contract(off)

namespace ntlb {

// the NF4 codebook (NTLB_NF4_CODEBOOK, ntlb_device.h)
__constant__ float kNF4[16] = NTLB_NF4_CODEBOOK;
// the same values as compile-time constants (folded into immediates)
constexpr float kNF4c[16] = NTLB_NF4_CODEBOOK;
__constant__ float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

enum LowFmt : int { FMT_NF4 = 0, FMT_MXFP4 = 1, FMT_FP8P = 2 };


// ---------------------------------------------------------------------------
// element codes
// ---------------------------------------------------------------------------
// NF4 index of c = clamp(w/s): the pair of codebook entries bracketing c
// decides (every other entry is farther by at least the codebook gap); ties
// go to the lower index; NaN gives 0 as torch.argmin does on an all-NaN row.
// The bracket comes from a four-level binary search over the ascending
// codebook (base = the number of entries 1..15 at or below c), each level's
// probe picked from compile-time constants by selects, so the lookup never
// indexes memory.  It replaced a linear scan of all 15 entries (four VALU
// instructions each); the two agree on every float in [-1, 1], on both
// infinities and on NaN (an exhaustive host comparison).
__device__ __forceinline__ uint32_t nf4_index(float c) {
  constexpr const float* cb = kNF4c;
  if (!(c == c)) return 0;
  float lo = cb[0], hi = cb[15];
  bool b;
  float t = cb[8];
  b = t <= c;
  const bool b3 = b;
  lo = b ? t : lo;
  hi = b ? hi : t;
  t = b3 ? cb[12] : cb[4];
  b = t <= c;
  const bool b2 = b;
  lo = b ? t : lo;
  hi = b ? hi : t;
  t = b3 ? (b2 ? cb[14] : cb[10]) : (b2 ? cb[6] : cb[2]);
  b = t <= c;
  const bool b1 = b;
  lo = b ? t : lo;
  hi = b ? hi : t;
  t = b3 ? (b2 ? (b1 ? cb[15] : cb[13]) : (b1 ? cb[11] : cb[9])) : (b2 ? (b1 ? cb[7] : cb[5]) : (b1 ? cb[3] : cb[1]));
  b = t <= c;
  lo = b ? t : lo;
  hi = b ? hi : t;
  const uint32_t base = (b3 ? 8u : 0u) | (b2 ? 4u : 0u) | (b1 ? 2u : 0u) | (b ? 1u : 0u);
  if (base >= 15) return 15;
  const float d0 = fabsf(c - lo);
  const float d1 = fabsf(c - hi);
  return (d1 < d0) ? base + 1 : base;
}

// e2m1 round to nearest even with saturation; the sign of v is kept
__device__ __forceinline__ uint32_t e2m1_code(float v) {
  const float a = fabsf(v);
  uint32_t c = (a > 0.25f) + (a >= 0.75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) + (a >= 3.5f) + (a > 5.0f);
  if (!(a == a)) c = 0;
  return c | ((__float_as_uint(v) >> 28) & 8u);
}

__device__ __forceinline__ float e2m1_value(uint32_t c) {
  const float v = kE2M1[c & 7u];
  return (c & 8u) ? -v : v;
}

// e8m0 shared exponent of a 32-element block from its amax bits
__device__ __forceinline__ uint32_t mx_scale_byte(uint32_t amax_bits) {
  if (amax_bits >= 0x7F800000u) return 0xFFu;  // NaN or inf in the block
  if (amax_bits == 0u) return 0u;               // 2^-127
  int e;
  const uint32_t ef = amax_bits >> 23;
  if (ef != 0) {
    e = (int)ef - 127;
  } else {  // subnormal amax: position of the top set mantissa bit
    e = -127 - (__builtin_clz(amax_bits) - 9);
  }
  e -= 2;
  e = e < -127 ? -127 : (e > 127 ? 127 : e);
  return (uint32_t)(e + 127);
}

// ---------------------------------------------------------------------------
// NF4 refresh: block amax (atomics on |w| bits), scales, codes
// ---------------------------------------------------------------------------
template <int IN_DT>
__global__ void __launch_bounds__(256) flat_block_amax_kernel(const void* w, int64_t n, int64_t block,
                                                              uint32_t* amax_bits) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  uint32_t m[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) m[i] = (e0 + i < n) ? abs_bits(load_elem(w, IN_DT, e0 + i)) : 0u;
  if (block % 512 == 0) {
    // a wave covers 512 consecutive elements inside one block
    uint32_t mm = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) mm = max(mm, m[i]);
    mm = wave_max_u32(mm);
    if ((threadIdx.x & 63) == 0 && e0 < n && mm) atomicMax(amax_bits + e0 / block, mm);
  } else if (block % 8 == 0) {
    uint32_t mm = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) mm = max(mm, m[i]);
    if (e0 < n && mm) atomicMax(amax_bits + e0 / block, mm);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (e0 + i < n && m[i]) atomicMax(amax_bits + (e0 + i) / block, m[i]);
  }
}

// scale = amax when finite and > 0, else 1 (layers.py:98-100)
__global__ void amax_to_scale_kernel(const uint32_t* amax_bits, int64_t nb, float* scales) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < nb) {
    const uint32_t b = amax_bits[i];
    const float a = __uint_as_float(b);
    scales[i] = (b < 0x7F800000u && a > 0.0f) ? a : 1.0f;
  }
}

template <int IN_DT>
__global__ void __launch_bounds__(256) nf4_quant_kernel(const void* w, int64_t n, int64_t block, const float* scales,
                                                        uint8_t* packed) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 >= n) return;
  uint32_t idx[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t e = e0 + i;
    if (e < n) {
      float c = load_elem(w, IN_DT, e) / scales[e / block];
      c = (c < -1.0f) ? -1.0f : c;
      c = (c > 1.0f) ? 1.0f : c;
      idx[i] = nf4_index(c);
    } else {
      idx[i] = 0;
    }
  }
  const int64_t nbytes = (n + 1) / 2;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t bidx = e0 / 2 + j;
    if (bidx < nbytes) packed[bidx] = (uint8_t)(idx[2 * j] | (idx[2 * j + 1] << 4));
  }
}

template <int FMT>
__global__ void __launch_bounds__(256) lowbit_dequant_kernel(const uint8_t* packed, const void* scales, int64_t n,
                                                             int64_t block, void* out, int out_dtype) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 >= n) return;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t e = e0 + i;
    if (e >= n) break;
    const uint32_t byte = packed[e >> 1];
    const uint32_t c = (e & 1) ? (byte >> 4) : (byte & 15u);
    float v;
    if constexpr (FMT == FMT_NF4) {
      v = kNF4[c] * reinterpret_cast<const float*>(scales)[e / block];
    } else {
      const uint32_t sb = reinterpret_cast<const uint8_t*>(scales)[e >> 5];
      v = (sb == 0xFFu) ? __uint_as_float(0x7FC00000u) : ldexpf(e2m1_value(c), (int)sb - 127);
    }
    store_elem(out, out_dtype, e, v);
  }
}

// The same dequantization, 16 consecutive weights per thread (e0 % 16 == 0)
// under one scale (the scale block is a multiple of 16; MXFP4's 32-element
// blocks always are): one 8- or 16-byte code load, the scale once, and
// 16-byte stores.  The 4-bit code values come from a 16-entry table in LDS
// (one entry per bank, so any mix of codes reads without conflicts).  Each
// value is computed as above -- codebook value times scale in fp32 (NF4),
// e2m1 value times 2^(e - 127) (MXFP4), e4m3 value times scale (FP8P) -- and
// rounded to the output dtype by the same functions, so the output is
// bit-identical to the element-wise kernels.  POW2: the block is 2^bshift
// elements (a shift finds the scale), else a 64-bit division.
template <int FMT, int OUT_DT, bool POW2>
__global__ void __launch_bounds__(256) dequant16_kernel(const uint8_t* codes, const void* scales, int64_t n16,
                                                        int64_t block, int bshift, void* out) {
  __shared__ float table[16];
  if (threadIdx.x < 16) {
    if constexpr (FMT == FMT_NF4) table[threadIdx.x] = kNF4[threadIdx.x];
    else table[threadIdx.x] = e2m1_value(threadIdx.x);
  }
  __syncthreads();
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= n16) return;
  const int64_t e0 = t * 16;
  float v[16];
  if constexpr (FMT == FMT_FP8P) {
    const uint4 q = *reinterpret_cast<const uint4*>(codes + e0);
    const float s = reinterpret_cast<const float*>(scales)[POW2 ? (e0 >> bshift) : (e0 / block)];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = e4m3_to_f32((w[i >> 2] >> (8 * (i & 3))) & 0xFFu) * s;
  } else {
    const uint2 q = *reinterpret_cast<const uint2*>(codes + (e0 >> 1));
    const uint32_t w[2] = {q.x, q.y};
    float s = 0.0f;
    int ex = 0;
    bool nan_block = false;
    if constexpr (FMT == FMT_NF4) {
      s = reinterpret_cast<const float*>(scales)[POW2 ? (e0 >> bshift) : (e0 / block)];
    } else {
      const uint32_t sb = reinterpret_cast<const uint8_t*>(scales)[e0 >> 5];
      nan_block = sb == 0xFFu;
      ex = (int)sb - 127;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float c = table[(w[i >> 3] >> (4 * (i & 7))) & 15u];
      if constexpr (FMT == FMT_NF4)
        v[i] = c * s;
      else
        v[i] = nan_block ? __uint_as_float(0x7FC00000u) : ldexpf(c, ex);
    }
  }
  if constexpr (OUT_DT == DT_F32) {
    float4* o = reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + e0);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
  } else {
    uint32_t h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (OUT_DT == DT_BF16) {
        h[j] = (uint32_t)f32_to_bf16_bits(v[2 * j]) | ((uint32_t)f32_to_bf16_bits(v[2 * j + 1]) << 16);
      } else {
        h[j] = (uint32_t)__half_as_ushort(f32_to_f16(v[2 * j])) |
               ((uint32_t)__half_as_ushort(f32_to_f16(v[2 * j + 1])) << 16);
      }
    }
    uint4* o = reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + e0);
    o[0] = make_uint4(h[0], h[1], h[2], h[3]);
    o[1] = make_uint4(h[4], h[5], h[6], h[7]);
  }
}

// MXFP4 refresh: 4 lanes (a DPP quad) per 32-element block
template <int IN_DT>
__global__ void __launch_bounds__(256) mxfp4_quant_kernel(const void* w, int64_t n, uint8_t* packed,
                                                          uint8_t* scales) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  float v[8];
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = (e0 + i < n) ? load_elem(w, IN_DT, e0 + i) : 0.0f;
    m = max(m, abs_bits(v[i]));
  }
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));
  if (e0 >= n) return;
  const uint32_t sb = mx_scale_byte(m);
  if ((threadIdx.x & 3) == 0) scales[e0 >> 5] = (uint8_t)sb;
  uint32_t c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = (sb == 0xFFu) ? 0u : e2m1_code(ldexpf(v[i], 127 - (int)sb));
  const int64_t nbytes = (n + 1) / 2;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t bidx = e0 / 2 + j;
    if (bidx < nbytes) packed[bidx] = (uint8_t)(c[2 * j] | (c[2 * j + 1] << 4));
  }
}

// ---------------------------------------------------------------------------
// Persistent FP8 (layers.py:104-127): scale = amax per block (a row for
// per_channel, everything for per_tensor), code = e4m3(clamp(w/s, +-448)),
// dequantized value = e4m3 value * scale.
// ---------------------------------------------------------------------------
template <int IN_DT>
__global__ void __launch_bounds__(256) fp8p_quant_kernel(const void* w, int64_t n, int64_t block, const float* scales,
                                                         uint8_t* codes) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 >= n) return;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t e = e0 + i;
    if (e >= n) break;
    float v = load_elem(w, IN_DT, e) / scales[e / block];
    v = (v < -448.0f) ? -448.0f : v;
    v = (v > 448.0f) ? 448.0f : v;
    codes[e] = (uint8_t)e4m3_rne(v);
  }
}

__global__ void __launch_bounds__(256) fp8p_dequant_kernel(const uint8_t* codes, const float* scales, int64_t n,
                                                           int64_t block, void* out, int out_dtype) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 >= n) return;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t e = e0 + i;
    if (e >= n) break;
    store_elem(out, out_dtype, e, e4m3_to_f32(codes[e]) * scales[e / block]);
  }
}

// Dequantize n weights: the 16-per-thread kernel when n, the scale block and
// the pointers allow it, else the element-wise kernel.
template <int FMT>
static void launch_dequant(const uint8_t* codes, const void* scales, int64_t n, int64_t block, void* out,
                           int out_dtype, hipStream_t st) {
  const bool vec = n % 16 == 0 && block % 16 == 0 && aligned(out, 16) && aligned(codes, FMT == FMT_FP8P ? 16 : 8) &&
                   cdiv(n / 16, 256) <= 0x7FFFFFFF;
  if (!vec) {
    if constexpr (FMT == FMT_FP8P)
      fp8p_dequant_kernel<<<(unsigned)cdiv(cdiv(n, 8), 256), 256, 0, st>>>(codes, reinterpret_cast<const float*>(
                                                                              scales), n, block, out, out_dtype);
    else
      lowbit_dequant_kernel<FMT><<<(unsigned)cdiv(cdiv(n, 8), 256), 256, 0, st>>>(codes, scales, n, block, out,
                                                                                   out_dtype);
    return;
  }
  const int64_t n16 = n / 16;
  const bool pow2 = (block & (block - 1)) == 0;
  const int bshift = pow2 ? __builtin_ctzll((unsigned long long)block) : 0;
  const dim3 grd((unsigned)cdiv(n16, 256)), blk(256);
  auto go = [&](auto outc) {
    constexpr int ODT = decltype(outc)::value;
    if (pow2)
      dequant16_kernel<FMT, ODT, true><<<grd, blk, 0, st>>>(codes, scales, n16, block, bshift, out);
    else
      dequant16_kernel<FMT, ODT, false><<<grd, blk, 0, st>>>(codes, scales, n16, block, bshift, out);
  };
  if (out_dtype == NTLB_BF16)
    go(std::integral_constant<int, DT_BF16>());
  else if (out_dtype == NTLB_F16)
    go(std::integral_constant<int, DT_F16>());
  else
    go(std::integral_constant<int, DT_F32>());
}

// ---------------------------------------------------------------------------
// AdamW step fused with the persistent low-bit refresh.
//
// One pass over a parameter: the PrecisionAdamW update of
// optimizer_runtime.py:68-116 on fp32 master, exp_avg and exp_avg_sq, the
// parameter copy in its own dtype, and -- for scale blocks of at most 2048
// elements -- the NF4 or persistent-FP8 codes and scales that
// refresh_persistent_lowbit_params (layers.py:353-407) would compute from
// that parameter copy.  The arithmetic is that of the reference's torch ops
// on the GPU, operation for operation: add with alpha is fma(alpha, b, a),
// addcmul is fma(value, t1*t2, self), addcdiv is fma(value, t1/t2, self), and
// division by a scalar multiplies by its float reciprocal.  The host turns the
// reference's Python-double scalars into the floats torch uses.
// ---------------------------------------------------------------------------
struct AdamArgs {
  float* mp;  // fp32 master
  const void* g;
  int g_dtype;
  float* m;
  float* v;
  void* p;  // optional parameter copy
  int p_dtype;
  int64_t n;
  float b1, omb1, b2, omb2, inv_bc2_sqrt, eps, decay, neg_step;
  int64_t block;  // power of two in [8, 2048]
  uint8_t* codes;
  float* scales;
};

enum RefreshFmt : int { REFRESH_NONE = 0, REFRESH_NF4 = 1, REFRESH_FP8 = 2 };

// NF4 indices (layers.py:156-169) or e4m3 codes of clamp(w/s, +-448)
// (layers.py:104-117) of 8 consecutive values w[0..8) at e0 with the scale s,
// stored at their place in codes (4 packed bytes, or 8 code bytes)
template <int RF>
__device__ __forceinline__ void quant8_store(const float (&w)[8], float s, int64_t e0, int64_t n, uint8_t* codes) {
  const bool full = e0 + 8 <= n;
  // w / s by the exact reciprocal sequence of the fp8 quantizers wherever
  // the scale allows it (fast_div_ok on s, which is the block amax or 1:
  // every quotient that can move a code, here |w/s| >= 2^-10 for e4m3 and
  // >= 0.039 for NF4, has a normal residual) and w is finite (a block with
  // an infinity or a NaN has scale 1, and inf * 1 - inf would give NaN where
  // the division gives inf), else by IEEE division: one division per 8
  // weights instead of 8 (the NF4 pass was bound by its VALU work)
  const bool fast = fast_div_ok<false>(__float_as_uint(s));
  const float rs = fast ? 1.0f / s : 1.0f;
  auto quot = [&](float x) {
    if (fast && __builtin_isfinite(x)) {
      const float y = x * rs;
      const float e = __builtin_fmaf(-y, s, x);
      return __builtin_copysignf(__builtin_fmaf(e, rs, y), x);
    }
    return x / s;
  };
  if constexpr (RF == REFRESH_NF4) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float c = quot(w[i]);
      c = (c < -1.0f) ? -1.0f : c;
      c = (c > 1.0f) ? 1.0f : c;
      word |= nf4_index(c) << (4 * i);
    }
    if (full) {
      *reinterpret_cast<uint32_t*>(codes + e0 / 2) = word;
    } else {
      const int64_t nbytes = (n + 1) / 2;
      for (int j = 0; j < 4; ++j)
        if (e0 / 2 + j < nbytes) codes[e0 / 2 + j] = (uint8_t)(word >> (8 * j));
    }
  } else {
    uint32_t c8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float c = quot(w[i]);
      c = (c < -448.0f) ? -448.0f : c;
      c = (c > 448.0f) ? 448.0f : c;
      c8[i] = e4m3_rne(c);
    }
    if (full) {
      *reinterpret_cast<uint2*>(codes + e0) = make_uint2(c8[0] | (c8[1] << 8) | (c8[2] << 16) | (c8[3] << 24),
                                                         c8[4] | (c8[5] << 8) | (c8[6] << 16) | (c8[7] << 24));
    } else {
      for (int i = 0; i < 8; ++i)
        if (e0 + i < n) codes[e0 + i] = (uint8_t)c8[i];
    }
  }
}

// Codes and scales of 8 consecutive values w[0..8) at e0 (thread tid of a
// 256-thread workgroup covering 2048 consecutive elements), for power-of-two
// scale blocks in [8, 2048]: the block amax is reduced over the block's
// block/8 threads (shuffles, then LDS across waves), scale = amax with
// _safe_scale (layers.py:86-101), then NF4 indices (layers.py:156-169) or
// e4m3 of clamp(w/s, +-448) (layers.py:104-117).  Every thread of the
// workgroup must call it (it may synchronize).
template <int RF>
__device__ __forceinline__ void refresh8(const float (&w)[8], uint32_t amax, int64_t e0, int64_t n, int64_t block,
                                         uint8_t* codes, float* scales, uint32_t* wave_amax, int tid) {
  const int lane = tid & 63, wave = tid >> 6;
  const int gthreads = (int)(block >> 3);
  for (int off = 1; off < gthreads && off < 64; off <<= 1) amax = max(amax, (uint32_t)__shfl_xor((int)amax, off));
  if (gthreads > 64) {
    if (lane == 0) wave_amax[wave] = amax;
    __syncthreads();
    const int wpg = gthreads >> 6;  // waves per block: 2 or 4
    const int w0 = (wave / wpg) * wpg;
    uint32_t mm = 0;
    for (int i = 0; i < wpg; ++i) mm = max(mm, wave_amax[w0 + i]);
    amax = mm;
  }
  if (e0 >= n) return;
  const float s = (amax < 0x7F800000u && amax != 0u) ? __uint_as_float(amax) : 1.0f;
  if ((tid & (gthreads - 1)) == 0) scales[e0 / block] = s;
  quant8_store<RF>(w, s, e0, n, codes);
}

// 8 consecutive values at e0 as fp32: one or two 16-byte loads when all 8 lie
// inside [0, n) (e0 % 8 == 0 keeps them aligned), else element by element
__device__ __forceinline__ void load8f(const void* p, int dtype, int64_t e0, int64_t n, float (&v)[8]) {
  if (e0 + 8 <= n) {
    if (dtype == DT_F32) {
      const float4 a = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + e0)[0];
      const float4 b = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + e0)[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      return;
    }
    const uint4 r = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + e0);
    const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (dtype == DT_BF16) {
        v[2 * i] = bf16_bits_to_f32(u[i] & 0xFFFFu);
        v[2 * i + 1] = bf16_bits_to_f32(u[i] >> 16);
      } else {
        v[2 * i] = __half2float(__ushort_as_half((unsigned short)(u[i] & 0xFFFFu)));
        v[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(u[i] >> 16)));
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (e0 + i < n) ? load_elem(p, dtype, e0 + i) : 0.0f;
}

__device__ __forceinline__ void store8f(float* p, int64_t e0, int64_t n, const float (&v)[8]) {
  if (e0 + 8 <= n) {
    reinterpret_cast<float4*>(p + e0)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p + e0)[1] = make_float4(v[4], v[5], v[6], v[7]);
    return;
  }
  for (int i = 0; i < 8; ++i)
    if (e0 + i < n) p[e0 + i] = v[i];
}

template <int RF>
__global__ void __launch_bounds__(256) adamw_refresh_kernel(AdamArgs a) {
#pragma clang fp contract(off)
  __shared__ uint32_t wave_amax[4];
  const int tid = threadIdx.x;
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + tid) * 8;
  float g[8], m[8], v[8], p[8], w[8];
  load8f(a.g, a.g_dtype, e0, a.n, g);
  load8f(a.m, DT_F32, e0, a.n, m);
  load8f(a.v, DT_F32, e0, a.n, v);
  load8f(a.mp, DT_F32, e0, a.n, p);
  uint32_t amax = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m[i] = m[i] * a.b1;                                  // exp_avg.mul_(beta1)
    m[i] = __builtin_fmaf(a.omb1, g[i], m[i]);           // .add_(grad, alpha=1-beta1)
    v[i] = v[i] * a.b2;                                  // exp_avg_sq.mul_(beta2)
    v[i] = __builtin_fmaf(a.omb2, g[i] * g[i], v[i]);    // .addcmul_(grad, grad, value=1-beta2)
    float d = __builtin_sqrtf(v[i]);                     // exp_avg_sq.sqrt()
    d = d * a.inv_bc2_sqrt;                              // .div_(bias_correction2 ** 0.5)
    d = d + a.eps;                                       // .add_(eps)
    p[i] = p[i] * a.decay;                               // main_param.mul_(1 - lr * weight_decay)
    p[i] = __builtin_fmaf(a.neg_step, m[i] / d, p[i]);   // .addcdiv_(exp_avg, denom, value=-step_size)
    w[i] = round_to_dtype(p[i], a.p_dtype);              // the tensor the refresh quantizes
    if (e0 + i < a.n) amax = max(amax, abs_bits(w[i]));  // NaN bits sort above every finite value
  }
  store8f(a.m, e0, a.n, m);
  store8f(a.v, e0, a.n, v);
  store8f(a.mp, e0, a.n, p);
  if (a.p) {  // param.data.copy_(main_param_f.to(param.dtype))
    if (a.p_dtype == DT_F32) {
      store8f(reinterpret_cast<float*>(a.p), e0, a.n, p);
    } else if (a.p_dtype == DT_BF16 && e0 + 8 <= a.n) {
      uint32_t u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        u[i] = (uint32_t)f32_to_bf16_bits(p[2 * i]) | ((uint32_t)f32_to_bf16_bits(p[2 * i + 1]) << 16);
      *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(a.p) + e0) = make_uint4(u[0], u[1], u[2], u[3]);
    } else {
      for (int i = 0; i < 8; ++i)
        if (e0 + i < a.n) store_elem(a.p, a.p_dtype, e0 + i, p[i]);
    }
  }
  if constexpr (RF != REFRESH_NONE) refresh8<RF>(w, amax, e0, a.n, a.block, a.codes, a.scales, wave_amax, tid);
}

// One-pass block quantizer of a flat tensor for power-of-two blocks in
// [8, 2048]: the persistent NF4 / FP8 quantization without the separate amax
// pass and its atomics.
// Two-pass persistent quantization for blocks the one-pass kernel does not
// take (a row of more than 2048 values for per_channel, or the whole tensor
// for per_tensor), over a 16-byte aligned flat tensor.  Pass 1: the block
// maxima; each workgroup takes 2048-element chunks blockIdx.x, +gridDim.x,
// and reduces a chunk over its four waves before one atomic (one block: the
// workgroup keeps its maximum over all its chunks and issues one atomic in
// all).  The wave-per-512-elements kernel above put every wave's atomic on
// the one address of a per_tensor scale: 1.4 ms at the c5 weight.
template <int IN_DT>
__global__ void __launch_bounds__(256) flat_amax_chunks_kernel(const void* w, int64_t n, int64_t block,
                                                               int64_t nchunks, uint32_t* amax_bits) {
  __shared__ uint32_t red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool one = n <= block;  // uniform
  uint32_t run = 0;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t e0 = c * 2048 + (int64_t)threadIdx.x * 8;
    float v[8];
    load8f(w, IN_DT, e0, n, v);
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (e0 + i < n) m = max(m, abs_bits(v[i]));
    if (one) {
      run = max(run, m);
      continue;
    }
    // block % 2048 == 0: the chunk lies inside block c*2048 / block
    m = wave_max_u32(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t mm = max(max(red[0], red[1]), max(red[2], red[3]));
      if (mm) atomicMax(amax_bits + (c * 2048) / block, mm);
    }
    __syncthreads();
  }
  if (one) {
    run = wave_max_u32(run);
    if (lane == 0) red[wave] = run;
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t mm = max(max(red[0], red[1]), max(red[2], red[3]));
      if (mm) atomicMax(amax_bits, mm);
    }
  }
}

// Pass 2: 8 consecutive values per thread (block % 8 == 0: one scale each)
template <int RF>
__global__ void __launch_bounds__(256) flat_quant8_kernel(const void* w, int w_dtype, int64_t n, int64_t block,
                                                          const float* scales, uint8_t* codes) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 >= n) return;
  float v[8];
  load8f(w, w_dtype, e0, n, v);
  quant8_store<RF>(v, scales[e0 / block], e0, n, codes);
}

template <int RF>
__global__ void __launch_bounds__(256) quant_blocks_onepass(const void* w_in, int w_dtype, int64_t n, int64_t block,
                                                            uint8_t* codes, float* scales) {
  __shared__ uint32_t wave_amax[4];
  const int tid = threadIdx.x;
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + tid) * 8;
  float w[8];
  load8f(w_in, w_dtype, e0, n, w);
  uint32_t amax = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (e0 + i < n) amax = max(amax, abs_bits(w[i]));
  refresh8<RF>(w, amax, e0, n, block, codes, scales, wave_amax, tid);
}

static bool onepass_block(int64_t block) { return block >= 8 && block <= 2048 && (block & (block - 1)) == 0; }

// ---------------------------------------------------------------------------
// Dequant-fused GEMM  Y[M,N] = X[M,K] (bf16) . deq(W)[N,K]^T, fp32 accumulate.
// 256x256 output tile, 8 waves of 128x64, K step 64 bf16 (128-byte rows, the
// same swizzled tile layout as the fp8 kernel).  X tiles move global -> LDS
// directly; each thread dequantizes 32 weights (16 packed bytes, or 32 e4m3
// bytes) of one B row per K step into bf16 in LDS.  The codes and the block
// scale of block kt+1 are fetched into registers in the middle of step kt-1
// and decoded into the idle stage during step kt, one 16-byte chunk per odd
// 16-row group, so the VALU work interleaves with the matrix cores.  The
// 4-bit formats decode through the 16 bf16 products value * scale, built once
// per step in registers and looked up with byte permutes (a codebook in LDS
// made the kernel LDS-bound); e4m3 decodes with the hardware convert.  The
// two stages are distinct LDS objects and the K loop is unrolled by two (see
// the fp8 kernel): the copies in flight never alias the fragment reads, so no
// read waits for them.
// MFMA: v_mfma_f32_16x16x32_bf16, B tile as the first operand so each lane
// holds four consecutive output columns.  bf16 rounding is the hardware RNE
// pack-convert (v_cvt_pk_bf16_f32), the same rounding as f32_to_bf16_bits.
// ---------------------------------------------------------------------------
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int FBM = 256, FBN = 256, FBK = 64;  // FBK in bf16 elements: 128 bytes per row
constexpr int FROW = 128;                       // bytes per tile row
constexpr int FT = 256 * FROW;                  // 32 KiB per operand tile
constexpr int F_EPI_ROWS = 32;
constexpr int F_EPI_PITCH = 64 * 4 + 16;
static_assert(F_EPI_ROWS * F_EPI_PITCH <= FT / 2, "epilogue slice exceeds half an operand tile");

// 16-lane fragment reads are bank-conflict free for 8- and 16-lane phases
// (the permutation of the fp8 GEMM)
__device__ __forceinline__ int fswz_perm(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int fswz(int r, int c) { return r * FROW + ((c ^ fswz_perm(r)) << 4); }

__device__ __forceinline__ v8i frag32(const uint8_t* tile, int row0, int lane) {
  const int r = row0 + (lane & 15);
  const int g = lane >> 4;
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + fswz(r, 2 * g));
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + fswz(r, 2 * g + 1));
  v8i f;
  f[0] = (int)lo.x; f[1] = (int)lo.y; f[2] = (int)lo.z; f[3] = (int)lo.w;
  f[4] = (int)hi.x; f[5] = (int)hi.y; f[6] = (int)hi.z; f[7] = (int)hi.w;
  return f;
}

// two K=32 bf16 MFMAs over a 32-byte-per-lane fragment pair (64 K values)
__device__ __forceinline__ v4f mma_bf16_64(const v8i& p, const v8i& q, v4f acc) {
  typedef int v4i_t __attribute__((ext_vector_type(4)));
  const v4i_t pl = {p[0], p[1], p[2], p[3]}, ph = {p[4], p[5], p[6], p[7]};
  const v4i_t ql = {q[0], q[1], q[2], q[3]}, qh = {q[4], q[5], q[6], q[7]};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, pl), __builtin_bit_cast(v8bf, ql), acc, 0, 0,
                                                0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ph), __builtin_bit_cast(v8bf, qh), acc, 0, 0,
                                                0);
  return acc;
}

struct FusedArgs {
  const uint16_t* x;  // bf16 [M, K], row stride ldx
  int64_t ldx;
  const uint8_t* w;   // codes of the flat [N, K] weight: packed nibbles (NF4, MXFP4) or e4m3 bytes (FP8P)
  const void* scales;  // NF4, FP8P: fp32 per block; MXFP4: e8m0 per 32
  int64_t block;       // NF4/FP8P block (divides K, multiple of 32) or 0 for one tensor scale
  int64_t M, N, K;
  void* y;
  int y_dtype;
  int64_t ldy;
  int vec_out;
  const void* bias;  // optional [N], added in fp32 before the output rounding
  int bias_dtype;
  // split-K tail (ntlb_splitk.h): workgroups at or past split_base take K
  // range (q % split_s) of tile split_base + q / split_s
  int split_base, split_s;
  float* ws;
  uint32_t* ws_count;
};

// Scales of one weight row: the scale of the 32 weights [k0, k0+32) is
// row[k0 / blk] (NF4 fp32 multiplier) or the e8m0 byte row[k0 / 32] (MXFP4,
// carried in the float's bits).  A tensor-wide NF4 scale is a row of one
// entry with blk past any K.  K < 2^31 keeps the division in 32 bits.
struct RowScales {
  const void* row;
  uint32_t blk;
};

template <int FMT>
__device__ __forceinline__ RowScales fused_row_scales(const FusedArgs& g, int64_t n) {
  RowScales r;
  if constexpr (FMT == FMT_NF4 || FMT == FMT_FP8P) {
    const float* sc = reinterpret_cast<const float*>(g.scales);
    r.row = g.block ? sc + n * (g.K / g.block) : sc;
    r.blk = g.block ? (uint32_t)g.block : 0x40000000u;
  } else {
    r.row = reinterpret_cast<const uint8_t*>(g.scales) + n * (g.K >> 5);
    r.blk = 32;
  }
  return r;
}

template <int FMT>
__device__ __forceinline__ float fused_scale(const RowScales& r, uint32_t k0) {
  if constexpr (FMT == FMT_NF4 || FMT == FMT_FP8P)
    return reinterpret_cast<const float*>(r.row)[k0 / r.blk];
  else
    return __uint_as_float((uint32_t)reinterpret_cast<const uint8_t*>(r.row)[k0 >> 5]);
}

// The raw codes of 32 weights: 16 packed bytes (4-bit formats) or 32 e4m3
// bytes (FP8P, second half in b)
struct Raw32 {
  uint4 a, b;
};

// e4m3 weights 8j..8j+7 of the 32 of tile row r, half h: layers.py:121-127,
// the code's value (hardware decode, exact for every code, NaN codes to NaN)
// times the scale in fp32, rounded to bf16
__device__ __forceinline__ void dequant8_fp8_to_lds(const Raw32& raw, float s, int j, uint8_t* tile, int r, int h) {
  const uint32_t words[8] = {raw.a.x, raw.a.y, raw.a.z, raw.a.w, raw.b.x, raw.b.y, raw.b.z, raw.b.w};
  uint32_t out[4];
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)words[2 * j + w], false);
    const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)words[2 * j + w], true);
    const v2bf p0 = {(__bf16)(lo[0] * s), (__bf16)(lo[1] * s)};
    const v2bf p1 = {(__bf16)(hi[0] * s), (__bf16)(hi[1] * s)};
    out[2 * w] = __builtin_bit_cast(uint32_t, p0);
    out[2 * w + 1] = __builtin_bit_cast(uint32_t, p1);
  }
  *reinterpret_cast<uint4*>(tile + fswz(r, h * 4 + j)) = make_uint4(out[0], out[1], out[2], out[3]);
}

// The 16 bf16 weight values an NF4 thread can meet in one K step (all 32 of
// its weights share one scale): codebook value times scale in fp32, then
// bf16 (layers.py:172-184), held as two byte tables -- lo[q] / hi[q] carry
// the low / high bytes of entries 4q..4q+3 -- so a code is looked up with
// byte permutes instead of a memory read per weight.
struct Lut16 {
  uint32_t lo[4], hi[4];
};

__device__ __forceinline__ Lut16 lut16_build(float s) {
  uint32_t p[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const v2bf t = {(__bf16)(kNF4c[2 * k] * s), (__bf16)(kNF4c[2 * k + 1] * s)};
    p[k] = __builtin_bit_cast(uint32_t, t);
  }
  Lut16 t;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    t.lo[q] = __builtin_amdgcn_perm(p[2 * q + 1], p[2 * q], 0x06040200u);
    t.hi[q] = __builtin_amdgcn_perm(p[2 * q + 1], p[2 * q], 0x07050301u);
  }
  return t;
}

// Low and high bytes of four entries: byte i of sel (0..7) indexes both
// halves of the table, byte i of half (i or 4 + i) then takes the entry from
// entries 0..7 or 8..15.
__device__ __forceinline__ void lut16_lookup(const Lut16& t, uint32_t sel, uint32_t half, uint32_t& lo,
                                             uint32_t& hi) {
  const uint32_t l0 = __builtin_amdgcn_perm(t.lo[1], t.lo[0], sel);
  const uint32_t l1 = __builtin_amdgcn_perm(t.lo[3], t.lo[2], sel);
  const uint32_t h0 = __builtin_amdgcn_perm(t.hi[1], t.hi[0], sel);
  const uint32_t h1 = __builtin_amdgcn_perm(t.hi[3], t.hi[2], sel);
  lo = __builtin_amdgcn_perm(l1, l0, half);
  hi = __builtin_amdgcn_perm(h1, h0, half);
}

// What a thread needs to decode its 32 weights of one K step: the byte
// tables (4-bit formats) or the scale (FP8P)
template <int FMT>
struct StepDecode {
  Lut16 t;
  float s;
  bool nan;
};

// MXFP4 takes no table: gfx950's v_cvt_scalef32_pk_bf16_fp4 turns two e2m1
// codes times the block's power of two into a bf16 pair in one instruction
// (exact: an e2m1 value times 2^(e-127) is a bf16 value, subnormal for the
// smallest e, or overflows to inf as the fp32 product does), so d.s holds
// 2^(e-127) as a float and d.nan marks the NaN scale byte 0xFF
template <int FMT>
__device__ __forceinline__ StepDecode<FMT> decode_begin(float s) {
  StepDecode<FMT> d;
  if constexpr (FMT == FMT_MXFP4) {
    const uint32_t e = __float_as_uint(s);
    d.s = __uint_as_float(e ? e << 23 : 0x00400000u);
    d.nan = e == 0xFFu;
  } else {
    d.s = s;
    if constexpr (FMT == FMT_NF4) d.t = lut16_build(s);
  }
  return d;
}

// weights 8j..8j+7 (4 packed bytes, low nibble first; or 8 e4m3 bytes) of
// the 32 of tile row r, half h, as one 16-byte LDS chunk
template <int FMT>
__device__ __forceinline__ void decode_chunk(const StepDecode<FMT>& d, const Raw32& rw, int j, uint8_t* tile, int r,
                                             int h) {
  if constexpr (FMT == FMT_FP8P) {
    dequant8_fp8_to_lds(rw, d.s, j, tile, r, h);
  } else if constexpr (FMT == FMT_MXFP4) {
    // byte b of the word holds weights 2b (low nibble) and 2b+1: the pair
    // the instruction returns in that order
    const uint32_t words[4] = {rw.a.x, rw.a.y, rw.a.z, rw.a.w};
    const uint32_t w = words[j];
    uint4 out = make_uint4(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, d.s, 0)),
                           __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, d.s, 1)),
                           __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, d.s, 2)),
                           __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, d.s, 3)));
    if (d.nan) out = make_uint4(0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u);
    *reinterpret_cast<uint4*>(tile + fswz(r, h * 4 + j)) = out;
  } else {
    const uint32_t words[4] = {rw.a.x, rw.a.y, rw.a.z, rw.a.w};
    const uint32_t w = words[j];
    uint32_t le, he, lo_, ho;
    // weights 0, 2, 4, 6 are the low nibbles, 1, 3, 5, 7 the high ones; bit 3
    // of a nibble picks the table half
    lut16_lookup(d.t, w & 0x07070707u, ((w >> 1) & 0x04040404u) | 0x03020100u, le, he);
    lut16_lookup(d.t, (w >> 4) & 0x07070707u, ((w >> 5) & 0x04040404u) | 0x03020100u, lo_, ho);
    const uint32_t l03 = __builtin_amdgcn_perm(lo_, le, 0x05010400u);  // low bytes of weights 0..3
    const uint32_t h03 = __builtin_amdgcn_perm(ho, he, 0x05010400u);
    const uint32_t l47 = __builtin_amdgcn_perm(lo_, le, 0x07030602u);
    const uint32_t h47 = __builtin_amdgcn_perm(ho, he, 0x07030602u);
    *reinterpret_cast<uint4*>(tile + fswz(r, h * 4 + j)) =
        make_uint4(__builtin_amdgcn_perm(h03, l03, 0x05010400u), __builtin_amdgcn_perm(h03, l03, 0x07030602u),
                   __builtin_amdgcn_perm(h47, l47, 0x05010400u), __builtin_amdgcn_perm(h47, l47, 0x07030602u));
  }
}

template <int FMT>
__global__ void __launch_bounds__(512, 1) gemm_lowbit_fused_kernel(FusedArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t fx0[FT];
  __shared__ __attribute__((aligned(16))) uint8_t fw0[FT];
  __shared__ __attribute__((aligned(16))) uint8_t fx1[FT];
  __shared__ __attribute__((aligned(16))) uint8_t fw1[FT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int num_n = (int)((g.N + FBN - 1) / FBN);
  const int num_m = (int)((g.M + FBM - 1) / FBM);
  // the whole-wave tiles are renumbered so each XCD walks a contiguous range;
  // the split tail's ranges keep their tile
  const SplitWork sw = split_work(blockIdx.x, g.split_base, g.split_s);
  int pid = sw.pid;
  if (sw.tail < 0) {
    const int nwg = g.split_s > 1 ? g.split_base : num_m * num_n;
    const int xcd = pid & 7, local = pid >> 3;
    const int per = nwg >> 3, extra = nwg & 7;
    pid = xcd * per + min(xcd, extra) + local;
  }
  constexpr int GROUP_M = 4;
  const int group = pid / (GROUP_M * num_n);
  const int first_m = group * GROUP_M;
  const int gsize = min(num_m - first_m, GROUP_M);
  const int in_group = pid - group * GROUP_M * num_n;
  const int64_t m0 = (int64_t)(first_m + in_group % gsize) * FBM;
  const int64_t n0 = (int64_t)(in_group / gsize) * FBN;


  // X tile: direct-to-LDS; wave w moves the 8-row groups w, w+8, w+16, w+24
  // (bit 3 of its rows is w & 1, so its lanes' swizzled chunks are the same
  // for all four groups); rows past M read zero
  __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)g.x, (short)0, (int)(g.M * g.ldx * 2), 0x00020000);
  const int xr = wave * 8 + (lane >> 3);
  const uint32_t x_off = (uint32_t)(((m0 + xr) * g.ldx) * 2 + (((lane & 7) ^ fswz_perm(xr)) * 16));
  const uint32_t x_grp = (uint32_t)(64 * g.ldx * 2);
  auto issue_x = [&](uint8_t* stage, int kt, int j) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(stage + (wave + 8 * j) * 8 * FROW), 16, x_off,
                                             (uint32_t)kt * FROW + j * x_grp, 0, 0);
  };
  // W: thread t dequantizes row t/2, half t%2 (32 weights = 16 packed bytes,
  // or 32 e4m3 bytes)
  constexpr bool BYTE_CODES = FMT == FMT_FP8P;
  const int br = tid >> 1, bh = tid & 1;
  const int64_t bn = min<int64_t>(n0 + br, g.N - 1);
  const uint8_t* wrow = BYTE_CODES ? g.w + bn * g.K + bh * 32 : g.w + bn * (g.K >> 1) + bh * 16;
  const RowScales wsc = fused_row_scales<FMT>(g, bn);

  const int nk = (int)(g.K / FBK);
  // K blocks [kb0, kb1) of this workgroup: all of them, or one split range
  const int kb0 = sw.tail >= 0 ? (int)((int64_t)sw.chunk * nk / g.split_s) : 0;
  const int kb1 = sw.tail >= 0 ? (int)((int64_t)(sw.chunk + 1) * nk / g.split_s) : nk;
  // the epilogue's arguments, kept in scalar registers through the K loop
  uintptr_t e_y = reinterpret_cast<uintptr_t>(g.y), e_bias = reinterpret_cast<uintptr_t>(g.bias);
  int64_t e_ldy = g.ldy, e_M = g.M, e_N = g.N;
  int e_f32 = g.y_dtype == DT_F32, e_vec = g.vec_out, e_bdt = g.bias_dtype;
  e_y = uniform64(e_y); e_ldy = uniform64(e_ldy); e_M = uniform64(e_M); e_N = uniform64(e_N);
  e_bias = uniform64(e_bias);
  e_f32 = __builtin_amdgcn_readfirstlane(e_f32); e_vec = __builtin_amdgcn_readfirstlane(e_vec);
  e_bdt = __builtin_amdgcn_readfirstlane(e_bdt);
  asm volatile("" : "+s"(e_y), "+s"(e_ldy), "+s"(e_M), "+s"(e_N), "+s"(e_f32), "+s"(e_vec));
  asm volatile("" : "+s"(e_bias), "+s"(e_bdt));
  v4f acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int j = 0; j < 4; ++j) issue_x(fx0, kb0, j);
  // packed weight bytes and scale of block kt+1 travel in registers during
  // step kt-1 and step kt: they are loaded at the middle of step kt-1, after
  // that step's X copies, and may stay in flight across its closing barrier.
  // Register set kt & 1 holds block kt+2 (written by step kt, read by step
  // kt+1), so with the K loop unrolled by two no set is copied.
  auto w_load = [&](int kb, Raw32& raw, float& sc) {
    if constexpr (BYTE_CODES) {
      raw.a = *reinterpret_cast<const uint4*>(wrow + (int64_t)kb * FBK);
      raw.b = *reinterpret_cast<const uint4*>(wrow + (int64_t)kb * FBK + 16);
    } else {
      raw.a = *reinterpret_cast<const uint4*>(wrow + (int64_t)kb * (FBK / 2));
    }
    sc = fused_scale<FMT>(wsc, (uint32_t)(kb * FBK + bh * 32));
  };
  Raw32 raw_pf0, raw_pf1;
  float sc_pf0, sc_pf1;
  {
    Raw32 raw0;
    float s0;
    w_load(kb0, raw0, s0);
    const StepDecode<FMT> d0 = decode_begin<FMT>(s0);
#pragma unroll
    for (int j = 0; j < 4; ++j) decode_chunk<FMT>(d0, raw0, j, fw0, br, bh);
  }
  w_load(min(kb0 + 1, kb1 - 1), raw_pf1, sc_pf1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  auto step = [&](auto bufc, int kt) {
    constexpr int BUF = decltype(bufc)::value;
    const uint8_t* ta = BUF ? fx1 : fx0;
    const uint8_t* tb = BUF ? fw1 : fw0;
    uint8_t* xa_next = BUF ? fx0 : fx1;
    uint8_t* wb_next = BUF ? fw0 : fw1;
    // unconditional copies of block kn (the last step reloads itself into
    // the idle stage) keep the step one basic block
    const int kn = min(kt + 1, kb1 - 1);

    StepDecode<FMT> dec;
    v8i bf[4];
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) bf[tn] = frag32(tb, wn * 64 + tn * 16, lane);
    v8i af = frag32(ta, wm * 128, lane);
#pragma unroll
    for (int tm = 0; tm < 8; ++tm) {
      v8i af_next;
      if (tm + 1 < 8) af_next = frag32(ta, wm * 128 + (tm + 1) * 16, lane);
      if (tm < 4) issue_x(xa_next, kn, tm);
      Raw32& r = BUF ? raw_pf0 : raw_pf1;
      float& s = BUF ? sc_pf0 : sc_pf1;
      // block kn's codes (loaded during the previous step) become visible to
      // the compiler at tm == 0; their decode is spread over the step, one
      // 16-byte chunk per odd tm, so it interleaves with the matrix-core work
      // instead of stalling it in one burst
      if (tm == 0) {
        asm volatile("" : "+v"(r.a.x), "+v"(r.a.y), "+v"(r.a.z), "+v"(r.a.w), "+v"(s));
        if constexpr (BYTE_CODES) asm volatile("" : "+v"(r.b.x), "+v"(r.b.y), "+v"(r.b.z), "+v"(r.b.w));
        dec = decode_begin<FMT>(s);
      }
      if (tm & 1) decode_chunk<FMT>(dec, r, tm >> 1, wb_next, br, bh);
      // block kn+1's loads go out after this step's X copies, as the last
      // vector-memory operations of the step
      if (tm == 4) w_load(min(kt + 2, kb1 - 1), BUF ? raw_pf1 : raw_pf0, BUF ? sc_pf1 : sc_pf0);
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) acc[tm][tn] = mma_bf16_64(bf[tn], af, acc[tm][tn]);
      if constexpr (FMT == FMT_MXFP4) {
        // the short hardware decode interleaved with the group's MFMAs, three
        // VALU instructions after each (MXFP4 1278-1291 -> 1309-1321 TFLOP/s
        // at c5; the same schedule left NF4 unchanged and slowed FP8P by 3%)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        }
      }
      asm volatile("" : "+v"(acc[tm][0]), "+v"(acc[tm][1]), "+v"(acc[tm][2]), "+v"(acc[tm][3])::"memory");
      if (tm + 1 < 8) af = af_next;
    }
    // vmcnt(1) lgkmcnt(0): vector loads complete in issue order, so every X
    // copy of this step has landed while the last weight load may still be
    // in flight; the dequant's LDS writes are done
    __builtin_amdgcn_s_waitcnt(0x0071);
    __syncthreads();
  };

  for (int kt = kb0; kt < kb1; kt += 2) {
    step(std::integral_constant<int, 0>(), kt);
    if (kt + 1 < kb1) step(std::integral_constant<int, 1>(), kt + 1);
  }
  // a split range publishes its partial; the last to arrive sums them in
  // range order and stores the tile
  if (sw.tail >= 0 && !split_exchange(acc, g.ws, g.ws_count, sw.tail, g.split_s, sw.chunk, tid)) return;

  // the tile origin and lane pass through an empty asm so that no epilogue
  // address arithmetic is hoisted above the K loop, where every register is
  // taken
  int64_t m0e = uniform64(m0), n0e = uniform64(n0);
  int lane_e = lane;
  asm volatile("" : "+s"(m0e), "+s"(n0e), "+v"(lane_e));
  // epilogue: each wave stages 32 rows of its 128x64 tile at a time in a
  // 16 KiB slice of the idle operand tiles; 16-byte row-contiguous stores.
  // One straight-line body per output dtype, interior tiles without bounds
  // checks, and the arguments it needs held in scalar registers from before
  // the K loop (re-loading them after it costs scalar-cache misses).
  const int slab = wave >> 1;
  uint8_t* stage_w = (slab == 0 ? fx0 : slab == 1 ? fw0 : slab == 2 ? fx1 : fw1) + (wave & 1) * (FT / 2);
  // bias of this lane's 16 output columns (4 per 16-column block), in fp32
  if (e_bias) {
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = min<int64_t>(n0e + wn * 64 + tn * 16 + (lane_e >> 4) * 4 + i, e_N - 1);
        const float b = load_elem(reinterpret_cast<const void*>(e_bias), e_bdt, n);
#pragma unroll
        for (int tm = 0; tm < 8; ++tm) acc[tm][tn][i] = acc[tm][tn][i] + b;
      }
    }
  }
  auto store_tile = [&](auto f32c, auto fullc) {
    constexpr bool OUT_F32 = decltype(f32c)::value;
    constexpr bool FULL = decltype(fullc)::value;
    constexpr int pitch = OUT_F32 ? F_EPI_PITCH : (64 * 2 + 16);
    constexpr int esz = OUT_F32 ? 4 : 2;
    constexpr int cpr = OUT_F32 ? 16 : 8;
    constexpr int epc = 16 / esz;
#pragma unroll
    for (int part = 0; part < 4; ++part) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int tm = part * 2 + t;
        const int rloc = t * 16 + (lane_e & 15);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
          const v4f v = acc[tm][tn];
          uint8_t* dst = stage_w + rloc * pitch + (tn * 16 + (lane_e >> 4) * 4) * esz;
          if constexpr (OUT_F32) {
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
          } else {
            const v2bf p0 = {(__bf16)v[0], (__bf16)v[1]}, p1 = {(__bf16)v[2], (__bf16)v[3]};
            *reinterpret_cast<uint2*>(dst) =
                make_uint2(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1));
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's slice is written
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < cpr / 2; ++j) {
        const int q = lane_e + 64 * j;
        const int row = q / cpr, c = q % cpr;
        const int64_t m = m0e + wm * 128 + part * F_EPI_ROWS + row;
        const int64_t n = n0e + wn * 64 + c * epc;
        const uint8_t* src = stage_w + row * pitch + c * 16;
        uint8_t* ydst = reinterpret_cast<uint8_t*>(e_y) + (m * e_ldy + n) * esz;
        if constexpr (FULL) {
          store16_nt(ydst, src);
          continue;
        }
        if (m >= e_M || n >= e_N) continue;
        if (e_vec && n + epc <= e_N) {
          store16_nt(ydst, src);
        } else {
          using E = std::conditional_t<esz == 4, uint32_t, uint16_t>;
#pragma nounroll
          for (int e = 0; e < epc && n + e < e_N; ++e)
            reinterpret_cast<E*>(ydst)[e] = reinterpret_cast<const E*>(src)[e];
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // the re-reads are done before the next part overwrites
      __builtin_amdgcn_wave_barrier();
    }
  };
  const bool full = e_vec && m0e + FBM <= e_M && n0e + FBN <= e_N;
  if (e_f32) {
    if (full)
      store_tile(std::true_type(), std::true_type());
    else
      store_tile(std::true_type(), std::false_type());
  } else {
    if (full)
      store_tile(std::false_type(), std::true_type());
    else
      store_tile(std::false_type(), std::false_type());
  }
}

}  // namespace ntlb

using namespace ntlb;

// the two vectorized passes, when the tensor and its blocks allow them
template <int RF>
static bool flat_two_pass(const void* w, int w_dtype, int64_t n, int64_t block, uint32_t* amax_ws, uint8_t* codes,
                          float* scales, hipStream_t st) {
  if (!aligned(w, 16) || block % 8 != 0 || !(n <= block || block % 2048 == 0)) return false;
  const int64_t nb = cdiv(n, block);
  const int64_t nchunks = cdiv(n, 2048);
  const unsigned ga = (unsigned)std::min<int64_t>(nchunks, 2048);
  if (w_dtype == NTLB_BF16)
    flat_amax_chunks_kernel<DT_BF16><<<ga, 256, 0, st>>>(w, n, block, nchunks, amax_ws);
  else if (w_dtype == NTLB_F32)
    flat_amax_chunks_kernel<DT_F32><<<ga, 256, 0, st>>>(w, n, block, nchunks, amax_ws);
  else
    flat_amax_chunks_kernel<DT_F16><<<ga, 256, 0, st>>>(w, n, block, nchunks, amax_ws);
  amax_to_scale_kernel<<<(unsigned)cdiv(nb, 256), 256, 0, st>>>(amax_ws, nb, scales);
  flat_quant8_kernel<RF><<<(unsigned)cdiv(cdiv(n, 8), 256), 256, 0, st>>>(w, w_dtype, n, block, scales, codes);
  return true;
}

extern "C" int ntlb_nf4_quant(const void* w, int w_dtype, int64_t n, int64_t block, uint32_t* amax_ws,
                              uint8_t* packed, float* scales, void* stream) {
  const char* fn = "ntlb_nf4_quant";
  if (!valid_dtype(w_dtype)) return fail(NTLB_EINVAL, "%s: bad dtype", fn);
  if (n < 0 || block < 1) return fail(NTLB_EINVAL, "%s: bad size or block", fn);
  if (n == 0) return NTLB_OK;
  if (!w || !amax_ws || !packed || !scales) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (onepass_block(block) && aligned(w, 16)) {
    if (cdiv(cdiv(n, 8), 256) > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too large", fn);
    quant_blocks_onepass<REFRESH_NF4><<<(unsigned)cdiv(cdiv(n, 8), 256), 256, 0, as_stream(stream)>>>(
        w, w_dtype, n, block, packed, scales);
    return check_launch(fn);
  }
  const int64_t nb = cdiv(n, block);
  const int64_t threads = cdiv(n, 8);
  if (cdiv(threads, 256) > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too large", fn);
  hipStream_t st = as_stream(stream);
  if (flat_two_pass<REFRESH_NF4>(w, w_dtype, n, block, amax_ws, packed, scales, st)) return check_launch(fn);
  dim3 grd((unsigned)cdiv(threads, 256)), blk(256);
  if (w_dtype == NTLB_BF16)
    flat_block_amax_kernel<DT_BF16><<<grd, blk, 0, st>>>(w, n, block, amax_ws);
  else if (w_dtype == NTLB_F32)
    flat_block_amax_kernel<DT_F32><<<grd, blk, 0, st>>>(w, n, block, amax_ws);
  else
    flat_block_amax_kernel<DT_F16><<<grd, blk, 0, st>>>(w, n, block, amax_ws);
  amax_to_scale_kernel<<<(unsigned)cdiv(nb, 256), 256, 0, st>>>(amax_ws, nb, scales);
  if (w_dtype == NTLB_BF16)
    nf4_quant_kernel<DT_BF16><<<grd, blk, 0, st>>>(w, n, block, scales, packed);
  else if (w_dtype == NTLB_F32)
    nf4_quant_kernel<DT_F32><<<grd, blk, 0, st>>>(w, n, block, scales, packed);
  else
    nf4_quant_kernel<DT_F16><<<grd, blk, 0, st>>>(w, n, block, scales, packed);
  return check_launch(fn);
}

extern "C" int ntlb_nf4_dequant(const uint8_t* packed, const float* scales, int64_t n, int64_t block, void* out,
                                int out_dtype, void* stream) {
  const char* fn = "ntlb_nf4_dequant";
  if (!valid_dtype(out_dtype) || n < 0 || block < 1) return fail(NTLB_EINVAL, "%s: bad argument", fn);
  if (n == 0) return NTLB_OK;
  if (!packed || !scales || !out) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  launch_dequant<FMT_NF4>(packed, scales, n, block, out, out_dtype, as_stream(stream));
  return check_launch(fn);
}

extern "C" int ntlb_mxfp4_quant(const void* w, int w_dtype, int64_t n, uint8_t* packed, uint8_t* scales,
                                void* stream) {
  const char* fn = "ntlb_mxfp4_quant";
  if (!valid_dtype(w_dtype) || n < 0) return fail(NTLB_EINVAL, "%s: bad argument", fn);
  if (n == 0) return NTLB_OK;
  if (!w || !packed || !scales) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  dim3 grd((unsigned)cdiv(cdiv(n, 8), 256)), blk(256);
  hipStream_t st = as_stream(stream);
  if (w_dtype == NTLB_BF16)
    mxfp4_quant_kernel<DT_BF16><<<grd, blk, 0, st>>>(w, n, packed, scales);
  else if (w_dtype == NTLB_F32)
    mxfp4_quant_kernel<DT_F32><<<grd, blk, 0, st>>>(w, n, packed, scales);
  else
    mxfp4_quant_kernel<DT_F16><<<grd, blk, 0, st>>>(w, n, packed, scales);
  return check_launch(fn);
}

extern "C" int ntlb_mxfp4_dequant(const uint8_t* packed, const uint8_t* scales, int64_t n, void* out, int out_dtype,
                                  void* stream) {
  const char* fn = "ntlb_mxfp4_dequant";
  if (!valid_dtype(out_dtype) || n < 0) return fail(NTLB_EINVAL, "%s: bad argument", fn);
  if (n == 0) return NTLB_OK;
  if (!packed || !scales || !out) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  launch_dequant<FMT_MXFP4>(packed, scales, n, 32, out, out_dtype, as_stream(stream));
  return check_launch(fn);
}

// the split-K tail's minimum K blocks (64 bf16 each) per range
constexpr int FUSED_SPLIT_MIN_BLOCKS = 9;

static int fused_launch(int fmt, const char* fn, const void* x, int64_t ldx, const uint8_t* w, const void* scales,
                        int64_t block, const void* bias, int bias_dtype, int64_t M, int64_t N, int64_t K, void* y,
                        int y_dtype, int64_t ldy, void* workspace, int64_t ws_bytes, void* stream) {
  if (M < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (M == 0 || N == 0) return NTLB_OK;
  if (!x || !w || !scales || !y) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (K % FBK) return fail(NTLB_EUNSUPPORTED, "%s: K must be a multiple of %d", fn, FBK);
  if (ldx < K || (ldx % 8) || !aligned(x, 16) || !aligned(w, 16))
    return fail(NTLB_EINVAL, "%s: x needs ldx >= K, ldx %% 8 == 0, 16-byte alignment; w 16-byte alignment", fn);
  if (!(y_dtype == NTLB_BF16 || y_dtype == NTLB_F32) || ldy < N)
    return fail(NTLB_EINVAL, "%s: output must be bf16 or fp32 with ldy >= N", fn);
  if (fmt != FMT_MXFP4 && block != 0 && (K % block || block % 32))
    return fail(NTLB_EUNSUPPORTED, "%s: the scale block must divide K and be a multiple of 32 (or 0 = tensor)", fn);
  if ((M + FBM) * ldx * 2 >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: X exceeds 2 GiB", fn);
  if (bias && !valid_dtype(bias_dtype)) return fail(NTLB_EINVAL, "%s: bad bias dtype", fn);
  const int64_t tiles = ((M + FBM - 1) / FBM) * ((N + FBN - 1) / FBN);
  if (tiles > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  FusedArgs g;
  g.x = reinterpret_cast<const uint16_t*>(x); g.ldx = ldx; g.w = w; g.scales = scales; g.block = block;
  g.M = M; g.N = N; g.K = K; g.y = y; g.y_dtype = y_dtype; g.ldy = ldy;
  g.vec_out = aligned(y, 16) && ((ldy * dtype_size(y_dtype)) % 16 == 0);
  g.bias = bias; g.bias_dtype = bias_dtype;
  g.split_base = (int)tiles; g.split_s = 1; g.ws = nullptr; g.ws_count = nullptr;
  int64_t grid_wgs = tiles;
  if (workspace) {
    if (!aligned(workspace, 256)) return fail(NTLB_EINVAL, "%s: workspace must be 256-byte aligned", fn);
    const SplitPlan plan = split_plan(tiles, (int)(K / FBK), FUSED_SPLIT_MIN_BLOCKS);
    if (plan.s > 1 && ws_bytes >= split_ws_bytes(plan)) {
      g.split_base = plan.base; g.split_s = plan.s;
      g.ws_count = reinterpret_cast<uint32_t*>(workspace);
      g.ws = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + split_count_bytes());
      grid_wgs = (int64_t)plan.base + (int64_t)plan.tail * plan.s;
    }
  }
  dim3 grd((unsigned)grid_wgs), blk(512);
  if (fmt == FMT_NF4)
    gemm_lowbit_fused_kernel<FMT_NF4><<<grd, blk, 0, as_stream(stream)>>>(g);
  else if (fmt == FMT_MXFP4)
    gemm_lowbit_fused_kernel<FMT_MXFP4><<<grd, blk, 0, as_stream(stream)>>>(g);
  else
    gemm_lowbit_fused_kernel<FMT_FP8P><<<grd, blk, 0, as_stream(stream)>>>(g);
  return check_launch(fn);
}

extern "C" int ntlb_gemm_nf4(const void* x, int64_t ldx, const uint8_t* w_packed, const float* w_scales,
                             int64_t block, int64_t M, int64_t N, int64_t K, void* y, int y_dtype, int64_t ldy,
                             void* stream) {
  return fused_launch(FMT_NF4, "ntlb_gemm_nf4", x, ldx, w_packed, w_scales, block, nullptr, 0, M, N, K, y, y_dtype,
                      ldy, nullptr, 0, stream);
}

extern "C" int ntlb_gemm_fp8p(const void* x, int64_t ldx, const uint8_t* w_codes, const float* w_scales,
                              int64_t block, int64_t M, int64_t N, int64_t K, void* y, int y_dtype, int64_t ldy,
                              void* stream) {
  return fused_launch(FMT_FP8P, "ntlb_gemm_fp8p", x, ldx, w_codes, w_scales, block, nullptr, 0, M, N, K, y,
                      y_dtype, ldy, nullptr, 0, stream);
}

extern "C" int ntlb_gemm_mxfp4(const void* x, int64_t ldx, const uint8_t* w_packed, const uint8_t* w_scales,
                               int64_t M, int64_t N, int64_t K, void* y, int y_dtype, int64_t ldy, void* stream) {
  if (K % 32) return fail(NTLB_EUNSUPPORTED, "ntlb_gemm_mxfp4: K must be a multiple of 32");
  return fused_launch(FMT_MXFP4, "ntlb_gemm_mxfp4", x, ldx, w_packed, w_scales, 32, nullptr, 0, M, N, K, y,
                      y_dtype, ldy, nullptr, 0, stream);
}

extern "C" int64_t ntlb_gemm_lowbit_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % FBK) return 0;
  const int64_t tiles = ((M + FBM - 1) / FBM) * ((N + FBN - 1) / FBN);
  if (tiles > 0x7FFFFFFF) return 0;
  return split_ws_bytes(split_plan(tiles, (int)(K / FBK), FUSED_SPLIT_MIN_BLOCKS));
}

extern "C" int ntlb_gemm_lowbit_ws(int fmt, const void* x, int64_t ldx, const uint8_t* w, const void* w_scales,
                                   int64_t block, const void* bias, int bias_dtype, int64_t M, int64_t N, int64_t K,
                                   void* y, int y_dtype, int64_t ldy, void* workspace, int64_t ws_bytes,
                                   void* stream) {
  const char* fn = "ntlb_gemm_lowbit_ws";
  if (fmt == NTLB_LOWBIT_MXFP4) {
    if (K % 32) return fail(NTLB_EUNSUPPORTED, "%s: MXFP4 needs K %% 32 == 0", fn);
    return fused_launch(FMT_MXFP4, fn, x, ldx, w, w_scales, 32, bias, bias_dtype, M, N, K, y, y_dtype, ldy,
                        workspace, ws_bytes, stream);
  }
  if (fmt != NTLB_LOWBIT_NF4 && fmt != NTLB_LOWBIT_FP8P) return fail(NTLB_EINVAL, "%s: bad format %d", fn, fmt);
  return fused_launch(fmt == NTLB_LOWBIT_NF4 ? FMT_NF4 : FMT_FP8P, fn, x, ldx, w, w_scales, block, bias, bias_dtype,
                      M, N, K, y, y_dtype, ldy, workspace, ws_bytes, stream);
}

extern "C" int ntlb_fp8_persistent_quant(const void* w, int w_dtype, int64_t n, int64_t block, uint32_t* amax_ws,
                                         uint8_t* codes, float* scales, void* stream) {
  const char* fn = "ntlb_fp8_persistent_quant";
  if (!valid_dtype(w_dtype) || n < 0 || block < 1) return fail(NTLB_EINVAL, "%s: bad argument", fn);
  if (n == 0) return NTLB_OK;
  if (!w || !amax_ws || !codes || !scales) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (onepass_block(block) && aligned(w, 16)) {
    if (cdiv(cdiv(n, 8), 256) > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too large", fn);
    quant_blocks_onepass<REFRESH_FP8><<<(unsigned)cdiv(cdiv(n, 8), 256), 256, 0, as_stream(stream)>>>(
        w, w_dtype, n, block, codes, scales);
    return check_launch(fn);
  }
  const int64_t nb = cdiv(n, block);
  if (cdiv(cdiv(n, 8), 256) > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too large", fn);
  dim3 grd((unsigned)cdiv(cdiv(n, 8), 256)), blk(256);
  hipStream_t st = as_stream(stream);
  if (flat_two_pass<REFRESH_FP8>(w, w_dtype, n, block, amax_ws, codes, scales, st)) return check_launch(fn);
  if (w_dtype == NTLB_BF16)
    flat_block_amax_kernel<DT_BF16><<<grd, blk, 0, st>>>(w, n, block, amax_ws);
  else if (w_dtype == NTLB_F32)
    flat_block_amax_kernel<DT_F32><<<grd, blk, 0, st>>>(w, n, block, amax_ws);
  else
    flat_block_amax_kernel<DT_F16><<<grd, blk, 0, st>>>(w, n, block, amax_ws);
  amax_to_scale_kernel<<<(unsigned)cdiv(nb, 256), 256, 0, st>>>(amax_ws, nb, scales);
  if (w_dtype == NTLB_BF16)
    fp8p_quant_kernel<DT_BF16><<<grd, blk, 0, st>>>(w, n, block, scales, codes);
  else if (w_dtype == NTLB_F32)
    fp8p_quant_kernel<DT_F32><<<grd, blk, 0, st>>>(w, n, block, scales, codes);
  else
    fp8p_quant_kernel<DT_F16><<<grd, blk, 0, st>>>(w, n, block, scales, codes);
  return check_launch(fn);
}

extern "C" int ntlb_fp8_persistent_dequant(const uint8_t* codes, const float* scales, int64_t n, int64_t block,
                                           void* out, int out_dtype, void* stream) {
  const char* fn = "ntlb_fp8_persistent_dequant";
  if (!valid_dtype(out_dtype) || n < 0 || block < 1) return fail(NTLB_EINVAL, "%s: bad argument", fn);
  if (n == 0) return NTLB_OK;
  if (!codes || !scales || !out) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  launch_dequant<FMT_FP8P>(codes, scales, n, block, out, out_dtype, as_stream(stream));
  return check_launch(fn);
}

extern "C" int ntlb_adamw_step_refresh(float* main_param, const void* grad, int grad_dtype, float* exp_avg,
                                       float* exp_avg_sq, void* param, int param_dtype, int64_t n, float beta1,
                                       float one_minus_beta1, float beta2, float one_minus_beta2, float inv_bc2_sqrt,
                                       float eps, float decay, float neg_step_size, int refresh, int64_t block,
                                       uint8_t* codes, float* scales, void* stream) {
  const char* fn = "ntlb_adamw_step_refresh";
  if (n < 0) return fail(NTLB_EINVAL, "%s: negative size", fn);
  if (!valid_dtype(grad_dtype) || (param && !valid_dtype(param_dtype)))
    return fail(NTLB_EINVAL, "%s: bad grad or param dtype", fn);
  if (refresh != REFRESH_NONE && refresh != REFRESH_NF4 && refresh != REFRESH_FP8)
    return fail(NTLB_EINVAL, "%s: bad refresh format %d", fn, refresh);
  if (refresh != REFRESH_NONE) {
    if (block < 8 || block > 2048 || (block & (block - 1)))
      return fail(NTLB_EUNSUPPORTED, "%s: fused refresh needs a power-of-two block in [8, 2048]", fn);
    if (!codes || !scales) return fail(NTLB_EINVAL, "%s: NULL codes or scales", fn);
  }
  if (n == 0) return NTLB_OK;
  if (!main_param || !grad || !exp_avg || !exp_avg_sq) return fail(NTLB_EINVAL, "%s: NULL state", fn);
  if (cdiv(cdiv(n, 8), 256) > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too large", fn);
  AdamArgs a;
  a.mp = main_param; a.g = grad; a.g_dtype = grad_dtype; a.m = exp_avg; a.v = exp_avg_sq;
  a.p = param; a.p_dtype = param ? param_dtype : NTLB_F32; a.n = n;
  a.b1 = beta1; a.omb1 = one_minus_beta1; a.b2 = beta2; a.omb2 = one_minus_beta2; a.inv_bc2_sqrt = inv_bc2_sqrt;
  a.eps = eps; a.decay = decay; a.neg_step = neg_step_size;
  a.block = refresh != REFRESH_NONE ? block : 8;
  a.codes = codes; a.scales = scales;
  dim3 grd((unsigned)cdiv(cdiv(n, 8), 256)), blk(256);
  hipStream_t st = as_stream(stream);
  if (refresh == REFRESH_NF4)
    adamw_refresh_kernel<REFRESH_NF4><<<grd, blk, 0, st>>>(a);
  else if (refresh == REFRESH_FP8)
    adamw_refresh_kernel<REFRESH_FP8><<<grd, blk, 0, st>>>(a);
  else
    adamw_refresh_kernel<REFRESH_NONE><<<grd, blk, 0, st>>>(a);
  return check_launch(fn);
}
