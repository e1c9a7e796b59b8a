// Device helpers shared by the gfx950 kernels of the low-bit linear path.
//
// Numerics follow nano-train's emulated backend (src/runtime/te_backend.py)
// bit for bit: fp32 division x / s (correctly rounded: hipcc's default), round
// half to even (torch.round), NaN-propagating amax (torch.amax), the
// _safe_scale rule of te_backend.py:74-79, and the comm-quant rule of
// src/models/moe.py:94-98.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ntlb {

enum Grid : int { GRID_INT = 0, GRID_E4M3 = 1 };
enum Rounding : int { ROUND_NEAREST = 0, ROUND_STOCHASTIC = 1 };
enum ScaleRule : int { SCALE_AFTER_DIVIDE = 0, SCALE_BEFORE_DIVIDE = 1 };
enum DType : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

// the 16 NF4 code values of src/layers.py:60-83, as fp32
#define NTLB_NF4_CODEBOOK                                                                                          \
  {-1.0f,       -0.6961928f, -0.52507305f, -0.3949175f, -0.28444138f, -0.18477343f, -0.09105004f, 0.0f,         \
   0.0795803f,  0.1609302f,  0.2461123f,   0.33791524f, 0.44070983f,  0.562617f,    0.72295684f,  1.0f}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

// 8 bytes (two words) stored with the non-temporal hint
__device__ __forceinline__ void store8_nt(void* dst, uint32_t lo, uint32_t hi) {
  typedef unsigned int u32x2_nt __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(1))) u32x2_nt* global_u32x2_nt;
  const u32x2_nt v = {lo, hi};
  __builtin_nontemporal_store(v, (global_u32x2_nt)dst);
}

// 16 bytes stored with the non-temporal hint (a vector store with the nt
// bit), for GEMM outputs that the kernel never reads back.  Measured at the
// c2 shape: the GEMM runs 4-5% faster with its read traffic unchanged, and
// the quantizers launched after it no longer slow down behind its output
// (X 1x128: 41 -> 32 us, W 128x128: 80 -> 70 us).
__device__ __forceinline__ void store16_nt(void* dst, const void* src) {
  typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(1))) u32x4_nt* global_u32x4_nt;
  __builtin_nontemporal_store(*reinterpret_cast<const u32x4_nt*>(src), (global_u32x4_nt)dst);
}

// a 64-bit value that is the same in every lane, as a scalar (lets values
// the compiler cannot prove uniform be pinned in scalar registers)
template <typename T>
__device__ __forceinline__ T uniform64(T v) {
  const uint64_t u = (uint64_t)v;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
  return (T)(((uint64_t)hi << 32) | lo);
}

// fp32 -> bf16 round to nearest even; NaN stays NaN (quiet bit set).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  // a select, not an early return: inside unrolled loops a per-element branch
  // turns into exec-mask control flow around every conversion
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x40u;
  return (uint16_t)(((u & 0x7FFFFFFFu) > 0x7F800000u) ? qnan : rne);
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon et al., SC'11).  The stochastic-rounding contract:
// element e of a call keyed (seed, offset) uses word e%4 of
// Philox(counter = {lo(e/4), hi(e/4), lo(offset), hi(offset)}, key = seed).
// ---------------------------------------------------------------------------
struct Philox4 {
  uint32_t v[4];
};

__device__ __forceinline__ Philox4 philox4x32_10(uint64_t group, uint64_t offset, uint64_t seed) {
  uint32_t c0 = (uint32_t)group, c1 = (uint32_t)(group >> 32);
  uint32_t c2 = (uint32_t)offset, c3 = (uint32_t)(offset >> 32);
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    // three-input xor in one v_bitop3_b32 (truth table 0x96), where two
    // v_xor_b32 would otherwise follow every product
    c0 = __builtin_amdgcn_bitop3_b32(hi1, c1, k0, 0x96);
    c1 = lo1;
    c2 = __builtin_amdgcn_bitop3_b32(hi0, c3, k1, 0x96);
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  Philox4 o;
  o.v[0] = c0;
  o.v[1] = c1;
  o.v[2] = c2;
  o.v[3] = c3;
  return o;
}

__device__ __forceinline__ float sr_uniform(uint32_t r) {
#pragma clang fp contract(off)
  return (float)(r >> 8) * 0x1p-24f;
}

// ---------------------------------------------------------------------------
// e4m3fn (OCP) encode / decode, bit-exact with torch's float8_e4m3fn cast on
// the clamped range the quantizers use.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t e4m3_rne(float v) {
#pragma clang fp contract(off)
  uint32_t bits = __float_as_uint(v);
  uint32_t sign = (bits >> 24) & 0x80u;
  uint32_t ab = bits & 0x7FFFFFFFu;
  float a = __uint_as_float(ab);
  uint32_t code;
  if (ab > 0x7F800000u || a > 464.0f) {
    code = 0x7Fu;
  } else if (a < 0x1p-6f) {
    code = (uint32_t)__builtin_rintf(a * 512.0f);  // multiples of 2^-9; 8 == min normal
  } else {
    uint32_t r = ab + 0x7FFFFu + ((ab >> 20) & 1u);  // RNE at the 3rd mantissa bit
    code = (r >> 20) - (120u << 3);                  // rebias exponent 127 -> 7
  }
  return sign | code;
}

// Stochastic rounding onto the e4m3 grid (the e4m3 counterpart of the
// te_backend.py:61-65 rule): the 20 bits of |v| just below its e4m3 spacing
// (truncated) plus the top 20 bits of the Philox word r carry into the code,
// i.e. |v| rounds away from zero iff frac20 + (r >> 12) >= 2^20, sign kept.
// This is the rounding of gfx950's v_cvt_sr_fp8_f32, which the tile paths use
// (tests/hip/fp8_sr_cvt_probe.hip compares the two over every fp32 |v| <=
// 448).  |v| <= 448 on entry (the callers clamp first); there frac20 is 0 at
// 448, so no draw rounds past the largest finite code.
__device__ __forceinline__ uint32_t e4m3_sr(float v, uint32_t r) {
  const uint32_t bits = __float_as_uint(v);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t ab = bits & 0x7FFFFFFFu;
  if (ab > 0x7F800000u) return sign | 0x7Fu;
  if (ab >= 0x43E00000u) return sign | 0x7Eu;  // >= 448
  const uint32_t e8 = ab >> 23;
  uint32_t trunc, f20;
  if (e8 >= 121u) {  // |v| >= 2^-6: 3 mantissa bits, then 20
    trunc = ((e8 - 120u) << 3) + ((ab >> 20) & 7u);
    f20 = ab & 0xFFFFFu;
  } else {  // subnormal e4m3 (spacing 2^-9): |v| * 512 = m >> sh, fp32 denormals as exponent 1
    const uint32_t m = (ab & 0x7FFFFFu) | (e8 ? 0x800000u : 0u);
    const uint32_t sh = 141u - (e8 ? e8 : 1u);  // 21 .. 140
    trunc = sh < 32u ? m >> sh : 0u;
    f20 = sh - 20u < 32u ? (m >> (sh - 20u)) & 0xFFFFFu : 0u;
  }
  return sign | min(trunc + ((f20 + (r >> 12)) >> 20), 0x7Eu);
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
#pragma clang fp contract(off)
  uint32_t ef = (c >> 3) & 0xFu, m = c & 7u;
  float v;
  if (ef == 0xFu && m == 7u) {
    v = __uint_as_float(0x7FC00000u);
  } else if (ef == 0u) {
    v = (float)m * 0x1p-9f;
  } else {
    v = __uint_as_float(((ef + 120u) << 23) | (m << 20));
  }
  return (c & 0x80u) ? -v : v;
}

// ---------------------------------------------------------------------------
// scales
// ---------------------------------------------------------------------------
// |x| bits for a NaN-propagating max: unsigned order of non-negative floats is
// their numeric order, and every NaN compares above +inf.
__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }

__device__ __forceinline__ float scale_from_amax_bits(uint32_t amax_bits, float qmaxf, int rule) {
#pragma clang fp contract(off)
  float amax = __uint_as_float(amax_bits);
  if (rule == SCALE_BEFORE_DIVIDE) {
    if (!(amax_bits < 0x7F800000u) || !(amax > 0.0f)) return 1.0f;
    return amax / qmaxf;
  }
  float s = amax / qmaxf;
  bool ok = (__float_as_uint(s) & 0x7FFFFFFFu) < 0x7F800000u && s > 0.0f;
  return ok ? s : 1.0f;
}

// ---------------------------------------------------------------------------
// one element: te_backend.py:101-106 (int grid) / the e4m3 recipe
// returns the code byte (low 8 bits) and writes q (as the reference holds it)
// ---------------------------------------------------------------------------
template <int GRID, bool SR>
__device__ __forceinline__ uint32_t quant_one(float x, float s, float qmaxf, uint32_t rbits, float& q) {
#pragma clang fp contract(off)
  float v = x / s;
  if constexpr (GRID == GRID_INT) {
    float t;
    if constexpr (SR) {
      float u = sr_uniform(rbits);
      t = (v >= 0.0f) ? __builtin_floorf(v + u) : __builtin_ceilf(v - u);
    } else {
      t = __builtin_rintf(v);
    }
    t = (t < -qmaxf) ? -qmaxf : t;
    t = (t > qmaxf) ? qmaxf : t;
    q = t;
    bool nan = (__float_as_uint(t) & 0x7FFFFFFFu) > 0x7F800000u;
    return nan ? 0x80u : ((uint32_t)(int32_t)t & 0xFFu);
  } else {
    v = (v < -448.0f) ? -448.0f : v;
    v = (v > 448.0f) ? 448.0f : v;
    uint32_t c;
    if constexpr (SR) {
      c = e4m3_sr(v, rbits);
    } else {
      c = e4m3_rne(v);
    }
    q = e4m3_to_f32(c);
    return c;
  }
}

// ---------------------------------------------------------------------------
// DPP reductions over the 16 lanes of a row
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  // quad xor 1, quad xor 2, half-row mirror, row mirror
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = row16_max_u32(v);
  // combine the four rows of the wave
  v = max(v, (uint32_t)__shfl_xor((int)v, 16));
  v = max(v, (uint32_t)__shfl_xor((int)v, 32));
  return v;
}

// v to f16 (round to nearest even) from the fp32 value as it stands.  The
// fence keeps the compiler from folding a preceding fp32 multiply or add into
// a mixed-precision instruction (v_fma_mixlo_f16), which rounds the exact
// result once instead of rounding to fp32 and then to f16 as fp32 arithmetic
// followed by a cast does: -38.078125 is an f16 tie only after the fp32
// rounding of the product that gives it.
__device__ __forceinline__ __half f32_to_f16(float v) {
  asm("" : "+v"(v));
  return __float2half(v);
}

__device__ __forceinline__ float load_elem(const void* p, int dtype, int64_t idx) {
  if (dtype == DT_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[idx]);
  if (dtype == DT_F16) return __half2float(((const __half*)p)[idx]);
  return ((const float*)p)[idx];
}

// v rounded to dtype (round to nearest even, as store_elem and torch's .to())
// and widened back to fp32
__device__ __forceinline__ float round_to_dtype(float v, int dtype) {
  if (dtype == DT_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (dtype == DT_F16) return __half2float(f32_to_f16(v));
  return v;
}

__device__ __forceinline__ void store_elem(void* p, int dtype, int64_t idx, float v) {
  if (dtype == DT_BF16) {
    ((uint16_t*)p)[idx] = f32_to_bf16_bits(v);
  } else if (dtype == DT_F16) {
    ((__half*)p)[idx] = f32_to_f16(v);
  } else {
    ((float*)p)[idx] = v;
  }
}

}  // namespace ntlb
