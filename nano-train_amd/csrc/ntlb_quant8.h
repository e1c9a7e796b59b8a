// Shared 8-element quantization helpers of the low-bit kernels: the Philox
// stochastic-rounding words, the per-element reference path, and the fast
// tile path (exact reciprocal division, hardware e4m3 convert).  Used by the
// quantizers and by GEMM epilogues that quantize their output.  Every fp32
// operation here rounds on its own (no contraction), as the reference's torch
// ops do.
#pragma once

#include "ntlb_device.h"

namespace ntlb {

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
// v_pk_max_u16 on two packed halves
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}

// The 8 SR words for source elements e0 .. e0+7.
template <bool SR>
__device__ __forceinline__ void sr_words(uint64_t e0, uint64_t seed, uint64_t offset, uint32_t (&rb)[8]) {
  if constexpr (SR) {
    if ((e0 & 3u) == 0) {
      Philox4 p0 = philox4x32_10(e0 >> 2, offset, seed);
      Philox4 p1 = philox4x32_10((e0 >> 2) + 1, offset, seed);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rb[i] = p0.v[i];
        rb[4 + i] = p1.v[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint64_t e = e0 + i;
        Philox4 p = philox4x32_10(e >> 2, offset, seed);
        uint32_t j = (uint32_t)(e & 3u);
        rb[i] = j == 0 ? p.v[0] : (j == 1 ? p.v[1] : (j == 2 ? p.v[2] : p.v[3]));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) rb[i] = 0;
  }
}

// Quantize N (8 or 4) values with one scale; returns the codes packed in two
// words (hi is 0 for N = 4) and whether any q was NaN.  Writes dq when
// requested.
template <int GRID, bool SR, int N>
__device__ __forceinline__ bool quant8(const float (&v)[N], float s, float qmaxf, const uint32_t (&rb)[N],
                                       uint32_t& lo, uint32_t& hi, float (&q)[N]) {
#pragma clang fp contract(off)
  static_assert(N == 8 || N == 4, "8 or 4 values");
  uint32_t c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  bool nan = false;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    c[i] = quant_one<GRID, SR>(v[i], s, qmaxf, rb[i], q[i]);
    nan |= (__float_as_uint(q[i]) & 0x7FFFFFFFu) > 0x7F800000u;
  }
  lo = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
  hi = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
  return nan;
}

// Quantize 8 values of a tile with scale s whose amax bits are m.  A tile
// holding a NaN takes the per-element reference path (and reports it); every
// other tile clamps with min/max, divides with the fast exact sequence when
// its amax allows, and rounds to e4m3 in hardware under round to nearest.
//
// The fast sequence y = x*r, e = fma(-y, s, x), q = fma(e, r, y) with
// r = RN(1/s) equals RN(x/s) for every pair of fp32 significands (all 2^46
// pairs checked on the CPU by tests/cpu/division_check.c) as long as no
// intermediate underflows or overflows.  Round to nearest takes it for amax bits in
// [0x1A000000, 0x7B800000] (2^-75 .. 2^120): there every quotient that can
// move a code (|x/s| >= 2^-11) has a normal residual.  Stochastic rounding
// needs the quotient exactly wherever v + u can round differently, down to
// |x/s| = 2^-34 (e4m3 subnormals: 512*v + u), so it takes the sequence for
// amax bits in [0x30000000, 0x7B800000] (2^-31 .. 2^120), where those
// residuals are normal; smaller quotients stay below 2^-34 either way.
template <bool SR>
__device__ __forceinline__ bool fast_div_ok(uint32_t m) {
  return m >= (SR ? 0x30000000u : 0x1A000000u) && m <= 0x7B800000u;
}

// The codes (and, with DQ, the values q as the reference holds them) of N
// quotients x/s already clamped to [-qmax, qmax]: the int grid rounds them
// (to nearest, or stochastically with the bits rb), e4m3 converts them in
// hardware.
template <int GRID, bool SR, bool DQ, int N>
__device__ __forceinline__ void codes_from_quotients(const float (&vq)[N], const uint32_t (&rb)[N], float qmaxf,
                                                     uint32_t& lo, uint32_t& hi, float (&q)[N]) {
#pragma clang fp contract(off)
  if constexpr (GRID == GRID_INT) {
    uint32_t c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < N; ++i) {
      float t;
      if constexpr (SR) {
        // floor(v + u) for v >= 0 and ceil(v - u) = -floor(|v| + u) below
        // (round to nearest is symmetric), so one floor, negated for
        // v < 0 (te_backend.py:61-65); v = -0 counts as v >= 0 there and
        // gives +0, so the sign comes from the comparison, not from v.
        // The reference clamps after rounding (:102-106): at the clamp,
        // qmax + u rounds to qmax + 1 in fp32 when u >= 1 - 2^-18
        const float uu = sr_uniform(rb[i]);
        const float w = __builtin_floorf(__builtin_fabsf(vq[i]) + uu);
        t = vq[i] >= 0.0f ? w : -w;
        t = __builtin_amdgcn_fmed3f(t, -qmaxf, qmaxf);
      } else {
        t = __builtin_rintf(vq[i]);
      }
      q[i] = t;
      c[i] = (uint32_t)(int32_t)t & 0xFFu;
    }
    lo = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
    hi = N == 8 ? (c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24)) : 0u;
  } else {
    uint32_t c[8];
    hi = 0;
    if constexpr (!SR) {
      lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(vq[0], vq[1], 0, false);
      lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(vq[2], vq[3], (int)lo, true);
      if constexpr (N == 8) {
        hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(vq[4 % N], vq[5 % N], 0, false);
        hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(vq[6 % N], vq[7 % N], (int)hi, true);
      }
    } else {
      // the hardware stochastic convert, whose rounding is e4m3_sr's (the
      // clamped quotients are finite and at most 448)
      lo = (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(vq[0], (int)rb[0], 0, 0);
      lo = (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(vq[1], (int)rb[1], (int)lo, 1);
      lo = (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(vq[2], (int)rb[2], (int)lo, 2);
      lo = (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(vq[3], (int)rb[3], (int)lo, 3);
      if constexpr (N == 8) {
        hi = (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(vq[4 % N], (int)rb[4 % N], 0, 0);
        hi = (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(vq[5 % N], (int)rb[5 % N], (int)hi, 1);
        hi = (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(vq[6 % N], (int)rb[6 % N], (int)hi, 2);
        hi = (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(vq[7 % N], (int)rb[7 % N], (int)hi, 3);
      }
    }
    c[0] = lo & 0xFF; c[1] = (lo >> 8) & 0xFF; c[2] = (lo >> 16) & 0xFF; c[3] = lo >> 24;
    c[4] = hi & 0xFF; c[5] = (hi >> 8) & 0xFF; c[6] = (hi >> 16) & 0xFF; c[7] = hi >> 24;
    if constexpr (DQ) {
#pragma unroll
      for (int i = 0; i < N; ++i) q[i] = e4m3_to_f32(c[i]);
    }
  }
}

// rs is 1/s (IEEE, correctly rounded) wherever fast_div_ok(m) holds; it is
// not read otherwise.
template <int GRID, bool SR, bool DQ, int N>
__device__ __forceinline__ bool quant8_tile_rs(const float (&v)[N], uint32_t m, float s, float rs, float qmaxf,
                                               const uint32_t (&rb)[N], uint32_t& lo, uint32_t& hi, float (&q)[N]) {
#pragma clang fp contract(off)
  static_assert(N == 8 || N == 4, "8 or 4 values");
  if (m > 0x7F800000u || !(s > 0.0f)) {
    // NaN in the tile, or a scale that underflowed to zero (the rule that
    // divides the amax after checking it: x / 0 is NaN or +-inf): reference
    // semantics element by element
    quant8<GRID, SR>(v, s, qmaxf, rb, lo, hi, q);
    return true;
  } else {
    float vq[N];
    // x/s by the fast sequence (with the sign of x, so that -0 and signed
    // tiny quotients keep their sign) where fast_div_ok holds, else by IEEE
    // division.  No NaN reaches the clamp here (NaN tiles took the path
    // above; x/s is finite or +-inf), so the single-instruction median is
    // the clamp
    if (fast_div_ok<SR>(m)) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const float y = v[i] * rs;
        const float e = __builtin_fmaf(-y, s, v[i]);
        float z = __builtin_copysignf(__builtin_fmaf(e, rs, y), v[i]);
        vq[i] = __builtin_amdgcn_fmed3f(z, -qmaxf, qmaxf);
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        float z = v[i] / s;
        vq[i] = __builtin_amdgcn_fmed3f(z, -qmaxf, qmaxf);
      }
    }
    codes_from_quotients<GRID, SR, DQ, N>(vq, rb, qmaxf, lo, hi, q);
  }
  return false;
}

// Eight values with a scale each (s[i], from amax bits that all pass
// fast_div_ok, rs[i] = 1/s[i] correctly rounded): the fast exact division of
// quant8_tile_rs element by element.  The amax bits exclude NaN and
// infinity, so no NaN reaches the clamp.
template <int GRID, bool SR, bool DQ>
__device__ __forceinline__ void quant8_cols_rs(const float (&v)[8], const float (&s)[8], const float (&rs)[8],
                                               float qmaxf, const uint32_t (&rb)[8], uint32_t& lo, uint32_t& hi,
                                               float (&q)[8]) {
#pragma clang fp contract(off)
  float vq[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y = v[i] * rs[i];
    const float e = __builtin_fmaf(-y, s[i], v[i]);
    const float z = __builtin_copysignf(__builtin_fmaf(e, rs[i], y), v[i]);
    vq[i] = __builtin_amdgcn_fmed3f(z, -qmaxf, qmaxf);
  }
  codes_from_quotients<GRID, SR, DQ, 8>(vq, rb, qmaxf, lo, hi, q);
}

template <int GRID, bool SR, bool DQ>
__device__ __forceinline__ bool quant8_tile(const float (&v)[8], uint32_t m, float s, float qmaxf,
                                            const uint32_t (&rb)[8], uint32_t& lo, uint32_t& hi, float (&q)[8]) {
#pragma clang fp contract(off)
  const float rs = fast_div_ok<SR>(m) ? 1.0f / s : 1.0f;
  return quant8_tile_rs<GRID, SR, DQ>(v, m, s, rs, qmaxf, rb, lo, hi, q);
}

}  // namespace ntlb
