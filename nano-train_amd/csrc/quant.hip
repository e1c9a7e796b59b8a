// Quantizers of the low-bit linear path for gfx950.
//
//   tile 1x128    : te_backend.py:82-110      (activation tiles)
//   block 128x128 : te_backend.py:113-149     (weight blocks, + transposed codes)
//   grouped       : te_backend.py:165-185     (tensor / channel) and
//                   moe.py:123-140            (comm-quant strips)
//   128x1 (transposed output): the DeepSeek-V3 wgrad operands
//
// All of them are HBM-bound: each element is read once (bf16 or fp32) and
// written once as a code byte, plus one fp32 scale per group.  Loads are
// 16-byte vectors, one 128-element tile per 16 lanes (one DPP row), so the
// tile amax is a 4-step DPP reduction that never leaves the row.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "ntlb_device.h"
#include "ntlb_host.h"

// every fp32 operation rounds on its own, as the reference's torch ops do
#pragma clang fp contract(off)

namespace ntlb {

struct QuantArgs {
  const void* x;
  int64_t R, K, ldx;
  float qmaxf;
  int scale_rule;
  uint64_t seed, offset;
  uint8_t* codes;
  int64_t ldc;
  float* scales;
  int64_t s_row, s_col;
  void* dq;
  int dq_dtype;
  int64_t lddq;
  int32_t* nan_rows;
};

// Load 8 consecutive elements [k0, k0+8) of a row as fp32, zero past K.
template <int IN_DT, bool VEC>
__device__ __forceinline__ void load8(const void* base, int64_t row_off, int64_t k0, int64_t K, float (&v)[8]) {
  if (VEC && k0 + 8 <= K) {
    if constexpr (IN_DT == DT_BF16) {
      uint4 raw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + row_off + k0);
      uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      }
    } else if constexpr (IN_DT == DT_F32) {
      const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + row_off + k0);
      float4 a = p[0], b = p[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      const __half* p = reinterpret_cast<const __half*>(base) + row_off + k0;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = __half2float(p[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int64_t k = k0 + i;
      v[i] = (k < K) ? load_elem(base, IN_DT, row_off + k) : 0.0f;
    }
  }
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

// Quantize 8 values with one scale; returns the codes packed in two words
// and whether any q was NaN.  Writes dq when requested.
template <int GRID, bool SR>
__device__ __forceinline__ bool quant8(const float (&v)[8], float s, float qmaxf, const uint32_t (&rb)[8],
                                       uint32_t& lo, uint32_t& hi, float (&q)[8]) {
  uint32_t c[8];
  bool nan = false;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    c[i] = quant_one<GRID, SR>(v[i], s, qmaxf, rb[i], q[i]);
    nan |= (__float_as_uint(q[i]) & 0x7FFFFFFFu) > 0x7F800000u;
  }
  lo = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
  hi = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
  return nan;
}

__device__ __forceinline__ void store_dq8(void* dq, int dq_dtype, int64_t row_off, int64_t k0, int64_t K,
                                          const float (&q)[8], float s) {
  if (dq_dtype == DT_BF16 && k0 + 8 <= K && ((row_off + k0) & 7) == 0) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)f32_to_bf16_bits(q[2 * i] * s) | ((uint32_t)f32_to_bf16_bits(q[2 * i + 1] * s) << 16);
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(dq) + row_off + k0) = make_uint4(w[0], w[1], w[2], w[3]);
    return;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (k0 + i < K) store_elem(dq, dq_dtype, row_off + k0 + i, q[i] * s);
}

// ---------------------------------------------------------------------------
// 1x128 tiles: one tile per 16-lane DPP row, two tiles in flight per row.
// ---------------------------------------------------------------------------
template <int IN_DT, int GRID, bool SR, bool VEC>
__global__ void __launch_bounds__(256) quant_tile_1x128_kernel(QuantArgs a) {
  const int lane16 = threadIdx.x & 15;
  const int64_t T = (a.K + 127) >> 7;
  const int64_t n_tiles = a.R * T;
  const int64_t rows_per_grid = (int64_t)gridDim.x * 16;  // 16 DPP rows per workgroup
  int64_t slot = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  constexpr int U = 2;
  for (int64_t base = slot; base < n_tiles; base += rows_per_grid * U) {
    float v[U][8];
    int64_t tile[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      tile[u] = base + u * rows_per_grid;
      if (tile[u] < n_tiles) {
        int64_t r = tile[u] / T, t = tile[u] - r * T;
        load8<IN_DT, VEC>(a.x, r * a.ldx, t * 128 + lane16 * 8, a.K, v[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (tile[u] >= n_tiles) continue;  // uniform across the 16-lane row
      int64_t r = tile[u] / T, t = tile[u] - r * T;
      int64_t k0 = t * 128 + lane16 * 8;
      uint32_t m = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) m = max(m, abs_bits(v[u][i]));
      m = row16_max_u32(m);
      float s = scale_from_amax_bits(m, a.qmaxf, a.scale_rule);
      uint32_t rb[8];
      sr_words<SR>((uint64_t)(r * a.K + k0), a.seed, a.offset, rb);
      uint32_t lo, hi;
      float q[8];
      bool nan = quant8<GRID, SR>(v[u], s, a.qmaxf, rb, lo, hi, q);
      *reinterpret_cast<uint2*>(a.codes + r * a.ldc + k0) = make_uint2(lo, hi);
      if (lane16 == 0) a.scales[r * a.s_row + t * a.s_col] = s;
      if (a.dq) store_dq8(a.dq, a.dq_dtype, r * a.lddq, k0, a.K, q, s);
      if (nan && a.nan_rows) atomicOr(a.nan_rows + r, 1);
    }
  }
}

// ---------------------------------------------------------------------------
// 128x128 blocks: one workgroup per block, the block held in registers
// between the amax pass and the quantize pass (one HBM read).
// ---------------------------------------------------------------------------
struct BlockArgs {
  QuantArgs q;
  uint8_t* codes_t;
  int64_t ldct;
};

template <int IN_DT, int GRID, bool SR, bool VEC>
__global__ void __launch_bounds__(256) quant_block_128x128_kernel(BlockArgs ba) {
  const QuantArgs& a = ba.q;
  __shared__ uint32_t red[4];
  __shared__ uint8_t tile_t[128][128 + 4];
  const int tid = threadIdx.x;
  const int sub = tid & 15, rr = tid >> 4;
  const int64_t T = (a.K + 127) >> 7;
  const int64_t nb = blockIdx.x / T, kb = blockIdx.x - nb * T;
  const int64_t k0 = kb * 128 + sub * 8;
  float v[8][8];
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int64_t n = nb * 128 + rr + 16 * i;
    if (n < a.R) {
      load8<IN_DT, VEC>(a.x, n * a.ldx, k0, a.K, v[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) m = max(m, abs_bits(v[i][j]));
  }
  m = wave_max_u32(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = max(max(red[0], red[1]), max(red[2], red[3]));
  const float s = scale_from_amax_bits(m, a.qmaxf, a.scale_rule);
  if (tid == 0) a.scales[nb * a.s_row + kb * a.s_col] = s;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int64_t n = nb * 128 + rr + 16 * i;
    uint32_t rb[8];
    sr_words<SR>((uint64_t)(n * a.K + k0), a.seed, a.offset, rb);
    uint32_t lo, hi;
    float q[8];
    bool nan = quant8<GRID, SR>(v[i], s, a.qmaxf, rb, lo, hi, q);
    if (n < a.R) {
      *reinterpret_cast<uint2*>(a.codes + n * a.ldc + k0) = make_uint2(lo, hi);
      if (a.dq) store_dq8(a.dq, a.dq_dtype, n * a.lddq, k0, a.K, q, s);
      if (nan && a.nan_rows) atomicOr(a.nan_rows + n, 1);
    }
    if (ba.codes_t) {
      *reinterpret_cast<uint32_t*>(&tile_t[rr + 16 * i][sub * 8]) = lo;
      *reinterpret_cast<uint32_t*>(&tile_t[rr + 16 * i][sub * 8 + 4]) = hi;
    }
  }
  if (ba.codes_t) {
    __syncthreads();
    // transposed write: W^T row kr, 64 consecutive n per thread
    const int kr = tid >> 1, h = tid & 1;
    const int64_t krow = kb * 128 + kr;
    if (krow < a.K) {
      uint32_t w[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        int n0 = h * 64 + j * 4;
        w[j] = (uint32_t)tile_t[n0][kr] | ((uint32_t)tile_t[n0 + 1][kr] << 8) |
               ((uint32_t)tile_t[n0 + 2][kr] << 16) | ((uint32_t)tile_t[n0 + 3][kr] << 24);
      }
      uint4* dst = reinterpret_cast<uint4*>(ba.codes_t + krow * ba.ldct + nb * 128 + h * 64);
#pragma unroll
      for (int j = 0; j < 4; ++j) dst[j] = make_uint4(w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]);
    }
  }
}

// ---------------------------------------------------------------------------
// grouped amax (tensor / channel / strip) and quantization with group scales
// ---------------------------------------------------------------------------
template <int IN_DT>
__global__ void __launch_bounds__(256) amax_grouped_kernel(const void* x, int64_t R, int64_t K, int64_t ldx,
                                                           int64_t gr, int64_t gc, int64_t n_gc,
                                                           int64_t rows_per_block, uint32_t* amax_bits) {
  const int64_t kc = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;  // 8 columns per thread
  const int64_t r_begin = (int64_t)blockIdx.y * rows_per_block;
  const int64_t r_end = min(R, r_begin + rows_per_block);
  if (r_begin >= R) return;
  uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t cur_g = r_begin / gr;
  auto flush = [&](int64_t g) {
    if (kc >= K) return;
    if (gc == 1) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (kc + i < K && m[i]) atomicMax(amax_bits + g * n_gc + kc + i, m[i]);
    } else {
      // gc > 1: the 8 columns may straddle a group edge only if gc % 8 != 0
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (kc + i < K && m[i]) atomicMax(amax_bits + g * n_gc + (kc + i) / gc, m[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) m[i] = 0;
  };
  for (int64_t r = r_begin; r < r_end; ++r) {
    int64_t g = r / gr;
    if (g != cur_g) {
      flush(cur_g);
      cur_g = g;
    }
    if (kc < K) {
      float v[8];
      load8<IN_DT, false>(x, r * ldx, kc, K, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) m[i] = max(m[i], abs_bits(v[i]));
    }
  }
  if (gc > 1 && gc % 8 == 0) {
    // all 8 columns share one group: fold them first to cut atomics
    uint32_t mm = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) mm = max(mm, m[i]);
#pragma unroll
    for (int i = 0; i < 8; ++i) m[i] = (i == 0) ? mm : 0;
  }
  flush(cur_g);
}

__global__ void scales_from_amax_kernel(const uint32_t* amax_bits, int64_t n, float qmaxf, int rule,
                                        float* scales) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) scales[i] = scale_from_amax_bits(amax_bits[i], qmaxf, rule);
}

template <int IN_DT, int GRID, bool SR>
__global__ void __launch_bounds__(256) quant_grouped_kernel(QuantArgs a, int64_t gr, int64_t gc, int64_t n_gc) {
  const int64_t chunks_per_row = (a.K + 7) >> 3;
  const int64_t total = a.R * chunks_per_row;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < total; c += (int64_t)gridDim.x * 256) {
    int64_t r = c / chunks_per_row;
    int64_t k0 = (c - r * chunks_per_row) * 8;
    float v[8];
    load8<IN_DT, false>(a.x, r * a.ldx, k0, a.K, v);
    uint32_t rb[8];
    sr_words<SR>((uint64_t)(r * a.K + k0), a.seed, a.offset, rb);
    uint32_t cb[8];
    float q[8];
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int64_t k = k0 + i;
      float s = (k < a.K) ? a.scales[(r / gr) * n_gc + k / gc] : 1.0f;
      cb[i] = (k < a.K) ? quant_one<GRID, SR>(v[i], s, a.qmaxf, rb[i], q[i]) : 0u;
      if (k < a.K) {
        nan |= (__float_as_uint(q[i]) & 0x7FFFFFFFu) > 0x7F800000u;
        if (a.dq) store_elem(a.dq, a.dq_dtype, r * a.lddq + k, q[i] * s);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k0 + i < a.ldc) a.codes[r * a.ldc + k0 + i] = (uint8_t)cb[i];
    if (nan && a.nan_rows) atomicOr(a.nan_rows + r, 1);
  }
}

// ---------------------------------------------------------------------------
// 128x1 tiles with transposed output: codes_t [K, ldct] where row k holds
// column k of x in 128-row groups; scales_t(k, mb) = scales[k*s_row + mb*s_col].
// One workgroup per 128 x 64 region.
// ---------------------------------------------------------------------------
template <int IN_DT, int GRID, bool SR>
__global__ void __launch_bounds__(256) quant_tile_128x1_t_kernel(QuantArgs a) {
  __shared__ uint32_t colmax[32][64 + 1];
  __shared__ float colscale[64];
  __shared__ uint8_t tr[64][128 + 16];
  const int tid = threadIdx.x;
  const int c8 = tid & 7, slice = tid >> 3;  // 8 columns x 4 rows per thread
  const int64_t n_cb = (a.K + 63) / 64;
  const int64_t mb = blockIdx.x / n_cb, cb = blockIdx.x - mb * n_cb;
  const int64_t col0 = cb * 64 + c8 * 8;
  float v[4][8];
  uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int64_t r = mb * 128 + slice * 4 + i;
    if (r < a.R) {
      load8<IN_DT, false>(a.x, r * a.ldx, col0, a.K, v[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) m[j] = max(m[j], abs_bits(v[i][j]));
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) colmax[slice][c8 * 8 + j] = m[j];
  __syncthreads();
  if (tid < 64) {
    uint32_t mm = 0;
    for (int s = 0; s < 32; ++s) mm = max(mm, colmax[s][tid]);
    float sc = scale_from_amax_bits(mm, a.qmaxf, a.scale_rule);
    colscale[tid] = sc;
    int64_t col = cb * 64 + tid;
    if (col < a.K) a.scales[col * a.s_row + mb * a.s_col] = sc;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int64_t r = mb * 128 + slice * 4 + i;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int64_t col = col0 + j;
      float s = colscale[c8 * 8 + j];
      uint32_t rbits = 0;
      if constexpr (SR) {
        uint64_t e = (uint64_t)(r * a.K + col);
        Philox4 p = philox4x32_10(e >> 2, a.offset, a.seed);
        uint32_t w = (uint32_t)(e & 3u);
        rbits = w == 0 ? p.v[0] : (w == 1 ? p.v[1] : (w == 2 ? p.v[2] : p.v[3]));
      }
      float q;
      uint32_t c = quant_one<GRID, SR>(v[i][j], s, a.qmaxf, rbits, q);
      if (r >= a.R || col >= a.K) c = 0;
      tr[c8 * 8 + j][slice * 4 + i] = (uint8_t)c;
      if (r < a.R && col < a.K) {
        if (a.dq) store_elem(a.dq, a.dq_dtype, r * a.lddq + col, q * s);
        if (a.nan_rows && ((__float_as_uint(q) & 0x7FFFFFFFu) > 0x7F800000u)) atomicOr(a.nan_rows + r, 1);
      }
    }
  }
  __syncthreads();
  // 64 transposed rows of 128 bytes: 4 threads per row, 32 bytes each
  const int orow = tid >> 2, part = tid & 3;
  const int64_t col = cb * 64 + orow;
  if (col < a.K) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(&tr[orow][part * 32]);
    uint4* dst = reinterpret_cast<uint4*>(a.codes + col * a.ldc + mb * 128 + part * 32);
    dst[0] = make_uint4(src[0], src[1], src[2], src[3]);
    dst[1] = make_uint4(src[4], src[5], src[6], src[7]);
  }
}

// ---------------------------------------------------------------------------
// dispatch helpers
// ---------------------------------------------------------------------------
#define NTLB_DISPATCH_GRID_SR(GRIDV, SRV, ...)                         \
  do {                                                                  \
    if ((GRIDV) == GRID_INT) {                                          \
      if (SRV) {                                                        \
        constexpr int G_ = GRID_INT;                                    \
        constexpr bool S_ = true;                                       \
        __VA_ARGS__;                                                    \
      } else {                                                          \
        constexpr int G_ = GRID_INT;                                    \
        constexpr bool S_ = false;                                      \
        __VA_ARGS__;                                                    \
      }                                                                 \
    } else {                                                            \
      if (SRV) {                                                        \
        constexpr int G_ = GRID_E4M3;                                   \
        constexpr bool S_ = true;                                       \
        __VA_ARGS__;                                                    \
      } else {                                                          \
        constexpr int G_ = GRID_E4M3;                                   \
        constexpr bool S_ = false;                                      \
        __VA_ARGS__;                                                    \
      }                                                                 \
    }                                                                   \
  } while (0)

#define NTLB_DISPATCH_DT(DTV, ...)        \
  do {                                    \
    if ((DTV) == DT_BF16) {               \
      constexpr int D_ = DT_BF16;         \
      __VA_ARGS__;                        \
    } else if ((DTV) == DT_F32) {         \
      constexpr int D_ = DT_F32;          \
      __VA_ARGS__;                        \
    } else {                              \
      constexpr int D_ = DT_F16;          \
      __VA_ARGS__;                        \
    }                                     \
  } while (0)

static int check_common(const char* fn, const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int grid,
                        int qmax, int rounding, int scale_rule, const void* dq, int dq_dtype, int64_t lddq) {
  if (!x && R * K > 0) return fail(NTLB_EINVAL, "%s: x is NULL", fn);
  if (!valid_dtype(x_dtype)) return fail(NTLB_EINVAL, "%s: bad x dtype %d", fn, x_dtype);
  if (R < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (ldx < K) return fail(NTLB_EINVAL, "%s: ldx %lld < K %lld", fn, (long long)ldx, (long long)K);
  if (grid != NTLB_GRID_INT && grid != NTLB_GRID_E4M3) return fail(NTLB_EINVAL, "%s: bad grid %d", fn, grid);
  if (grid == NTLB_GRID_INT && (qmax < 1 || qmax > 127))
    return fail(NTLB_EINVAL, "%s: qmax %d outside [1, 127]", fn, qmax);
  if (rounding != NTLB_ROUND_NEAREST && rounding != NTLB_ROUND_STOCHASTIC)
    return fail(NTLB_EINVAL, "%s: bad rounding %d", fn, rounding);
  if (scale_rule != NTLB_SCALE_AFTER_DIVIDE && scale_rule != NTLB_SCALE_BEFORE_DIVIDE)
    return fail(NTLB_EINVAL, "%s: bad scale rule %d", fn, scale_rule);
  if (dq && !valid_dtype(dq_dtype)) return fail(NTLB_EINVAL, "%s: bad dq dtype %d", fn, dq_dtype);
  if (dq && lddq < K) return fail(NTLB_EINVAL, "%s: lddq < K", fn);
  return NTLB_OK;
}

static QuantArgs make_args(const void* x, int64_t R, int64_t K, int64_t ldx, int grid, int qmax, int scale_rule,
                           uint64_t seed, uint64_t offset, uint8_t* codes, int64_t ldc, float* scales,
                           int64_t s_row, int64_t s_col, void* dq, int dq_dtype, int64_t lddq, int32_t* nan_rows) {
  QuantArgs a;
  a.x = x;
  a.R = R;
  a.K = K;
  a.ldx = ldx;
  a.qmaxf = grid == NTLB_GRID_E4M3 ? 448.0f : (float)qmax;
  a.scale_rule = scale_rule;
  a.seed = seed;
  a.offset = offset;
  a.codes = codes;
  a.ldc = ldc;
  a.scales = scales;
  a.s_row = s_row;
  a.s_col = s_col;
  a.dq = dq;
  a.dq_dtype = dq_dtype;
  a.lddq = lddq;
  a.nan_rows = nan_rows;
  return a;
}

}  // namespace ntlb

using namespace ntlb;

extern "C" int ntlb_quant_tile_1x128(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int grid,
                                     int qmax, int rounding, int scale_rule, uint64_t seed, uint64_t offset,
                                     uint8_t* codes, int64_t ldc, float* scales, int64_t s_row, int64_t s_col,
                                     void* dq, int dq_dtype, int64_t lddq, int32_t* nan_rows, void* stream) {
  const char* fn = "ntlb_quant_tile_1x128";
  int rc = check_common(fn, x, x_dtype, R, K, ldx, grid, qmax, rounding, scale_rule, dq, dq_dtype, lddq);
  if (rc) return rc;
  const int64_t T = cdiv(K, 128);
  if (ldc < T * 128 || (ldc & 7)) return fail(NTLB_EINVAL, "%s: ldc must be >= ceil(K/128)*128 and a multiple of 8", fn);
  if (!codes || !scales) {
    if (R * K == 0) return NTLB_OK;
    return fail(NTLB_EINVAL, "%s: codes/scales NULL", fn);
  }
  if (!aligned(codes, 8)) return fail(NTLB_EINVAL, "%s: codes must be 8-byte aligned", fn);
  if (R * T == 0) return NTLB_OK;
  QuantArgs a = make_args(x, R, K, ldx, grid, qmax, scale_rule, seed, offset, codes, ldc, scales, s_row, s_col, dq,
                          dq_dtype, lddq, nan_rows);
  const bool vec = aligned(x, 16) && ((ldx * dtype_size(x_dtype)) % 16 == 0);
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  dim3 grd(grid_for(R * T, 32, 256 * 32)), blk(256);
  hipStream_t st = as_stream(stream);
  NTLB_DISPATCH_DT(x_dtype, NTLB_DISPATCH_GRID_SR(grid, sr, {
    if (vec)
      quant_tile_1x128_kernel<D_, G_, S_, true><<<grd, blk, 0, st>>>(a);
    else
      quant_tile_1x128_kernel<D_, G_, S_, false><<<grd, blk, 0, st>>>(a);
  }));
  return check_launch(fn);
}

extern "C" int ntlb_quant_block_128x128(const void* w, int w_dtype, int64_t N, int64_t K, int64_t ldw, int grid,
                                        int qmax, int rounding, int scale_rule, uint64_t seed, uint64_t offset,
                                        uint8_t* codes, int64_t ldc, uint8_t* codes_t, int64_t ldct, float* scales,
                                        int64_t s_row, int64_t s_col, void* dq, int dq_dtype, int64_t lddq,
                                        int32_t* nan_rows, void* stream) {
  const char* fn = "ntlb_quant_block_128x128";
  int rc = check_common(fn, w, w_dtype, N, K, ldw, grid, qmax, rounding, scale_rule, dq, dq_dtype, lddq);
  if (rc) return rc;
  const int64_t T = cdiv(K, 128), NB = cdiv(N, 128);
  if (ldc < T * 128 || (ldc & 7)) return fail(NTLB_EINVAL, "%s: ldc must be >= ceil(K/128)*128 and a multiple of 8", fn);
  if (codes_t && (ldct < NB * 128 || (ldct & 15) || !aligned(codes_t, 16)))
    return fail(NTLB_EINVAL, "%s: codes_t needs ldct >= ceil(N/128)*128, a multiple of 16, 16-byte aligned", fn);
  if (!codes || !scales) {
    if (N * K == 0) return NTLB_OK;
    return fail(NTLB_EINVAL, "%s: codes/scales NULL", fn);
  }
  if (!aligned(codes, 8)) return fail(NTLB_EINVAL, "%s: codes must be 8-byte aligned", fn);
  if (NB * T == 0) return NTLB_OK;
  BlockArgs ba;
  ba.q = make_args(w, N, K, ldw, grid, qmax, scale_rule, seed, offset, codes, ldc, scales, s_row, s_col, dq, dq_dtype,
                   lddq, nan_rows);
  ba.codes_t = codes_t;
  ba.ldct = ldct;
  const bool vec = aligned(w, 16) && ((ldw * dtype_size(w_dtype)) % 16 == 0);
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  if (NB * T > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many blocks", fn);
  dim3 grd((unsigned)(NB * T)), blk(256);
  hipStream_t st = as_stream(stream);
  NTLB_DISPATCH_DT(w_dtype, NTLB_DISPATCH_GRID_SR(grid, sr, {
    if (vec)
      quant_block_128x128_kernel<D_, G_, S_, true><<<grd, blk, 0, st>>>(ba);
    else
      quant_block_128x128_kernel<D_, G_, S_, false><<<grd, blk, 0, st>>>(ba);
  }));
  return check_launch(fn);
}

extern "C" int ntlb_amax_grouped(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr,
                                 int64_t gc, uint32_t* amax_bits, void* stream) {
  const char* fn = "ntlb_amax_grouped";
  if (!valid_dtype(x_dtype)) return fail(NTLB_EINVAL, "%s: bad dtype", fn);
  if (R < 0 || K < 0 || ldx < K || gr < 1 || gc < 1) return fail(NTLB_EINVAL, "%s: bad shape/group", fn);
  if (R * K == 0) return NTLB_OK;
  if (!x || !amax_bits) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  const int64_t n_gc = cdiv(K, gc);
  const int64_t col_blocks = cdiv(cdiv(K, 8), 256);
  // rows per workgroup: enough to amortize the atomics, enough groups to fill the GPU
  int64_t rpb = cdiv(R, cdiv(2048, col_blocks));
  if (rpb < 16) rpb = 16;
  const int64_t row_blocks = cdiv(R, rpb);
  if (row_blocks > 65535 || col_blocks > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: shape too large", fn);
  dim3 grd((unsigned)col_blocks, (unsigned)row_blocks), blk(256);
  hipStream_t st = as_stream(stream);
  NTLB_DISPATCH_DT(x_dtype, {
    amax_grouped_kernel<D_><<<grd, blk, 0, st>>>(x, R, K, ldx, gr, gc, n_gc, rpb, amax_bits);
  });
  return check_launch(fn);
}

extern "C" int ntlb_quant_grouped(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr,
                                  int64_t gc, const uint32_t* amax_bits, int grid, int qmax, int rounding,
                                  int scale_rule, uint64_t seed, uint64_t offset, uint8_t* codes, int64_t ldc,
                                  float* scales, void* dq, int dq_dtype, int64_t lddq, int32_t* nan_rows,
                                  void* stream) {
  const char* fn = "ntlb_quant_grouped";
  int rc = check_common(fn, x, x_dtype, R, K, ldx, grid, qmax, rounding, scale_rule, dq, dq_dtype, lddq);
  if (rc) return rc;
  if (gr < 1 || gc < 1) return fail(NTLB_EINVAL, "%s: bad group", fn);
  if (ldc < K) return fail(NTLB_EINVAL, "%s: ldc < K", fn);
  if (R * K == 0) return NTLB_OK;
  if (!codes || !scales || !amax_bits) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  const int64_t n_gr = cdiv(R, gr), n_gc = cdiv(K, gc);
  QuantArgs a = make_args(x, R, K, ldx, grid, qmax, scale_rule, seed, offset, codes, ldc, scales, 0, 0, dq, dq_dtype,
                          lddq, nan_rows);
  hipStream_t st = as_stream(stream);
  const int64_t ns = n_gr * n_gc;
  scales_from_amax_kernel<<<grid_for(ns, 256, 1 << 20), 256, 0, st>>>(amax_bits, ns, a.qmaxf, scale_rule, scales);
  rc = check_launch(fn);
  if (rc) return rc;
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  dim3 grd(grid_for(R * cdiv(K, 8), 256, 256 * 16)), blk(256);
  NTLB_DISPATCH_DT(x_dtype, NTLB_DISPATCH_GRID_SR(grid, sr, {
    quant_grouped_kernel<D_, G_, S_><<<grd, blk, 0, st>>>(a, gr, gc, n_gc);
  }));
  // ldc > K: padding columns beyond the 8-aligned chunks are not touched; callers
  // pass zero-initialised code buffers when ldc > round_up(K, 8).
  return check_launch(fn);
}

extern "C" int ntlb_quant_tile_128x1_t(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int grid,
                                       int qmax, int rounding, int scale_rule, uint64_t seed, uint64_t offset,
                                       uint8_t* codes_t, int64_t ldct, float* scales, int64_t s_row, int64_t s_col,
                                       void* dq, int dq_dtype, int64_t lddq, int32_t* nan_rows, void* stream) {
  const char* fn = "ntlb_quant_tile_128x1_t";
  int rc = check_common(fn, x, x_dtype, R, K, ldx, grid, qmax, rounding, scale_rule, dq, dq_dtype, lddq);
  if (rc) return rc;
  const int64_t MB = cdiv(R, 128), CB = cdiv(K, 64);
  if (ldct < MB * 128 || (ldct & 15) || (codes_t && !aligned(codes_t, 16)))
    return fail(NTLB_EINVAL, "%s: ldct must be >= ceil(R/128)*128, a multiple of 16, 16-byte aligned", fn);
  if (R * K == 0) return NTLB_OK;
  if (!codes_t || !scales) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (MB * CB > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many blocks", fn);
  QuantArgs a = make_args(x, R, K, ldx, grid, qmax, scale_rule, seed, offset, codes_t, ldct, scales, s_row, s_col,
                          dq, dq_dtype, lddq, nan_rows);
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  dim3 grd((unsigned)(MB * CB)), blk(256);
  hipStream_t st = as_stream(stream);
  NTLB_DISPATCH_DT(x_dtype, NTLB_DISPATCH_GRID_SR(grid, sr, {
    quant_tile_128x1_t_kernel<D_, G_, S_><<<grd, blk, 0, st>>>(a);
  }));
  return check_launch(fn);
}
