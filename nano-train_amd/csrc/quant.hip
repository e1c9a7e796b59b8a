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
#include <algorithm>
#include <hip/hip_runtime.h>
#include <mutex>

#include <type_traits>

#include "ntlb_device.h"
#include "ntlb_host.h"
#include "ntlb_quant8.h"

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
  // fast 1x128 path, fan-out (the expert-parallel send records and the
  // gather by expert): input row r goes to the output rows
  // fan_pos[r * fan_k + k], k < fan_k (clamped below fan_rows; a negative
  // entry writes nothing); output row p's NaN flag is nan_rows[p * nan_stride];
  // fan_nt stores the codes with the non-temporal hint
  const int32_t* fan_pos;
  int64_t fan_k, fan_rows;
  int64_t nan_stride;
  bool fan_nt;
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
// 1x128 tiles, fast path (bf16 or fp32 input, K a multiple of 8, 16-byte
// aligned rows).  Workgroup (bx, by) covers rows [16*bx, 16*bx+16) and tiles
// [TU*by, TU*by+TU): no integer division, every lane keeps TU 16-byte loads in
// flight, and 16 consecutive rows of one tile column write their scales
// contiguously in the tile-major layout.  The amax runs on packed bf16 bits
// (one op per two elements).  A tile whose amax is NaN takes the per-element
// path of the reference semantics; every other tile clamps with min/max.
// Under round to nearest the e4m3 rounding uses v_cvt_pk_fp8_f32 (checked
// bit-exact against the software rounding on every fp32 input with
// |v| <= 448).  Grids put the tile groups in x, so consecutive workgroups
// walk along a row and concurrent reads stay within the same DRAM pages.
// ---------------------------------------------------------------------------
constexpr int TILE_TU = 2;

// 8 consecutive elements as fp32 plus their |x| max (bits), from a chunk
// loaded raw: bf16 keeps 4 registers per chunk and reduces on packed halves.
template <int IN_DT>
struct Chunk8 {
  uint4 w[IN_DT == DT_F32 ? 2 : 1];
};

// NTL: loads with the non-temporal hint, for inputs read once and too large
// to stay in the caches
typedef unsigned int u32x4_ld __attribute__((ext_vector_type(4)));
template <bool NTL>
__device__ __forceinline__ uint4 load16(const void* p) {
  if constexpr (NTL) {
    const u32x4_ld v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_ld*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4*>(p);
  }
}

template <int IN_DT, bool NTL = false>
__device__ __forceinline__ void chunk_load(Chunk8<IN_DT>& c, const void* base, int64_t off, bool in) {
  if (!in) {
    c.w[0] = make_uint4(0, 0, 0, 0);
    if constexpr (IN_DT == DT_F32) c.w[1] = make_uint4(0, 0, 0, 0);
    return;
  }
  if constexpr (IN_DT == DT_F32) {
    const float* p = reinterpret_cast<const float*>(base) + off;
    c.w[0] = load16<NTL>(p);
    c.w[1] = load16<NTL>(p + 4);
  } else {
    c.w[0] = load16<NTL>(reinterpret_cast<const uint16_t*>(base) + off);
  }
}

template <int IN_DT>
__device__ __forceinline__ uint32_t chunk_amax(const Chunk8<IN_DT>& c) {
  if constexpr (IN_DT == DT_F32) {
    const uint32_t w[8] = {c.w[0].x, c.w[0].y, c.w[0].z, c.w[0].w, c.w[1].x, c.w[1].y, c.w[1].z, c.w[1].w};
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = max(m, w[i] & 0x7FFFFFFFu);
    return m;
  } else {
    uint32_t m2 = pk_max_u16(c.w[0].x & 0x7FFF7FFFu, c.w[0].y & 0x7FFF7FFFu);
    m2 = pk_max_u16(m2, c.w[0].z & 0x7FFF7FFFu);
    m2 = pk_max_u16(m2, c.w[0].w & 0x7FFF7FFFu);
    return max(m2 & 0xFFFFu, m2 >> 16) << 16;
  }
}

template <int IN_DT>
__device__ __forceinline__ void chunk_floats(const Chunk8<IN_DT>& c, float (&v)[8]) {
  if constexpr (IN_DT == DT_F32) {
    const uint32_t w[8] = {c.w[0].x, c.w[0].y, c.w[0].z, c.w[0].w, c.w[1].x, c.w[1].y, c.w[1].z, c.w[1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(w[i]);
  } else {
    const uint32_t w[4] = {c.w[0].x, c.w[0].y, c.w[0].z, c.w[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
}

template <int IN_DT, bool NTL = false>
__device__ __forceinline__ void tile_loads(Chunk8<IN_DT> (&c)[TILE_TU], const QuantArgs& a, int64_t r, int t0,
                                           int T, int lane16) {
#pragma unroll
  for (int u = 0; u < TILE_TU; ++u) {
    const int64_t k0 = (int64_t)(t0 + u) * 128 + lane16 * 8;
    chunk_load<IN_DT, NTL>(c[u], a.x, r * a.ldx + k0, r < a.R && t0 + u < T && k0 < a.K);
  }
}

// The fan-out form (expert-parallel send records): the TILE_TU tiles of input
// row r, each written to the fan_k output rows fan_pos[r * fan_k + f].  Round
// to nearest quantizes a tile once; stochastic rounding draws each output
// row's bits from its own element index.  A record's adjacent tile scales go
// out in one store.
template <int IN_DT, int GRID, bool SR>
__device__ __forceinline__ void tile_quant_fan(const Chunk8<IN_DT> (&c)[TILE_TU], const QuantArgs& a, int64_t r,
                                               int t0, int T, int lane16) {
  float v[TILE_TU][8], s[TILE_TU];
  uint32_t m[TILE_TU], lo[TILE_TU], hi[TILE_TU];
  bool nan[TILE_TU];
#pragma unroll
  for (int u = 0; u < TILE_TU; ++u) {
    chunk_floats<IN_DT>(c[u], v[u]);
    m[u] = row16_max_u32(chunk_amax<IN_DT>(c[u]));
    s[u] = scale_from_amax_bits(m[u], a.qmaxf, a.scale_rule);
    if constexpr (!SR) {
      uint32_t rb[8];
      float q[8];
      nan[u] = quant8_tile<GRID, false, false>(v[u], m[u], s[u], a.qmaxf, rb, lo[u], hi[u], q);
    }
  }
  const int nt = min(TILE_TU, T - t0);
  for (int64_t f = 0; f < a.fan_k; ++f) {
    const int32_t pr = a.fan_pos[r * a.fan_k + f];
    if (pr < 0) continue;  // an assignment a capacity limit dropped
    const int64_t p = min<int64_t>(pr, a.fan_rows - 1);
    bool any_nan = false;
#pragma unroll
    for (int u = 0; u < TILE_TU; ++u) {
      if (u >= nt) break;
      const int64_t k0 = (int64_t)(t0 + u) * 128 + lane16 * 8;
      if constexpr (SR) {
        uint32_t rb[8];
        float q[8];
        sr_words<true>((uint64_t)(p * a.K + k0), a.seed, a.offset, rb);
        nan[u] = quant8_tile<GRID, true, false>(v[u], m[u], s[u], a.qmaxf, rb, lo[u], hi[u], q);
      }
      any_nan |= nan[u];
      // the dispatch records go out with the non-temporal hint: 10% faster
      // at c4 (76 -> 68 us); the send-back pack measured 7% slower with it,
      // and the rows gathered by expert feed the next GEMM, so both store
      // normally
      if (a.fan_nt)
        store8_nt(a.codes + p * a.ldc + k0, lo[u], hi[u]);
      else
        *reinterpret_cast<uint2*>(a.codes + p * a.ldc + k0) = make_uint2(lo[u], hi[u]);
    }
    if (lane16 == 0) {
      float* sp = a.scales + p * a.s_row + (int64_t)t0 * a.s_col;
      if (TILE_TU == 2 && nt == 2 && a.s_col == 1 && (reinterpret_cast<uintptr_t>(sp) & 7) == 0) {
        *reinterpret_cast<float2*>(sp) = make_float2(s[0], s[TILE_TU - 1]);
      } else {
#pragma unroll
        for (int u = 0; u < TILE_TU; ++u)
          if (u < nt) sp[u * a.s_col] = s[u];
      }
      if (any_nan && a.nan_rows) atomicOr(a.nan_rows + p * a.nan_stride, 1);
    }
  }
}

template <int IN_DT, int GRID, bool SR, bool DQ, bool FAN>
__device__ __forceinline__ void tile_quant(const Chunk8<IN_DT> (&c)[TILE_TU], const QuantArgs& a, int64_t r, int t0,
                                           int T, int lane16) {
  if constexpr (FAN) {
    tile_quant_fan<IN_DT, GRID, SR>(c, a, r, t0, T, lane16);
    return;
  }
#pragma unroll
  for (int u = 0; u < TILE_TU; ++u) {
    const int t = t0 + u;
    if (t >= T) break;
    float v[8];
    chunk_floats<IN_DT>(c[u], v);
    uint32_t m = row16_max_u32(chunk_amax<IN_DT>(c[u]));
    const float s = scale_from_amax_bits(m, a.qmaxf, a.scale_rule);
    const int64_t k0 = (int64_t)t * 128 + lane16 * 8;
    uint32_t rb[8];
    sr_words<SR>((uint64_t)(r * a.K + k0), a.seed, a.offset, rb);
    uint32_t lo, hi;
    float q[8];
    const bool nan = quant8_tile<GRID, SR, DQ>(v, m, s, a.qmaxf, rb, lo, hi, q);
    if (nan && a.nan_rows && lane16 == 0) atomicOr(a.nan_rows + r * a.nan_stride, 1);
    *reinterpret_cast<uint2*>(a.codes + r * a.ldc + k0) = make_uint2(lo, hi);
    if (lane16 == 0) a.scales[r * a.s_row + (int64_t)t * a.s_col] = s;
    if constexpr (DQ) store_dq8(a.dq, a.dq_dtype, r * a.lddq, k0, a.K, q, s);
  }
}

// Workgroup (bx, by) covers tile columns [TU*bx, TU*bx+TU) of the row blocks
// by, by + gridDim.y, ... (16 rows each).  No prefetch: the lowest register
// count and the highest occupancy; the loop only runs when the grid is capped
// below the number of row blocks.
template <int IN_DT, int GRID, bool SR, bool DQ, bool FAN = false, bool NTL = false>
__global__ void __launch_bounds__(256) quant_tile_1x128_fast(QuantArgs a) {
  const int lane16 = threadIdx.x & 15;
  const int T = (int)((a.K + 127) >> 7);
  const int t0 = blockIdx.x * TILE_TU;
  const int64_t n_rb = (a.R + 15) >> 4;
  int64_t rb = blockIdx.y;  // row-block index
  if (rb >= n_rb) return;
  Chunk8<IN_DT> cur[TILE_TU];
  int64_t r = rb * 16 + (threadIdx.x >> 4);
  // the loads at the end of the body, not at its head: head-first, the
  // compiler gave the stochastic-rounding and dq variants 4-13 more VGPRs
  tile_loads<IN_DT, NTL>(cur, a, r, t0, T, lane16);
  for (;;) {
    if (r < a.R) tile_quant<IN_DT, GRID, SR, DQ, FAN>(cur, a, r, t0, T, lane16);  // whole 16-lane rows
    rb += gridDim.y;
    if (rb >= n_rb) return;
    r = rb * 16 + (threadIdx.x >> 4);
    tile_loads<IN_DT, NTL>(cur, a, r, t0, T, lane16);
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
  // fully unrolled so that v[i] stays in registers (a rolled loop indexes it
  // in scratch memory)
#pragma clang loop unroll(full)
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

// 128x128 blocks, fast path (bf16/fp32, K % 8 == 0, 16-byte aligned rows):
// one workgroup of 512 threads per block.
constexpr int BLK_THREADS = 512;
constexpr int BLK_ROWS = BLK_THREADS / 16;  // rows covered by one pass of the workgroup
constexpr int BLK_RPT = 128 / BLK_ROWS;     // rows per thread
constexpr int BLK_WAVES = BLK_THREADS / 64;

template <int IN_DT, bool NTL = false>
__device__ __forceinline__ void block_loads(Chunk8<IN_DT> (&ch)[BLK_RPT], const QuantArgs& a, int64_t nb, int64_t kb,
                                            int rr, int sub) {
  const int64_t k0 = kb * 128 + sub * 8;
#pragma unroll
  for (int i = 0; i < BLK_RPT; ++i) {
    const int64_t n = nb * 128 + rr + BLK_ROWS * i;
    chunk_load<IN_DT, NTL>(ch[i], a.x, n * a.ldx + k0, n < a.R && k0 < a.K);
  }
}

template <int IN_DT, int GRID, bool SR, bool DQ>
__device__ __forceinline__ void block_quant(const Chunk8<IN_DT> (&ch)[BLK_RPT], const BlockArgs& ba, int64_t nb,
                                            int64_t kb, int tid, uint32_t* red, uint8_t (*tile_t)[128 + 4]) {
  const QuantArgs& a = ba.q;
  const int sub = tid & 15, rr = tid >> 4;
  const int64_t k0 = kb * 128 + sub * 8;
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < BLK_RPT; ++i) m = max(m, chunk_amax<IN_DT>(ch[i]));
  m = wave_max_u32(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int w = 1; w < BLK_WAVES; ++w) m = max(m, red[w]);
  const float s = scale_from_amax_bits(m, a.qmaxf, a.scale_rule);
  if (tid == 0) a.scales[nb * a.s_row + kb * a.s_col] = s;
  // fully unrolled even when the stochastic-rounding body is large: a rolled
  // loop would index ch[] at run time and move it to scratch memory
#pragma clang loop unroll(full)
  for (int i = 0; i < BLK_RPT; ++i) {
    const int64_t n = nb * 128 + rr + BLK_ROWS * i;
    float v[8];
    chunk_floats<IN_DT>(ch[i], v);
    uint32_t rb[8];
    sr_words<SR>((uint64_t)(n * a.K + k0), a.seed, a.offset, rb);
    uint32_t lo, hi;
    float q[8];
    const bool nan = quant8_tile<GRID, SR, DQ>(v, m, s, a.qmaxf, rb, lo, hi, q);
    if (n < a.R && k0 < a.K) {
      *reinterpret_cast<uint2*>(a.codes + n * a.ldc + k0) = make_uint2(lo, hi);
      if constexpr (DQ) store_dq8(a.dq, a.dq_dtype, n * a.lddq, k0, a.K, q, s);
    } else if (n < a.R && k0 < a.ldc) {
      *reinterpret_cast<uint2*>(a.codes + n * a.ldc + k0) = make_uint2(0, 0);
    }
    if (nan && a.nan_rows && n < a.R) {
      bool row_nan = false;
#pragma unroll
      for (int j = 0; j < 8; ++j) row_nan |= (__float_as_uint(v[j]) & 0x7FFFFFFFu) > 0x7F800000u;
      if (row_nan) atomicOr(a.nan_rows + n, 1);
    }
    if (ba.codes_t) {
      *reinterpret_cast<uint32_t*>(&tile_t[rr + BLK_ROWS * i][sub * 8]) = lo;
      *reinterpret_cast<uint32_t*>(&tile_t[rr + BLK_ROWS * i][sub * 8 + 4]) = hi;
    }
  }
  if (ba.codes_t) {
    __syncthreads();
    // W^T rows: 128 rows x 128 bytes, 16-byte pieces spread over the workgroup
    for (int piece = tid; piece < 128 * 8; piece += BLK_THREADS) {
      const int kr = piece >> 3, h = piece & 7;
      const int64_t krow = kb * 128 + kr;
      if (krow < a.K) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int n0 = h * 16 + j * 4;
          w[j] = (uint32_t)tile_t[n0][kr] | ((uint32_t)tile_t[n0 + 1][kr] << 8) |
                 ((uint32_t)tile_t[n0 + 2][kr] << 16) | ((uint32_t)tile_t[n0 + 3][kr] << 24);
        }
        *reinterpret_cast<uint4*>(ba.codes_t + krow * ba.ldct + nb * 128 + h * 16) = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }
  __syncthreads();  // red[] and tile_t are reused by the next block
}

// 128x128 blocks, fast path (bf16/fp32, K % 8 == 0, 16-byte aligned rows):
// thread (rr, sub) holds rows rr + BLK_ROWS*i, columns sub*8 .. sub*8+7 of a
// block as raw chunks between the amax pass and the quantize pass (one HBM
// read).  Workgroup (kb, nb0) covers column block kb of the row blocks nb0,
// nb0 + gridDim.y, ...: consecutive workgroups walk column blocks.
template <int IN_DT, int GRID, bool SR, bool DQ, bool NTL = false>
__global__ void __launch_bounds__(BLK_THREADS) quant_block_128x128_fast(BlockArgs ba) {
  __shared__ uint32_t red[BLK_WAVES];
  __shared__ uint8_t tile_t[128][128 + 4];
  const int tid = threadIdx.x;
  const int sub = tid & 15, rr = tid >> 4;
  const int64_t NB = (ba.q.R + 127) >> 7;
  const int64_t kb = blockIdx.x;
  int64_t nb = blockIdx.y;
  if (nb >= NB) return;
  Chunk8<IN_DT> cur[BLK_RPT];
  // loads at the end of the body, as in the 1x128 kernel (head-first took
  // 59 -> 83 VGPRs and halved the resident workgroups)
  block_loads<IN_DT, NTL>(cur, ba.q, nb, kb, rr, sub);
  for (;;) {
    block_quant<IN_DT, GRID, SR, DQ>(cur, ba, nb, kb, tid, red, tile_t);
    nb += gridDim.y;
    if (nb >= NB) return;
    block_loads<IN_DT, NTL>(cur, ba.q, nb, kb, rr, sub);
  }
}

// ---------------------------------------------------------------------------
// grouped amax (tensor / channel / strip) and quantization with group scales
// ---------------------------------------------------------------------------
// |x| maxima per (gr x gc) group.  Workgroup = 2048 columns (8 per thread)
// of rows [r_begin, r_end).  Groups of at least 8 columns reduce in LDS
// first, so the workgroup issues one global atomic per group it touches
// (the strip and tensor groups of the comm payloads would otherwise put
// every thread's atomic on a handful of addresses).
constexpr int AMAX_LDS_GROUPS = 2048 / 8 + 2;

template <int IN_DT, bool VEC>
__global__ void __launch_bounds__(256) amax_grouped_kernel(const void* x, int64_t R, int64_t K, int64_t ldx,
                                                           int64_t gr, int64_t gc, int64_t n_gc,
                                                           int64_t rows_per_block, uint32_t* amax_bits) {
  __shared__ uint32_t sm[AMAX_LDS_GROUPS];
  const int64_t col0 = (int64_t)blockIdx.x * 2048;
  const int64_t kc = col0 + (int64_t)threadIdx.x * 8;  // 8 columns per thread
  const int64_t r_begin = (int64_t)blockIdx.y * rows_per_block;
  const int64_t r_end = min(R, r_begin + rows_per_block);
  if (r_begin >= R) return;  // the whole workgroup
  const bool lds = gc >= 8;
  const int64_t g0 = col0 / gc;
  const int64_t ngb = lds ? (min(col0 + 2048, K) - 1) / gc + 1 - g0 : 0;  // groups this workgroup's columns touch
  for (int64_t j = threadIdx.x; j < ngb; j += 256) sm[j] = 0;
  __syncthreads();
  uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  // every thread of the workgroup calls flush at the same rows (barriers inside)
  auto flush = [&](int64_t g) {
    if (lds) {
      if (kc < K) {
        if (gc % 8 == 0) {  // the 8 columns share one group
          uint32_t mm = 0;
#pragma unroll
          for (int i = 0; i < 8; ++i) mm = max(mm, m[i]);
          if (mm) atomicMax(&sm[kc / gc - g0], mm);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (kc + i < K && m[i]) atomicMax(&sm[(kc + i) / gc - g0], m[i]);
        }
      }
      __syncthreads();
      for (int64_t j = threadIdx.x; j < ngb; j += 256) {
        if (sm[j]) atomicMax(amax_bits + g * n_gc + g0 + j, sm[j]);
        sm[j] = 0;
      }
      __syncthreads();
    } else if (kc < K) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (kc + i < K && m[i]) atomicMax(amax_bits + g * n_gc + (kc + i) / gc, m[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) m[i] = 0;
  };
  int64_t cur_g = r_begin / gr;
  int64_t next_b = (cur_g + 1) * gr;  // first row of the next row group
  int64_t r = r_begin;
  while (r < r_end) {
    if (r >= next_b) {
      flush(cur_g);
      cur_g = r / gr;
      next_b = (cur_g + 1) * gr;
    }
    const int64_t lim = min(r_end, next_b);
    if (kc < K) {
      // four rows' loads in flight at a time (c4 payload, amax and
      // straight-through passes together: 288 -> 283 us)
      for (; r + 4 <= lim; r += 4) {
        float v[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) load8<IN_DT, VEC>(x, (r + u) * ldx, kc, K, v[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 8; ++i) m[i] = max(m[i], abs_bits(v[u][i]));
      }
      for (; r < lim; ++r) {
        float v[8];
        load8<IN_DT, VEC>(x, r * ldx, kc, K, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) m[i] = max(m[i], abs_bits(v[i]));
      }
    } else {
      r = lim;
    }
  }
  flush(cur_g);
}

// Row maxima (one group per row: gr = 1 and gc >= K, the weight `channel`
// granularity of te_backend.py:152-204): a wave per row, 8 columns per lane
// with four loads in flight, a wave reduction and one plain store per row
// (the group-flushing kernel below paid a barrier per row).
template <int IN_DT, bool VEC>
__global__ void __launch_bounds__(256) amax_rows_kernel(const void* x, int64_t R, int64_t K, int64_t ldx,
                                                        uint32_t* amax_bits) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;  // the whole wave
  uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t k = (int64_t)lane * 8;
  for (; k + 3 * 512 < K; k += 4 * 512) {
    float v[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) load8<IN_DT, VEC>(x, r * ldx, k + u * 512, K, v[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) m[i] = max(m[i], abs_bits(v[u][i]));
  }
  for (; k < K; k += 512) {
    float v[8];
    load8<IN_DT, VEC>(x, r * ldx, k, K, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) m[i] = max(m[i], abs_bits(v[i]));
  }
  uint32_t mm = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) mm = max(mm, m[i]);
  mm = wave_max_u32(mm);
  if (lane == 0) amax_bits[r] = max(amax_bits[r], mm);
}

// Group maxima, for groups narrower than 8 columns (channel granularity: one
// per column) and for tall groups.  amax_grouped_kernel's threads own
// distinct columns, so for one-column groups each of its workgroups issues
// one global atomic per column, and a 16-row workgroup pays as many atomics
// as loads (the c4 dispatch rows, 4096 x 7168: 1.8 million atomics on 7168
// addresses, 72 us).  Here a workgroup covers 512 columns and one row block
// of a single row group; its four waves take every fourth row of the block
// with four rows' loads in flight, the four partial maxima of each column
// meet in LDS, and wider groups meet again in LDS, so the workgroup issues
// one atomic per column (or per group) for four times the rows.  blockIdx.y
// = row group * bpg + block within the group.
template <int IN_DT, bool VEC>
__global__ void __launch_bounds__(256) amax_narrow_kernel(const void* x, int64_t R, int64_t K, int64_t ldx,
                                                          int64_t gr, int64_t gc, int64_t n_gc, int64_t rpb,
                                                          int64_t bpg, uint32_t* amax_bits) {
  __shared__ uint32_t sm[4][512];
  __shared__ uint32_t gm[512 + 2];  // the maxima of the column groups this workgroup touches (gc > 1)
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * 512;
  const int64_t kc = c0 + lane * 8;
  const int64_t g0 = c0 / gc;
  const int ngb = gc > 1 && c0 < K ? (int)((min(c0 + 512, K) - 1) / gc + 1 - g0) : 0;
  for (int j = threadIdx.x; j < ngb; j += 256) gm[j] = 0;
  const int64_t g = blockIdx.y / bpg;
  const int64_t g_end = min(R, (g + 1) * gr);
  const int64_t r_begin = g * gr + (blockIdx.y - g * bpg) * rpb;
  const int64_t r_end = min(g_end, r_begin + rpb);
  uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (kc < K) {
    int64_t r = r_begin + wv;
    for (; r + 12 < r_end; r += 16) {
      float v[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u) load8<IN_DT, VEC>(x, (r + 4 * u) * ldx, kc, K, v[u]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) m[i] = max(m[i], abs_bits(v[u][i]));
    }
    for (; r < r_end; r += 4) {
      float v[8];
      load8<IN_DT, VEC>(x, r * ldx, kc, K, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) m[i] = max(m[i], abs_bits(v[i]));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) sm[wv][lane * 8 + i] = m[i];
  __syncthreads();
  for (int j = threadIdx.x; j < 512; j += 256) {
    const int64_t k = c0 + j;
    const uint32_t mm = max(max(sm[0][j], sm[1][j]), max(sm[2][j], sm[3][j]));
    if (k < K && mm) {
      if (gc == 1)
        atomicMax(amax_bits + g * n_gc + k, mm);
      else
        atomicMax(&gm[k / gc - g0], mm);  // wider groups meet in LDS first
    }
  }
  if (gc > 1) {  // uniform
    __syncthreads();
    for (int j = threadIdx.x; j < ngb; j += 256)
      if (gm[j]) atomicMax(amax_bits + g * n_gc + g0 + j, gm[j]);
  }
}

typedef __bf16 v2bf_q __attribute__((ext_vector_type(2)));

// eight values rounded to a float dtype in place; bf16 by the hardware
// pack-convert (v_cvt_pk_bf16_f32, round to nearest even as f32_to_bf16_bits,
// a NaN stays a NaN)
template <int DT>
__device__ __forceinline__ void round8_dtype(float (&v)[8]) {
  if constexpr (DT == DT_BF16) {
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const v2bf_q p = {(__bf16)v[i], (__bf16)v[i + 1]};
      const uint32_t b = __builtin_bit_cast(uint32_t, p);
      v[i] = __uint_as_float(b << 16);
      v[i + 1] = __uint_as_float(b & 0xFFFF0000u);
    }
  } else if constexpr (DT == DT_F16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __half2float(f32_to_f16(v[i]));
  }
}

// moe.py:79-143 in one pass: each element quantized with its group's scale
// (from the group amaxes) and written as the value the reference's
// straight-through expression forms, tensor + (dq - tensor) in the tensor's
// dtype, with dq = q * scale rounded to that dtype.  One scale lookup per 8
// elements when gc % 8 == 0.  Thread (x, t) owns the 8-element chunk
// blockIdx.x*256 + t of rows blockIdx.y, blockIdx.y + gridDim.y, ...: its
// column group indices are fixed, and the row group takes one 32-bit
// division per row (the host keeps R and gr below 2^31), and the group
// scales are looked up again only when the row group changes.  A grid-stride
// walk over flat chunk indices paid three 64-bit divisions and a scale lookup
// per chunk and was VALU-bound (c4 payload, strip groups: 240 us at 98% VALU
// busy; with the amax pass and the workgroup counts below, 337 -> 274 us, and
// channel groups 651 -> 370 us).
template <int IN_DT, int GRID, bool SR, bool VEC>
__global__ void __launch_bounds__(256) comm_quant_ste_kernel(QuantArgs a, const uint32_t* amax_bits, int64_t gr,
                                                             int64_t gc, int64_t n_gc, void* out, int64_t ldo) {
#pragma clang fp contract(off)
  const int64_t chunks_per_row = (a.K + 7) >> 3;
  const int64_t kc = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (kc >= chunks_per_row) return;
  const int64_t k0 = kc * 8;
  const bool chunk_scale = gc % 8 == 0;
  // column groups of the chunk (chunk_scale: one for all 8 elements; the
  // host keeps n_gc below 2^31)
  int kg[8];
  if (chunk_scale) {
    kg[0] = (int)(k0 / gc);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) kg[i] = (int)min<int64_t>(gc == 1 ? k0 + i : (k0 + i) / gc, n_gc - 1);
  }
  const uint32_t gr32 = (uint32_t)gr;
  // the chunk's scales (and, with one group per chunk, its amax and
  // reciprocal), looked up again only when the row group changes: the
  // branch is uniform, as r is
  uint32_t gcur = 0xFFFFFFFFu, m = 0;
  float rs = 1.0f, sv[8], rsv[8];
  bool fast = false;  // every element's group allows the fast exact division
  for (int64_t r = blockIdx.y; r < a.R; r += gridDim.y) {
    float v[8];
    load8<IN_DT, VEC>(a.x, r * a.ldx, k0, a.K, v);
    uint32_t rb[8];
    sr_words<SR>((uint64_t)(r * a.K + k0), a.seed, a.offset, rb);
    const uint32_t g = (uint32_t)r / gr32;
    if (g != gcur) {
      gcur = g;
      const int64_t grow = (int64_t)g * n_gc;
      if (chunk_scale) {
        m = amax_bits[grow + kg[0]];
        const float s = scale_from_amax_bits(m, a.qmaxf, a.scale_rule);
        rs = fast_div_ok<SR>(m) ? 1.0f / s : 1.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) sv[i] = s;
      } else {
        fast = true;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t mi = amax_bits[grow + kg[i]];
          sv[i] = scale_from_amax_bits(mi, a.qmaxf, a.scale_rule);
          fast = fast && fast_div_ok<SR>(mi);
          rsv[i] = 1.0f / sv[i];
        }
      }
    }
    float q[8];
    if (chunk_scale) {
      // one group for the chunk: the tile quantizers' path (exact reciprocal
      // division where the group amax allows it, per element with a NaN)
      uint32_t lo, hi;
      (void)quant8_tile_rs<GRID, SR, true>(v, m, sv[0], rs, a.qmaxf, rb, lo, hi, q);
    } else if (fast) {
      // a group per element (channel): the same exact division element by
      // element (c4 payload, channel groups with the amax pass: 329 us before)
      uint32_t lo, hi;
      quant8_cols_rs<GRID, SR, true>(v, sv, rsv, a.qmaxf, rb, lo, hi, q);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) (void)quant_one<GRID, SR>(v[i], sv[i], a.qmaxf, rb[i], q[i]);
    }
    // dq = q * scale in the tensor's dtype, then tensor + (dq - tensor) in it
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = q[i] * sv[i];
    round8_dtype<IN_DT>(o);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = o[i] - v[i];
    round8_dtype<IN_DT>(o);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = v[i] + o[i];
    if (VEC && IN_DT == DT_BF16 && k0 + 8 <= a.K) {
      // the last rounding gives the stored bits (the hardware pack-convert)
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v2bf_q pk = {(__bf16)o[2 * i], (__bf16)o[2 * i + 1]};
        w[i] = __builtin_bit_cast(uint32_t, pk);
      }
      // non-temporal: the straight-through value at c4 takes 335 us instead of 365
      store16_nt(reinterpret_cast<uint16_t*>(out) + r * ldo + k0, w);
    } else {
      round8_dtype<IN_DT>(o);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k0 + i < a.K) store_elem(out, IN_DT, r * ldo + k0 + i, o[i]);
    }
  }
}

__global__ void scales_from_amax_kernel(const uint32_t* amax_bits, int64_t n, float qmaxf, int rule,
                                        float* scales) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) scales[i] = scale_from_amax_bits(amax_bits[i], qmaxf, rule);
}

template <int IN_DT, int GRID, bool SR, bool VEC>
// Thread (x, t) owns the 8-column chunk blockIdx.x*256 + t of rows
// blockIdx.y, blockIdx.y + gridDim.y, ..., as the comm-quant pass: column
// groups fixed per thread, one 32-bit division per row for the row group, and
// the chunk's scales read again only when the row group changes.
__global__ void __launch_bounds__(256) quant_grouped_kernel(QuantArgs a, const uint32_t* amax_bits, int64_t gr,
                                                            int64_t gc, int64_t n_gc) {
#pragma clang fp contract(off)
  const int64_t chunks_per_row = (a.K + 7) >> 3;
  const int64_t kc = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (kc >= chunks_per_row) return;
  const int64_t k0 = kc * 8;
  int kg[8];  // the host keeps n_gc below 2^31
#pragma unroll
  for (int i = 0; i < 8; ++i) kg[i] = (int)min<int64_t>(gc == 1 ? k0 + i : (k0 + i) / gc, n_gc - 1);
  const uint32_t gr32 = (uint32_t)gr;
  // one group for the chunk's 8 columns (gc % 8 == 0): the tile quantizers'
  // path, the exact reciprocal division where the group amax allows it and
  // the hardware e4m3 convert; a group per column where all eight amaxes
  // allow the division: the same element by element; else element by
  // element by IEEE division (the quantizer with its amax pass, c2 X [8192,
  // 7168] with a tensor scale: 98 -> 81 us on the int grid, 130 -> 94 us for
  // e4m3; channel scales, e4m3: 120 -> 97 us)
  const bool chunk_scale = gc % 8 == 0;
  uint32_t gcur = 0xFFFFFFFFu, m = 0;
  float sv[8], rsv[8];
  bool fast = false;
  for (int64_t r = blockIdx.y; r < a.R; r += gridDim.y) {
    float v[8];
    load8<IN_DT, VEC>(a.x, r * a.ldx, k0, a.K, v);
    uint32_t rb[8];
    sr_words<SR>((uint64_t)(r * a.K + k0), a.seed, a.offset, rb);
    const uint32_t g = (uint32_t)r / gr32;
    if (g != gcur) {
      gcur = g;
      const float* srow = a.scales + (int64_t)g * n_gc;
      const uint32_t* mrow = amax_bits + (int64_t)g * n_gc;
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = (k0 + i < a.K) ? srow[kg[i]] : 1.0f;
      if (chunk_scale) {
        m = mrow[kg[0]];
        rsv[0] = fast_div_ok<SR>(m) ? 1.0f / sv[0] : 1.0f;
      } else {
        fast = true;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          fast = fast && (k0 + i >= a.K || fast_div_ok<SR>(mrow[kg[i]]));
          rsv[i] = 1.0f / sv[i];
        }
      }
    }
    uint32_t lo, hi;
    float q[8];
    if (chunk_scale) {
      (void)quant8_tile_rs<GRID, SR, true>(v, m, sv[0], rsv[0], a.qmaxf, rb, lo, hi, q);
    } else if (fast) {
      quant8_cols_rs<GRID, SR, true>(v, sv, rsv, a.qmaxf, rb, lo, hi, q);
    } else {
      uint32_t cb[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) cb[i] = quant_one<GRID, SR>(v[i], sv[i], a.qmaxf, rb[i], q[i]);
      lo = cb[0] | (cb[1] << 8) | (cb[2] << 16) | (cb[3] << 24);
      hi = cb[4] | (cb[5] << 8) | (cb[6] << 16) | (cb[7] << 24);
    }
    // columns past K: their values load as zero and quantize to code 0
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k0 + i < a.K) nan |= (__float_as_uint(q[i]) & 0x7FFFFFFFu) > 0x7F800000u;
    if (VEC && k0 + 8 <= a.ldc) {
      *reinterpret_cast<uint2*>(a.codes + r * a.ldc + k0) = make_uint2(lo, hi);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k0 + i < a.ldc) a.codes[r * a.ldc + k0 + i] = (uint8_t)((i < 4 ? lo : hi) >> (8 * (i & 3)));
    }
    if (a.dq) {
      if (VEC && a.dq_dtype == DT_BF16 && k0 + 8 <= a.K && ((r * a.lddq + k0) & 7) == 0 &&
          (reinterpret_cast<uintptr_t>(a.dq) & 15) == 0) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[i] = (uint32_t)f32_to_bf16_bits(q[2 * i] * sv[2 * i]) |
                 ((uint32_t)f32_to_bf16_bits(q[2 * i + 1] * sv[2 * i + 1]) << 16);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(a.dq) + r * a.lddq + k0) = make_uint4(w[0], w[1], w[2], w[3]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (k0 + i < a.K) store_elem(a.dq, a.dq_dtype, r * a.lddq + k0 + i, q[i] * sv[i]);
      }
    }
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
        if (a.nan_rows && ((__float_as_uint(q) & 0x7FFFFFFFu) > 0x7F800000u)) atomicOr(a.nan_rows + col, 1);
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


// 128x1 tiles with transposed codes, for 8-aligned K and 16-byte aligned rows.
// A workgroup covers 128 rows x 8*CW columns (CW = 16 or 32) with 16*CW
// threads; thread t owns columns cb*8*CW + 8*(t % CW) + [0, 8) of rows
// mb*128 + 8*(t / CW) + [0, 8), read as eight 16-byte row chunks (a wave reads
// 64/CW full 16*CW-byte row segments per load).  The single-output pass takes
// CW = 32 under round to nearest: its 512-byte row segments read faster than
// 256-byte ones (c3 dY: 83.5 -> 78.0 us; 1024-byte segments, with one
// 1024-thread workgroup per CU, 106 us).  Column amax: packed per thread, shuffles across the row groups of
// a wave, LDS across the waves.  Each of the thread's columns then quantizes
// its 8 consecutive rows as one quant8_tile group (fast division and the
// hardware e4m3 convert where they apply), whose 8 codes are 8 consecutive
// bytes of the transposed row.  They are staged in LDS and leave as full
// 128-byte transposed rows, 16 bytes per lane; direct 8-byte stores would
// scatter 32-byte pieces over 16 rows per instruction.  Staging layout
// (128-byte rows, no padding; 64 banks of 4 bytes): transposed row cl sits at
// row cl ^ ((cl >> 3) & 1) and its 8-byte slot for row group rg at
// rg ^ (2*((cl >> 4) & 7) | ((cl >> 7) & 1)).  A 32-lane phase of the 8-byte
// writes (one column parity j; 16 columns of 2 row groups, or 32 columns of
// one) then covers both 128-byte halves of a 256-byte bank window, 16
// distinct slots in each: conflict-free.  16-byte piece k of a row holds row
// groups 2k and 2k+1, swapped when bit 7 of cl is set.  Each 16-lane phase of
// the 16-byte reads takes 8 pieces of two adjacent rows, one from each half:
// conflict-free too.  The per-column arrays (maxima, scales, reciprocals) skip
// one word after every 64 columns, so that the 16 columns cc*8 + j a
// half-wave reads at once fall on 16 banks.  nan_rows, when given, is indexed
// by transposed row (source column).
//
// With DUAL the same pass also writes the 1x128 tiles of x, described by ar
// (codes, ldc, scales, s_row, s_col, nan_rows and the SR offset): row i of a
// thread's chunks is 8 columns of one 1x128 tile, whose other 120 columns are
// held by the 15 lanes of the same row group, so a 16-lane max gives the tile
// amax.  One read of dY feeds both the dgrad and the wgrad operands.
//
// With SHARED (stochastic rounding, both outputs keyed at the same seed and
// offset) an element's word is the same for both layouts, so each Philox
// block is drawn once: the 1x128 codes are formed four columns at a time
// inside the 128x1 pass's two halves, from the same words.
template <int IN_DT, int GRID, bool SR, bool DQ, bool DUAL = false, int CW = 16, bool SHARED = false>
__global__ void __launch_bounds__(16 * CW) quant_tile_128x1_t_fast(QuantArgs a, QuantArgs ar = QuantArgs()) {
  static_assert(CW == 16 || (CW == 32 && !DUAL), "128 or 256 columns per workgroup; the dual pass takes 128");
  constexpr int NCOL = 8 * CW, NW = CW / 4;  // columns and waves of the workgroup
  constexpr int NPC = NCOL + NCOL / 64;      // per-column array length (pc() skips a word per 64)
  // staged transposed row of column cl, its 8-byte slot for row group rg and
  // its 16-byte piece k; per-column array index of column c
  auto trow = [](int cl) { return cl ^ ((cl >> 3) & 1); };
  auto tslot = [](int cl, int rg) { return rg ^ ((2 * ((cl >> 4) & 7)) | ((cl >> 7) & 1)); };
  auto tpiece = [](int cl, int k) { return k ^ ((cl >> 4) & 7); };
  auto pc = [](int c) { return c + (c >> 6); };
  __shared__ uint32_t wmax[NW][NPC];
  __shared__ uint32_t rmax[DUAL ? 128 : 1];
  // per column (and, with DUAL, per row tile): amax bits, scale, 1/scale,
  // computed once per workgroup by one thread each
  __shared__ __attribute__((aligned(16))) uint32_t cm[NPC];
  __shared__ __attribute__((aligned(16))) float cs[NPC], crs[NPC];
  __shared__ __attribute__((aligned(16))) uint32_t rm[DUAL ? 128 : 1];
  __shared__ __attribute__((aligned(16))) float rs_[DUAL ? 128 : 1], rrs[DUAL ? 128 : 1];
  __shared__ __attribute__((aligned(16))) uint8_t tcodes[NCOL * 128];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cc = tid & (CW - 1), rg = tid / CW;
  const int64_t n_cb = (a.K + NCOL - 1) / NCOL;
  // workgroup pid takes column block pid % n_cb of row block
  // (pid / n_cb + 7 * column block) mod n_mb: consecutive workgroups walk the
  // column blocks, and the skew spreads the row blocks that run at one time
  // over all of them, so concurrent transposed stores land at many offsets of
  // the transposed rows instead of a few (c3 dY: 87 -> 82 us).  The dual pass
  // keeps the plain walk (row block pid / n_cb): its row-major 1x128 stores
  // want concurrent workgroups on the same rows (skewed: 128 -> 137 us)
  const int64_t n_mb = (a.R + 127) / 128;
  const int64_t q = (int64_t)blockIdx.x / n_cb, cb = (int64_t)blockIdx.x - q * n_cb;
  const int64_t mb = DUAL ? q : (q + 7 * cb) % n_mb;
  const int64_t col0 = cb * NCOL + cc * 8;
  const int64_t row0 = mb * 128 + rg * 8;
  const bool col_in = col0 < a.K;  // K % 8 == 0: a chunk is wholly in or out

  Chunk8<IN_DT> c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) chunk_load<IN_DT>(c[i], a.x, (row0 + i) * a.ldx + col0, col_in && row0 + i < a.R);

  // column |x| maxima as fp32 bit patterns (NaN above every finite value):
  // per thread, then across the row groups of the wave, then (in LDS) across
  // the waves
  if constexpr (IN_DT == DT_F32) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t mm = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint4 w = c[i].w[j >> 2];
        const uint32_t b = (j & 3) == 0 ? w.x : (j & 3) == 1 ? w.y : (j & 3) == 2 ? w.z : w.w;
        mm = max(mm, b & 0x7FFFFFFFu);
      }
      if constexpr (CW == 16) mm = max(mm, (uint32_t)__shfl_xor((int)mm, 16));
      mm = max(mm, (uint32_t)__shfl_xor((int)mm, 32));
      if (lane < CW) wmax[wave][pc(cc * 8 + j)] = mm;
    }
  } else {
    uint32_t m2[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      m2[0] = pk_max_u16(m2[0], c[i].w[0].x & 0x7FFF7FFFu);
      m2[1] = pk_max_u16(m2[1], c[i].w[0].y & 0x7FFF7FFFu);
      m2[2] = pk_max_u16(m2[2], c[i].w[0].z & 0x7FFF7FFFu);
      m2[3] = pk_max_u16(m2[3], c[i].w[0].w & 0x7FFF7FFFu);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (CW == 16) m2[k] = pk_max_u16(m2[k], (uint32_t)__shfl_xor((int)m2[k], 16));
      m2[k] = pk_max_u16(m2[k], (uint32_t)__shfl_xor((int)m2[k], 32));
      if (lane < CW) {
        wmax[wave][pc(cc * 8 + 2 * k)] = m2[k] << 16;
        wmax[wave][pc(cc * 8 + 2 * k + 1)] = m2[k] & 0xFFFF0000u;
      }
    }
  }
  if constexpr (DUAL) {
    // 1x128 tile amax of each of the 128 rows: the 16 lanes of a row group
    // hold the tile's 128 columns
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t mr = row16_max_u32(chunk_amax<IN_DT>(c[i]));
      if (cc == 0) rmax[rg * 8 + i] = mr;
    }
  }
  __syncthreads();
  if (tid < NCOL) {
    const int c = pc(tid);
    uint32_t mm = wmax[0][c];
#pragma unroll
    for (int w = 1; w < NW; ++w) mm = max(mm, wmax[w][c]);
    const float sc = scale_from_amax_bits(mm, a.qmaxf, a.scale_rule);
    cm[c] = mm;
    cs[c] = sc;
    crs[c] = fast_div_ok<SR>(mm) ? 1.0f / sc : 1.0f;
  } else if (DUAL) {
    const int r = tid - 128;
    const uint32_t mm = rmax[r];
    const float sc = scale_from_amax_bits(mm, ar.qmaxf, ar.scale_rule);
    rm[r] = mm;
    rs_[r] = sc;
    rrs[r] = fast_div_ok<SR>(mm) ? 1.0f / sc : 1.0f;
  }
  __syncthreads();

  if constexpr (DUAL && !SHARED) {
    // 1x128 tiles: tile cb of rows row0..row0+7; pad columns [K, ldc) get
    // zero codes like every other 1x128 output (fully unrolled: c[] must stay
    // in registers)
#pragma clang loop unroll(full)
    for (int i = 0; i < 8; ++i) {
      const int64_t r = row0 + i;
      const int rl = rg * 8 + i;
      const uint32_t mr = rm[rl];
      const float sr = rs_[rl];
      float v[8];
      chunk_floats<IN_DT>(c[i], v);
      uint32_t rbr[8];
      sr_words<SR>((uint64_t)(r * a.K + col0), ar.seed, ar.offset, rbr);
      uint32_t lo, hi;
      float q[8];
      const bool nan = quant8_tile_rs<GRID, SR, false>(v, mr, sr, rrs[rl], ar.qmaxf, rbr, lo, hi, q);
      if (r < a.R) {
        *reinterpret_cast<uint2*>(ar.codes + r * ar.ldc + col0) = make_uint2(lo, hi);
        if (cc == 0) {
          ar.scales[r * ar.s_row + cb * ar.s_col] = sr;
          if (nan && ar.nan_rows) atomicOr(ar.nan_rows + r, 1);
        }
      }
    }
  }

  // SR words in two halves: columns 4h..4h+3 of every row share one Philox
  // block (K % 8 == 0 and col0 % 8 == 0 align the element index), so only
  // 32 words are live at a time.  Fully unrolled: a rolled loop would index
  // c[] by h at run time and move it to scratch memory
  uint32_t dlo[8];     // SHARED: each row's 1x128 codes of columns 0..3
  uint32_t dnan = 0;   // SHARED: NaN seen in row i's tile (bit i)
#pragma clang loop unroll(full)
  for (int h = 0; h < 2; ++h) {
  uint32_t rb[8][4];  // [row i][column j - 4h]
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if constexpr (SR) {
      const Philox4 p = philox4x32_10((((uint64_t)((row0 + i) * a.K + col0)) >> 2) + h, a.offset, a.seed);
#pragma unroll
      for (int u = 0; u < 4; ++u) rb[i][u] = p.v[u];
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) rb[i][u] = 0;
    }
  }
  if constexpr (DUAL && SHARED) {
    // the 1x128 codes of columns 4h..4h+3 of each row, from the same words
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rl = rg * 8 + i;
      float v8[8];
      chunk_floats<IN_DT>(c[i], v8);
      const float v4[4] = {v8[4 * h], v8[4 * h + 1], v8[4 * h + 2], v8[4 * h + 3]};
      const uint32_t rb4[4] = {rb[i][0], rb[i][1], rb[i][2], rb[i][3]};
      uint32_t w, w_unused;
      float q4[4];
      const bool nan = quant8_tile_rs<GRID, SR, false>(v4, rm[rl], rs_[rl], rrs[rl], ar.qmaxf, rb4, w, w_unused, q4);
      if (h == 0) {
        dlo[i] = w;
        dnan |= (nan ? 1u : 0u) << i;
      } else {
        const int64_t r = row0 + i;
        if (r < a.R) {
          *reinterpret_cast<uint2*>(ar.codes + r * ar.ldc + col0) = make_uint2(dlo[i], w);
          if (cc == 0) {
            ar.scales[r * ar.s_row + cb * ar.s_col] = rs_[rl];
            if ((nan || ((dnan >> i) & 1u)) && ar.nan_rows) atomicOr(ar.nan_rows + r, 1);
          }
        }
      }
    }
  }

#pragma clang loop unroll(full)
  for (int jj = 0; jj < 4; ++jj) {
    const int j = 4 * h + jj;
    const int cl = cc * 8 + j;
    const int64_t col = col0 + j;
    const uint32_t mj = cm[pc(cl)];
    const float s = cs[pc(cl)];
    float v[8];
    uint32_t rbj[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (IN_DT == DT_F32) {
        const uint4 w = c[i].w[j >> 2];
        v[i] = __uint_as_float((j & 3) == 0 ? w.x : (j & 3) == 1 ? w.y : (j & 3) == 2 ? w.z : w.w);
      } else {
        const uint4 w = c[i].w[0];
        const uint32_t b = (j >> 1) == 0 ? w.x : (j >> 1) == 1 ? w.y : (j >> 1) == 2 ? w.z : w.w;
        v[i] = __uint_as_float((j & 1) ? (b & 0xFFFF0000u) : (b << 16));
      }
      rbj[i] = rb[i][jj];
    }
    uint32_t lo, hi;
    float q[8];
    const bool nan = quant8_tile_rs<GRID, SR, DQ>(v, mj, s, crs[pc(cl)], a.qmaxf, rbj, lo, hi, q);
    *reinterpret_cast<uint2*>(tcodes + trow(cl) * 128 + tslot(cl, rg) * 8) = make_uint2(lo, hi);
    if (col_in) {
      if (rg == 0) {
        a.scales[col * a.s_row + mb * a.s_col] = s;
        if (nan && a.nan_rows) atomicOr(a.nan_rows + col, 1);
      }
      if constexpr (DQ) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (row0 + i < a.R) store_elem(a.dq, a.dq_dtype, (row0 + i) * a.lddq + col, q[i] * s);
      }
    }
  }
  }
  __syncthreads();
  // NCOL transposed rows of 128 bytes (rows past R hold zero codes, inside ldct)
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int qi = p * 16 * CW + tid;
    const int cl = qi >> 3, k = qi & 7;
    const int64_t col = cb * NCOL + cl;
    if (col < a.K) {
      uint4 v = *reinterpret_cast<const uint4*>(tcodes + trow(cl) * 128 + tpiece(cl, k) * 16);
      if (CW > 16 && (cl & 128)) v = make_uint4(v.z, v.w, v.x, v.y);  // row groups 2k, 2k+1 in order
      // the single-output pass stores its transposed rows with the
      // non-temporal hint (c3 dY: 100 -> 88 us); the dual pass, which also
      // writes the 1x128 codes, measured slower with it (128 -> 136 us)
      if constexpr (DUAL)
        *reinterpret_cast<uint4*>(a.codes + col * a.ldc + mb * 128 + k * 16) = v;
      else
        store16_nt(a.codes + col * a.ldc + mb * 128 + k * 16, &v);
    }
  }
}


// ---------------------------------------------------------------------------
// dequantize: out[i, k] = value(code[i, k]) * scale(i, k), cast to out dtype.
// scale(i, k) = scales[(i >> r_shift) * s_row + (k >> c_shift) * s_col]
// (r_shift/c_shift 0 or 7 cover rows, 128-blocks, tiles and strips; a zero
// stride broadcasts).  The receive side of the comm-quant wire format.
// ---------------------------------------------------------------------------
template <int GRID>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* codes, int64_t ldc, const float* scales,
                                                      int64_t s_row, int64_t s_col, int r_shift, int c_shift,
                                                      int64_t R, int64_t K, void* out, int out_dtype, int64_t ldo) {
  const int64_t chunks_per_row = (K + 7) >> 3;
  const int64_t total = R * chunks_per_row;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < total; c += (int64_t)gridDim.x * 256) {
    const int64_t r = c / chunks_per_row;
    const int64_t k0 = (c - r * chunks_per_row) * 8;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = k0 + i;
      if (k < K) {
        const uint32_t cd = codes[r * ldc + k];
        const float q = (GRID == GRID_E4M3) ? e4m3_to_f32(cd)
                                            : (cd == 0x80u ? __uint_as_float(0x7FC00000u) : (float)(int8_t)cd);
        v[i] = q * scales[(r >> r_shift) * s_row + (k >> c_shift) * s_col];
      } else {
        v[i] = 0.0f;
      }
    }
    store_dq8(out, out_dtype, r * ldo, k0, K, v, 1.0f);
  }
}
// Dequantize, fast path: K and ldc multiples of 8, one scale per 128
// columns (c_shift 7).  Thread = 8 columns, walking rows; no division.  e4m3
// through the hardware converter (v_cvt_pk_f32_fp8), bf16 output in 16-byte
// stores when BF16V (f32_to_bf16_bits rounding, as store_elem).
typedef float v2f_q __attribute__((ext_vector_type(2)));

template <int GRID, bool BF16V>
__global__ void __launch_bounds__(256) dequant_fast_kernel(const uint8_t* codes, int64_t ldc, const float* scales,
                                                           int64_t s_row, int64_t s_col, int r_shift, int64_t R,
                                                           int64_t K, void* out, int out_dtype, int64_t ldo) {
  const int64_t k0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (k0 >= K) return;
  for (int64_t r = blockIdx.y; r < R; r += gridDim.y) {
    const uint2 cw = *reinterpret_cast<const uint2*>(codes + r * ldc + k0);
    const float s = scales[(r >> r_shift) * s_row + (k0 >> 7) * s_col];
    float v[8];
    const uint32_t wd[2] = {cw.x, cw.y};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if constexpr (GRID == GRID_E4M3) {
        const v2f_q lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)wd[h], false);
        const v2f_q hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)wd[h], true);
        v[4 * h + 0] = lo[0] * s;
        v[4 * h + 1] = lo[1] * s;
        v[4 * h + 2] = hi[0] * s;
        v[4 * h + 3] = hi[1] * s;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t c = (wd[h] >> (8 * i)) & 0xFFu;
          v[4 * h + i] = (c == 0x80u ? __uint_as_float(0x7FC00000u) : (float)(int8_t)c) * s;
        }
      }
    }
    if constexpr (BF16V) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)f32_to_bf16_bits(v[2 * i]) | ((uint32_t)f32_to_bf16_bits(v[2 * i + 1]) << 16);
      // non-temporal: the c4 payload dequant takes 120 us instead of 150
      store16_nt(reinterpret_cast<uint16_t*>(out) + r * ldo + k0, w);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) store_elem(out, out_dtype, r * ldo + k0 + i, v[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// dispatch helpers
// ---------------------------------------------------------------------------
// Round-to-nearest inputs larger than this stream through the caches with
// the non-temporal load hint.  At c2/c3: W (264 MB) 77 -> 66 us in the
// 128x128 pass, dY (302 MB) 79 -> 72 us in the 1x128 pass; X at c2 (117 MB)
// measured 31 -> 33 us with it and keeps plain loads.  The 128x1 pass reads
// 16-column strips that share cache lines with the neighbouring strips, and
// the hint slowed it (83 -> 91-96 us), so it has none.  Stochastic rounding
// is VALU-bound and keeps plain loads.
constexpr int64_t NT_LOAD_MIN_BYTES = (int64_t)128 << 20;

template <int DT, int G, bool S>
static void launch_tile_fast_nodq(bool ntl, dim3 grd, dim3 blk, hipStream_t st, const QuantArgs& a) {
  if constexpr (!S) {
    if (ntl) {
      quant_tile_1x128_fast<DT, G, S, false, false, true><<<grd, blk, 0, st>>>(a);
      return;
    }
  }
  quant_tile_1x128_fast<DT, G, S, false><<<grd, blk, 0, st>>>(a);
}

template <int DT, int G, bool S>
static void launch_block_fast_nodq(bool ntl, dim3 grd, dim3 blk, hipStream_t st, const BlockArgs& ba) {
  if constexpr (!S) {
    if (ntl) {
      quant_block_128x128_fast<DT, G, S, false, true><<<grd, blk, 0, st>>>(ba);
      return;
    }
  }
  quant_block_128x128_fast<DT, G, S, false><<<grd, blk, 0, st>>>(ba);
}

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
  a.fan_pos = nullptr;
  a.fan_k = 1;
  a.fan_rows = R;
  a.nan_stride = 1;
  a.fan_nt = false;
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
  hipStream_t st = as_stream(stream);
  const bool fast_ok = vec && (K % 8 == 0) && (x_dtype == NTLB_BF16 || x_dtype == NTLB_F32) &&
                       (!dq || (dq_dtype == NTLB_BF16 && aligned(dq, 16) && (lddq % 8) == 0)) &&
                       cdiv(T, TILE_TU) <= 0x7FFFFFFF;
  if (fast_ok) {
    // one row block per workgroup, up to 65535 in y; the kernel's row-block
    // loop covers the rest
    const int64_t n_rb = cdiv(R, 16), n_tg = cdiv(T, TILE_TU);
    dim3 fgrd((unsigned)n_tg, (unsigned)std::min<int64_t>(n_rb, 65535));
    dim3 fblk(256);
    if (dq) {
      NTLB_DISPATCH_GRID_SR(grid, sr, {
        if (x_dtype == NTLB_BF16)
          quant_tile_1x128_fast<DT_BF16, G_, S_, true><<<fgrd, fblk, 0, st>>>(a);
        else
          quant_tile_1x128_fast<DT_F32, G_, S_, true><<<fgrd, fblk, 0, st>>>(a);
      });
    } else {
      const bool ntl = R * ldx * dtype_size(x_dtype) > NT_LOAD_MIN_BYTES;
      NTLB_DISPATCH_GRID_SR(grid, sr, {
        if (x_dtype == NTLB_BF16)
          launch_tile_fast_nodq<DT_BF16, G_, S_>(ntl, fgrd, fblk, st, a);
        else
          launch_tile_fast_nodq<DT_F32, G_, S_>(ntl, fgrd, fblk, st, a);
      });
    }
    return check_launch(fn);
  }
  dim3 grd(grid_for(R * T, 32, 256 * 32)), blk(256);
  NTLB_DISPATCH_DT(x_dtype, NTLB_DISPATCH_GRID_SR(grid, sr, {
    if (vec)
      quant_tile_1x128_kernel<D_, G_, S_, true><<<grd, blk, 0, st>>>(a);
    else
      quant_tile_1x128_kernel<D_, G_, S_, false><<<grd, blk, 0, st>>>(a);
  }));
  return check_launch(fn);
}

extern "C" int ntlb_quant_tile_1x128_fanout(const void* x, int x_dtype, int64_t T, int64_t K, int64_t ldx,
                                            const int32_t* pos, int64_t fan_k, int64_t rows, int grid, int qmax,
                                            int rounding, int scale_rule, uint64_t seed, uint64_t offset,
                                            uint8_t* codes, int64_t ldc, float* scales, int64_t s_row, int64_t s_col,
                                            int32_t* nan_rows, void* stream) {
  const char* fn = "ntlb_quant_tile_1x128_fanout";
  int rc = check_common(fn, x, x_dtype, T, K, ldx, grid, qmax, rounding, scale_rule, nullptr, 0, 0);
  if (rc) return rc;
  if (fan_k < 1 || rows < 0 || T * fan_k > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: bad fan_k or rows", fn);
  const int64_t Tt = cdiv(K, 128);
  if (ldc < Tt * 128 || (ldc & 7)) return fail(NTLB_EINVAL, "%s: ldc must be >= ceil(K/128)*128 and a multiple of 8", fn);
  if (T == 0 || rows == 0 || K == 0) return NTLB_OK;
  if (!codes || !scales || !pos) return fail(NTLB_EINVAL, "%s: codes/scales/pos NULL", fn);
  const bool vec = aligned(x, 16) && ((ldx * dtype_size(x_dtype)) % 16 == 0);
  if (!(vec && K % 8 == 0 && (x_dtype == NTLB_BF16 || x_dtype == NTLB_F32) && aligned(codes, 8) &&
        ldc % 8 == 0))
    return fail(NTLB_EUNSUPPORTED, "%s: needs bf16/fp32 rows, K %% 8 == 0, 16-byte aligned rows, 8-byte aligned codes",
                fn);
  QuantArgs a = make_args(x, T, K, ldx, grid, qmax, scale_rule, seed, offset, codes, ldc, scales, s_row, s_col,
                          nullptr, 0, 0, nan_rows);
  a.fan_pos = pos;
  a.fan_k = fan_k;
  a.fan_rows = rows;
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  hipStream_t st = as_stream(stream);
  const int64_t n_rb = cdiv(T, 16), n_tg = cdiv(Tt, TILE_TU);
  dim3 fgrd((unsigned)n_tg, (unsigned)std::min<int64_t>(n_rb, 65535)), fblk(256);
  NTLB_DISPATCH_GRID_SR(grid, sr, {
    if (x_dtype == NTLB_BF16)
      quant_tile_1x128_fast<DT_BF16, G_, S_, false, true><<<fgrd, fblk, 0, st>>>(a);
    else
      quant_tile_1x128_fast<DT_F32, G_, S_, false, true><<<fgrd, fblk, 0, st>>>(a);
  });
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
  hipStream_t st = as_stream(stream);
  const bool fast_ok = vec && (K % 8 == 0) && (w_dtype == NTLB_BF16 || w_dtype == NTLB_F32) &&
                       (!dq || (dq_dtype == NTLB_BF16 && aligned(dq, 16) && (lddq % 8) == 0)) &&
                       T <= 0x7FFFFFFF;
  if (fast_ok) {
    // one row block per workgroup, up to 65535 in y; the kernel's row-block
    // loop covers the rest
    dim3 fgrd((unsigned)T, (unsigned)std::min<int64_t>(NB, 65535));
    dim3 fblk(BLK_THREADS);
    if (dq) {
      NTLB_DISPATCH_GRID_SR(grid, sr, {
        if (w_dtype == NTLB_BF16)
          quant_block_128x128_fast<DT_BF16, G_, S_, true><<<fgrd, fblk, 0, st>>>(ba);
        else
          quant_block_128x128_fast<DT_F32, G_, S_, true><<<fgrd, fblk, 0, st>>>(ba);
      });
    } else {
      const bool ntl = N * ldw * dtype_size(w_dtype) > NT_LOAD_MIN_BYTES;
      NTLB_DISPATCH_GRID_SR(grid, sr, {
        if (w_dtype == NTLB_BF16)
          launch_block_fast_nodq<DT_BF16, G_, S_>(ntl, fgrd, fblk, st, ba);
        else
          launch_block_fast_nodq<DT_F32, G_, S_>(ntl, fgrd, fblk, st, ba);
      });
    }
    return check_launch(fn);
  }
  dim3 grd((unsigned)(NB * T)), blk(256);
  NTLB_DISPATCH_DT(w_dtype, NTLB_DISPATCH_GRID_SR(grid, sr, {
    if (vec)
      quant_block_128x128_kernel<D_, G_, S_, true><<<grd, blk, 0, st>>>(ba);
    else
      quant_block_128x128_kernel<D_, G_, S_, false><<<grd, blk, 0, st>>>(ba);
  }));
  return check_launch(fn);
}

// the grouped amax pass into amax_bits (validated, non-empty shapes)
static int amax_grouped_launch(const char* fn, const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx,
                               int64_t gr, int64_t gc, uint32_t* amax_bits, hipStream_t st) {
  const int64_t n_gc = cdiv(K, gc);
  // narrow groups, and any groups at least 64 rows tall: about 1024
  // workgroups of at least 64 rows, none straddling a row group (many short
  // row groups take the kernel below).  Strip and tensor groups of the c4
  // payload (32768 x 7168): 99.8 -> 90.5 and 98.7 -> 94.8 us against the
  // kernel below
  const int64_t cb = cdiv(K, 512);
  const int64_t ge = std::min(gr, R);
  const int64_t nrpb = std::min(ge, std::max<int64_t>(64, cdiv(R, cdiv(1024, cb))));
  const int64_t bpg = cdiv(ge, nrpb);
  const int64_t nb = cdiv(R, ge) * bpg;
  if (gr == 1 && gc >= K) {
    const bool vec = K % 8 == 0 && ldx % 8 == 0 && aligned(x, 16);
    if (cdiv(R, 4) > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: shape too large", fn);
    NTLB_DISPATCH_DT(x_dtype, {
      if (vec)
        amax_rows_kernel<D_, true><<<(unsigned)cdiv(R, 4), 256, 0, st>>>(x, R, K, ldx, amax_bits);
      else
        amax_rows_kernel<D_, false><<<(unsigned)cdiv(R, 4), 256, 0, st>>>(x, R, K, ldx, amax_bits);
    });
    return check_launch(fn);
  }
  if ((gc < 8 || ge >= 64) && nb <= 65535 && cb <= 0x7FFFFFFF) {
    const int64_t rpb = nrpb;
    dim3 grd((unsigned)cb, (unsigned)nb), blk(256);
    const bool vec = K % 8 == 0 && ldx % 8 == 0 && aligned(x, 16);
    NTLB_DISPATCH_DT(x_dtype, {
      if (vec)
        amax_narrow_kernel<D_, true><<<grd, blk, 0, st>>>(x, R, K, ldx, gr, gc, n_gc, rpb, bpg, amax_bits);
      else
        amax_narrow_kernel<D_, false><<<grd, blk, 0, st>>>(x, R, K, ldx, gr, gc, n_gc, rpb, bpg, amax_bits);
    });
    return check_launch(fn);
  }
  const int64_t col_blocks = cdiv(cdiv(K, 8), 256);
  // rows per workgroup: enough to amortize the atomics, enough groups to fill
  // the GPU.  About 1024 workgroups (c4 payload with the straight-through
  // pass: strip groups 282 us, channel groups 373; 2048: 283 and 416; 512:
  // 336 and 411; 8192: 285 and 610)
  int64_t rpb = cdiv(R, cdiv(1024, col_blocks));
  if (rpb < 16) rpb = 16;
  const int64_t row_blocks = cdiv(R, rpb);
  if (row_blocks > 65535 || col_blocks > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: shape too large", fn);
  dim3 grd((unsigned)col_blocks, (unsigned)row_blocks), blk(256);
  const bool vec = K % 8 == 0 && ldx % 8 == 0 && aligned(x, 16);
  NTLB_DISPATCH_DT(x_dtype, {
    if (vec)
      amax_grouped_kernel<D_, true><<<grd, blk, 0, st>>>(x, R, K, ldx, gr, gc, n_gc, rpb, amax_bits);
    else
      amax_grouped_kernel<D_, false><<<grd, blk, 0, st>>>(x, R, K, ldx, gr, gc, n_gc, rpb, amax_bits);
  });
  return check_launch(fn);
}

extern "C" int ntlb_amax_grouped(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr,
                                 int64_t gc, uint32_t* amax_bits, void* stream) {
  const char* fn = "ntlb_amax_grouped";
  if (!valid_dtype(x_dtype)) return fail(NTLB_EINVAL, "%s: bad dtype", fn);
  if (R < 0 || K < 0 || ldx < K || gr < 1 || gc < 1) return fail(NTLB_EINVAL, "%s: bad shape/group", fn);
  if (R * K == 0) return NTLB_OK;
  if (!x || !amax_bits) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  return amax_grouped_launch(fn, x, x_dtype, R, K, ldx, gr, gc, amax_bits, as_stream(stream));
}

extern "C" int ntlb_comm_quant_dequant(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr,
                                       int64_t gc, const uint32_t* amax_bits, int grid, int qmax, int rounding,
                                       int scale_rule, uint64_t seed, uint64_t offset, void* out, int64_t ldo,
                                       void* stream) {
  const char* fn = "ntlb_comm_quant_dequant";
  int rc = check_common(fn, x, x_dtype, R, K, ldx, grid, qmax, rounding, scale_rule, nullptr, 0, 0);
  if (rc) return rc;
  if (gr < 1 || gc < 1 || ldo < K) return fail(NTLB_EINVAL, "%s: bad group or ldo", fn);
  if (R * K == 0) return NTLB_OK;
  if (!amax_bits || !out) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  QuantArgs a = make_args(x, R, K, ldx, grid, qmax, scale_rule, seed, offset, nullptr, 0, nullptr, 0, 0, nullptr, 0,
                          0, nullptr);
  const int64_t n_gc = cdiv(K, gc);
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  const bool vec = K % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 && aligned(x, 16) && aligned(out, 16);
  // the kernel's row group is a 32-bit division: rows and row groups below
  // 2^31 (a row group at least as tall as the tensor is one group)
  if (R >= ((int64_t)1 << 31) || n_gc >= ((int64_t)1 << 31))
    return fail(NTLB_EUNSUPPORTED, "%s: 2^31 or more rows or column groups", fn);
  if (gr > R) gr = R;
  // x: 256 chunks of 8 columns per workgroup; y: rows, strided; about 8192
  // workgroups (c4 payload with the amax pass, strip groups: 271-277 us;
  // 4096: 282-289, 2048: 290-296, 16384: 265-273 but channel groups 381-384
  // against 368-370)
  const int64_t gx = cdiv(cdiv(K, 8), 256);
  if (gx > 0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: rows too long", fn);
  dim3 grd((unsigned)gx, (unsigned)std::max<int64_t>(1, std::min<int64_t>(R, std::min<int64_t>(65535, 8192 / gx)))),
      blk(256);
  hipStream_t st = as_stream(stream);
  NTLB_DISPATCH_DT(x_dtype, NTLB_DISPATCH_GRID_SR(grid, sr, {
    if (vec)
      comm_quant_ste_kernel<D_, G_, S_, true><<<grd, blk, 0, st>>>(a, amax_bits, gr, gc, n_gc, out, ldo);
    else
      comm_quant_ste_kernel<D_, G_, S_, false><<<grd, blk, 0, st>>>(a, amax_bits, gr, gc, n_gc, out, ldo);
  }));
  return check_launch(fn);
}

// arguments of the grouped quantizer shared by its two entry points
static int quant_grouped_check(const char* fn, const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx,
                               int64_t gr, int64_t gc, int grid, int qmax, int rounding, int scale_rule,
                               const uint8_t* codes, int64_t ldc, const float* scales, void* dq, int dq_dtype,
                               int64_t lddq) {
  int rc = check_common(fn, x, x_dtype, R, K, ldx, grid, qmax, rounding, scale_rule, dq, dq_dtype, lddq);
  if (rc) return rc;
  if (gr < 1 || gc < 1) return fail(NTLB_EINVAL, "%s: bad group", fn);
  if (ldc < K) return fail(NTLB_EINVAL, "%s: ldc < K", fn);
  if (R * K == 0) return NTLB_OK;
  if (!codes || !scales) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  return NTLB_OK;
}

// scales from the group amaxes, then the codes (validated, non-empty shapes)
static int quant_grouped_launch(const char* fn, const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx,
                                int64_t gr, int64_t gc, const uint32_t* amax_bits, int grid, int qmax, int rounding,
                                int scale_rule, uint64_t seed, uint64_t offset, uint8_t* codes, int64_t ldc,
                                float* scales, void* dq, int dq_dtype, int64_t lddq, int32_t* nan_rows,
                                hipStream_t st) {
  const int64_t n_gr = cdiv(R, gr), n_gc = cdiv(K, gc);
  QuantArgs a = make_args(x, R, K, ldx, grid, qmax, scale_rule, seed, offset, codes, ldc, scales, 0, 0, dq, dq_dtype,
                          lddq, nan_rows);
  const int64_t ns = n_gr * n_gc;
  scales_from_amax_kernel<<<grid_for(ns, 256, 1 << 20), 256, 0, st>>>(amax_bits, ns, a.qmaxf, scale_rule, scales);
  int rc = check_launch(fn);
  if (rc) return rc;
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  if (R >= ((int64_t)1 << 31) || n_gc >= ((int64_t)1 << 31))
    return fail(NTLB_EUNSUPPORTED, "%s: 2^31 or more rows or column groups", fn);
  if (gr > R) gr = R;  // one row group either way; the kernel divides in 32 bits
  const int64_t gx = cdiv(cdiv(K, 8), 256);
  if (gx > 0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: rows too long", fn);
  // about 4096 workgroups (8192 measured slower: c2 X with channel scales
  // 92 -> 116 us, the per-thread scale set-up amortized over fewer rows)
  dim3 grd((unsigned)gx, (unsigned)std::max<int64_t>(1, std::min<int64_t>(R, std::min<int64_t>(65535, 4096 / gx)))),
      blk(256);
  // vector loads and 8-byte code stores where rows and pitches allow
  const bool vec = K % 8 == 0 && ldx % 8 == 0 && ldc % 8 == 0 && aligned(x, 16) && aligned(codes, 8);
  NTLB_DISPATCH_DT(x_dtype, NTLB_DISPATCH_GRID_SR(grid, sr, {
    if (vec)
      quant_grouped_kernel<D_, G_, S_, true><<<grd, blk, 0, st>>>(a, amax_bits, gr, gc, n_gc);
    else
      quant_grouped_kernel<D_, G_, S_, false><<<grd, blk, 0, st>>>(a, amax_bits, gr, gc, n_gc);
  }));
  // ldc > K: padding columns beyond the 8-aligned chunks are not touched; callers
  // pass zero-initialised code buffers when ldc > round_up(K, 8).
  return check_launch(fn);
}

extern "C" int ntlb_quant_grouped(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr,
                                  int64_t gc, const uint32_t* amax_bits, int grid, int qmax, int rounding,
                                  int scale_rule, uint64_t seed, uint64_t offset, uint8_t* codes, int64_t ldc,
                                  float* scales, void* dq, int dq_dtype, int64_t lddq, int32_t* nan_rows,
                                  void* stream) {
  const char* fn = "ntlb_quant_grouped";
  int rc = quant_grouped_check(fn, x, x_dtype, R, K, ldx, gr, gc, grid, qmax, rounding, scale_rule, codes, ldc,
                               scales, dq, dq_dtype, lddq);
  if (rc || R * K == 0) return rc;
  if (!amax_bits) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  return quant_grouped_launch(fn, x, x_dtype, R, K, ldx, gr, gc, amax_bits, grid, qmax, rounding, scale_rule, seed,
                              offset, codes, ldc, scales, dq, dq_dtype, lddq, nan_rows, as_stream(stream));
}

// ---------------------------------------------------------------------------
// The grouped quantizer without a caller workspace, for callers that cannot
// allocate (code under graph capture, serving loops): the amax accumulator
// lives in `scratch`, one copy per GPU, held until the process ends.  Every
// call on a GPU shares that GPU's copy, so calls that overlap on one GPU
// (concurrent streams) race; calls in one stream order are safe.
// ---------------------------------------------------------------------------
constexpr int64_t NOALLOC_MAX_GROUPS = 1 << 16;  // 256 KiB of uint32 amaxes
static __device__ __align__(256) uint32_t scratch[NOALLOC_MAX_GROUPS];

__global__ void __launch_bounds__(256) fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = v;
}

// device address of `scratch` on the current device, looked up once per device
static int scratch_on_current_device(const char* fn, uint32_t** out) {
  static std::mutex mu;
  static uint32_t* addr[64] = {nullptr};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) return fail(NTLB_ELAUNCH, "%s: no current device", fn);
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(NTLB_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed: %s", fn, hipGetErrorString(e));
    addr[dev] = reinterpret_cast<uint32_t*>(p);
  }
  *out = addr[dev];
  return NTLB_OK;
}

extern "C" int ntlb_quant_grouped_noalloc(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr,
                                          int64_t gc, int grid, int qmax, int rounding, int scale_rule, uint64_t seed,
                                          uint64_t offset, uint8_t* codes, int64_t ldc, float* scales, void* dq,
                                          int dq_dtype, int64_t lddq, int32_t* nan_rows, void* stream) {
  const char* fn = "ntlb_quant_grouped_noalloc";
  int rc = quant_grouped_check(fn, x, x_dtype, R, K, ldx, gr, gc, grid, qmax, rounding, scale_rule, codes, ldc,
                               scales, dq, dq_dtype, lddq);
  if (rc || R * K == 0) return rc;
  const int64_t groups = cdiv(R, gr) * cdiv(K, gc);
  if (groups > NOALLOC_MAX_GROUPS)
    return fail(NTLB_EINVAL, "%s: %lld scale groups exceed the %lld this entry point holds (use ntlb_amax_grouped + "
                "ntlb_quant_grouped with a workspace)", fn, (long long)groups, (long long)NOALLOC_MAX_GROUPS);
  uint32_t* amax = nullptr;
  rc = scratch_on_current_device(fn, &amax);
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  // the previous call's amaxes are still there: clear what this call uses
  // (a fill kernel, so the call can also be captured in a graph)
  fill_u32_kernel<<<grid_for(groups, 256, 1024), 256, 0, st>>>(amax, groups, 0u);
  rc = check_launch(fn);
  if (rc) return rc;
  rc = amax_grouped_launch(fn, x, x_dtype, R, K, ldx, gr, gc, amax, st);
  if (rc) return rc;
  return quant_grouped_launch(fn, x, x_dtype, R, K, ldx, gr, gc, amax, grid, qmax, rounding, scale_rule, seed,
                              offset, codes, ldc, scales, dq, dq_dtype, lddq, nan_rows, st);
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
  hipStream_t st = as_stream(stream);
  if (K % 8 == 0 && ldx % 8 == 0 && aligned(x, 16) && (x_dtype == NTLB_BF16 || x_dtype == NTLB_F32) &&
      cdiv(R, 128) * cdiv(K, 128) <= 0x7FFFFFFF) {
    // round to nearest: 256-column workgroups (CW = 32); stochastic
    // rounding, whose Philox work makes it VALU-bound, keeps 128 columns
    // (CW = 16), since at 512 threads its register use allows one workgroup
    // per CU (c3 dY: 156 -> 222 us)
    const int cw = sr ? 16 : 32;
    dim3 grd((unsigned)(cdiv(R, 128) * cdiv(K, 8 * cw))), blk(16 * cw);
#define NTLB_T128(DT_, DQ_)                                                                      \
  do {                                                                                           \
    if constexpr (S_) quant_tile_128x1_t_fast<DT_, G_, S_, DQ_, false, 16><<<grd, blk, 0, st>>>(a); \
    else quant_tile_128x1_t_fast<DT_, G_, S_, DQ_, false, 32><<<grd, blk, 0, st>>>(a);              \
  } while (0)
    if (x_dtype == NTLB_BF16) {
      NTLB_DISPATCH_GRID_SR(grid, sr, {
        if (dq) NTLB_T128(DT_BF16, true);
        else NTLB_T128(DT_BF16, false);
      });
    } else {
      NTLB_DISPATCH_GRID_SR(grid, sr, {
        if (dq) NTLB_T128(DT_F32, true);
        else NTLB_T128(DT_F32, false);
      });
    }
#undef NTLB_T128
    return check_launch(fn);
  }
  dim3 grd((unsigned)(MB * CB)), blk(256);
  NTLB_DISPATCH_DT(x_dtype, NTLB_DISPATCH_GRID_SR(grid, sr, {
    quant_tile_128x1_t_kernel<D_, G_, S_><<<grd, blk, 0, st>>>(a);
  }));
  return check_launch(fn);
}

extern "C" int ntlb_quant_dual_1x128_128x1(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx,
                                           int grid, int qmax, int rounding, int scale_rule, uint64_t seed,
                                           uint64_t offset_rows, uint64_t offset_cols, uint8_t* codes, int64_t ldc,
                                           float* scales, int64_t s_row, int64_t s_col, int32_t* nan_rows,
                                           uint8_t* codes_t, int64_t ldct, float* scales_t, int64_t st_row,
                                           int64_t st_col, int32_t* nan_cols, void* stream) {
  const char* fn = "ntlb_quant_dual_1x128_128x1";
  int rc = check_common(fn, x, x_dtype, R, K, ldx, grid, qmax, rounding, scale_rule, nullptr, NTLB_BF16, 0);
  if (rc) return rc;
  if (!(x_dtype == NTLB_BF16 || x_dtype == NTLB_F32) || K % 8 || ldx % 8 || (x && !aligned(x, 16)))
    return fail(NTLB_EUNSUPPORTED, "%s: needs bf16 or fp32 input, K %% 8 == 0, ldx %% 8 == 0, 16-byte rows", fn);
  const int64_t T = cdiv(K, 128), MB = cdiv(R, 128);
  if (ldc < T * 128 || ldc % 16 || (codes && !aligned(codes, 16)))
    return fail(NTLB_EINVAL, "%s: ldc must be >= ceil(K/128)*128, a multiple of 16, 16-byte aligned", fn);
  if (ldct < MB * 128 || ldct % 16 || (codes_t && !aligned(codes_t, 16)))
    return fail(NTLB_EINVAL, "%s: ldct must be >= ceil(R/128)*128, a multiple of 16, 16-byte aligned", fn);
  if (R * K == 0) return NTLB_OK;
  if (!codes || !scales || !codes_t || !scales_t) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (MB * T > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many blocks", fn);
  QuantArgs ac = make_args(x, R, K, ldx, grid, qmax, scale_rule, seed, offset_cols, codes_t, ldct, scales_t, st_row,
                           st_col, nullptr, 0, 0, nan_cols);
  QuantArgs ar = make_args(x, R, K, ldx, grid, qmax, scale_rule, seed, offset_rows, codes, ldc, scales, s_row, s_col,
                           nullptr, 0, 0, nan_rows);
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  hipStream_t st = as_stream(stream);
  dim3 grd((unsigned)(MB * T)), blk(256);
  if (sr && offset_rows == offset_cols) {
    // one Philox draw per element for both layouts
    if (x_dtype == NTLB_BF16) {
      if (grid == NTLB_GRID_E4M3)
        quant_tile_128x1_t_fast<DT_BF16, GRID_E4M3, true, false, true, 16, true><<<grd, blk, 0, st>>>(ac, ar);
      else
        quant_tile_128x1_t_fast<DT_BF16, GRID_INT, true, false, true, 16, true><<<grd, blk, 0, st>>>(ac, ar);
    } else {
      if (grid == NTLB_GRID_E4M3)
        quant_tile_128x1_t_fast<DT_F32, GRID_E4M3, true, false, true, 16, true><<<grd, blk, 0, st>>>(ac, ar);
      else
        quant_tile_128x1_t_fast<DT_F32, GRID_INT, true, false, true, 16, true><<<grd, blk, 0, st>>>(ac, ar);
    }
    return check_launch(fn);
  }
  if (x_dtype == NTLB_BF16) {
    NTLB_DISPATCH_GRID_SR(grid, sr, {
      quant_tile_128x1_t_fast<DT_BF16, G_, S_, false, true><<<grd, blk, 0, st>>>(ac, ar);
    });
  } else {
    NTLB_DISPATCH_GRID_SR(grid, sr, {
      quant_tile_128x1_t_fast<DT_F32, G_, S_, false, true><<<grd, blk, 0, st>>>(ac, ar);
    });
  }
  return check_launch(fn);
}

extern "C" int ntlb_dequant(int grid, const uint8_t* codes, int64_t ldc, const float* scales, int64_t s_row,
                            int64_t s_col, int r_shift, int c_shift, int64_t R, int64_t K, void* out, int out_dtype,
                            int64_t ldo, void* stream) {
  const char* fn = "ntlb_dequant";
  if (grid != NTLB_GRID_INT && grid != NTLB_GRID_E4M3) return fail(NTLB_EINVAL, "%s: bad grid %d", fn, grid);
  if (R < 0 || K < 0 || ldc < K || ldo < K) return fail(NTLB_EINVAL, "%s: bad shape", fn);
  if (!(r_shift == 0 || r_shift == 7) || !(c_shift == 0 || c_shift == 7))
    return fail(NTLB_EINVAL, "%s: shifts must be 0 or 7", fn);
  if (!valid_dtype(out_dtype)) return fail(NTLB_EINVAL, "%s: bad output dtype", fn);
  if (R * K == 0) return NTLB_OK;
  if (!codes || !scales || !out) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  hipStream_t st = as_stream(stream);
  if (c_shift == 7 && K % 8 == 0 && ldc % 8 == 0 && aligned(codes, 8)) {
    const int64_t gx = cdiv(K / 8, 256);
    const int64_t gy = std::min<int64_t>(R, std::max<int64_t>(1, (256 * 16) / gx));
    dim3 fgrd((unsigned)gx, (unsigned)std::min<int64_t>(gy, 65535)), fblk(256);
    const bool bf16v = out_dtype == NTLB_BF16 && ldo % 8 == 0 && aligned(out, 16);
    auto launch = [&](auto gridc, auto vecc) {
      dequant_fast_kernel<decltype(gridc)::value, decltype(vecc)::value><<<fgrd, fblk, 0, st>>>(
          codes, ldc, scales, s_row, s_col, r_shift, R, K, out, out_dtype, ldo);
    };
    using E = std::integral_constant<int, GRID_E4M3>;
    using I = std::integral_constant<int, GRID_INT>;
    using T = std::true_type;
    using F = std::false_type;
    if (grid == NTLB_GRID_E4M3) {
      if (bf16v) launch(E(), T()); else launch(E(), F());
    } else {
      if (bf16v) launch(I(), T()); else launch(I(), F());
    }
    return check_launch(fn);
  }
  dim3 grd(grid_for(R * cdiv(K, 8), 256, 256 * 16)), blk(256);
  if (grid == NTLB_GRID_E4M3)
    dequant_kernel<GRID_E4M3><<<grd, blk, 0, st>>>(codes, ldc, scales, s_row, s_col, r_shift, c_shift, R, K, out,
                                                   out_dtype, ldo);
  else
    dequant_kernel<GRID_INT><<<grd, blk, 0, st>>>(codes, ldc, scales, s_row, s_col, r_shift, c_shift, R, K, out,
                                                  out_dtype, ldo);
  return check_launch(fn);
}

// Expert-parallel send records (the record layout is described in ep.hip):
// assignment a goes to record p = pos[a], whose metadata is token a / K, slot
// a % K, local expert topk_idx[a] % experts_per_rank and routing weight
// topk_w[a], with the NaN flag cleared for the quantizer to set.
// Bytes [pad_off, m_off) of a record (the padding of a value record; none
// in a code record) are zeroed, 16 at a time.
__device__ __forceinline__ void ep_zero_pad(uint8_t* r, int64_t pad_off, int64_t m_off) {
  for (int64_t b = pad_off; b < m_off; b += 16) *reinterpret_cast<uint4*>(r + b) = make_uint4(0, 0, 0, 0);
}

__global__ void __launch_bounds__(256) ep_meta_kernel(uint8_t* rec, int64_t R, int64_t m_off, int64_t A,
                                                      const int32_t* pos, const void* topk_idx, int idx_dt,
                                                      const void* topk_w, int w_dt, int64_t K, int64_t epr,
                                                      int64_t pad_off) {
  const int64_t a = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (a >= A) return;
  const int64_t p = min<int64_t>(max<int32_t>(pos[a], 0), A - 1);
  ep_zero_pad(rec + p * R, pad_off, m_off);
  const int64_t e = idx_dt == 1 ? reinterpret_cast<const int64_t*>(topk_idx)[a]
                                : (int64_t) reinterpret_cast<const int32_t*>(topk_idx)[a];
  const float w = load_elem(topk_w, w_dt, a);
  int32_t* m = reinterpret_cast<int32_t*>(rec + p * R + m_off);
  *reinterpret_cast<int4*>(m) = make_int4((int32_t)(a / K), (int32_t)(a % K), (int32_t)(e % epr), 0);
  *reinterpret_cast<int4*>(m + 4) = make_int4(__float_as_int(w), 0, 0, 0);
}

// Return records (the expert side of the combine, moe.py:926-962): row i of
// the expert outputs goes to record p = pos[i] with token_idx[i], slot_idx[i],
// the optional local expert and weight, and the NaN flag cleared.
__global__ void __launch_bounds__(256) ep_meta_rows_kernel(uint8_t* rec, int64_t R, int64_t m_off, int64_t n,
                                                           const int32_t* pos, const int32_t* token_idx,
                                                           const int32_t* slot_idx, const int32_t* local_expert,
                                                           const float* weight, int64_t pad_off) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t p = min<int64_t>(max<int32_t>(pos[i], 0), n - 1);
  ep_zero_pad(rec + p * R, pad_off, m_off);
  int32_t* m = reinterpret_cast<int32_t*>(rec + p * R + m_off);
  *reinterpret_cast<int4*>(m) = make_int4(token_idx[i], slot_idx[i], local_expert ? local_expert[i] : 0, 0);
  *reinterpret_cast<int4*>(m + 4) = make_int4(weight ? __float_as_int(weight[i]) : 0, 0, 0, 0);
}

// Records quantized with the reference's comm-quant scales (moe.py:93-140):
// one scale per gc-column group over all rows, from the group amaxes of
// ntlb_amax_grouped, each element through the same quant_one as
// quant_grouped_kernel.  A thread takes 8 columns of one input row (zero past
// K, up to the record's whole tiles Hp) and writes them to the fan_k records
// fan_pos[r * fan_k + f], each with its own SR bits (element index p*K + col).
template <int IN_DT, int GRID, bool SR>
__global__ void __launch_bounds__(256) ep_pack_grouped_kernel(QuantArgs a, const uint32_t* amax_bits, int64_t gc,
                                                              int64_t n_gc, int64_t Hp) {
  const int64_t cpr = Hp >> 3;
  const int64_t total = a.R * cpr;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < total; c += (int64_t)gridDim.x * 256) {
    const int64_t r = c / cpr;
    const int64_t k0 = (c - r * cpr) * 8;
    float v[8];
    load8<IN_DT, true>(a.x, r * a.ldx, k0, a.K, v);
    // a group spans whole tiles (gc % 128 == 0) or all columns (n_gc == 1)
    const float s = scale_from_amax_bits(amax_bits[min<int64_t>(k0 / gc, n_gc - 1)], a.qmaxf, a.scale_rule);
    for (int64_t f = 0; f < a.fan_k; ++f) {
      const int64_t p = min<int64_t>(max<int32_t>(a.fan_pos[r * a.fan_k + f], 0), a.fan_rows - 1);
      uint32_t rb[8];
      sr_words<SR>((uint64_t)(p * a.K + k0), a.seed, a.offset, rb);
      uint32_t cb[8];
      float q[8];
      bool nan = false;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        cb[i] = quant_one<GRID, SR>(v[i], s, a.qmaxf, rb[i], q[i]);
        nan |= (__float_as_uint(q[i]) & 0x7FFFFFFFu) > 0x7F800000u;
      }
      const uint32_t lo = cb[0] | (cb[1] << 8) | (cb[2] << 16) | (cb[3] << 24);
      const uint32_t hi = cb[4] | (cb[5] << 8) | (cb[6] << 16) | (cb[7] << 24);
      *reinterpret_cast<uint2*>(a.codes + p * a.ldc + k0) = make_uint2(lo, hi);
      if ((k0 & 127) == 0) a.scales[p * a.s_row + (k0 >> 7)] = s;
      if (nan && a.nan_rows) atomicOr(a.nan_rows + p * a.nan_stride, 1);
    }
  }
}

// Value records: the reference's wire values themselves, as
// _comm_quant_dequant (moe.py:79-143) leaves them in the send buffer of
// _dispatch_tokens (moe.py:805-814) and _combine_remote_outputs
// (moe.py:983-990).  Any column grouping, including one scale per column
// (channel granularity, moe.py:112-121), whose scales a record's tile scales
// cannot carry.  Thread (x, t) owns the 8-column chunk blockIdx.x*256 + t of
// input rows blockIdx.y, blockIdx.y + gridDim.y, ...; its group scales are
// read once (one row group spans every row).  Each element is quantized with
// its group's scale (SR element index p*H + column of record p) and written
// as tensor + (dq - tensor) in the input dtype, dq = q * scale rounded to it,
// the expression comm_quant_ste_kernel evaluates; input row r goes to the
// fan_k records fan_pos[r * fan_k + f] at byte p*R + 2 or 4 per column.
template <int IN_DT, int GRID, bool SR>
__global__ void __launch_bounds__(256) ep_pack_values_kernel(QuantArgs a, const uint32_t* amax_bits, int64_t gc,
                                                             int64_t n_gc, uint8_t* rec, int64_t R) {
#pragma clang fp contract(off)
  const int64_t k0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (k0 >= a.K) return;  // K % 8 == 0: whole chunks
  // the chunk's group scales, and their reciprocals where every one of the
  // eight allows the fast exact division (quant8_tile_rs's condition)
  float sv[8], rs[8];
  bool fast = true;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t m = amax_bits[min<int64_t>((k0 + i) / gc, n_gc - 1)];
    sv[i] = scale_from_amax_bits(m, a.qmaxf, a.scale_rule);
    fast = fast && fast_div_ok<SR>(m);
    rs[i] = 1.0f / sv[i];
  }
  constexpr int64_t esz = IN_DT == DT_F32 ? 4 : 2;
  // one row at a time: loading four rows ahead measured slower (c4 return
  // pack 358 -> 368 us, the stochastic dispatch pack 243 -> 260)
  for (int64_t r = blockIdx.y; r < a.R; r += gridDim.y) {
    float v[8];
    load8<IN_DT, true>(a.x, r * a.ldx, k0, a.K, v);
    {
      uint32_t w[8];  // the value's bits (bf16: 4 words)
      for (int64_t f = 0; f < a.fan_k; ++f) {
        const int64_t p = min<int64_t>(max<int32_t>(a.fan_pos[r * a.fan_k + f], 0), a.fan_rows - 1);
        if (SR || f == 0) {  // round to nearest: one value for every copy
          float o[8];
          uint32_t rb[8];
          sr_words<SR>((uint64_t)(p * a.K + k0), a.seed, a.offset, rb);
          float q[8];
          if (fast) {
            uint32_t lo, hi;
            quant8_cols_rs<GRID, SR, true>(v, sv, rs, a.qmaxf, rb, lo, hi, q);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) (void)quant_one<GRID, SR>(v[i], sv[i], a.qmaxf, rb[i], q[i]);
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = q[i] * sv[i];
          round8_dtype<IN_DT>(o);
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = o[i] - v[i];
          round8_dtype<IN_DT>(o);
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = v[i] + o[i];
          // the last rounding gives the stored bits: bf16 pairs by the
          // hardware pack-convert (round to nearest even), fp32 as is
          if constexpr (IN_DT == DT_BF16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const v2bf_q pk = {(__bf16)o[2 * i], (__bf16)o[2 * i + 1]};
              w[i] = __builtin_bit_cast(uint32_t, pk);
            }
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i] = __float_as_uint(o[i]);
          }
        }
        uint8_t* dst = rec + p * R + k0 * esz;  // 16-byte aligned: R % 16 == 0, k0 % 8 == 0
        // non-temporal: the records go to the exchange, not to the next
        // kernel (c4 return pack: 443 -> 419 us)
        store16_nt(dst, w);
        if constexpr (IN_DT == DT_F32) store16_nt(dst + 16, w + 4);
      }
    }
  }
}

// Shared by the dispatch and return packs: rows x [n_in, H] quantized into
// records (codes, tile scales, NaN flag; the metadata kernels run first),
// input row r going to the fan_k records fan_pos[r * fan_k + f].
static int ep_pack_payload(const char* fn, const void* x, int x_dtype, int64_t n_in, int64_t H, int64_t ldx,
                           const int32_t* fan_pos, int64_t fan_k, int64_t n_rec, const uint32_t* amax_bits,
                           int64_t gc, int grid, int qmax, int rounding, int scale_rule, uint64_t seed,
                           uint64_t offset, uint8_t* records, hipStream_t st) {
  const int64_t R = ntlb_ep_record_bytes(H);
  const int64_t s_off = (H + 127) / 128 * 128, m_off = R - 32;
  const int64_t Tt = cdiv(H, 128);
  QuantArgs a = make_args(x, n_in, H, ldx, grid, qmax, scale_rule, seed, offset, records, R,
                          reinterpret_cast<float*>(records + s_off), R / 4, 1, nullptr, 0, 0,
                          reinterpret_cast<int32_t*>(records + m_off + 12));
  a.fan_pos = fan_pos;
  a.fan_k = fan_k;
  a.fan_rows = n_rec;
  a.nan_stride = R / 4;
  a.fan_nt = fan_k > 1;
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  if (amax_bits) {
    dim3 grd(grid_for(n_in * (s_off >> 3), 256, 256 * 16)), blk(256);
    const int64_t n_gc = cdiv(H, gc);
    NTLB_DISPATCH_GRID_SR(grid, sr, {
      if (x_dtype == NTLB_BF16)
        ep_pack_grouped_kernel<DT_BF16, G_, S_><<<grd, blk, 0, st>>>(a, amax_bits, gc, n_gc, s_off);
      else
        ep_pack_grouped_kernel<DT_F32, G_, S_><<<grd, blk, 0, st>>>(a, amax_bits, gc, n_gc, s_off);
    });
    return check_launch(fn);
  }
  const int64_t n_rb = cdiv(n_in, 16), n_tg = cdiv(Tt, TILE_TU);
  dim3 fgrd((unsigned)n_tg, (unsigned)std::min<int64_t>(n_rb, 65535)), fblk(256);
  NTLB_DISPATCH_GRID_SR(grid, sr, {
    if (x_dtype == NTLB_BF16)
      quant_tile_1x128_fast<DT_BF16, G_, S_, false, true><<<fgrd, fblk, 0, st>>>(a);
    else
      quant_tile_1x128_fast<DT_F32, G_, S_, false, true><<<fgrd, fblk, 0, st>>>(a);
  });
  return check_launch(fn);
}

static int ep_check_payload(const char* fn, const void* x, int x_dtype, int64_t H, int64_t ldx,
                            const uint32_t* amax_bits, int64_t gc, const uint8_t* records) {
  const bool vec = aligned(x, 16) && ((ldx * dtype_size(x_dtype)) % 16 == 0);
  if (!(vec && H % 8 == 0 && (x_dtype == NTLB_BF16 || x_dtype == NTLB_F32) && aligned(records, 16) &&
        cdiv(cdiv(H, 128), TILE_TU) <= 65535))
    return fail(NTLB_EUNSUPPORTED, "%s: needs bf16/fp32 rows, H %% 8 == 0, 16-byte aligned rows and records", fn);
  if (amax_bits && (gc < 1 || (gc % 128 != 0 && gc < H)))
    return fail(NTLB_EINVAL, "%s: a scale group spans whole 128-column tiles (gc %% 128 == 0) or all H columns", fn);
  return NTLB_OK;
}

extern "C" int ntlb_ep_pack_records_grouped(const void* tokens, int x_dtype, int64_t T, int64_t H, int64_t ldt,
                                            const int32_t* pos, const void* topk_idx, int idx_dtype,
                                            const void* topk_w, int w_dtype, int64_t K, int64_t experts_per_rank,
                                            const uint32_t* amax_bits, int64_t gc, int grid, int qmax, int rounding,
                                            int scale_rule, uint64_t seed, uint64_t offset, uint8_t* records,
                                            void* stream) {
  const char* fn = "ntlb_ep_pack_records";
  if (K < 1 || experts_per_rank < 1 || T < 0 || (idx_dtype != 0 && idx_dtype != 1) || !valid_dtype(w_dtype))
    return fail(NTLB_EINVAL, "%s: bad argument", fn);
  const int64_t A = T * K;
  if (A > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: more than 2^31 assignments", fn);
  int rc = check_common(fn, tokens, x_dtype, T, H, ldt, grid, qmax, rounding, scale_rule, nullptr, 0, 0);
  if (rc) return rc;
  if (A == 0 || H == 0) return NTLB_OK;
  if (!pos || !topk_idx || !topk_w || !records) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  rc = ep_check_payload(fn, tokens, x_dtype, H, ldt, amax_bits, gc, records);
  if (rc) return rc;
  const int64_t R = ntlb_ep_record_bytes(H);
  hipStream_t st = as_stream(stream);
  ep_meta_kernel<<<(unsigned)cdiv(A, 256), 256, 0, st>>>(records, R, R - 32, A, pos, topk_idx, idx_dtype, topk_w,
                                                          w_dtype, K, experts_per_rank, R - 32);
  rc = check_launch(fn);
  if (rc) return rc;
  // each token row read once, quantized, and written to its K records
  return ep_pack_payload(fn, tokens, x_dtype, T, H, ldt, pos, K, A, amax_bits, gc, grid, qmax, rounding, scale_rule,
                         seed, offset, records, st);
}

extern "C" int ntlb_ep_pack_records(const void* tokens, int x_dtype, int64_t T, int64_t H, int64_t ldt,
                                    const int32_t* pos, const void* topk_idx, int idx_dtype, const void* topk_w,
                                    int w_dtype, int64_t K, int64_t experts_per_rank, int grid, int qmax,
                                    int rounding, int scale_rule, uint64_t seed, uint64_t offset, uint8_t* records,
                                    void* stream) {
  return ntlb_ep_pack_records_grouped(tokens, x_dtype, T, H, ldt, pos, topk_idx, idx_dtype, topk_w, w_dtype, K,
                                      experts_per_rank, nullptr, 0, grid, qmax, rounding, scale_rule, seed, offset,
                                      records, stream);
}

extern "C" int ntlb_ep_pack_return(const void* x, int x_dtype, int64_t n, int64_t H, int64_t ldx, const int32_t* pos,
                                   const int32_t* token_idx, const int32_t* slot_idx, const int32_t* local_expert,
                                   const float* weight, const uint32_t* amax_bits, int64_t gc, int grid, int qmax,
                                   int rounding, int scale_rule, uint64_t seed, uint64_t offset, uint8_t* records,
                                   void* stream) {
  const char* fn = "ntlb_ep_pack_return";
  if (n < 0 || n > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: need 0 <= n < 2^31", fn);
  int rc = check_common(fn, x, x_dtype, n, H, ldx, grid, qmax, rounding, scale_rule, nullptr, 0, 0);
  if (rc) return rc;
  if (n == 0 || H == 0) return NTLB_OK;
  if (!pos || !token_idx || !slot_idx || !records) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  rc = ep_check_payload(fn, x, x_dtype, H, ldx, amax_bits, gc, records);
  if (rc) return rc;
  const int64_t R = ntlb_ep_record_bytes(H);
  hipStream_t st = as_stream(stream);
  ep_meta_rows_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(records, R, R - 32, n, pos, token_idx, slot_idx,
                                                               local_expert, weight, R - 32);
  rc = check_launch(fn);
  if (rc) return rc;
  return ep_pack_payload(fn, x, x_dtype, n, H, ldx, pos, 1, n, amax_bits, gc, grid, qmax, rounding, scale_rule, seed,
                         offset, records, st);
}

extern "C" int64_t ntlb_ep_value_record_bytes(int64_t H, int dtype) {
  if (H <= 0 || !valid_dtype(dtype)) return 0;
  // whole 128-byte lines: every record's payload starts on a line
  return (H * dtype_size(dtype) + 32 + 127) / 128 * 128;
}

// Value-record payload of rows x [n_in, H]: the metadata kernels run first.
static int ep_pack_values_payload(const char* fn, const void* x, int x_dtype, int64_t n_in, int64_t H, int64_t ldx,
                                  const int32_t* fan_pos, int64_t fan_k, int64_t n_rec, const uint32_t* amax_bits,
                                  int64_t gc, int grid, int qmax, int rounding, int scale_rule, uint64_t seed,
                                  uint64_t offset, uint8_t* records, int64_t R, hipStream_t st) {
  QuantArgs a = make_args(x, n_in, H, ldx, grid, qmax, scale_rule, seed, offset, nullptr, 0, nullptr, 0, 0, nullptr, 0,
                          0, nullptr);
  a.fan_pos = fan_pos;
  a.fan_k = fan_k;
  a.fan_rows = n_rec;
  const int64_t n_gc = cdiv(H, gc);
  const int64_t gx = cdiv(H / 8, 256);
  dim3 grd((unsigned)gx, (unsigned)std::max<int64_t>(1, std::min<int64_t>(n_in, std::min<int64_t>(65535, 8192 / gx)))),
      blk(256);
  const bool sr = rounding == NTLB_ROUND_STOCHASTIC;
  NTLB_DISPATCH_GRID_SR(grid, sr, {
    if (x_dtype == NTLB_BF16)
      ep_pack_values_kernel<DT_BF16, G_, S_><<<grd, blk, 0, st>>>(a, amax_bits, gc, n_gc, records, R);
    else
      ep_pack_values_kernel<DT_F32, G_, S_><<<grd, blk, 0, st>>>(a, amax_bits, gc, n_gc, records, R);
  });
  return check_launch(fn);
}

static int ep_check_values(const char* fn, const void* x, int x_dtype, int64_t H, int64_t ldx,
                           const uint32_t* amax_bits, int64_t gc, const uint8_t* records) {
  const bool vec = aligned(x, 16) && ((ldx * dtype_size(x_dtype)) % 16 == 0);
  if (!(vec && H % 8 == 0 && (x_dtype == NTLB_BF16 || x_dtype == NTLB_F32) && aligned(records, 16) &&
        cdiv(H / 8, 256) <= 65535))
    return fail(NTLB_EUNSUPPORTED, "%s: needs bf16/fp32 rows, H %% 8 == 0, 16-byte aligned rows and records", fn);
  if (!amax_bits || gc < 1) return fail(NTLB_EINVAL, "%s: needs the group amaxes and gc >= 1", fn);
  if (cdiv(H, gc) >= ((int64_t)1 << 31)) return fail(NTLB_EUNSUPPORTED, "%s: 2^31 or more column groups", fn);
  return NTLB_OK;
}

extern "C" int ntlb_ep_pack_values(const void* tokens, int x_dtype, int64_t T, int64_t H, int64_t ldt,
                                   const int32_t* pos, const void* topk_idx, int idx_dtype, const void* topk_w,
                                   int w_dtype, int64_t K, int64_t experts_per_rank, const uint32_t* amax_bits,
                                   int64_t gc, int grid, int qmax, int rounding, int scale_rule, uint64_t seed,
                                   uint64_t offset, uint8_t* records, void* stream) {
  const char* fn = "ntlb_ep_pack_values";
  if (K < 1 || experts_per_rank < 1 || T < 0 || (idx_dtype != 0 && idx_dtype != 1) || !valid_dtype(w_dtype))
    return fail(NTLB_EINVAL, "%s: bad argument", fn);
  const int64_t A = T * K;
  if (A > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: more than 2^31 assignments", fn);
  int rc = check_common(fn, tokens, x_dtype, T, H, ldt, grid, qmax, rounding, scale_rule, nullptr, 0, 0);
  if (rc) return rc;
  if (A == 0 || H == 0) return NTLB_OK;
  if (!pos || !topk_idx || !topk_w || !records) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  rc = ep_check_values(fn, tokens, x_dtype, H, ldt, amax_bits, gc, records);
  if (rc) return rc;
  const int64_t R = ntlb_ep_value_record_bytes(H, x_dtype);
  hipStream_t st = as_stream(stream);
  ep_meta_kernel<<<(unsigned)cdiv(A, 256), 256, 0, st>>>(records, R, R - 32, A, pos, topk_idx, idx_dtype, topk_w,
                                                          w_dtype, K, experts_per_rank, H * dtype_size(x_dtype));
  rc = check_launch(fn);
  if (rc) return rc;
  return ep_pack_values_payload(fn, tokens, x_dtype, T, H, ldt, pos, K, A, amax_bits, gc, grid, qmax, rounding,
                                scale_rule, seed, offset, records, R, st);
}

extern "C" int ntlb_ep_pack_return_values(const void* x, int x_dtype, int64_t n, int64_t H, int64_t ldx,
                                          const int32_t* pos, const int32_t* token_idx, const int32_t* slot_idx,
                                          const int32_t* local_expert, const float* weight,
                                          const uint32_t* amax_bits, int64_t gc, int grid, int qmax, int rounding,
                                          int scale_rule, uint64_t seed, uint64_t offset, uint8_t* records,
                                          void* stream) {
  const char* fn = "ntlb_ep_pack_return_values";
  if (n < 0 || n > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: need 0 <= n < 2^31", fn);
  int rc = check_common(fn, x, x_dtype, n, H, ldx, grid, qmax, rounding, scale_rule, nullptr, 0, 0);
  if (rc) return rc;
  if (n == 0 || H == 0) return NTLB_OK;
  if (!pos || !token_idx || !slot_idx || !records) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  rc = ep_check_values(fn, x, x_dtype, H, ldx, amax_bits, gc, records);
  if (rc) return rc;
  const int64_t R = ntlb_ep_value_record_bytes(H, x_dtype);
  hipStream_t st = as_stream(stream);
  ep_meta_rows_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(records, R, R - 32, n, pos, token_idx, slot_idx,
                                                               local_expert, weight, H * dtype_size(x_dtype));
  rc = check_launch(fn);
  if (rc) return rc;
  return ep_pack_values_payload(fn, x, x_dtype, n, H, ldx, pos, 1, n, amax_bits, gc, grid, qmax, rounding, scale_rule,
                                seed, offset, records, R, st);
}
