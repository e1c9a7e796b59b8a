// Expert-parallel dispatch wire format: the one-GPU share of the MoE payload
// exchange of moe.py:670-863 (_build_send_partitions, _dispatch_tokens) and
// of the receive-side grouping of _run_local_experts (moe.py:888-923).
//
// The reference sends five tensors per direction (comm-quantized tokens
// dequantized to bf16, token index, slot index, local expert index, routing
// weight), each with its own all-to-all after a count exchange.  Here every
// routed (token, slot) assignment is one fixed-size record, so one byte
// all-to-all carries everything:
//
//   bytes [0, S_OFF)         e4m3 / int-grid codes of the token row (1x128 tiles;
//                            the columns past H hold zero codes)
//   bytes [S_OFF, +4*ceil(H/128))  the row's fp32 tile scales
//   bytes [M_OFF, +32)       int32 token index, int32 top-k slot, int32 local
//                            expert, int32 NaN flag, fp32 routing weight, 3
//                            reserved words (zero)
//
// with S_OFF = 128*ceil(H/128) (whole tiles, the GEMM's padded K), M_OFF =
// S_OFF + round_up(4*ceil(H/128), 16) and the record size M_OFF + 32
// (ntlb_ep_record_bytes).
//
// Sender: ntlb_ep_partition orders the T*K assignments by destination rank
// (expert / experts_per_rank), stable in assignment order as the reference's
// boolean masks are; ntlb_ep_pack_records (quant.hip) writes the records in
// that order.  Receiver: ntlb_ep_partition on the records' local-expert field
// groups them by local expert, stable in arrival order as the reference's
// per-expert nonzero() is; ntlb_ep_unpack_records gathers codes, scales and
// metadata in that order for the grouped GEMM.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "ntlb_device.h"
#include "ntlb_host.h"

namespace ntlb {

constexpr int EP_BLOCK = 256;  // keys per partition block
constexpr int EP_MAX_BUCKETS = 4096;
constexpr int EP_SCAN_THREADS = 1024;
constexpr int EP_MAX_RANKS = 256;

__device__ __forceinline__ int64_t ep_key(const uint8_t* keys, int key_dt, int64_t stride, int64_t i) {
  const uint8_t* p = keys + i * stride;
  return key_dt == 1 ? *reinterpret_cast<const int64_t*>(p) : (int64_t) * reinterpret_cast<const int32_t*>(p);
}

// bucket of key i: key / divisor, clamped into [0, buckets) so that a bad key
// can never index out of bounds (such input has no meaning to preserve)
__device__ __forceinline__ int ep_bucket(const uint8_t* keys, int key_dt, int64_t stride, int64_t i, int64_t divisor,
                                         int buckets) {
  int64_t b = ep_key(keys, key_dt, stride, i) / divisor;
  b = b < 0 ? 0 : (b >= buckets ? buckets - 1 : b);
  return (int)b;
}

// pass 1: histogram of each block of EP_BLOCK keys, stored bucket-major,
// hist[bucket * nb + block], so that one exclusive scan of the whole array
// gives every (bucket, block) its first output position
__global__ void __launch_bounds__(EP_BLOCK) ep_hist_kernel(const uint8_t* keys, int key_dt, int64_t stride, int64_t n,
                                                           int64_t divisor, int buckets, int32_t* hist) {
  extern __shared__ int32_t h[];
  for (int d = threadIdx.x; d < buckets; d += EP_BLOCK) h[d] = 0;
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * EP_BLOCK + threadIdx.x;
  if (i < n) atomicAdd(&h[ep_bucket(keys, key_dt, stride, i, divisor, buckets)], 1);
  __syncthreads();
  for (int d = threadIdx.x; d < buckets; d += EP_BLOCK) hist[(int64_t)d * gridDim.x + blockIdx.x] = h[d];
}

// exclusive scan of one value per thread over a workgroup of EP_SCAN_THREADS;
// *total = the sum of all values
__device__ __forceinline__ int32_t ep_block_scan(int32_t v, int32_t* wsum, int32_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int32_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t y = __shfl_up(x, d, 64);
    x += lane >= d ? y : 0;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t a = 0;
    for (int k = 0; k < EP_SCAN_THREADS / 64; ++k) {
      const int32_t c = wsum[k];
      wsum[k] = a;
      a += c;
    }
    wsum[EP_SCAN_THREADS / 64] = a;
  }
  __syncthreads();
  *total = wsum[EP_SCAN_THREADS / 64];
  return wsum[w] + x - v;
}

// pass 2 (one workgroup): the bucket-major histogram becomes each (bucket,
// block)'s first output position; counts[d] and offsets[d] (exclusive scan,
// offsets[buckets] = n).  Each thread owns a contiguous segment: sum, scan of
// the sums, then the segment rewritten with its running prefix.
__global__ void __launch_bounds__(EP_SCAN_THREADS) ep_scan_kernel(int32_t* hist, int64_t nb, int buckets,
                                                                  int64_t* counts, int32_t* offsets) {
  __shared__ int32_t base[EP_MAX_BUCKETS + 1];
  __shared__ int32_t wsum[EP_SCAN_THREADS / 64 + 1];
  for (int d = threadIdx.x; d <= buckets; d += EP_SCAN_THREADS) base[d] = 0;  // n == 0: every offset is 0
  const int64_t L = nb * buckets;
  const int64_t seg = (L + EP_SCAN_THREADS - 1) / EP_SCAN_THREADS;
  const int64_t lo = min<int64_t>(L, (int64_t)threadIdx.x * seg), hi = min<int64_t>(L, lo + seg);
  int32_t s = 0;
  for (int64_t j = lo; j < hi; ++j) s += hist[j];
  int32_t total;
  int32_t run = ep_block_scan(s, wsum, &total);  // its barriers also order the base[] clears above
  if (nb > 0) {
    int64_t d = (lo + nb - 1) / nb, next = d * nb;  // first bucket starting at or after lo
    for (int64_t j = lo; j < hi; ++j) {
      if (j == next) {
        base[d] = run;  // bucket d starts with block 0
        ++d;
        next += nb;
      }
      const int32_t c = hist[j];
      hist[j] = run;
      run += c;
    }
  }
  if (threadIdx.x == 0) base[buckets] = total;
  __syncthreads();
  for (int d = threadIdx.x; d <= buckets; d += EP_SCAN_THREADS) {
    if (offsets) offsets[d] = base[d];
    if (counts && d < buckets) counts[d] = base[d + 1] - base[d];
  }
}

// pass 3: pos[i] = first position of (bucket, block) + number of earlier keys
// of the block in the same bucket (stable); inv[pos[i]] = i
__global__ void __launch_bounds__(EP_BLOCK) ep_place_kernel(const uint8_t* keys, int key_dt, int64_t stride,
                                                            int64_t n, int64_t divisor, int buckets,
                                                            const int32_t* start, int32_t* pos, int32_t* inv) {
  __shared__ int32_t kb[EP_BLOCK];
  const int64_t i = (int64_t)blockIdx.x * EP_BLOCK + threadIdx.x;
  const int b = i < n ? ep_bucket(keys, key_dt, stride, i, divisor, buckets) : -1;
  kb[threadIdx.x] = b;
  __syncthreads();
  if (i >= n) return;
  int rank = 0;
  for (int j = 0; j < (int)threadIdx.x; ++j) rank += kb[j] == b ? 1 : 0;
  const int32_t p = start[(int64_t)b * gridDim.x + blockIdx.x] + rank;
  if (pos) pos[i] = p;
  if (inv) inv[p] = (int32_t)i;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// prefix of the received counts per source rank, passed by value
struct RankOffsets {
  int32_t v[EP_MAX_RANKS + 1];
};

// receiver gather: output row i < rows is record inv[i] of the n records; codes, scales (at
// scales[i*s_row + t*s_col]), NaN flag and metadata, and the source rank of
// the record (the s with ro.v[s] <= inv[i] < ro.v[s+1]).  A wave per row; the
// vector path issues up to eight 16-byte loads per lane before their stores.
// TILES: a code record (Hp code bytes, then tile scales); otherwise a value
// record (Hp payload bytes, no scales)
template <bool VEC, bool TILES = true>
__global__ void __launch_bounds__(256) ep_gather_kernel(const uint8_t* __restrict__ rec, int64_t n, int64_t rows,
                                                        int64_t Hp,
                                                        int64_t R, int64_t s_off, int64_t m_off,
                                                        const int32_t* __restrict__ inv, RankOffsets ro, int ep_size,
                                                        uint8_t* __restrict__ codes, int64_t ldc,
                                                        float* __restrict__ scales, int64_t s_row, int64_t s_col,
                                                        int32_t* nan_rows, int32_t* token_idx, int32_t* slot_idx,
                                                        int32_t* src_rank, float* weight) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // four rows per workgroup, a wave each
  const int lane = threadIdx.x & 63;
  if (i >= rows) return;
  const int64_t src = min<int64_t>(max<int32_t>(inv[i], 0), n - 1);  // a record index, clamped into the n records
  const uint8_t* r = rec + src * R;
  uint8_t* out = codes + i * ldc;
  const int64_t nt = TILES ? Hp >> 7 : 0;
  const float* sc = reinterpret_cast<const float*>(r + s_off);
  const int32_t* m = reinterpret_cast<const int32_t*>(r + m_off);
  // lane l < nt takes tile scale l, lanes 0-4 the metadata words (token, slot,
  // local expert, NaN flag, weight); both loads clamped into the record
  float s_l = TILES ? sc[min<int64_t>(lane, nt - 1)] : 0.f;
  int32_t m_l = m[min(lane, 7)];
  if constexpr (VEC) {
    constexpr int U = 8;
    for (int64_t c0 = 0; c0 < Hp; c0 += 64 * 16 * U) {
      // offsets clamped into the row (Hp >= 128): a lane past the end loads and
      // stores the row's last 16 bytes again, the same bytes to the same place,
      // which keeps the eight loads unconditional and ahead of the stores
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = min<int64_t>(c0 + (int64_t)(u * 64 + lane) * 16, Hp - 16);
        v[u] = *reinterpret_cast<const u32x4*>(r + c);
      }
      // the loads all complete here, before the first store (left alone, the
      // scheduler pairs each load with its store and waits on each)
      asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]),
                   "+v"(v[7]), "+v"(s_l), "+v"(m_l));
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = min<int64_t>(c0 + (int64_t)(u * 64 + lane) * 16, Hp - 16);
        *reinterpret_cast<u32x4*>(out + c) = v[u];
      }
    }
  } else {
    for (int64_t c = lane; c < Hp; c += 64) out[c] = r[c];
  }
  if constexpr (TILES) {
    if (lane < nt) scales[i * s_row + lane * s_col] = s_l;
    for (int64_t t = 64 + lane; t < nt; t += 64) scales[i * s_row + t * s_col] = sc[t];
  }
  if (lane == 0 && token_idx) token_idx[i] = m_l;
  if (lane == 1 && slot_idx) slot_idx[i] = m_l;
  if (lane == 3 && nan_rows) nan_rows[i] = m_l;
  if (lane == 4 && weight) weight[i] = __int_as_float(m_l);
  if (lane == 5 && src_rank) {
    int lo = 0, hi = ep_size - 1;  // the last s with ro.v[s] <= src
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (ro.v[mid] <= src) lo = mid; else hi = mid - 1;
    }
    src_rank[i] = lo;
  }
}

// ---------------------------------------------------------------------------
// Combine (moe.py:964-1038): every returned record is the expert output of one
// (token, slot) assignment; out[t] = sum over the token's slots of
// w[t, slot] * dequant(record), formed as the reference's index_add_ into
// zeros forms it on the CPU: each product rounded to the output dtype (a
// tensor op of that dtype), the products summed in fp32 in arrival order --
// for one token, ascending global expert id (ranks in order, local experts in
// order) -- and the sum rounded once.
// ---------------------------------------------------------------------------
constexpr int EP_COMBINE_MAX_K = 32;

__global__ void __launch_bounds__(256) ep_slot_fill_kernel(int32_t* slot_map, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) slot_map[i] = -1;
}

// slot_map[token * K + slot] = the record carrying that assignment; records
// whose (token, slot) lies outside [0, T) x [0, K) are ignored
__global__ void __launch_bounds__(256) ep_slot_scatter_kernel(const uint8_t* rec, int64_t n, int64_t R, int64_t m_off,
                                                              int64_t T, int K, int32_t* slot_map) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= n) return;
  const int32_t* m = reinterpret_cast<const int32_t*>(rec + r * R + m_off);
  const int32_t t = m[0], k = m[1];
  if (t >= 0 && t < T && k >= 0 && k < K) slot_map[(int64_t)t * K + k] = (int32_t)r;
}

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// two floats rounded to bf16 by the hardware pack-convert (v_cvt_pk_bf16_f32,
// round to nearest even like f32_to_bf16_bits; a NaN stays a NaN), as their
// packed bits
__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
  const v2bf p = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, p);
}

// the eight codes of two words as floats: e4m3 by the hardware converter
// (v_cvt_pk_f32_fp8, OCP e4m3fn), the int grid as int8 with -128 the NaN code
template <int GRID>
__device__ __forceinline__ void decode8(uint2 cw, float (&q)[8]) {
  const uint32_t wd[2] = {cw.x, cw.y};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if constexpr (GRID == GRID_E4M3) {
      const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)wd[h], false);
      const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)wd[h], true);
      q[4 * h + 0] = lo[0];
      q[4 * h + 1] = lo[1];
      q[4 * h + 2] = hi[0];
      q[4 * h + 3] = hi[1];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t c = (wd[h] >> (8 * i)) & 0xFFu;
        q[4 * h + i] = c == 0x80u ? __uint_as_float(0x7FC00000u) : (float)(int8_t)c;
      }
    }
  }
}

// eight values rounded to the output dtype (in place)
template <int OUT_DT>
__device__ __forceinline__ void round8(float (&v)[8]) {
  if constexpr (OUT_DT == DT_BF16) {
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const uint32_t b = bf16x2_bits(v[i], v[i + 1]);
      v[i] = __uint_as_float(b << 16);
      v[i + 1] = __uint_as_float(b & 0xFFFF0000u);
    }
  } else if constexpr (OUT_DT == DT_F16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __half2float(f32_to_f16(v[i]));
  }
}

// one workgroup per token; thread j owns columns [8j + 2048i, +8)
template <int GRID, int OUT_DT>
__global__ void __launch_bounds__(256) ep_combine_kernel(const uint8_t* rec, int64_t n, int64_t R, int64_t s_off,
                                                         int64_t H, const int32_t* slot_map, const void* topk_idx,
                                                         int idx_dt, const void* topk_w, int w_dt, int K, void* out,
                                                         int64_t ldo, int vec_out) {
#pragma clang fp contract(off)  // each product and sum rounds on its own, as the reference's torch ops do
  __shared__ int64_t s_e[EP_COMBINE_MAX_K];
  __shared__ int32_t s_rec[EP_COMBINE_MAX_K];
  __shared__ float s_w[EP_COMBINE_MAX_K];
  const int64_t t = blockIdx.x;
  const int k = threadIdx.x;
  if (k < K) {
    const int64_t a = t * K + k;
    s_e[k] = idx_dt == 1 ? reinterpret_cast<const int64_t*>(topk_idx)[a]
                         : (int64_t) reinterpret_cast<const int32_t*>(topk_idx)[a];
  }
  __syncthreads();
  if (k < K) {
    // slot k's place in ascending expert id (ties, which routing does not
    // produce, keep slot order)
    const int64_t ek = s_e[k];
    int rank = 0;
    for (int j = 0; j < K; ++j) rank += (s_e[j] < ek || (s_e[j] == ek && j < k)) ? 1 : 0;
    s_rec[rank] = slot_map[t * K + k];
    s_w[rank] = load_elem(topk_w, w_dt, t * K + k);
  }
  __syncthreads();
  for (int64_t c0 = (int64_t)threadIdx.x * 8; c0 < H; c0 += 256 * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; n > 0 && j0 < K; j0 += 8) {  // n == 0: nothing came back, the outputs are zero
      // up to eight records' codes and scales in flight at once: slots past K
      // or without a record read record 0 and are not added
      uint2 cw[8];
      float sc[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = min(j0 + u, K - 1);
        const uint8_t* rp = rec + (int64_t)max(s_rec[j], 0) * R;
        cw[u] = *reinterpret_cast<const uint2*>(rp + c0);
        sc[u] = reinterpret_cast<const float*>(rp + s_off)[c0 >> 7];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u;
        if (j >= K || s_rec[j] < 0) continue;  // past K, or dropped by a capacity limit: never returned
        float v[8];
        decode8<GRID>(cw[u], v);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = v[i] * sc[u];
        round8<OUT_DT>(v);  // the dequantized row in the output dtype
        const float w = s_w[j];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = v[i] * w;
        round8<OUT_DT>(v);  // the product, a tensor op of the output dtype
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = acc[i] + v[i];
      }
    }
    // the one rounding of the sum
    if constexpr (OUT_DT == DT_BF16) {
      uint32_t pk[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pk[i] = bf16x2_bits(acc[2 * i], acc[2 * i + 1]);
      uint16_t* o = reinterpret_cast<uint16_t*>(out) + t * ldo + c0;
      if (vec_out) {
        store16_nt(o, pk);  // token rows the next layer reads: 4% faster at c4 with the hint
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (uint16_t)(pk[i >> 1] >> (16 * (i & 1)));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) store_elem(out, OUT_DT, t * ldo + c0 + i, acc[i]);
    }
  }
}

// Single-rank combine of the local expert outputs (moe.py:1087-1088 and
// :489-490, `output[token_indices] += expert_out * weights` once per expert in
// ascending expert id): one workgroup of 128 threads per token t; thread j
// owns columns [8j + 1024i, +8) (H 7168: seven chunks each, none idle; 256
// threads left half the last pass idle).  Slot s of t names row pos[t*K + s] of y (rows in expert
// order, clamped below n; negative: dropped by a capacity limit, adds
// nothing).  Per expert,
// the product is rounded to the promoted dtype of y and w (ROUND_P: both the
// output dtype) and the sum to the output dtype, as the two torch ops do.
constexpr int COMBINE_ROWS_THREADS = 128;

template <int OUT_DT, bool ROUND_P>
__global__ void __launch_bounds__(COMBINE_ROWS_THREADS) moe_combine_rows_kernel(const void* y, int64_t ldy, int64_t n,
                                                               const int32_t* pos,
                                                               const void* topk_idx, int idx_dt, const void* topk_w,
                                                               int w_dt, int K, int64_t H, void* out, int64_t ldo,
                                                               int vec) {
#pragma clang fp contract(off)  // each product and sum rounds on its own
  __shared__ int64_t s_e[EP_COMBINE_MAX_K];
  __shared__ int32_t s_row[EP_COMBINE_MAX_K];
  __shared__ float s_w[EP_COMBINE_MAX_K];
  const int64_t t = blockIdx.x;
  const int k = threadIdx.x;
  if (k < K) {
    const int64_t a = t * K + k;
    s_e[k] = idx_dt == 1 ? reinterpret_cast<const int64_t*>(topk_idx)[a]
                         : (int64_t) reinterpret_cast<const int32_t*>(topk_idx)[a];
  }
  __syncthreads();
  if (k < K) {
    // slot k's place in ascending expert id (ties, which routing does not
    // produce, keep slot order)
    const int64_t ek = s_e[k];
    int rank = 0;
    for (int j = 0; j < K; ++j) rank += (s_e[j] < ek || (s_e[j] == ek && j < k)) ? 1 : 0;
    s_row[rank] = pos[t * K + k];
    s_w[rank] = load_elem(topk_w, w_dt, t * K + k);
  }
  __syncthreads();
  if constexpr (OUT_DT == DT_BF16) {
    if (vec && K <= 8) {
      // bf16 rows, up to 8 slots: the raw 16-byte chunks of two column steps
      // (all slots) are loaded before either is summed, twice the loads in
      // flight of the general loop below (c4 combine: 127 -> 112 us; three or
      // four steps measured the same, seven slower).  Same operation order,
      // so the same bits.
      constexpr int64_t STEP = COMBINE_ROWS_THREADS * 8;
      constexpr int D = 2;
      for (int64_t c0 = (int64_t)threadIdx.x * 8; c0 < H; c0 += D * STEP) {
        uint4 raw[D][8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int j = min(u, K - 1);
          const uint16_t* rowp = reinterpret_cast<const uint16_t*>(y) + min<int64_t>(max(s_row[j], 0), n - 1) * ldy;
#pragma unroll
          for (int h = 0; h < D; ++h)
            raw[h][u] = c0 + h * STEP < H ? *reinterpret_cast<const uint4*>(rowp + c0 + h * STEP) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int h = 0; h < D; ++h) {
          if (c0 + h * STEP >= H) break;
          float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            if (u >= K || s_row[u] < 0) continue;
            const uint32_t ww[4] = {raw[h][u].x, raw[h][u].y, raw[h][u].z, raw[h][u].w};
            float p[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              p[2 * i] = __uint_as_float(ww[i] << 16) * s_w[u];
              p[2 * i + 1] = __uint_as_float(ww[i] & 0xFFFF0000u) * s_w[u];
            }
            if constexpr (ROUND_P) round8<OUT_DT>(p);  // expert_out * weights in the output dtype
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = acc[i] + p[i];
            round8<OUT_DT>(acc);  // output[token_indices] += ..., an op of the output dtype
          }
          uint32_t pk[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) pk[i] = bf16x2_bits(acc[2 * i], acc[2 * i + 1]);
          // non-temporal, as the EP combine's token rows (c4: 111 -> 106 us)
          store16_nt(reinterpret_cast<uint16_t*>(out) + t * ldo + c0 + h * STEP, pk);
        }
      }
      return;
    }
  }
  for (int64_t c0 = (int64_t)threadIdx.x * 8; c0 < H; c0 += COMBINE_ROWS_THREADS * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < K; j0 += 8) {
      // up to eight rows in flight at once: slots past K or dropped read row
      // 0 of y and are not added
      float v[8][8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = min(j0 + u, K - 1);
        const int64_t off = min<int64_t>(max(s_row[j], 0), n - 1) * ldy + c0;
        if constexpr (OUT_DT == DT_BF16) {
          if (vec) {
            const uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(y) + off);
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              v[u][2 * i] = __uint_as_float(ww[i] << 16);
              v[u][2 * i + 1] = __uint_as_float(ww[i] & 0xFFFF0000u);
            }
            continue;
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[u][i] = c0 + i < H ? load_elem(y, OUT_DT, off + i) : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u;
        if (j >= K || s_row[j] < 0) continue;
        const float w = s_w[j];
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = v[u][i] * w;
        if constexpr (ROUND_P) round8<OUT_DT>(p);  // expert_out * weights in the output dtype
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = acc[i] + p[i];
        round8<OUT_DT>(acc);  // output[token_indices] += ..., an op of the output dtype
      }
    }
    if constexpr (OUT_DT == DT_BF16) {
      if (vec) {
        uint32_t pk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pk[i] = bf16x2_bits(acc[2 * i], acc[2 * i + 1]);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + t * ldo + c0) =
            make_uint4(pk[0], pk[1], pk[2], pk[3]);
        continue;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (c0 + i < H) store_elem(out, OUT_DT, t * ldo + c0 + i, acc[i]);
  }
}

// The combine over records that carry the reference's wire values instead of
// codes (the channel comm-quant: moe.py:112-121 applied to the send-back
// buffer, whose per-column scales a record's tile scales cannot hold): the
// payload is a row of VAL_DT values at the record's start, the metadata at
// R - 32.  The sum is ep_combine_kernel's: per token, the kept slots in
// ascending expert id, each value in the output dtype times its weight
// rounded to it, added in fp32, rounded once.
template <int VAL_DT, int OUT_DT>
__global__ void __launch_bounds__(256) ep_combine_values_kernel(const uint8_t* rec, int64_t n, int64_t R, int64_t H,
                                                                const int32_t* slot_map, const void* topk_idx,
                                                                int idx_dt, const void* topk_w, int w_dt, int K,
                                                                void* out, int64_t ldo, int vec_out) {
#pragma clang fp contract(off)
  __shared__ int64_t s_e[EP_COMBINE_MAX_K];
  __shared__ int32_t s_rec[EP_COMBINE_MAX_K];
  __shared__ float s_w[EP_COMBINE_MAX_K];
  const int64_t t = blockIdx.x;
  const int k = threadIdx.x;
  if (k < K) {
    const int64_t a = t * K + k;
    s_e[k] = idx_dt == 1 ? reinterpret_cast<const int64_t*>(topk_idx)[a]
                         : (int64_t) reinterpret_cast<const int32_t*>(topk_idx)[a];
  }
  __syncthreads();
  if (k < K) {
    const int64_t ek = s_e[k];
    int rank = 0;
    for (int j = 0; j < K; ++j) rank += (s_e[j] < ek || (s_e[j] == ek && j < k)) ? 1 : 0;
    s_rec[rank] = slot_map[t * K + k];
    s_w[rank] = load_elem(topk_w, w_dt, t * K + k);
  }
  __syncthreads();
  constexpr int esz = VAL_DT == DT_F32 ? 4 : 2;
  for (int64_t c0 = (int64_t)threadIdx.x * 8; c0 < H; c0 += 256 * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; n > 0 && j < K; ++j) {
      if (s_rec[j] < 0) continue;  // dropped by a capacity limit: never returned
      const uint8_t* rp = rec + (int64_t)s_rec[j] * R + c0 * esz;
      float v[8];
      if constexpr (VAL_DT == DT_F32) {
        const uint4 a = *reinterpret_cast<const uint4*>(rp), b = *reinterpret_cast<const uint4*>(rp + 16);
        const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(u[i]);
      } else {
        const uint4 a = *reinterpret_cast<const uint4*>(rp);
        const uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t hb = (u[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
          v[i] = VAL_DT == DT_BF16 ? bf16_bits_to_f32(hb) : __half2float(__ushort_as_half((unsigned short)hb));
        }
      }
      round8<OUT_DT>(v);  // the received row in the output dtype
      const float w = s_w[j];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = v[i] * w;
      round8<OUT_DT>(v);  // the product, a tensor op of the output dtype
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = acc[i] + v[i];
    }
    if constexpr (OUT_DT == DT_BF16) {
      uint32_t pk[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pk[i] = bf16x2_bits(acc[2 * i], acc[2 * i + 1]);
      uint16_t* o = reinterpret_cast<uint16_t*>(out) + t * ldo + c0;
      if (vec_out) {
        store16_nt(o, pk);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (uint16_t)(pk[i >> 1] >> (16 * (i & 1)));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) store_elem(out, OUT_DT, t * ldo + c0 + i, acc[i]);
    }
  }
}

}  // namespace ntlb

using namespace ntlb;

extern "C" int64_t ntlb_ep_record_bytes(int64_t H) {
  if (H <= 0) return 0;
  const int64_t s_off = (H + 127) / 128 * 128;
  const int64_t m_off = s_off + ((H + 127) / 128 * 4 + 15) / 16 * 16;
  return m_off + 32;
}

extern "C" int ntlb_ep_partition(const void* keys, int key_dtype, int64_t key_stride, int64_t n, int64_t divisor,
                                 int buckets, int32_t* pos, int32_t* inv, int64_t* counts, int32_t* offsets,
                                 int32_t* ws, int64_t ws_elems, void* stream) {
  const char* fn = "ntlb_ep_partition";
  if (n < 0 || n > 0x7FFFFFFF || divisor < 1 || buckets < 1 || buckets > EP_MAX_BUCKETS)
    return fail(NTLB_EINVAL, "%s: need 0 <= n < 2^31, divisor >= 1 and 1 <= buckets <= %d", fn, EP_MAX_BUCKETS);
  if (key_dtype != 0 && key_dtype != 1) return fail(NTLB_EINVAL, "%s: key_dtype is 0 (int32) or 1 (int64)", fn);
  const int64_t ksz = key_dtype ? 8 : 4;
  if (key_stride < ksz || key_stride % ksz) return fail(NTLB_EINVAL, "%s: key_stride must be a multiple of the key size", fn);
  if (n > 0 && (!keys || !aligned(keys, ksz))) return fail(NTLB_EINVAL, "%s: keys NULL or misaligned", fn);
  const int64_t nb = cdiv(n, EP_BLOCK);
  if (n > 0 && (!ws || ws_elems < nb * buckets)) return fail(NTLB_EINVAL, "%s: workspace needs %lld int32", fn,
                                                             (long long)(nb * buckets));
  hipStream_t st = as_stream(stream);
  const uint8_t* k = reinterpret_cast<const uint8_t*>(keys);
  if (n > 0)
    ep_hist_kernel<<<(unsigned)nb, EP_BLOCK, buckets * sizeof(int32_t), st>>>(k, key_dtype, key_stride, n, divisor,
                                                                             buckets, ws);
  ep_scan_kernel<<<1, EP_SCAN_THREADS, 0, st>>>(ws, nb, buckets, counts, offsets);
  if (n > 0)
    ep_place_kernel<<<(unsigned)nb, EP_BLOCK, 0, st>>>(k, key_dtype, key_stride, n, divisor, buckets, ws, pos, inv);
  return check_launch(fn);
}

extern "C" int ntlb_ep_unpack_records(const uint8_t* records, int64_t n, int64_t H, const int32_t* inv, int64_t rows,
                                      const int64_t* recv_offsets, int ep_size, uint8_t* codes, int64_t ldc,
                                      float* scales, int64_t s_row, int64_t s_col, int32_t* nan_rows,
                                      int32_t* token_idx, int32_t* slot_idx, int32_t* src_rank, float* weight,
                                      void* stream) {
  const char* fn = "ntlb_ep_unpack_records";
  const int64_t Hp = (H + 127) / 128 * 128;  // codes with their zero padding
  if (n < 0 || n > 0x7FFFFFFF || rows < 0 || (rows > 0 && n == 0) || H <= 0 || ldc < Hp)
    return fail(NTLB_EINVAL, "%s: bad shape (0 <= n < 2^31, rows >= 0 with records to read, ldc >= 128*ceil(H/128))",
                fn);
  RankOffsets ro{};
  if (src_rank) {
    if (!recv_offsets || ep_size < 1 || ep_size > EP_MAX_RANKS)
      return fail(NTLB_EINVAL, "%s: src_rank needs recv_offsets and 1 <= ep_size <= %d", fn, EP_MAX_RANKS);
    if (recv_offsets[0] != 0 || recv_offsets[ep_size] != n)
      return fail(NTLB_EINVAL, "%s: recv_offsets must run from 0 to n", fn);
    for (int s = 0; s <= ep_size; ++s) {
      if (s > 0 && recv_offsets[s] < recv_offsets[s - 1])
        return fail(NTLB_EINVAL, "%s: recv_offsets must not decrease", fn);
      ro.v[s] = (int32_t)recv_offsets[s];
    }
  }
  if (rows == 0) return NTLB_OK;
  if (!records || !inv || !codes || !scales) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (!aligned(records, 16)) return fail(NTLB_EINVAL, "%s: records must be 16-byte aligned", fn);
  const int64_t R = ntlb_ep_record_bytes(H);
  const int64_t s_off = Hp;
  const int64_t m_off = R - 32;
  const bool vec = aligned(codes, 16) && ldc % 16 == 0;
  dim3 grd((unsigned)cdiv(rows, 4)), blk(256);
  hipStream_t st = as_stream(stream);
  if (vec)
    ep_gather_kernel<true><<<grd, blk, 0, st>>>(records, n, rows, Hp, R, s_off, m_off, inv, ro, ep_size, codes, ldc, scales,
                                                 s_row, s_col, nan_rows, token_idx, slot_idx, src_rank, weight);
  else
    ep_gather_kernel<false><<<grd, blk, 0, st>>>(records, n, rows, Hp, R, s_off, m_off, inv, ro, ep_size, codes, ldc, scales,
                                                  s_row, s_col, nan_rows, token_idx, slot_idx, src_rank, weight);
  return check_launch(fn);
}

extern "C" int ntlb_ep_unpack_values(const uint8_t* records, int64_t n, int64_t H, int val_dtype, const int32_t* inv,
                                     int64_t rows, const int64_t* recv_offsets, int ep_size, void* values, int64_t ldv,
                                     int32_t* token_idx, int32_t* slot_idx, int32_t* src_rank, float* weight,
                                     void* stream) {
  const char* fn = "ntlb_ep_unpack_values";
  if (n < 0 || n > 0x7FFFFFFF || rows < 0 || (rows > 0 && n == 0) || H <= 0 || H % 8 != 0 || ldv < H ||
      !valid_dtype(val_dtype))
    return fail(NTLB_EINVAL, "%s: bad shape or dtype (0 <= n < 2^31, rows >= 0 with records to read, H %% 8 == 0, "
                "ldv >= H)", fn);
  RankOffsets ro{};
  if (src_rank) {
    if (!recv_offsets || ep_size < 1 || ep_size > EP_MAX_RANKS)
      return fail(NTLB_EINVAL, "%s: src_rank needs recv_offsets and 1 <= ep_size <= %d", fn, EP_MAX_RANKS);
    if (recv_offsets[0] != 0 || recv_offsets[ep_size] != n)
      return fail(NTLB_EINVAL, "%s: recv_offsets must run from 0 to n", fn);
    for (int s = 0; s <= ep_size; ++s) {
      if (s > 0 && recv_offsets[s] < recv_offsets[s - 1])
        return fail(NTLB_EINVAL, "%s: recv_offsets must not decrease", fn);
      ro.v[s] = (int32_t)recv_offsets[s];
    }
  }
  if (rows == 0) return NTLB_OK;
  if (!records || !inv || !values) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  const int64_t esz = dtype_size(val_dtype);
  if (!aligned(records, 16) || !aligned(values, 16) || (ldv * esz) % 16)
    return fail(NTLB_EINVAL, "%s: records and value rows must be 16-byte aligned", fn);
  const int64_t R = ntlb_ep_value_record_bytes(H, val_dtype);
  dim3 grd((unsigned)cdiv(rows, 4)), blk(256);
  ep_gather_kernel<true, false><<<grd, blk, 0, as_stream(stream)>>>(
      records, n, rows, H * esz, R, 0, R - 32, inv, ro, ep_size, reinterpret_cast<uint8_t*>(values), ldv * esz,
      nullptr, 0, 0, nullptr, token_idx, slot_idx, src_rank, weight);
  return check_launch(fn);
}

extern "C" int ntlb_ep_combine_values(const uint8_t* records, int64_t n, int64_t H, int val_dtype,
                                      const void* topk_idx, int idx_dtype, const void* topk_w, int w_dtype, int64_t T,
                                      int64_t K, void* out, int out_dtype, int64_t ldo, int32_t* slot_map,
                                      void* stream) {
  const char* fn = "ntlb_ep_combine_values";
  if (n < 0 || n > 0x7FFFFFFF || T < 0 || K < 1 || K > EP_COMBINE_MAX_K || H <= 0 || H % 8 != 0 || ldo < H)
    return fail(NTLB_EINVAL, "%s: bad shape (H %% 8 == 0, 1 <= K <= %d, ldo >= H)", fn, EP_COMBINE_MAX_K);
  if ((idx_dtype != 0 && idx_dtype != 1) || !valid_dtype(w_dtype) || !valid_dtype(out_dtype) || !valid_dtype(val_dtype))
    return fail(NTLB_EINVAL, "%s: bad dtype", fn);
  if (T == 0) return NTLB_OK;
  if (!topk_idx || !topk_w || !out || !slot_map || (n > 0 && !records)) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (n > 0 && !aligned(records, 16)) return fail(NTLB_EINVAL, "%s: records must be 16-byte aligned", fn);
  if (T * K > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: more than 2^31 assignments", fn);
  const int64_t R = ntlb_ep_value_record_bytes(H, val_dtype);
  hipStream_t st = as_stream(stream);
  ep_slot_fill_kernel<<<(unsigned)cdiv(T * K, 256), 256, 0, st>>>(slot_map, T * K);
  if (n > 0)
    ep_slot_scatter_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(records, n, R, R - 32, T, (int)K, slot_map);
  const int vec = aligned(out, 16) && ldo % 8 == 0;
  auto launch = [&](auto valc, auto outc) {
    ep_combine_values_kernel<decltype(valc)::value, decltype(outc)::value><<<(unsigned)T, 256, 0, st>>>(
        records, n, R, H, slot_map, topk_idx, idx_dtype, topk_w, w_dtype, (int)K, out, ldo, vec);
  };
  using B = std::integral_constant<int, DT_BF16>;
  using F = std::integral_constant<int, DT_F32>;
  using Hh = std::integral_constant<int, DT_F16>;
  auto by_out = [&](auto valc) {
    if (out_dtype == NTLB_BF16) launch(valc, B()); else if (out_dtype == NTLB_F32) launch(valc, F()); else launch(valc, Hh());
  };
  if (val_dtype == NTLB_BF16) by_out(B()); else if (val_dtype == NTLB_F32) by_out(F()); else by_out(Hh());
  return check_launch(fn);
}

extern "C" int ntlb_ep_combine(const uint8_t* records, int64_t n, int64_t H, const void* topk_idx, int idx_dtype,
                               const void* topk_w, int w_dtype, int64_t T, int64_t K, int grid, void* out,
                               int out_dtype, int64_t ldo, int32_t* slot_map, void* stream) {
  const char* fn = "ntlb_ep_combine";
  if (n < 0 || n > 0x7FFFFFFF || T < 0 || K < 1 || K > EP_COMBINE_MAX_K || H <= 0 || H % 8 != 0 || ldo < H)
    return fail(NTLB_EINVAL, "%s: bad shape (H %% 8 == 0, 1 <= K <= %d, ldo >= H)", fn, EP_COMBINE_MAX_K);
  if ((idx_dtype != 0 && idx_dtype != 1) || !valid_dtype(w_dtype) || !valid_dtype(out_dtype) ||
      (grid != NTLB_GRID_INT && grid != NTLB_GRID_E4M3))
    return fail(NTLB_EINVAL, "%s: bad dtype or grid", fn);
  if (T == 0) return NTLB_OK;
  if (!topk_idx || !topk_w || !out || !slot_map || (n > 0 && !records)) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (n > 0 && !aligned(records, 16)) return fail(NTLB_EINVAL, "%s: records must be 16-byte aligned", fn);
  if (T * K > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: more than 2^31 assignments", fn);
  const int64_t R = ntlb_ep_record_bytes(H);
  const int64_t s_off = (H + 127) / 128 * 128;
  hipStream_t st = as_stream(stream);
  ep_slot_fill_kernel<<<(unsigned)cdiv(T * K, 256), 256, 0, st>>>(slot_map, T * K);
  if (n > 0)
    ep_slot_scatter_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(records, n, R, R - 32, T, (int)K, slot_map);
  const int vec = aligned(out, 16) && ldo % 8 == 0;
  auto launch = [&](auto gridc, auto outc) {
    ep_combine_kernel<decltype(gridc)::value, decltype(outc)::value><<<(unsigned)T, 256, 0, st>>>(
        records, n, R, s_off, H, slot_map, topk_idx, idx_dtype, topk_w, w_dtype, (int)K, out, ldo, vec);
  };
  using I = std::integral_constant<int, GRID_INT>;
  using E = std::integral_constant<int, GRID_E4M3>;
  using B = std::integral_constant<int, DT_BF16>;
  using F = std::integral_constant<int, DT_F32>;
  using Hh = std::integral_constant<int, DT_F16>;
  if (grid == NTLB_GRID_E4M3) {
    if (out_dtype == NTLB_BF16) launch(E(), B()); else if (out_dtype == NTLB_F32) launch(E(), F()); else launch(E(), Hh());
  } else {
    if (out_dtype == NTLB_BF16) launch(I(), B()); else if (out_dtype == NTLB_F32) launch(I(), F()); else launch(I(), Hh());
  }
  return check_launch(fn);
}

extern "C" int ntlb_moe_combine_rows(const void* y, int64_t ldy, int64_t n, const int32_t* pos, const void* topk_idx,
                                     int idx_dtype, const void* topk_w, int w_dtype, int64_t T, int64_t K,
                                     int64_t H, void* out, int out_dtype, int64_t ldo, void* stream) {
  const char* fn = "ntlb_moe_combine_rows";
  if (T < 0 || H < 0 || n < 0 || K < 1 || K > EP_COMBINE_MAX_K || (idx_dtype != 0 && idx_dtype != 1) ||
      !valid_dtype(w_dtype) || !valid_dtype(out_dtype))
    return fail(NTLB_EINVAL, "%s: bad argument (1 <= K <= %d)", fn, EP_COMBINE_MAX_K);
  if (ldy < H || ldo < H) return fail(NTLB_EINVAL, "%s: ldy and ldo must be >= H", fn);
  if (T == 0 || H == 0) return NTLB_OK;
  if (!out || !pos || !topk_idx || !topk_w || (n > 0 && !y)) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (n == 0) return fail(NTLB_EINVAL, "%s: no expert rows for %lld tokens", fn, (long long)T);
  hipStream_t st = as_stream(stream);
  const int vec = aligned(y, 16) && aligned(out, 16) && ldy % 8 == 0 && ldo % 8 == 0 && H % 8 == 0;
  // the product rounds to the output dtype when torch's promotion of (y, w)
  // is that dtype: w of the same dtype, which is not fp32
  const bool round_p = w_dtype == out_dtype && out_dtype != NTLB_F32;
  auto launch = [&](auto outc, auto rpc) {
    moe_combine_rows_kernel<decltype(outc)::value, decltype(rpc)::value><<<(unsigned)T, COMBINE_ROWS_THREADS, 0, st>>>(
        y, ldy, n, pos, topk_idx, idx_dtype, topk_w, w_dtype, (int)K, H, out, ldo, vec);
  };
  using B = std::integral_constant<int, DT_BF16>;
  using F = std::integral_constant<int, DT_F32>;
  using Hh = std::integral_constant<int, DT_F16>;
  using Y = std::integral_constant<bool, true>;
  using N = std::integral_constant<bool, false>;
  if (out_dtype == NTLB_BF16) {
    if (round_p) launch(B(), Y()); else launch(B(), N());
  } else if (out_dtype == NTLB_F16) {
    if (round_p) launch(Hh(), Y()); else launch(Hh(), N());
  } else {
    launch(F(), N());
  }
  return check_launch(fn);
}
