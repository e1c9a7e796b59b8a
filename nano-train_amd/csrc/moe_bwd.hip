// The routed expert loop's capacity keep and the elementwise parts of its
// backward (src/models/moe.py:1062-1093 and :476-491 of nano-train, where each
// expert's rows pass through ExpertMLP, moe.py:190-193, and
// `output[token_indices] += expert_out * weights`):
//
//   moe_capacity_keep: per expert, the rows torch.topk(sort_weights,
//     k=capacity, sorted=True) keeps (moe.py:1077-1081, :482-486), highest
//     routing weight first, as a new row order, its offset table and the
//     assignment -> row map (-1 for a dropped assignment);
//   moe_combine_backward: the gradient of the combine: dY[row] =
//     d_out[token] * w in y's dtype and d_w = sum over H of d_out[token] *
//     y[row] in fp32, each product first rounded to y's dtype when w has
//     that 16-bit dtype (autograd's mul backward forms the bf16 products,
//     then sums them);
//   swiglu_backward: the gradient of gated = silu(gate) * up through torch's
//     bf16 op sequence (F.silu, mul), in B's interleaved gate / up columns.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "ntlb_device.h"
#include "ntlb_host.h"

namespace ntlb {

constexpr int CAP_THREADS = 256;

// kept rows per expert (all of them when capacity <= 0) and their prefix
__global__ void __launch_bounds__(CAP_THREADS) capacity_offsets_kernel(const int32_t* offsets, int n_experts,
                                                                       int64_t capacity, int32_t* offsets_out,
                                                                       int64_t* counts_out) {
  if (threadIdx.x != 0) return;
  int32_t acc = 0;
  offsets_out[0] = 0;
  for (int e = 0; e < n_experts; ++e) {
    int64_t n = (int64_t)offsets[e + 1] - offsets[e];
    if (capacity > 0 && n > capacity) n = capacity;
    counts_out[e] = n;
    acc += (int32_t)n;
    offsets_out[e + 1] = acc;
  }
}

__global__ void __launch_bounds__(CAP_THREADS) fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

// Workgroup (e, c) ranks rows c*256 .. c*256+255 of expert e.  A row's rank
// is the number of the expert's rows with a larger weight, or an equal
// weight and a lower row (the order torch.topk(sorted=True) lists them in
// when the weights are distinct; equal weights keep row order).  Rows ranked
// below the capacity move to offsets_out[e] + rank.
__global__ void __launch_bounds__(CAP_THREADS) capacity_rank_kernel(const int32_t* inv, const int32_t* offsets,
                                                                    const void* topk_w, int w_dt, int64_t capacity,
                                                                    const int32_t* offsets_out, int32_t* pos_out,
                                                                    int32_t* inv_out) {
  __shared__ float s_w[CAP_THREADS];
  const int e = blockIdx.x;
  const int64_t lo = offsets[e], n = (int64_t)offsets[e + 1] - lo;
  const int64_t i = (int64_t)blockIdx.y * CAP_THREADS + threadIdx.x;
  if ((int64_t)blockIdx.y * CAP_THREADS >= n) return;  // the whole workgroup: no row of this expert here
  const bool live = i < n;
  const int32_t a = live ? inv[lo + i] : 0;
  const float wi = live ? load_elem(topk_w, w_dt, a) : 0.f;
  int64_t rank = i;
  if (capacity > 0 && n > capacity) {
    rank = 0;
    for (int64_t j0 = 0; j0 < n; j0 += CAP_THREADS) {
      const int64_t j = j0 + threadIdx.x;
      s_w[threadIdx.x] = j < n ? load_elem(topk_w, w_dt, inv[lo + j]) : 0.f;
      __syncthreads();
      const int lim = (int)min<int64_t>(CAP_THREADS, n - j0);
      for (int q = 0; q < lim; ++q) {
        const float wj = s_w[q];
        rank += (wj > wi || (wj == wi && j0 + q < i)) ? 1 : 0;
      }
      __syncthreads();
    }
  }
  if (!live) return;
  const int64_t kept = capacity > 0 && n > capacity ? capacity : n;
  if (rank < kept) {
    const int32_t row = offsets_out[e] + (int32_t)rank;
    pos_out[a] = row;
    inv_out[row] = a;
  }
}

constexpr int CB_THREADS = 256;
constexpr int CB_MAX_K = 8;  // slots per token (unrolled: the per-slot state stays in registers)

// one workgroup per token: its slots' dY rows and routing-weight gradients
template <int DT>
__global__ void __launch_bounds__(CB_THREADS) combine_backward_kernel(const void* d_out, int64_t ldo, const void* y,
                                                                      int64_t ldy, const int32_t* pos,
                                                                      const void* topk_w, int w_dt, int K, int64_t H,
                                                                      void* dy, int64_t lddy, void* d_w, int vec) {
#pragma clang fp contract(off)
  __shared__ float red[CB_MAX_K][CB_THREADS / 64];
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x;
  // w of y's 16-bit dtype: the products d * y are that dtype's (mul of two
  // bf16 tensors), rounded before the sum
  const bool rnd_prod = DT != DT_F32 && w_dt == DT;
  int32_t row[CB_MAX_K];
  float w[CB_MAX_K], dot[CB_MAX_K];
#pragma unroll
  for (int s = 0; s < CB_MAX_K; ++s) {
    row[s] = s < K ? pos[t * K + s] : -1;
    w[s] = s < K ? load_elem(topk_w, w_dt, t * K + s) : 0.f;
    dot[s] = 0.f;
  }
  const char* dor = static_cast<const char*>(d_out) + t * ldo * (DT == DT_F32 ? 4 : 2);
  constexpr int esz = DT == DT_F32 ? 4 : 2;
  constexpr int per = 16 / esz;  // elements per 16-byte chunk
  if (vec) {
    for (int64_t c = (int64_t)tid * per; c < H; c += (int64_t)CB_THREADS * per) {
      const uint4 dv = *reinterpret_cast<const uint4*>(dor + c * esz);
      float d[per];
      if constexpr (DT == DT_F32) {
        d[0] = __uint_as_float(dv.x); d[1] = __uint_as_float(dv.y); d[2] = __uint_as_float(dv.z); d[3] = __uint_as_float(dv.w);
      } else {
        const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint32_t h = (dw[q >> 1] >> (16 * (q & 1))) & 0xFFFFu;
          d[q] = DT == DT_BF16 ? bf16_bits_to_f32(h) : __half2float(__ushort_as_half((unsigned short)h));
        }
      }
#pragma unroll
      for (int s = 0; s < CB_MAX_K; ++s) {
        if (row[s] < 0) continue;
        const char* yr = static_cast<const char*>(y) + ((int64_t)row[s] * ldy + c) * esz;
        char* dyr = static_cast<char*>(dy) + ((int64_t)row[s] * lddy + c) * esz;
        const uint4 yv = *reinterpret_cast<const uint4*>(yr);
        float yy[per];
        if constexpr (DT == DT_F32) {
          yy[0] = __uint_as_float(yv.x); yy[1] = __uint_as_float(yv.y); yy[2] = __uint_as_float(yv.z); yy[3] = __uint_as_float(yv.w);
        } else {
          const uint32_t yw[4] = {yv.x, yv.y, yv.z, yv.w};
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const uint32_t h = (yw[q >> 1] >> (16 * (q & 1))) & 0xFFFFu;
            yy[q] = DT == DT_BF16 ? bf16_bits_to_f32(h) : __half2float(__ushort_as_half((unsigned short)h));
          }
        }
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < per; ++q) dot[s] += rnd_prod ? round_to_dtype(d[q] * yy[q], DT) : d[q] * yy[q];
        if constexpr (DT == DT_F32) {
#pragma unroll
          for (int q = 0; q < 4; ++q) o[q] = __float_as_uint(d[q] * w[s]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float p0 = d[2 * q] * w[s], p1 = d[2 * q + 1] * w[s];
            const uint32_t b0 = DT == DT_BF16 ? (uint32_t)f32_to_bf16_bits(p0) : (uint32_t)__half_as_ushort(f32_to_f16(p0));
            const uint32_t b1 = DT == DT_BF16 ? (uint32_t)f32_to_bf16_bits(p1) : (uint32_t)__half_as_ushort(f32_to_f16(p1));
            o[q] = b0 | (b1 << 16);
          }
        }
        *reinterpret_cast<uint4*>(dyr) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  } else {
    for (int64_t c = tid; c < H; c += CB_THREADS) {
      const float d = load_elem(d_out, DT, t * ldo + c);
#pragma unroll
      for (int s = 0; s < CB_MAX_K; ++s) {
        if (row[s] < 0) continue;
        const float yy = load_elem(y, DT, (int64_t)row[s] * ldy + c);
        dot[s] += rnd_prod ? round_to_dtype(d * yy, DT) : d * yy;
        store_elem(dy, DT, (int64_t)row[s] * lddy + c, d * w[s]);
      }
    }
  }
  // the dot products: wave sums, then the four waves' sums in order
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int s = 0; s < CB_MAX_K; ++s) {
    float v = dot[s];
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if (lane == 0) red[s][wave] = v;
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < CB_MAX_K; ++s) {
    if (tid == s && s < K) {
      const float v = ((red[s][0] + red[s][1]) + red[s][2]) + red[s][3];
      store_elem(d_w, w_dt, t * K + s, row[s] < 0 ? 0.f : v);
    }
  }
}

// silu(g) * u backward, 8 h columns per thread (one 16-byte chunk of dH, of
// gate and of up); h column j of row r is gate column 256*(j/128) + j%128
// and up column 256*(j/128) + 128 + j%128 of the interleaved layout
__global__ void __launch_bounds__(256) swiglu_backward_kernel(const uint16_t* dh, int64_t lddh, const uint16_t* gu,
                                                              int64_t ldgu, int64_t R, int64_t I, uint16_t* dgu,
                                                              int64_t lddgu) {
#pragma clang fp contract(off)
  const int64_t chunks = I / 8;
  const int64_t total = R * chunks;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += stride) {
    const int64_t r = q / chunks;
    const int64_t j = (q - r * chunks) * 8;
    const int64_t gc = (j >> 7) * 256 + (j & 127);
    const uint4 hv = *reinterpret_cast<const uint4*>(dh + r * lddh + j);
    const uint4 gv = *reinterpret_cast<const uint4*>(gu + r * ldgu + gc);
    const uint4 uv = *reinterpret_cast<const uint4*>(gu + r * ldgu + gc + 128);
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t og[4], ou[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      uint32_t rg = 0, ru = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float d = bf16_bits_to_f32((hw[p] >> (16 * h)) & 0xFFFFu);
        const float g = bf16_bits_to_f32((gw[p] >> (16 * h)) & 0xFFFFu);
        const float u = bf16_bits_to_f32((uw[p] >> (16 * h)) & 0xFFFFu);
        // forward: s = bf16(silu(g)) (F.silu on a bf16 tensor), gated = bf16(s * u)
        const float sig = 1.0f / (1.0f + expf(-g));
        const float s = bf16_bits_to_f32(f32_to_bf16_bits(g / (1.0f + expf(-g))));
        // mul backward: d_s = bf16(d * u), d_u = bf16(d * s)
        const float ds = bf16_bits_to_f32(f32_to_bf16_bits(d * u));
        const uint32_t du = f32_to_bf16_bits(d * s);
        // silu backward: dy * sigmoid * (1 + x * (1 - sigmoid)) in fp32
        const uint32_t dg = f32_to_bf16_bits((ds * sig) * (1.0f + g * (1.0f - sig)));
        rg |= dg << (16 * h);
        ru |= du << (16 * h);
      }
      og[p] = rg;
      ou[p] = ru;
    }
    *reinterpret_cast<uint4*>(dgu + r * lddgu + gc) = make_uint4(og[0], og[1], og[2], og[3]);
    *reinterpret_cast<uint4*>(dgu + r * lddgu + gc + 128) = make_uint4(ou[0], ou[1], ou[2], ou[3]);
  }
}

// one workgroup per token: d_tokens[t] = the token's kept slots' rows of dx,
// in descending expert id, the first taken as it is and each next one added
// in the output dtype (rounded per add): the order and roundings in which
// autograd accumulates the gradients of `tokens[token_indices]` over the
// expert loop (its later experts' backward runs first)
template <int DT, bool VEC>
__global__ void __launch_bounds__(CB_THREADS) token_grad_kernel(const void* dx, int64_t lddx, const int32_t* pos,
                                                                const void* topk_idx, int idx_dt, int K, int64_t H,
                                                                void* out, int64_t ldo) {
#pragma clang fp contract(off)
  __shared__ int32_t s_row[CB_MAX_K];
  const int64_t t = blockIdx.x;
  if (threadIdx.x == 0) {
    int64_t e[CB_MAX_K];
    int32_t r[CB_MAX_K];
#pragma unroll
    for (int s = 0; s < CB_MAX_K; ++s) {
      e[s] = s < K ? (idx_dt == 1 ? reinterpret_cast<const int64_t*>(topk_idx)[t * K + s]
                                  : (int64_t) reinterpret_cast<const int32_t*>(topk_idx)[t * K + s])
                   : -1;
      r[s] = s < K ? pos[t * K + s] : -1;
    }
    // descending expert id (distinct per token under top-k routing)
#pragma unroll
    for (int s = 0; s < CB_MAX_K; ++s) {
      int rank = 0;
#pragma unroll
      for (int q = 0; q < CB_MAX_K; ++q) rank += (e[q] > e[s] || (e[q] == e[s] && q < s)) ? 1 : 0;
#pragma unroll
      for (int q = 0; q < CB_MAX_K; ++q)
        if (q == rank) s_row[q] = r[s];
    }
  }
  __syncthreads();
  if constexpr (VEC) {
    // eight columns per thread: every kept slot's 16-byte chunk loaded before
    // the sum (element-wise 2-byte loads ran the c4 token gradient at 2 TB/s)
    const uint16_t* src = reinterpret_cast<const uint16_t*>(dx);
    uint16_t* dst = reinterpret_cast<uint16_t*>(out) + t * ldo;
    for (int64_t c0 = (int64_t)threadIdx.x * 8; c0 < H; c0 += CB_THREADS * 8) {
      uint4 raw[CB_MAX_K];
#pragma unroll
      for (int s = 0; s < CB_MAX_K; ++s) {
        const int32_t row = s_row[s];
        raw[s] = row >= 0 ? *reinterpret_cast<const uint4*>(src + (int64_t)row * lddx + c0) : make_uint4(0, 0, 0, 0);
      }
      bool any = false;
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < CB_MAX_K; ++s) {
        if (s_row[s] < 0) continue;
        const uint32_t w[4] = {raw[s].x, raw[s].y, raw[s].z, raw[s].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t hb = (w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
          const float v =
              DT == DT_BF16 ? __uint_as_float(hb << 16) : __half2float(__ushort_as_half((unsigned short)hb));
          acc[i] = any ? round_to_dtype(acc[i] + v, DT) : v;
        }
        any = true;
      }
      // the sums hold values of the dtype already (or a token without a kept
      // slot: zero): their bits, exactly
      uint32_t pk[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t lo, hi;
        if constexpr (DT == DT_BF16) {
          lo = __float_as_uint(acc[2 * i]) >> 16;
          hi = __float_as_uint(acc[2 * i + 1]) >> 16;
        } else {
          lo = __half_as_ushort(f32_to_f16(acc[2 * i]));
          hi = __half_as_ushort(f32_to_f16(acc[2 * i + 1]));
        }
        pk[i] = lo | (hi << 16);
      }
      *reinterpret_cast<uint4*>(dst + c0) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
    return;
  }
  for (int64_t c = threadIdx.x; c < H; c += CB_THREADS) {
    bool any = false;
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < CB_MAX_K; ++s) {
      const int32_t row = s_row[s];
      if (row < 0) continue;
      const float v = load_elem(dx, DT, (int64_t)row * lddx + c);
      acc = any ? round_to_dtype(acc + v, DT) : v;
      any = true;
    }
    store_elem(out, DT, t * ldo + c, any ? acc : 0.f);
  }
}

}  // namespace ntlb

using namespace ntlb;

extern "C" int ntlb_moe_token_grad(const void* dx, int64_t lddx, int dtype, const int32_t* pos, const void* topk_idx,
                                   int idx_dtype, int64_t T, int64_t K, int64_t H, void* out, int64_t ldo,
                                   void* stream) {
  const char* fn = "ntlb_moe_token_grad";
  if (T < 0 || H < 0 || K < 1 || K > CB_MAX_K || !valid_dtype(dtype) || (idx_dtype != 0 && idx_dtype != 1))
    return fail(NTLB_EINVAL, "%s: bad argument (1 <= K <= %d)", fn, CB_MAX_K);
  if (lddx < H || ldo < H) return fail(NTLB_EINVAL, "%s: ld smaller than H", fn);
  if (T == 0 || H == 0) return NTLB_OK;
  if (!dx || !pos || !topk_idx || !out) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  hipStream_t st = as_stream(stream);
  const bool vec = H % 8 == 0 && lddx % 8 == 0 && ldo % 8 == 0 && aligned(dx, 16) && aligned(out, 16);
  auto launch = [&](auto dtc, auto vecc) {
    token_grad_kernel<decltype(dtc)::value, decltype(vecc)::value><<<(unsigned)T, CB_THREADS, 0, st>>>(
        dx, lddx, pos, topk_idx, idx_dtype, (int)K, H, out, ldo);
  };
  using B = std::integral_constant<int, DT_BF16>;
  using Hh = std::integral_constant<int, DT_F16>;
  using Y = std::true_type;
  using N = std::false_type;
  if (dtype == NTLB_BF16) {
    if (vec) launch(B(), Y()); else launch(B(), N());
  } else if (dtype == NTLB_F16) {
    if (vec) launch(Hh(), Y()); else launch(Hh(), N());
  } else {
    launch(std::integral_constant<int, DT_F32>(), N());  // fp32: the element loop
  }
  return check_launch(fn);
}

extern "C" int ntlb_moe_capacity_keep(const int32_t* inv, const int32_t* offsets, int n_experts, int64_t rows,
                                      int64_t n_assign, const void* topk_w, int w_dtype, int64_t capacity,
                                      int32_t* pos_out, int32_t* inv_out, int32_t* offsets_out, int64_t* counts_out,
                                      void* stream) {
  const char* fn = "ntlb_moe_capacity_keep";
  if (n_experts < 1 || rows < 0 || n_assign < rows || !valid_dtype(w_dtype))
    return fail(NTLB_EINVAL, "%s: bad argument", fn);
  if (!offsets || !offsets_out || !counts_out || !pos_out || (rows > 0 && (!inv || !inv_out || !topk_w)))
    return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (rows >= (int64_t)0x7FFFFFFF || n_experts > 65535) return fail(NTLB_EUNSUPPORTED, "%s: too large", fn);
  hipStream_t st = as_stream(stream);
  if (n_assign > 0) fill_i32_kernel<<<grid_for(n_assign, CAP_THREADS), CAP_THREADS, 0, st>>>(pos_out, n_assign, -1);
  // rows past the kept count read -1 (a gather over inv_out must not meet stale indices)
  if (rows > 0) fill_i32_kernel<<<grid_for(rows, CAP_THREADS), CAP_THREADS, 0, st>>>(inv_out, rows, -1);
  capacity_offsets_kernel<<<1, CAP_THREADS, 0, st>>>(offsets, n_experts, capacity, offsets_out, counts_out);
  if (rows > 0) {
    const int64_t chunks = (rows + CAP_THREADS - 1) / CAP_THREADS;  // bounds every expert's row count
    if (chunks > 65535) return fail(NTLB_EUNSUPPORTED, "%s: too many rows", fn);
    capacity_rank_kernel<<<dim3((unsigned)n_experts, (unsigned)chunks), CAP_THREADS, 0, st>>>(
        inv, offsets, topk_w, w_dtype, capacity, offsets_out, pos_out, inv_out);
  }
  return check_launch(fn);
}

extern "C" int ntlb_moe_combine_backward(const void* d_out, int64_t ldo, const void* y, int64_t ldy, int dtype,
                                         const int32_t* pos, const void* topk_w, int w_dtype, int64_t T, int64_t K,
                                         int64_t H, void* dy, int64_t lddy, void* d_w, void* stream) {
  const char* fn = "ntlb_moe_combine_backward";
  if (T < 0 || H < 0 || K < 1 || K > CB_MAX_K || !valid_dtype(dtype) || !valid_dtype(w_dtype))
    return fail(NTLB_EINVAL, "%s: bad argument (1 <= K <= %d)", fn, CB_MAX_K);
  if (ldo < H || ldy < H || lddy < H) return fail(NTLB_EINVAL, "%s: ld smaller than H", fn);
  if (T == 0) return NTLB_OK;
  if (!d_out || !y || !pos || !topk_w || !dy || !d_w) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  const int esz = dtype_size(dtype);
  const int per = 16 / esz;
  const int vec = aligned(d_out, 16) && aligned(y, 16) && aligned(dy, 16) && ldo % per == 0 && ldy % per == 0 &&
                  lddy % per == 0 && H % per == 0;
  hipStream_t st = as_stream(stream);
  if (dtype == NTLB_BF16)
    combine_backward_kernel<DT_BF16><<<(unsigned)T, CB_THREADS, 0, st>>>(d_out, ldo, y, ldy, pos, topk_w, w_dtype,
                                                                          (int)K, H, dy, lddy, d_w, vec);
  else if (dtype == NTLB_F16)
    combine_backward_kernel<DT_F16><<<(unsigned)T, CB_THREADS, 0, st>>>(d_out, ldo, y, ldy, pos, topk_w, w_dtype,
                                                                         (int)K, H, dy, lddy, d_w, vec);
  else
    combine_backward_kernel<DT_F32><<<(unsigned)T, CB_THREADS, 0, st>>>(d_out, ldo, y, ldy, pos, topk_w, w_dtype,
                                                                         (int)K, H, dy, lddy, d_w, vec);
  return check_launch(fn);
}

extern "C" int ntlb_swiglu_backward(const uint16_t* dh, int64_t lddh, const uint16_t* gu, int64_t ldgu, int64_t R,
                                    int64_t I, uint16_t* dgu, int64_t lddgu, void* stream) {
  const char* fn = "ntlb_swiglu_backward";
  if (R < 0 || I < 0 || I % 128) return fail(NTLB_EINVAL, "%s: I must be a multiple of 128", fn);
  if (R == 0 || I == 0) return NTLB_OK;
  if (!dh || !gu || !dgu) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (lddh < I || ldgu < 2 * I || lddgu < 2 * I || lddh % 8 || ldgu % 8 || lddgu % 8 || !aligned(dh, 16) ||
      !aligned(gu, 16) || !aligned(dgu, 16))
    return fail(NTLB_EINVAL, "%s: bf16 rows need ld %% 8 == 0 and 16-byte alignment", fn);
  const int64_t total = R * (I / 8);
  swiglu_backward_kernel<<<grid_for(total, 256), 256, 0, as_stream(stream)>>>(dh, lddh, gu, ldgu, R, I, dgu, lddgu);
  return check_launch(fn);
}
