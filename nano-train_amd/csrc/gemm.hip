// Blockwise-scaled GEMM for gfx950:
//   Y[M,N] = sum_kb sa(m,kb) * sb(n,kb) * (A_kb[m,:] . B_kb[n,:])  (+ bias)
// The F.linear of te_backend.py:253-259 with both operands kept as codes and
// scales.  Each 128-wide K block is one MFMA chain on the matrix cores:
//   e4m3 codes: v_mfma_scale_f32_16x16x128_f8f6f4 (unit e8m0 scales), fp32 out
//   int-grid codes: 2x v_mfma_i32_16x16x64_i8, exact int32 partials
//     (|partial| <= 128*127^2 < 2^24, so the int32 -> fp32 conversion is exact)
// and the partial tile is promoted into the fp32 accumulator with
// sa(m,kb)*sb(n,kb) in VALU.
//
// Block tile 128x128, K step 128 (= one scale block), 256 threads as 2x2 waves
// of 64x64.  A and B tiles go global -> registers -> LDS (double buffered,
// 16-byte chunks XOR-swizzled by row so the MFMA fragment reads are
// bank-conflict free); the next K block's loads are in flight while the current
// one is multiplied.
#include <hip/hip_runtime.h>

#include "ntlb_device.h"
#include "ntlb_host.h"

namespace ntlb {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct GemmArgs {
  const uint8_t* a;
  int64_t lda;
  const float* sa;
  int64_t sa_row, sa_col;
  int a_shift;
  const uint8_t* b;
  int64_t ldb;
  const float* sb;
  int64_t sb_row, sb_col;
  int b_shift;
  int64_t M, N, Kp;
  const void* bias;
  int bias_dtype;
  void* y;
  int y_dtype;
  int64_t ldy;
  const int32_t* nan_a;
  const int32_t* nan_b;
};

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int TILE_BYTES = BM * BK;  // 16 KiB per operand tile

// byte offset of 16-byte chunk c of row r inside a swizzled 128x128 tile
__device__ __forceinline__ int swz(int r, int c) { return r * BK + ((c ^ (r & 7)) << 4); }

// MFMA fragment for a 16-row group: row = lane%16, 32 K bytes from group lane/16.
// A and B use the same (lane group, byte) -> K mapping, so the products pair up.
__device__ __forceinline__ v8i load_frag(const uint8_t* tile, int row0, int lane) {
  const int r = row0 + (lane & 15);
  const int g = lane >> 4;
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + swz(r, 2 * g));
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + swz(r, 2 * g + 1));
  v8i f;
  f[0] = (int)lo.x; f[1] = (int)lo.y; f[2] = (int)lo.z; f[3] = (int)lo.w;
  f[4] = (int)hi.x; f[5] = (int)hi.y; f[6] = (int)hi.z; f[7] = (int)hi.w;
  return f;
}

template <int GRID>
__device__ __forceinline__ v4f mma_block(const v8i& a, const v8i& b) {
  if constexpr (GRID == GRID_E4M3) {
    v4f z = {0.f, 0.f, 0.f, 0.f};
    // fmt 0 = e4m3 for both operands; e8m0 scale 127 = 2^0
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
  } else {
    v4i z = {0, 0, 0, 0};
    v4i a0 = {a[0], a[1], a[2], a[3]}, a1 = {a[4], a[5], a[6], a[7]};
    v4i b0 = {b[0], b[1], b[2], b[3]}, b1 = {b[4], b[5], b[6], b[7]};
    v4i p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, z, 0, 0, 0);
    p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, p, 0, 0, 0);
    v4f f = {(float)p[0], (float)p[1], (float)p[2], (float)p[3]};
    return f;
  }
}

template <int GRID, bool B_UNIFORM>
__global__ void __launch_bounds__(256, 2) gemm_blockscaled_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][TILE_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][TILE_BYTES];
  __shared__ __attribute__((aligned(16))) float lds_sa[2][BM];
  __shared__ __attribute__((aligned(16))) float lds_sb[2][BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // workgroup -> output tile: undo the round-robin XCD dispatch so that each
  // XCD walks a contiguous range, then a grouped (8 row-tiles) raster order.
  const int num_m = (int)((g.M + BM - 1) / BM), num_n = (int)((g.N + BN - 1) / BN);
  const int nwg = num_m * num_n;
  int pid = blockIdx.x;
  {
    const int xcd = pid & 7, local = pid >> 3;
    const int per = nwg >> 3, extra = nwg & 7;
    pid = xcd * per + min(xcd, extra) + local;
  }
  constexpr int GROUP_M = 8;
  const int group = pid / (GROUP_M * num_n);
  const int first_m = group * GROUP_M;
  const int gsize = min(num_m - first_m, GROUP_M);
  const int in_group = pid - group * GROUP_M * num_n;
  const int tile_m = first_m + in_group % gsize;
  const int tile_n = in_group / gsize;
  const int64_t m0 = (int64_t)tile_m * BM, n0 = (int64_t)tile_n * BN;

  // global -> LDS copy assignment: chunk c of rows (tid>>3) + 32*i
  const int cc = tid & 7, cr = tid >> 3;
  const uint8_t* a_src[4];
  const uint8_t* b_src[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int64_t ra = min<int64_t>(m0 + cr + 32 * i, g.M - 1);
    int64_t rb = min<int64_t>(n0 + cr + 32 * i, g.N - 1);
    a_src[i] = g.a + ra * g.lda + cc * 16;
    b_src[i] = g.b + rb * g.ldb + cc * 16;
  }
  // scale copy: threads 0..127 fetch sa for rows m0+tid, 128..255 fetch sb
  const int64_t srow = (tid < BM) ? min<int64_t>(m0 + tid, g.M - 1) : min<int64_t>(n0 + tid - BM, g.N - 1);
  const float* s_src = (tid < BM) ? g.sa + (srow >> g.a_shift) * g.sa_row : g.sb + (srow >> g.b_shift) * g.sb_row;
  const int64_t s_step = (tid < BM) ? g.sa_col : g.sb_col;
  const float* sb_uniform = g.sb + (n0 >> g.b_shift) * g.sb_row;

  const int nk = (int)(g.Kp / BK);
  uint4 ra[4], rb[4];
  float rs;

  auto gload = [&](int kt) {
    const int64_t koff = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ra[i] = *reinterpret_cast<const uint4*>(a_src[i] + koff);
      rb[i] = *reinterpret_cast<const uint4*>(b_src[i] + koff);
    }
    rs = s_src[kt * s_step];
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = cr + 32 * i;
      *reinterpret_cast<uint4*>(&lds_a[buf][swz(r, cc)]) = ra[i];
      *reinterpret_cast<uint4*>(&lds_b[buf][swz(r, cc)]) = rb[i];
    }
    if (tid < BM)
      lds_sa[buf][tid] = rs;
    else
      lds_sb[buf][tid - BM] = rs;
  };

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

  gload(0);
  lstore(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);

    const uint8_t* ta = lds_a[buf];
    const uint8_t* tb = lds_b[buf];
    v8i bf[4];
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) bf[tn] = load_frag(tb, wn * 64 + tn * 16, lane);
    float sbv[4];
    if constexpr (B_UNIFORM) {
      const float s = sb_uniform[(int64_t)kt * g.sb_col];
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) sbv[tn] = s;
    } else {
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) sbv[tn] = lds_sb[buf][wn * 64 + tn * 16 + (lane & 15)];
    }
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      const v8i af = load_frag(ta, wm * 64 + tm * 16, lane);
      const float4 sa4 = *reinterpret_cast<const float4*>(&lds_sa[buf][wm * 64 + tm * 16 + (lane >> 4) * 4]);
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
        const v4f d = mma_block<GRID>(af, bf[tn]);
        acc[tm][tn][0] += d[0] * (sa4.x * sbv[tn]);
        acc[tm][tn][1] += d[1] * (sa4.y * sbv[tn]);
        acc[tm][tn][2] += d[2] * (sa4.z * sbv[tn]);
        acc[tm][tn][3] += d[3] * (sa4.w * sbv[tn]);
      }
    }
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue: NaN flags, bias, cast, store (16 lanes cover 16 consecutive columns)
#pragma unroll
  for (int tn = 0; tn < 4; ++tn) {
    const int64_t col = n0 + wn * 64 + tn * 16 + (lane & 15);
    if (col >= g.N) continue;
    float bias = 0.f;
    if (g.bias) bias = load_elem(g.bias, g.bias_dtype, col);
    const bool nan_col = g.nan_b && g.nan_b[col];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + wm * 64 + tm * 16 + (lane >> 4) * 4 + i;
        if (row >= g.M) continue;
        float v = acc[tm][tn][i] + bias;
        if (nan_col || (g.nan_a && g.nan_a[row])) v = __uint_as_float(0x7FC00000u);
        store_elem(g.y, g.y_dtype, row * g.ldy + col, v);
      }
    }
  }
}

}  // namespace ntlb

using namespace ntlb;

extern "C" int ntlb_gemm_blockscaled(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                                     int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb, const float* sb,
                                     int64_t sb_row, int64_t sb_col, int b_shift, int64_t M, int64_t N, int64_t Kp,
                                     const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                                     const int32_t* nan_a, const int32_t* nan_b, void* stream) {
  const char* fn = "ntlb_gemm_blockscaled";
  if (grid != NTLB_GRID_INT && grid != NTLB_GRID_E4M3) return fail(NTLB_EINVAL, "%s: bad grid %d", fn, grid);
  if (M < 0 || N < 0 || Kp < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (Kp % 128) return fail(NTLB_EINVAL, "%s: Kp %lld is not a multiple of 128", fn, (long long)Kp);
  if (M == 0 || N == 0) return NTLB_OK;
  if (!a || !b || !sa || !sb || !y) return fail(NTLB_EINVAL, "%s: NULL operand", fn);
  if (lda < Kp || ldb < Kp || (lda % 16) || (ldb % 16) || !aligned(a, 16) || !aligned(b, 16))
    return fail(NTLB_EINVAL, "%s: code matrices need ld >= Kp, ld %% 16 == 0 and 16-byte alignment", fn);
  if (!(a_shift == 0 || a_shift == 7) || !(b_shift == 0 || b_shift == 7))
    return fail(NTLB_EINVAL, "%s: scale shifts must be 0 or 7", fn);
  if (!valid_dtype(y_dtype) || ldy < N) return fail(NTLB_EINVAL, "%s: bad output dtype or ldy", fn);
  if (bias && !valid_dtype(bias_dtype)) return fail(NTLB_EINVAL, "%s: bad bias dtype", fn);
  if (Kp == 0) return fail(NTLB_EUNSUPPORTED, "%s: K == 0", fn);
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  GemmArgs g;
  g.a = a; g.lda = lda; g.sa = sa; g.sa_row = sa_row; g.sa_col = sa_col; g.a_shift = a_shift;
  g.b = b; g.ldb = ldb; g.sb = sb; g.sb_row = sb_row; g.sb_col = sb_col; g.b_shift = b_shift;
  g.M = M; g.N = N; g.Kp = Kp;
  g.bias = bias; g.bias_dtype = bias_dtype;
  g.y = y; g.y_dtype = y_dtype; g.ldy = ldy;
  g.nan_a = nan_a; g.nan_b = nan_b;
  // B's scale is uniform over a 128-column tile for 128x128 blocks and tensor scales
  const bool b_uniform = (b_shift == 7) || (sb_row == 0);
  hipStream_t st = as_stream(stream);
  dim3 grd((unsigned)tiles), blk(256);
  if (grid == NTLB_GRID_E4M3) {
    if (b_uniform)
      gemm_blockscaled_kernel<GRID_E4M3, true><<<grd, blk, 0, st>>>(g);
    else
      gemm_blockscaled_kernel<GRID_E4M3, false><<<grd, blk, 0, st>>>(g);
  } else {
    if (b_uniform)
      gemm_blockscaled_kernel<GRID_INT, true><<<grd, blk, 0, st>>>(g);
    else
      gemm_blockscaled_kernel<GRID_INT, false><<<grd, blk, 0, st>>>(g);
  }
  return check_launch(fn);
}
