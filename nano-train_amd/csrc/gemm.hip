// Blockwise-scaled GEMM for gfx950:
//   Y[M,N] = sum_kb sa(m,kb) * sb(n,kb) * (A_kb[m,:] . B_kb[n,:])  (+ bias)
// The F.linear of te_backend.py:253-259 with both operands kept as codes and
// scales.  Each 128-wide K block is one MFMA chain on the matrix cores:
//   e4m3 codes: v_mfma_f32_16x16x128_f8f6f4 (the scaled builtin with zero
//     scale operands, which selects the unscaled encoding), fp32 out
//   int-grid codes: 2x v_mfma_i32_16x16x64_i8, exact int32 partials
//     (|partial| <= 128*127^2 < 2^24, so the int32 -> fp32 conversion is exact)
// and the partial tile is promoted into the fp32 accumulator with
// sa(m,kb)*sb(n,kb) in VALU, one FMA per accumulator per K block.
//
// Tiling: 256x256 output tile per workgroup, K step 128 (= one scale block),
// 512 threads = 8 waves as 2 (M) x 4 (N), each wave 128x64.  The MFMA is fed
// with the B tile as its first operand and the A tile as its second, so each
// lane's four results are four consecutive output columns of one row: one
// A-scale per lane per 16-row group, and 8-byte packed writes in the epilogue.
//
// Operand tiles move global -> LDS with global_load_lds_dwordx4 (no register
// staging), double buffered; the next K block streams in while the current
// one is multiplied.  16-byte chunks are XOR-swizzled by row so the fragment
// reads are bank-conflict free.  The epilogue stages each wave's tile through
// LDS and writes full 128-byte row segments.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "ntlb_device.h"
#include "ntlb_host.h"
#include "ntlb_quant8.h"
#include "ntlb_splitk.h"

namespace ntlb {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

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
  int vec_out;  // y 16-byte aligned with 16-byte row pitch
  // grouped (per-expert) mode: rows of A sorted by expert, expert e owns rows
  // [offsets[e], offsets[e+1]) and multiplies B + e*b_estride (codes) with
  // scales sb + e*sb_estride
  const int32_t* offsets;
  int n_experts;
  int64_t b_estride, sb_estride;
  // SwiGLU epilogue (EPI_SWIGLU): B's rows come in 128-row blocks alternating
  // gate block t and up block t, so output tile columns [0,128) are gate and
  // [128,256) up for h columns n0/2 + [0,128).  h = bf16(silu(bf16(gate)) *
  // bf16(up)) is quantized per 1x128 tile (one tile per output tile row).
  uint16_t* h;    // optional bf16 h [M, I], row stride ldh
  int64_t ldh;
  uint8_t* hc;    // h codes [M, ldhc]
  int64_t ldhc;
  float* hs;      // h scales: hs[row * hs_row + tile * hs_col]
  int64_t hs_row, hs_col;
  int32_t* h_nan;  // optional per-row NaN flags of h
  uint16_t* gu;   // optional bf16 gate / up outputs [M, 2I] in B's interleaved column order, row stride ldgu
  int64_t ldgu;
  float h_qmaxf;
  int h_sr, h_scale_rule;
  uint64_t h_seed, h_offset;
  int64_t I;  // width of h = N / 2
  // Split-K tail (dense, EPI_STORE): workgroups at or past split_base take K
  // chunk (q % split_s) of tile split_base + q / split_s, q = pid - split_base;
  // the chunks' fp32 partials meet in ws and the last one to finish sums them
  // in chunk order and stores the tile.
  int split_base, split_s;
  float* ws;             // [tail tiles][split_s][NTHREADS * 128] fp32
  uint32_t* ws_count;    // per tail tile; zero between calls (the kernel resets it)
};

// Epilogues: store the tile as bf16 (EPI_STORE), fp32 or fp16, or the
// SwiGLU + 1x128 quantization of the expert MLP.  The output dtype is part of
// the kernel so that each kernel holds one straight-line store path.
constexpr int EPI_STORE = 0, EPI_SWIGLU = 1, EPI_STORE_F32 = 2, EPI_STORE_F16 = 3;

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int NTHREADS = 512;
constexpr int TILE_A = BM * BK, TILE_B = BN * BK;  // 32 KiB each
// epilogue: each wave stages 32 rows of its 128x64 tile at a time inside a
// 16 KiB slice of the (then idle) operand buffers
constexpr int EPI_ROWS = 32;
constexpr int EPI_PITCH_F32 = 64 * 4 + 16;  // bytes per staged row (fp32)
constexpr int EPI_PITCH_16 = 64 * 2 + 16;   // bytes per staged row (bf16 / fp16)
static_assert(EPI_ROWS * EPI_PITCH_F32 <= TILE_A / 2, "epilogue slice exceeds half an operand buffer");
static_assert(NTHREADS == SPLIT_THREADS, "the split-K exchange assumes 512 threads and acc[8][4]");

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Byte offset of 16-byte chunk c of row r inside a swizzled [rows][128] tile.
// A fragment read has 16 lanes read 16 consecutive rows at one logical chunk;
// the permutation f(r) = (r & 7) ^ bit3(r) gives rows 0-7 eight distinct
// chunks (conflict-free in 8-lane phases over 128 bytes of banks) and gives
// every 16-row window distinct (row parity, chunk) pairs (conflict-free in
// 16-lane phases over 256 bytes of banks).
__device__ __forceinline__ int swz_perm(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int swz(int r, int c) { return r * BK + ((c ^ swz_perm(r)) << 4); }

// MFMA fragment of 16 rows: row = lane%16, 32 K bytes of group lane/16.
// Both operands use the same (lane group, byte) -> K mapping, so the products pair up.
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

// D[i][j] = sum_k P[i][k] Q[j][k] for a 16x16 tile; lane l holds D[4*(l/16)+r][l%16]
template <int GRID>
__device__ __forceinline__ v4f mma_block(const v8i& p, const v8i& q) {
  if constexpr (GRID == GRID_E4M3) {
    v4f z = {0.f, 0.f, 0.f, 0.f};
    // fmt 0 = e4m3 for both operands.  Zero scale operands select the
    // unscaled encoding (v_mfma_f32_16x16x128_f8f6f4, no v_mfma_ld_scale
    // prefix); its products equal those of unit e8m0 scales (127) bit for bit
    // over the whole config-2 output, and the c2 GEMM runs 1.5% faster.
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(p, q, z, 0, 0, 0, 0, 0, 0);
  } else {
    v4i z = {0, 0, 0, 0};
    v4i p0 = {p[0], p[1], p[2], p[3]}, p1 = {p[4], p[5], p[6], p[7]};
    v4i q0 = {q[0], q[1], q[2], q[3]}, q1 = {q[4], q[5], q[6], q[7]};
    v4i s = __builtin_amdgcn_mfma_i32_16x16x64_i8(p0, q0, z, 0, 0, 0);
    s = __builtin_amdgcn_mfma_i32_16x16x64_i8(p1, q1, s, 0, 0, 0);
    v4f f = {(float)s[0], (float)s[1], (float)s[2], (float)s[3]};
    return f;
  }
}

// The raw MFMA result of one 16x16 block over one K block (fp32 for e4m3,
// int32 for the int grid: at most 128 * 127^2 in magnitude, exact in fp32)
// and its conversion, so that a pipelined promotion can keep the raw form
// until it is consumed.
template <int GRID>
using raw_t = typename std::conditional<GRID == GRID_E4M3, v4f, v4i>::type;

template <int GRID>
__device__ __forceinline__ raw_t<GRID> mma_raw(const v8i& p, const v8i& q) {
  if constexpr (GRID == GRID_E4M3) {
    return mma_block<GRID>(p, q);
  } else {
    v4i z = {0, 0, 0, 0};
    v4i p0 = {p[0], p[1], p[2], p[3]}, p1 = {p[4], p[5], p[6], p[7]};
    v4i q0 = {q[0], q[1], q[2], q[3]}, q1 = {q[4], q[5], q[6], q[7]};
    v4i s = __builtin_amdgcn_mfma_i32_16x16x64_i8(p0, q0, z, 0, 0, 0);
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(p1, q1, s, 0, 0, 0);
  }
}

template <int GRID>
__device__ __forceinline__ v4f raw_f32(const raw_t<GRID>& r) {
  if constexpr (GRID == GRID_E4M3) {
    return r;
  } else {
    return (v4f){(float)r[0], (float)r[1], (float)r[2], (float)r[3]};
  }
}

// Direct-to-LDS copies of one K block through buffer resources: wave w moves
// the 8-row groups w, w+8, w+16, w+24 (1 KiB each) of A and of B, so bit 3 of
// every row it writes equals w & 1.  Lane i lands at byte 16*i of its group
// (row i/8, physical chunk i%8) and fetches logical chunk (i%8) ^ swz_perm(row),
// which is therefore the same for all four groups: its 32-bit row offset is
// fixed for the whole K loop and the group / K offsets ride in the scalar
// offset.  Rows past M (or N) lie beyond the resource's num_records and read
// as zero.
struct StageSrc {
  __amdgpu_buffer_rsrc_t ra, rb;
  uint32_t a_off, b_off;   // per-lane byte offset of row (wave*8 + lane/8), chunk c
  uint32_t a_grp, b_grp;   // 64 rows of A / B in bytes
};

// group j (0..3) of this wave's share of K block kt, for A and for B
__device__ __forceinline__ void issue_group(const StageSrc& s, uint8_t* lds_a, uint8_t* lds_b, int kt, int wave,
                                            int j) {
  const uint32_t koff = (uint32_t)kt * BK;
  const int r0 = (wave + 8 * j) * 8;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(s.ra, (lds_ptr_t)(lds_a + r0 * BK), 16, s.a_off, koff + j * s.a_grp, 0,
                                           0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(s.rb, (lds_ptr_t)(lds_b + r0 * BK), 16, s.b_off, koff + j * s.b_grp, 0,
                                           0);
}

// The two pipeline stages live in distinct LDS objects and the K loop is
// unrolled by two, so every fragment read names one object and every
// direct-to-LDS copy another: the compiler can then see that the copies in
// flight for the next K block do not alias the reads of the current one, and
// keeps them in flight across the whole MFMA phase instead of waiting on them
// before the first read.
template <int GRID, bool SR>
__device__ __forceinline__ void swiglu_quant_rows(const GemmArgs& g, const uint8_t* s0, const uint8_t* s1,
                                                  const uint8_t* s2, const uint8_t* s3, int64_t m0, int64_t n0,
                                                  int tid);

// staged epilogue rows: slab k (one of the four 32 KiB stage buffers) holds
// tile rows 64k .. 64k+63, 512 bytes each
__device__ __forceinline__ uint8_t* slab_row(uint8_t* s0, uint8_t* s1, uint8_t* s2, uint8_t* s3, int r) {
  const int k = r >> 6;
  return (k == 0 ? s0 : k == 1 ? s1 : k == 2 ? s2 : s3) + (r & 63) * 512;
}

template <int GRID, bool B_UNIFORM, bool GROUPED, int EPI = EPI_STORE>
__global__ void __launch_bounds__(NTHREADS, 1) gemm_blockscaled_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_a0[TILE_A];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b0[TILE_B];
  __shared__ __attribute__((aligned(16))) uint8_t lds_a1[TILE_A];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b1[TILE_B];
  __shared__ __attribute__((aligned(16))) float lds_s0[BM + BN];  // A row scales, then B row scales
  __shared__ __attribute__((aligned(16))) float lds_s1[BM + BN];

  // the wave index through readfirstlane: the compiler then keeps everything
  // derived from it (fragment bases, the copies' LDS destinations) in scalar
  // registers instead of 28 VGPRs
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;

  // workgroup -> output tile: undo the round-robin XCD dispatch so each XCD
  // walks a contiguous range, then a grouped raster (GROUP_M row-tiles)
  const int num_n = (int)((g.N + BN - 1) / BN);
  // Workgroup pid runs on XCD pid % 8; xcd_local() renumbers the first nwg
  // pids so each XCD walks a contiguous range of tiles (its own L2 then holds
  // neighbouring tiles).  It is a bijection on [0, nwg).
  auto xcd_local = [](int p, int nwg) {
    const int xcd = p & 7, local = p >> 3;
    const int per = nwg >> 3, extra = nwg & 7;
    return xcd * per + min(xcd, extra) + local;
  };
  int pid = blockIdx.x;
  int split_tail = -1, split_chunk = 0;
  int64_t m0, n0;
  if constexpr (GROUPED) {
    // experts in order, each one's tiles in the grouped raster of the dense
    // case (GROUP_M row tiles sweep all n tiles).  The workgroups are not
    // renumbered into a contiguous range per XCD as in the dense case:
    // consecutive tiles go to consecutive XCDs, so every XCD gets its share
    // of each expert's ragged last row tile, whose waves past the expert's
    // end issue no MFMAs.  Contiguous ranges gave the XCDs that hold the
    // small experts about a fifth less work than those with the large ones
    // (c4: 1.884-1.897 ms per step against 1.841-1.851 round robin).
    // The offset table is read once, in parallel, into LDS (the first stage
    // buffer, free until the first copy) and searched there; a walk over
    // global memory would be one dependent load per expert.  The grid is an
    // upper bound on the tile count: workgroups past the last tile return.
    int32_t* tab = reinterpret_cast<int32_t*>(lds_a0);
    for (int i = tid; i <= g.n_experts; i += NTHREADS) tab[i] = g.offsets[i];
    __syncthreads();
    int e = 0, before = 0, tiles_m = 0;
    int64_t lo = 0, hi = 0;
    for (; e < g.n_experts; ++e) {
      lo = tab[e];
      hi = tab[e + 1];
      tiles_m = (int)((hi - lo + BM - 1) / BM);
      if (pid < before + tiles_m * num_n) break;
      before += tiles_m * num_n;
    }
    __syncthreads();  // the table's LDS is a copy target from here on
    if (e >= g.n_experts) return;  // beyond the last expert's tiles: the grid is an upper bound
    constexpr int GROUP_M = 4;
    const int l = pid - before;
    const int group = l / (GROUP_M * num_n);
    const int first_m = group * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    const int in_group = l - group * GROUP_M * num_n;
    m0 = lo + (int64_t)(first_m + in_group % gsize) * BM;
    n0 = (int64_t)(in_group / gsize) * BN;
    g.M = hi;  // rows at or past the expert's end are not stored
    g.b += (int64_t)e * g.b_estride;
    g.sb += (int64_t)e * g.sb_estride;
    if (g.nan_b) g.nan_b += (int64_t)e * g.N;
  } else {
    const SplitWork sw = split_work(pid, g.split_base, g.split_s);
    split_tail = sw.tail;
    split_chunk = sw.chunk;
    pid = sw.tail >= 0 ? sw.pid : xcd_local(pid, g.split_s > 1 ? g.split_base : (int)gridDim.x);
    const int num_m = (int)((g.M + BM - 1) / BM);
    constexpr int GROUP_M = 4;
    const int group = pid / (GROUP_M * num_n);
    const int first_m = group * GROUP_M;
    const int gsize = min(num_m - first_m, GROUP_M);
    const int in_group = pid - group * GROUP_M * num_n;
    m0 = (int64_t)(first_m + in_group % gsize) * BM;
    n0 = (int64_t)(in_group / gsize) * BN;
  }

  // scale fetch: thread t < 256 owns sa of row m0+t, t >= 256 sb of row n0+t-256
  const bool own_a = tid < BM;
  const int64_t srow = own_a ? min<int64_t>(m0 + tid, g.M - 1) : min<int64_t>(n0 + tid - BM, g.N - 1);
  const float* s_src = own_a ? g.sa + (srow >> g.a_shift) * g.sa_row : g.sb + (srow >> g.b_shift) * g.sb_row;
  const int64_t s_step = own_a ? g.sa_col : g.sb_col;

  // What the store epilogue reads of the arguments, loaded now and kept in
  // scalar registers through the K loop: re-loading them after the loop
  // costs a scalar-cache miss per use.
  uintptr_t e_y = reinterpret_cast<uintptr_t>(g.y), e_bias = reinterpret_cast<uintptr_t>(g.bias);
  uintptr_t e_nan_a = reinterpret_cast<uintptr_t>(g.nan_a), e_nan_b = reinterpret_cast<uintptr_t>(g.nan_b);
  int64_t e_ldy = g.ldy, e_M = g.M, e_N = g.N;
  int e_misc = (g.vec_out ? 1 : 0) | (g.bias_dtype << 1);
  if constexpr (EPI != EPI_SWIGLU) {
    // uniform by construction (the grouped mapping derives M and nan_b from
    // the offset table in LDS, which the compiler treats as per-lane)
    e_y = uniform64(e_y); e_bias = uniform64(e_bias); e_nan_a = uniform64(e_nan_a); e_nan_b = uniform64(e_nan_b);
    e_ldy = uniform64(e_ldy); e_M = uniform64(e_M); e_N = uniform64(e_N);
    e_misc = __builtin_amdgcn_readfirstlane(e_misc);
    asm volatile("" : "+s"(e_y), "+s"(e_bias), "+s"(e_nan_a), "+s"(e_nan_b));
    asm volatile("" : "+s"(e_ldy), "+s"(e_M), "+s"(e_N), "+s"(e_misc));
  }

  const int nk = (int)(g.Kp / BK);
  // K blocks [kb0, kb1) of this workgroup: all of them, or one split chunk
  const int kb0 = split_tail >= 0 ? (int)((int64_t)split_chunk * nk / g.split_s) : 0;
  const int kb1 = split_tail >= 0 ? (int)((int64_t)(split_chunk + 1) * nk / g.split_s) : nk;

  StageSrc src;
  {
    const int r = wave * 8 + (lane >> 3);
    const int c = (lane & 7) ^ swz_perm(r);
    src.ra = __builtin_amdgcn_make_buffer_rsrc((void*)g.a, (short)0, (int)(g.M * g.lda), 0x00020000);
    src.rb = __builtin_amdgcn_make_buffer_rsrc((void*)g.b, (short)0, (int)(g.N * g.ldb), 0x00020000);
    src.a_off = (uint32_t)((m0 + r) * g.lda + c * 16);
    src.b_off = (uint32_t)((n0 + r) * g.ldb + c * 16);
    src.a_grp = (uint32_t)(64 * g.lda);
    src.b_grp = (uint32_t)(64 * g.ldb);
  }

  v4f acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
  // whether any of this wave's rows m0 + wm*128 .. +127 is below M (for a
  // grouped tile, the expert's end); uniform per wave
  bool rows_live = true;
  if constexpr (B_UNIFORM) rows_live = __builtin_amdgcn_readfirstlane((int)(m0 + wm * 128 < g.M)) != 0;

#pragma unroll
  for (int j = 0; j < 4; ++j) issue_group(src, lds_a0, lds_b0, kb0, wave, j);
  lds_s0[tid] = s_src[(int64_t)kb0 * s_step];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // one K block from stage BUF while stage BUF^1 fills with block kt + 1
  auto step = [&](auto bufc, int kt) {
    constexpr int BUF = decltype(bufc)::value;
    const uint8_t* ta = BUF ? lds_a1 : lds_a0;
    const uint8_t* tb = BUF ? lds_b1 : lds_b0;
    const float* s_cur = BUF ? lds_s1 : lds_s0;
    // The copies into the idle stage are unconditional so the step is one
    // basic block: on the last K block they reload block kt (in bounds) into
    // the stage nobody reads again before the epilogue's barrier.
    const int kn = min(kt + 1, kb1 - 1);
    const float s_next = s_src[(int64_t)kn * s_step];

    if (B_UNIFORM && !rows_live) {
      // none of this wave's 128 rows is in the matrix (the last row tile of
      // an expert or of M): its share of the next block's copies only, no
      // fragments and no MFMAs; its accumulators stay zero and are never
      // stored.  The wave sharing its SIMD then has the matrix core alone.
#pragma unroll
      for (int j = 0; j < 4; ++j) issue_group(src, BUF ? lds_a0 : lds_a1, BUF ? lds_b0 : lds_b1, kn, wave, j);
    } else {
    v8i bf[4];
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) bf[tn] = load_frag(tb, wn * 64 + tn * 16, lane);

    float sbu = 0.f;
    v4f sbv[4];
    if constexpr (B_UNIFORM) {
      sbu = s_cur[BM + wn * 64];
    } else {
#pragma unroll
      for (int tn = 0; tn < 4; ++tn)
        sbv[tn] = *reinterpret_cast<const v4f*>(s_cur + BM + wn * 64 + tn * 16 + (lane >> 4) * 4);
    }
    // A fragments are double buffered by hand: the next 16-row group is read
    // from LDS while the current one is on the matrix cores.  The scheduling
    // fence keeps the compiler from hoisting all eight groups (64 VGPRs) at once.
    float sam_all[8];
#pragma unroll
    for (int tm = 0; tm < 8; ++tm) sam_all[tm] = s_cur[wm * 128 + tm * 16 + (lane & 15)];
    v8i af = load_frag(ta, wm * 128, lane);
    if constexpr (B_UNIFORM) {
      // The promotion is software pipelined: step tm issues group tm's four
      // blocks of MFMAs and promotes group tm-1's results meanwhile, one
      // block's MFMAs then one block's VALU work at a time (e4m3: 1 MFMA, 4
      // FMAs; int grid: 2 MFMAs, 4 converts and 4 FMAs), so the VALU never
      // waits on the MFMA it depends on.  The int32 partials stay raw until
      // then.  The per-column B scales of the other variant would spill here,
      // so that variant keeps the plain order.
      constexpr int MF = GRID == GRID_E4M3 ? 1 : 2, VA = GRID == GRID_E4M3 ? 4 : 8;
      raw_t<GRID> dp[4];
#pragma unroll
      for (int tm = 0; tm < 9; ++tm) {
        v8i af_next;
        raw_t<GRID> d[4];
        if (tm < 8) {
          if (tm + 1 < 8) af_next = load_frag(ta, wm * 128 + (tm + 1) * 16, lane);
          // the next block's copies go out one group per 16-row step, spread
          // over the first half of the MFMA phase
          if (tm < 4) issue_group(src, BUF ? lds_a0 : lds_a1, BUF ? lds_b0 : lds_b1, kn, wave, tm);
#pragma unroll
          for (int tn = 0; tn < 4; ++tn) d[tn] = mma_raw<GRID>(bf[tn], af);
        }
        if (tm > 0) {
          const float s = sam_all[tm - 1] * sbu;
#pragma unroll
          for (int tn = 0; tn < 4; ++tn) acc[tm - 1][tn] += raw_f32<GRID>(dp[tn]) * s;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);  // one block's MFMAs
            __builtin_amdgcn_sched_group_barrier(0x002, VA, 0);  // one block's promotion
          }
          // group tm-1's accumulators are final here, and no later LDS read
          // moves above this point
          asm volatile("" : "+v"(acc[tm - 1][0]), "+v"(acc[tm - 1][1]), "+v"(acc[tm - 1][2]),
                       "+v"(acc[tm - 1][3])::"memory");
        }
        if (tm < 8) {
#pragma unroll
          for (int tn = 0; tn < 4; ++tn) dp[tn] = d[tn];
          if (tm + 1 < 8) af = af_next;
        }
      }
    } else {
#pragma unroll
      for (int tm = 0; tm < 8; ++tm) {
        v8i af_next;
        if (tm + 1 < 8) af_next = load_frag(ta, wm * 128 + (tm + 1) * 16, lane);
        const float sam = sam_all[tm];
        if (tm < 4) issue_group(src, BUF ? lds_a0 : lds_a1, BUF ? lds_b0 : lds_b1, kn, wave, tm);
        v4f d[4];
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) d[tn] = mma_block<GRID>(bf[tn], af);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
          if constexpr (B_UNIFORM) {
            const float s = sam * sbu;
            acc[tm][tn] += d[tn] * s;
          } else {
            acc[tm][tn] += (d[tn] * sbv[tn]) * sam;
          }
        }
        // this group's accumulators are final here, and no later LDS read
        // moves above this point
        asm volatile("" : "+v"(acc[tm][0]), "+v"(acc[tm][1]), "+v"(acc[tm][2]), "+v"(acc[tm][3])::"memory");
        if (tm + 1 < 8) af = af_next;
      }
    }
    }
    (BUF ? lds_s0 : lds_s1)[tid] = s_next;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };

  for (int kt = kb0; kt < kb1; kt += 2) {
    step(std::integral_constant<int, 0>(), kt);
    if (kt + 1 < kb1) step(std::integral_constant<int, 1>(), kt + 1);
  }

  if constexpr (!GROUPED && EPI != EPI_SWIGLU) {
    // the last chunk to arrive sums all of them in chunk order and stores the tile
    if (split_tail >= 0 && !split_exchange(acc, g.ws, g.ws_count, split_tail, g.split_s, split_chunk, tid)) return;
  }

  if constexpr (EPI == EPI_SWIGLU) {
    // Stage the whole 256x256 tile as bf16 (the reference's Linear outputs):
    // slab k holds rows 64k..64k+63, 512 bytes per row, 16-byte units
    // XOR-swizzled by row so 16 lanes on 16 rows hit distinct banks.
    // NaN flags as bit masks (bit tm of the row flags, bit tn*4+q of the
    // column flags), loaded from clamped indices behind one uniform test per
    // pointer, so the staging below has no per-element branches
    uint32_t nan_rows = 0, nan_cols = 0;
    if (g.nan_a) {
#pragma unroll
      for (int tm = 0; tm < 8; ++tm)
        nan_rows |= (g.nan_a[min<int64_t>(m0 + wm * 128 + tm * 16 + (lane & 15), g.M - 1)] != 0 ? 1u : 0u) << tm;
    }
    if (g.nan_b) {
#pragma unroll
      for (int tn = 0; tn < 4; ++tn)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          nan_cols |= (g.nan_b[min<int64_t>(n0 + wn * 64 + tn * 16 + (lane >> 4) * 4 + q, g.N - 1)] != 0 ? 1u : 0u)
                      << (tn * 4 + q);
    }
    auto stage = [&](auto flagsc) {
      constexpr bool FLAGS = decltype(flagsc)::value;
#pragma unroll
      for (int tm = 0; tm < 8; ++tm) {
        const int r = wm * 128 + tm * 16 + (lane & 15);
        uint8_t* rowp = slab_row(lds_a0, lds_b0, lds_a1, lds_b1, r);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
          const int c = wn * 64 + tn * 16 + (lane >> 4) * 4;
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            v[q] = acc[tm][tn][q];
            if constexpr (FLAGS)
              v[q] = (((nan_rows >> tm) | (nan_cols >> (tn * 4 + q))) & 1u) ? __uint_as_float(0x7FC00000u) : v[q];
          }
          *reinterpret_cast<uint2*>(rowp + (((c >> 3) ^ (r & 15)) << 4) + (c & 4) * 2) =
              make_uint2((uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16),
                         (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16));
        }
      }
    };
    if (g.nan_a || g.nan_b)
      stage(std::true_type());
    else
      stage(std::false_type());
    __syncthreads();
    if (g.h_sr)
      swiglu_quant_rows<GRID, true>(g, lds_a0, lds_b0, lds_a1, lds_b1, m0, n0, tid);
    else
      swiglu_quant_rows<GRID, false>(g, lds_a0, lds_b0, lds_a1, lds_b1, m0, n0, tid);
    return;
  }

  // ---------------------------------------------------------------- epilogue
  // The tile origin passes through an empty asm here so that no address
  // arithmetic of the epilogue is hoisted above the K loop, where every
  // register is taken (hoisted values would be spilled across the loop).
  int lane_e = lane, wave_e = wave;
  asm volatile("" : "+s"(m0), "+s"(n0), "+v"(lane_e), "+s"(wave_e));
  // lane_e holds rows m = m0 + wm*128 + tm*16 + lane_e%16 and columns
  // n = n0 + wn*64 + tn*16 + 4*(lane_e/16) + r
  const int wm_e = wave_e >> 2, wn_e = wave_e & 3;
  const int slab = wave_e >> 1;
  uint8_t* stage_w = (slab == 0 ? lds_a0 : slab == 1 ? lds_b0 : slab == 2 ? lds_a1 : lds_b1) + (wave_e & 1) * (TILE_A / 2);
  const int64_t M = e_M, N = e_N, ldy = e_ldy;
  // bias and NaN flags: the indices are clamped into the matrix (values for
  // columns or rows past it are never stored), so the loads are
  // unconditional behind one uniform test per pointer; the flags are packed
  // into bit masks
  float bias[4][4];
#pragma unroll
  for (int tn = 0; tn < 4; ++tn)
#pragma unroll
    for (int r = 0; r < 4; ++r) bias[tn][r] = 0.f;
  if (e_bias) {
#pragma unroll
    for (int tn = 0; tn < 4; ++tn)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t n = min<int64_t>(n0 + wn_e * 64 + tn * 16 + (lane_e >> 4) * 4 + r, N - 1);
        bias[tn][r] = load_elem(reinterpret_cast<const void*>(e_bias), e_misc >> 1, n);
      }
  }
  uint32_t nan_cols = 0, nan_rows = 0;  // bit tn*4+r / bit tm
  if (e_nan_b) {
#pragma unroll
    for (int tn = 0; tn < 4; ++tn)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t n = min<int64_t>(n0 + wn_e * 64 + tn * 16 + (lane_e >> 4) * 4 + r, N - 1);
        nan_cols |= (reinterpret_cast<const int32_t*>(e_nan_b)[n] != 0 ? 1u : 0u) << (tn * 4 + r);
      }
  }
  if (e_nan_a) {
#pragma unroll
    for (int tm = 0; tm < 8; ++tm) {
      const int64_t m = min<int64_t>(m0 + wm_e * 128 + tm * 16 + (lane_e & 15), M - 1);
      nan_rows |= (reinterpret_cast<const int32_t*>(e_nan_a)[m] != 0 ? 1u : 0u) << tm;
    }
  }
  // Interior tiles (FULL) store without bounds checks; each wave stages and
  // re-reads only its own slice, so the waits between the two halves of a
  // pass are wave-local.
  constexpr int ODT = EPI == EPI_STORE_F32 ? DT_F32 : EPI == EPI_STORE_F16 ? DT_F16 : DT_BF16;
  auto store_tile = [&](auto fullc, auto flagsc) {
    constexpr bool FULL = decltype(fullc)::value;
    constexpr bool FLAGS = decltype(flagsc)::value;
    constexpr int esz = ODT == DT_F32 ? 4 : 2;
    constexpr int pitch = ODT == DT_F32 ? EPI_PITCH_F32 : EPI_PITCH_16;
#pragma unroll
    for (int part = 0; part < 4; ++part) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int tm = part * 2 + t;
        const int rloc = t * 16 + (lane_e & 15);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            v[r] = acc[tm][tn][r] + bias[tn][r];
            if constexpr (FLAGS) {
              const bool nan = ((nan_rows >> tm) | (nan_cols >> (tn * 4 + r))) & 1u;
              v[r] = nan ? __uint_as_float(0x7FC00000u) : v[r];
            }
          }
          uint8_t* dst = stage_w + rloc * pitch + (tn * 16 + (lane_e >> 4) * 4) * esz;
          if constexpr (ODT == DT_F32) {
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
          } else if constexpr (ODT == DT_BF16) {
            // hardware round-to-nearest-even pack (v_cvt_pk_bf16_f32)
            const v2bf p0 = {(__bf16)v[0], (__bf16)v[1]}, p1 = {(__bf16)v[2], (__bf16)v[3]};
            *reinterpret_cast<uint2*>(dst) =
                make_uint2(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1));
          } else {
            __half h[4] = {f32_to_f16(v[0]), f32_to_f16(v[1]), f32_to_f16(v[2]), f32_to_f16(v[3])};
            *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(h);
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
      __builtin_amdgcn_wave_barrier();
      // 32 rows x (128 or 256) bytes; 16-byte chunks, row-contiguous across lanes
      constexpr int chunks_per_row = 64 * esz / 16;
      constexpr int epc = 16 / esz;  // elements per chunk
#pragma unroll
      for (int j = 0; j < chunks_per_row / 2; ++j) {
        const int q = lane_e + 64 * j;
        const int row = q / chunks_per_row, c = q % chunks_per_row;
        const int64_t m = m0 + wm_e * 128 + part * EPI_ROWS + row;
        const int64_t n = n0 + wn_e * 64 + c * epc;
        const uint8_t* src = stage_w + row * pitch + c * 16;
        uint8_t* ydst = reinterpret_cast<uint8_t*>(e_y) + (m * ldy + n) * esz;
        if constexpr (FULL) {
          store16_nt(ydst, src);
          continue;
        }
        if (m >= M || n >= N) continue;
        if ((e_misc & 1) && n + epc <= N) {
          store16_nt(ydst, src);
        } else {
          // ragged edge or unaligned output: element by element
          using E = std::conditional_t<esz == 4, uint32_t, uint16_t>;
#pragma nounroll
          for (int e = 0; e < epc && n + e < N; ++e)
            reinterpret_cast<E*>(ydst)[e] = reinterpret_cast<const E*>(src)[e];
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // the re-reads are done before the next pass overwrites
      __builtin_amdgcn_wave_barrier();
    }
  };
  const bool full = (e_misc & 1) && m0 + BM <= M && n0 + BN <= N;
  if (e_nan_a || e_nan_b) {
    if (full)
      store_tile(std::true_type(), std::true_type());
    else
      store_tile(std::false_type(), std::true_type());
  } else {
    if (full)
      store_tile(std::true_type(), std::false_type());
    else
      store_tile(std::false_type(), std::false_type());
  }
}

// Thread t finishes row t/2 of the staged tile, h columns 64*(t%2) + [0,64):
// h = bf16(silu(gate) * up) with silu(x) = x / (1 + exp(-x)) in fp32 rounded
// to bf16 (F.silu on a bf16 tensor), the 1x128 tile amax shared with the
// partner lane t^1, then the tile's codes, scale, NaN flag and optional h.
template <int GRID, bool SR>
__device__ __forceinline__ void swiglu_quant_rows(const GemmArgs& g, const uint8_t* s0, const uint8_t* s1,
                                                  const uint8_t* s2, const uint8_t* s3, int64_t m0, int64_t n0,
                                                  int tid) {
#pragma clang fp contract(off)
  const int r = tid >> 1, hh = tid & 1;
  const int64_t m = m0 + r;
  const int64_t j0 = n0 / 2 + hh * 64;  // first h column of this thread
  uint8_t* rowp = slab_row(const_cast<uint8_t*>(s0), const_cast<uint8_t*>(s1), const_cast<uint8_t*>(s2),
                           const_cast<uint8_t*>(s3), r);
  // pass 1: h in bf16, written back over this thread's own gate units (no
  // other thread reads them), and the |h| maximum
  uint32_t amax = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uint8_t* gp = rowp + (((hh * 8 + k) ^ (r & 15)) << 4);
    const uint4 gw = *reinterpret_cast<const uint4*>(gp);
    const uint4 uw = *reinterpret_cast<const uint4*>(rowp + (((16 + hh * 8 + k) ^ (r & 15)) << 4));
    if (g.gu && m < g.M) {
      // the projections' bf16 outputs, kept for the SwiGLU backward
      uint16_t* gup = g.gu + m * g.ldgu + n0 + hh * 64 + k * 8;
      *reinterpret_cast<uint4*>(gup) = gw;
      *reinterpret_cast<uint4*>(gup + 128) = uw;
    }
    const uint32_t gg[4] = {gw.x, gw.y, gw.z, gw.w}, uu[4] = {uw.x, uw.y, uw.z, uw.w};
    uint32_t hb[4];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float gv = bf16_bits_to_f32((gg[q >> 1] >> (16 * (q & 1))) & 0xFFFFu);
      const float uv = bf16_bits_to_f32((uu[q >> 1] >> (16 * (q & 1))) & 0xFFFFu);
      const float sg = bf16_bits_to_f32(f32_to_bf16_bits(gv / (1.0f + expf(-gv))));
      const uint32_t h = f32_to_bf16_bits(sg * uv);
      amax = max(amax, (h & 0x7FFFu) << 16);
      hb[q >> 1] = (q & 1) ? (hb[q >> 1] | (h << 16)) : h;
    }
    *reinterpret_cast<uint4*>(gp) = make_uint4(hb[0], hb[1], hb[2], hb[3]);
  }
  amax = max(amax, (uint32_t)__shfl_xor((int)amax, 1));
  const float s = scale_from_amax_bits(amax, g.h_qmaxf, g.h_scale_rule);
  const float rs = fast_div_ok<SR>(amax) ? 1.0f / s : 1.0f;
  if (m >= g.M) return;
  // pass 2: codes (and h) 8 columns at a time from the bf16 h in LDS
  bool nan = false;
  for (int k = 0; k < 8; ++k) {
    const uint4 hw = *reinterpret_cast<const uint4*>(rowp + (((hh * 8 + k) ^ (r & 15)) << 4));
    const uint32_t hh4[4] = {hw.x, hw.y, hw.z, hw.w};
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = bf16_bits_to_f32((hh4[q >> 1] >> (16 * (q & 1))) & 0xFFFFu);
    uint32_t rb[8];
    sr_words<SR>((uint64_t)(m * g.I + j0 + k * 8), g.h_seed, g.h_offset, rb);
    uint32_t lo, hi;
    float q[8];
    nan |= quant8_tile_rs<GRID, SR, false>(v, amax, s, rs, g.h_qmaxf, rb, lo, hi, q);
    *reinterpret_cast<uint2*>(g.hc + m * g.ldhc + j0 + k * 8) = make_uint2(lo, hi);
    if (g.h) *reinterpret_cast<uint4*>(g.h + m * g.ldh + j0 + k * 8) = hw;
  }
  if (hh == 0) {
    g.hs[m * g.hs_row + (n0 / 256) * g.hs_col] = s;
    if (nan && g.h_nan) atomicOr(g.h_nan + m, 1);
  }
}

}  // namespace ntlb

using namespace ntlb;

// the store kernel for the output dtype
template <int GRID, bool B_UNIFORM, bool GROUPED>
static void launch_store(const GemmArgs& g, dim3 grd, dim3 blk, hipStream_t st) {
  if (g.y_dtype == DT_F32)
    gemm_blockscaled_kernel<GRID, B_UNIFORM, GROUPED, EPI_STORE_F32><<<grd, blk, 0, st>>>(g);
  else if (g.y_dtype == DT_F16)
    gemm_blockscaled_kernel<GRID, B_UNIFORM, GROUPED, EPI_STORE_F16><<<grd, blk, 0, st>>>(g);
  else
    gemm_blockscaled_kernel<GRID, B_UNIFORM, GROUPED, EPI_STORE><<<grd, blk, 0, st>>>(g);
}

// the split-K tail's minimum K blocks per range (K 1024, 8 blocks: 25 us
// split, 16 unsplit)
constexpr int SPLIT_MIN_BLOCKS = 9;

extern "C" int64_t ntlb_gemm_workspace_bytes(int64_t M, int64_t N, int64_t Kp) {
  if (M <= 0 || N <= 0 || Kp <= 0 || Kp % BK) return 0;
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > 0x7FFFFFFF) return 0;
  return split_ws_bytes(split_plan(tiles, (int)(Kp / BK), SPLIT_MIN_BLOCKS));
}

extern "C" int ntlb_gemm_blockscaled_ws(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                                        int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb, const float* sb,
                                        int64_t sb_row, int64_t sb_col, int b_shift, int64_t M, int64_t N,
                                        int64_t Kp, const void* bias, int bias_dtype, void* y, int y_dtype,
                                        int64_t ldy, const int32_t* nan_a, const int32_t* nan_b, void* workspace,
                                        int64_t ws_bytes, void* stream) {
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
  // buffer resources address each operand with 32-bit byte offsets
  if ((M + BM) * lda >= (int64_t)0x7FFFFFFF || (N + BN) * ldb >= (int64_t)0x7FFFFFFF)
    return fail(NTLB_EUNSUPPORTED, "%s: an operand exceeds 2 GiB of codes", fn);
  GemmArgs g{};
  g.a = a; g.lda = lda; g.sa = sa; g.sa_row = sa_row; g.sa_col = sa_col; g.a_shift = a_shift;
  g.b = b; g.ldb = ldb; g.sb = sb; g.sb_row = sb_row; g.sb_col = sb_col; g.b_shift = b_shift;
  g.M = M; g.N = N; g.Kp = Kp;
  g.bias = bias; g.bias_dtype = bias_dtype;
  g.y = y; g.y_dtype = y_dtype; g.ldy = ldy;
  g.nan_a = nan_a; g.nan_b = nan_b;
  g.vec_out = aligned(y, 16) && ((ldy * dtype_size(y_dtype)) % 16 == 0);
  g.offsets = nullptr; g.n_experts = 0; g.b_estride = 0; g.sb_estride = 0;
  g.split_base = (int)tiles; g.split_s = 1; g.ws = nullptr; g.ws_count = nullptr;
  int64_t grid_wgs = tiles;
  if (workspace) {
    if (!aligned(workspace, 256)) return fail(NTLB_EINVAL, "%s: workspace must be 256-byte aligned", fn);
    const SplitPlan plan = split_plan(tiles, (int)(Kp / BK), SPLIT_MIN_BLOCKS);
    if (plan.s > 1 && ws_bytes >= split_ws_bytes(plan)) {
      g.split_base = plan.base; g.split_s = plan.s;
      g.ws_count = reinterpret_cast<uint32_t*>(workspace);
      g.ws = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + split_count_bytes());
      grid_wgs = (int64_t)plan.base + (int64_t)plan.tail * plan.s;
    }
  }
  // B's scale is uniform over each wave's 64 columns for 128x128 blocks and tensor scales
  const bool b_uniform = (b_shift == 7) || (sb_row == 0);
  hipStream_t st = as_stream(stream);
  dim3 grd((unsigned)grid_wgs), blk(NTHREADS);
  if (grid == NTLB_GRID_E4M3) {
    if (b_uniform)
      launch_store<GRID_E4M3, true, false>(g, grd, blk, st);
    else
      launch_store<GRID_E4M3, false, false>(g, grd, blk, st);
  } else {
    if (b_uniform)
      launch_store<GRID_INT, true, false>(g, grd, blk, st);
    else
      launch_store<GRID_INT, false, false>(g, grd, blk, st);
  }
  return check_launch(fn);
}

extern "C" int ntlb_gemm_blockscaled(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                                     int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb, const float* sb,
                                     int64_t sb_row, int64_t sb_col, int b_shift, int64_t M, int64_t N, int64_t Kp,
                                     const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                                     const int32_t* nan_a, const int32_t* nan_b, void* stream) {
  return ntlb_gemm_blockscaled_ws(grid, a, lda, sa, sa_row, sa_col, a_shift, b, ldb, sb, sb_row, sb_col, b_shift, M,
                                  N, Kp, bias, bias_dtype, y, y_dtype, ldy, nan_a, nan_b, nullptr, 0, stream);
}

extern "C" int ntlb_gemm_grouped_blockscaled(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                                             int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb,
                                             int64_t b_estride, const float* sb, int64_t sb_row, int64_t sb_col,
                                             int b_shift, int64_t sb_estride, const int32_t* offsets, int n_experts,
                                             int64_t M_total, int64_t N, int64_t Kp, void* y, int y_dtype,
                                             int64_t ldy, const int32_t* nan_a, const int32_t* nan_b, void* stream) {
  const char* fn = "ntlb_gemm_grouped_blockscaled";
  if (grid != NTLB_GRID_INT && grid != NTLB_GRID_E4M3) return fail(NTLB_EINVAL, "%s: bad grid %d", fn, grid);
  if (M_total < 0 || N < 0 || Kp < 0 || n_experts < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (Kp % 128) return fail(NTLB_EINVAL, "%s: Kp %lld is not a multiple of 128", fn, (long long)Kp);
  if (M_total == 0 || N == 0 || n_experts == 0) return NTLB_OK;
  if (!a || !b || !sa || !sb || !y || !offsets) return fail(NTLB_EINVAL, "%s: NULL operand", fn);
  if (lda < Kp || ldb < Kp || (lda % 16) || (ldb % 16) || !aligned(a, 16) || !aligned(b, 16) ||
      (b_estride % 16) || b_estride < N * ldb)
    return fail(NTLB_EINVAL, "%s: code matrices need ld >= Kp, ld %% 16 == 0, 16-byte alignment and "
                "b_estride >= N*ldb", fn);
  if (!(a_shift == 0 || a_shift == 7) || !(b_shift == 0 || b_shift == 7))
    return fail(NTLB_EINVAL, "%s: scale shifts must be 0 or 7", fn);
  if (!valid_dtype(y_dtype) || ldy < N) return fail(NTLB_EINVAL, "%s: bad output dtype or ldy", fn);
  if (Kp == 0) return fail(NTLB_EUNSUPPORTED, "%s: K == 0", fn);
  if ((M_total + BM) * lda >= (int64_t)0x7FFFFFFF || (N + BN) * ldb >= (int64_t)0x7FFFFFFF)
    return fail(NTLB_EUNSUPPORTED, "%s: an operand exceeds 2 GiB of codes", fn);
  if ((int64_t)(n_experts + 1) * 4 > TILE_A)
    return fail(NTLB_EUNSUPPORTED, "%s: more than %d experts", fn, TILE_A / 4 - 1);
  const int64_t tiles = ((M_total + BM - 1) / BM + n_experts) * ((N + BN - 1) / BN);
  if (tiles > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  GemmArgs g{};
  g.a = a; g.lda = lda; g.sa = sa; g.sa_row = sa_row; g.sa_col = sa_col; g.a_shift = a_shift;
  g.b = b; g.ldb = ldb; g.sb = sb; g.sb_row = sb_row; g.sb_col = sb_col; g.b_shift = b_shift;
  g.M = M_total; g.N = N; g.Kp = Kp;
  g.bias = nullptr; g.bias_dtype = 0;
  g.y = y; g.y_dtype = y_dtype; g.ldy = ldy;
  g.nan_a = nan_a; g.nan_b = nan_b;
  g.vec_out = aligned(y, 16) && ((ldy * dtype_size(y_dtype)) % 16 == 0);
  g.offsets = offsets; g.n_experts = n_experts; g.b_estride = b_estride; g.sb_estride = sb_estride;
  g.split_base = 0; g.split_s = 1; g.ws = nullptr; g.ws_count = nullptr;
  const bool b_uniform = (b_shift == 7) || (sb_row == 0);
  hipStream_t st = as_stream(stream);
  dim3 grd((unsigned)tiles), blk(NTHREADS);
  if (grid == NTLB_GRID_E4M3) {
    if (b_uniform)
      launch_store<GRID_E4M3, true, true>(g, grd, blk, st);
    else
      launch_store<GRID_E4M3, false, true>(g, grd, blk, st);
  } else {
    if (b_uniform)
      launch_store<GRID_INT, true, true>(g, grd, blk, st);
    else
      launch_store<GRID_INT, false, true>(g, grd, blk, st);
  }
  return check_launch(fn);
}

// ---------------------------------------------------------------------------
// SwiGLU + 1x128 quantization epilogue: the expert MLP's gate and up
// projections (moe.py:190-193: F.silu(gate_proj(x)) * up_proj(x)) in one GEMM
// over B rows interleaved in 128-row blocks (gate block t, then up block t),
// writing h's 1x128 codes (the down projection's A operand) and optionally h.
// ---------------------------------------------------------------------------
static int swiglu_common(const char* fn, GemmArgs& g, int grid, int64_t N, uint16_t* h, int64_t ldh, uint8_t* hc,
                         int64_t ldhc, float* hs, int64_t hs_row, int64_t hs_col, int32_t* h_nan, int qmax,
                         int rounding, int scale_rule, uint64_t seed, uint64_t offset) {
  if (N % 256) return fail(NTLB_EUNSUPPORTED, "%s: N = 2*I must be a multiple of 256 (I a multiple of 128)", fn);
  const int64_t I = N / 2;
  if (!hc || !hs) return fail(NTLB_EINVAL, "%s: NULL h codes or scales", fn);
  if (ldhc < I || ldhc % 16 || !aligned(hc, 16))
    return fail(NTLB_EINVAL, "%s: h codes need ldhc >= I, ldhc %% 16 == 0, 16-byte alignment", fn);
  if (h && (ldh < I || ldh % 8 || !aligned(h, 16)))
    return fail(NTLB_EINVAL, "%s: h needs ldh >= I, ldh %% 8 == 0, 16-byte alignment", fn);
  if (grid == NTLB_GRID_INT && (qmax < 1 || qmax > 127)) return fail(NTLB_EINVAL, "%s: qmax outside [1, 127]", fn);
  if (rounding != NTLB_ROUND_NEAREST && rounding != NTLB_ROUND_STOCHASTIC)
    return fail(NTLB_EINVAL, "%s: bad rounding %d", fn, rounding);
  if (scale_rule != NTLB_SCALE_AFTER_DIVIDE && scale_rule != NTLB_SCALE_BEFORE_DIVIDE)
    return fail(NTLB_EINVAL, "%s: bad scale rule %d", fn, scale_rule);
  g.h = h; g.ldh = ldh; g.hc = hc; g.ldhc = ldhc; g.hs = hs; g.hs_row = hs_row; g.hs_col = hs_col; g.h_nan = h_nan;
  g.h_qmaxf = grid == NTLB_GRID_E4M3 ? 448.0f : (float)qmax;
  g.h_sr = rounding == NTLB_ROUND_STOCHASTIC;
  g.h_scale_rule = scale_rule;
  g.h_seed = seed; g.h_offset = offset; g.I = I;
  g.y = nullptr; g.y_dtype = NTLB_BF16; g.ldy = 0; g.vec_out = 0; g.bias = nullptr; g.bias_dtype = 0;
  return NTLB_OK;
}

extern "C" int ntlb_gemm_swiglu_quant(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                                      int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb, const float* sb,
                                      int64_t sb_row, int64_t sb_col, int64_t M, int64_t N, int64_t Kp,
                                      const int32_t* nan_a, const int32_t* nan_b, uint16_t* h, int64_t ldh,
                                      uint8_t* hc, int64_t ldhc, float* hs, int64_t hs_row, int64_t hs_col,
                                      int32_t* h_nan, int qmax, int rounding, int scale_rule, uint64_t seed,
                                      uint64_t offset, void* stream) {
  const char* fn = "ntlb_gemm_swiglu_quant";
  if (grid != NTLB_GRID_INT && grid != NTLB_GRID_E4M3) return fail(NTLB_EINVAL, "%s: bad grid %d", fn, grid);
  if (M < 0 || N < 0 || Kp < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (Kp % 128 || Kp == 0) return fail(NTLB_EINVAL, "%s: Kp must be a positive multiple of 128", fn);
  if (M == 0 || N == 0) return NTLB_OK;
  if (!a || !b || !sa || !sb) return fail(NTLB_EINVAL, "%s: NULL operand", fn);
  if (lda < Kp || ldb < Kp || (lda % 16) || (ldb % 16) || !aligned(a, 16) || !aligned(b, 16))
    return fail(NTLB_EINVAL, "%s: code matrices need ld >= Kp, ld %% 16 == 0 and 16-byte alignment", fn);
  if (!(a_shift == 0 || a_shift == 7)) return fail(NTLB_EINVAL, "%s: a_shift must be 0 or 7", fn);
  if ((M + BM) * lda >= (int64_t)0x7FFFFFFF || (N + BN) * ldb >= (int64_t)0x7FFFFFFF)
    return fail(NTLB_EUNSUPPORTED, "%s: an operand exceeds 2 GiB of codes", fn);
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  GemmArgs g{};
  g.a = a; g.lda = lda; g.sa = sa; g.sa_row = sa_row; g.sa_col = sa_col; g.a_shift = a_shift;
  g.b = b; g.ldb = ldb; g.sb = sb; g.sb_row = sb_row; g.sb_col = sb_col; g.b_shift = 7;
  g.M = M; g.N = N; g.Kp = Kp;
  g.nan_a = nan_a; g.nan_b = nan_b;
  g.offsets = nullptr; g.n_experts = 0; g.b_estride = 0; g.sb_estride = 0;
  g.split_base = 0; g.split_s = 1; g.ws = nullptr; g.ws_count = nullptr;
  int rc = swiglu_common(fn, g, grid, N, h, ldh, hc, ldhc, hs, hs_row, hs_col, h_nan, qmax, rounding, scale_rule,
                         seed, offset);
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  dim3 grd((unsigned)tiles), blk(NTHREADS);
  if (grid == NTLB_GRID_E4M3)
    gemm_blockscaled_kernel<GRID_E4M3, true, false, EPI_SWIGLU><<<grd, blk, 0, st>>>(g);
  else
    gemm_blockscaled_kernel<GRID_INT, true, false, EPI_SWIGLU><<<grd, blk, 0, st>>>(g);
  return check_launch(fn);
}

extern "C" int ntlb_gemm_grouped_swiglu_quant(int grid, const uint8_t* a, int64_t lda, const float* sa,
                                              int64_t sa_row, int64_t sa_col, int a_shift, const uint8_t* b,
                                              int64_t ldb, int64_t b_estride, const float* sb, int64_t sb_row,
                                              int64_t sb_col, int64_t sb_estride, const int32_t* offsets,
                                              int n_experts, int64_t M_total, int64_t N, int64_t Kp,
                                              const int32_t* nan_a, const int32_t* nan_b, uint16_t* h, int64_t ldh,
                                              uint8_t* hc, int64_t ldhc, float* hs, int64_t hs_row, int64_t hs_col,
                                              int32_t* h_nan, int qmax, int rounding, int scale_rule, uint64_t seed,
                                              uint64_t offset, void* stream) {
  return ntlb_gemm_grouped_swiglu_quant_gu(grid, a, lda, sa, sa_row, sa_col, a_shift, b, ldb, b_estride, sb, sb_row,
                                           sb_col, sb_estride, offsets, n_experts, M_total, N, Kp, nan_a, nan_b, h,
                                           ldh, hc, ldhc, hs, hs_row, hs_col, h_nan, qmax, rounding, scale_rule, seed,
                                           offset, nullptr, 0, stream);
}

extern "C" int ntlb_gemm_grouped_swiglu_quant_gu(int grid, const uint8_t* a, int64_t lda, const float* sa,
                                                 int64_t sa_row, int64_t sa_col, int a_shift, const uint8_t* b,
                                                 int64_t ldb, int64_t b_estride, const float* sb, int64_t sb_row,
                                                 int64_t sb_col, int64_t sb_estride, const int32_t* offsets,
                                                 int n_experts, int64_t M_total, int64_t N, int64_t Kp,
                                                 const int32_t* nan_a, const int32_t* nan_b, uint16_t* h, int64_t ldh,
                                                 uint8_t* hc, int64_t ldhc, float* hs, int64_t hs_row, int64_t hs_col,
                                                 int32_t* h_nan, int qmax, int rounding, int scale_rule, uint64_t seed,
                                                 uint64_t offset, uint16_t* gu, int64_t ldgu, void* stream) {
  const char* fn = "ntlb_gemm_grouped_swiglu_quant";
  if (grid != NTLB_GRID_INT && grid != NTLB_GRID_E4M3) return fail(NTLB_EINVAL, "%s: bad grid %d", fn, grid);
  if (M_total < 0 || N < 0 || Kp < 0 || n_experts < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (Kp % 128 || Kp == 0) return fail(NTLB_EINVAL, "%s: Kp must be a positive multiple of 128", fn);
  if (M_total == 0 || N == 0 || n_experts == 0) return NTLB_OK;
  if (!a || !b || !sa || !sb || !offsets) return fail(NTLB_EINVAL, "%s: NULL operand", fn);
  if (lda < Kp || ldb < Kp || (lda % 16) || (ldb % 16) || !aligned(a, 16) || !aligned(b, 16) ||
      (b_estride % 16) || b_estride < N * ldb)
    return fail(NTLB_EINVAL, "%s: code matrices need ld >= Kp, ld %% 16 == 0, 16-byte alignment and "
                "b_estride >= N*ldb", fn);
  if (!(a_shift == 0 || a_shift == 7)) return fail(NTLB_EINVAL, "%s: a_shift must be 0 or 7", fn);
  if ((M_total + BM) * lda >= (int64_t)0x7FFFFFFF || (N + BN) * ldb >= (int64_t)0x7FFFFFFF)
    return fail(NTLB_EUNSUPPORTED, "%s: an operand exceeds 2 GiB of codes", fn);
  if ((int64_t)(n_experts + 1) * 4 > TILE_A)
    return fail(NTLB_EUNSUPPORTED, "%s: more than %d experts", fn, TILE_A / 4 - 1);
  const int64_t tiles = ((M_total + BM - 1) / BM + n_experts) * ((N + BN - 1) / BN);
  if (tiles > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  GemmArgs g{};
  g.a = a; g.lda = lda; g.sa = sa; g.sa_row = sa_row; g.sa_col = sa_col; g.a_shift = a_shift;
  g.b = b; g.ldb = ldb; g.sb = sb; g.sb_row = sb_row; g.sb_col = sb_col; g.b_shift = 7;
  g.M = M_total; g.N = N; g.Kp = Kp;
  g.nan_a = nan_a; g.nan_b = nan_b;
  g.offsets = offsets; g.n_experts = n_experts; g.b_estride = b_estride; g.sb_estride = sb_estride;
  g.split_base = 0; g.split_s = 1; g.ws = nullptr; g.ws_count = nullptr;
  if (gu && (ldgu < N || ldgu % 8 || !aligned(gu, 16)))
    return fail(NTLB_EINVAL, "%s: the gate/up output needs ld >= N, ld %% 8 == 0 and 16-byte alignment", fn);
  g.gu = gu; g.ldgu = ldgu;
  int rc = swiglu_common(fn, g, grid, N, h, ldh, hc, ldhc, hs, hs_row, hs_col, h_nan, qmax, rounding, scale_rule,
                         seed, offset);
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  dim3 grd((unsigned)tiles), blk(NTHREADS);
  if (grid == NTLB_GRID_E4M3)
    gemm_blockscaled_kernel<GRID_E4M3, true, true, EPI_SWIGLU><<<grd, blk, 0, st>>>(g);
  else
    gemm_blockscaled_kernel<GRID_INT, true, true, EPI_SWIGLU><<<grd, blk, 0, st>>>(g);
  return check_launch(fn);
}
