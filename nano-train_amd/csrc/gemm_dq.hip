// GEMM over dequantized operands for gfx950:
//   Y[M,N] = A[M,:] . B[N,:]^T (+ bias), fp32 accumulation,
// where each operand reaches the matrix cores as the values the reference's
// emulated backend multiplies: bf16(q * s) or fp32(q * s) decoded from codes
// and scales in the tile prologue (te_backend.py:173-202 casts every
// dequantized operand back to the input dtype before its fp32 F.linear), or
// a plain bf16 / fp32 matrix (the gradient dY).  Products of bf16 values are
// exact in fp32, so on bf16 operands v_mfma_f32_16x16x32_bf16 computes the
// reference's fp32 GEMM up to the order of the fp32 additions; fp32 operands
// run v_mfma_f32_16x16x4_f32.
//
// Serves:
//   the reference-exact forward      Y  = bf16(dq(X)) . bf16(dq(W))^T + b   (te_backend.py:229-260)
//   the straight-through dgrad       dX = dY . bf16(dq(W))                  (autograd of te_backend.py:253-259)
//   the straight-through wgrad       dW = dY^T . bf16(dq(X))
//   plain GEMMs over dequantized tensors (granularities whose scales vary
//   along the contraction element by element)
//   the persistent layers' dgrad       dX = dY . deq(W)                     (layers.py:409-436 straight through)
//
// Operand sources (one per operand, a template parameter):
//   SRC_DIRECT : bf16/fp32 [rows, >= Kc] row-major, contraction contiguous;
//                global -> LDS with buffer_load ... lds, no registers
//   SRC_CODES  : uint8 codes [rows, ldc], contraction contiguous, fp32
//                scales; each thread decodes 32 (bf16) or 16 (fp32) codes of
//                one row per K step
//   SRC_TDIRECT: bf16/fp32 stored transposed, element (r, c) at p[c*ld + r]
//                (the contraction is the slow index: dY^T in wgrad); each
//                thread loads an 8x4 (bf16) or 4x4 (fp32) block and writes
//                it transposed
//   SRC_TCODES : codes stored transposed, (r, c) at codes[c*ldc + r] (W for
//                dgrad, X for wgrad), decoded and written transposed
//   SRC_TNF4   : a persistent NF4 weight stored transposed, its nibbles flat
//                row-major over [contraction, rows] (two per byte, the even
//                element low): codebook value times scale, for the dgrad of
//                a persistent layer without a dequantized copy
//   SRC_PCODES : a persistent NF4 or FP8 weight [rows, K] row-major (NF4
//                nibbles flat, two per byte), contraction contiguous, one
//                scale per row or one for all; values past K are zero (the
//                next row's codes follow in memory): the forward of a
//                persistent layer over fp32 activations or a K that is not
//                a multiple of 64
//   SRC_TR     : bf16 stored transposed, as SRC_TDIRECT, copied global ->
//                LDS as stored (buffer_load ... lds, no registers, no VALU)
//                and read back transposed by gfx950's ds_read_b64_tr_b16;
//                the host picks it for every bf16 SRC_TDIRECT operand
//                except the wgrad that sums its dY rows into db
// Scales of a coded operand: s(r, c) = s[(r >> r_shift)*s_r + (c >> c_shift)*s_c].
//
// Tiling: 256x256 output tile per workgroup, K step of 128 bytes per row (64
// bf16 or 32 fp32), 512 threads = 8 waves as 2 (M) x 4 (N), each wave
// 128x64, the LDS layout and fragment reads of the blockwise fp8 GEMM
// (16-byte chunks XOR-swizzled by row).  Register-staged operands load block
// kt+2 at the end of step kt (in flight across the barrier) and decode it
// into the idle stage during step kt+1, two 16-byte chunks per thread at
// 16-row groups 4 and 6, so the VALU decode interleaves with the MFMAs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "ntlb_device.h"
#include "ntlb_host.h"
#include "ntlb_splitk.h"

namespace ntlb {
namespace gdq {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int SRC_DIRECT = 0, SRC_CODES = 1, SRC_TDIRECT = 2, SRC_TCODES = 3, SRC_TNF4 = 4, SRC_PCODES = 5,
              SRC_TR = 6;
// the code format of a SRC_PCODES operand (the GRID parameter): e4m3 codes,
// or NF4 nibbles
constexpr int GRID_NF4 = 2;

constexpr float kNF4v[16] = NTLB_NF4_CODEBOOK;
constexpr int EL_BF16 = 0, EL_F32 = 1;

constexpr int TM = 256, TN = 256;  // output tile
constexpr int ROWB = 128;          // bytes per tile row per K step
constexpr int TILE = 256 * ROWB;   // 32 KiB per operand stage
constexpr int NT = 512;
constexpr int EPI_ROWS = 32;
constexpr int EPI_PITCH_F32 = 64 * 4 + 16;
constexpr int EPI_PITCH_16 = 64 * 2 + 16;
static_assert(EPI_ROWS * EPI_PITCH_F32 <= TILE / 2, "epilogue slice exceeds half a stage");

template <int EL>
struct ElemT {
  static constexpr int bytes = EL == EL_BF16 ? 2 : 4;
  static constexpr int kstep = ROWB / bytes;  // contraction elements per K step
};

// 16-byte chunk c of row r inside a [256][128-byte] tile: rows 0-7 get eight
// distinct chunks and every 16-row window distinct (row parity, chunk) pairs,
// so the 16-lane fragment reads are bank-conflict free
__device__ __forceinline__ int sw_perm(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int sw(int r, int c) { return r * ROWB + ((c ^ sw_perm(r)) << 4); }

// MFMA fragment of 16 rows: row = lane%16, bytes [32g, 32g+32) of the row with
// g = lane/16; both operands use this map, so the products pair up
__device__ __forceinline__ v8i frag(const uint8_t* tile, int row0, int lane) {
  const int r = row0 + (lane & 15);
  const int g = lane >> 4;
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + sw(r, 2 * g));
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + sw(r, 2 * g + 1));
  v8i f;
  f[0] = (int)lo.x; f[1] = (int)lo.y; f[2] = (int)lo.z; f[3] = (int)lo.w;
  f[4] = (int)hi.x; f[5] = (int)hi.y; f[6] = (int)hi.z; f[7] = (int)hi.w;
  return f;
}

// SRC_TR stages: [64 contraction rows][256 operand rows] bf16, 512 bytes per
// contraction row, the 16-byte chunk c (operand rows 8c..8c+7) of row k at
// tr_off(k, c).  ds_read_b64_tr_b16 hands lane i of each 16-lane group the
// four 16-bit values that lanes 4j + i/4 (j = 0..3) loaded at position i%4
// (measured on gfx950).  So when lane 4j + q of the group loads operand rows
// row0 + 4q .. 4q+3 of contraction row kk + j, lane i receives operand row
// row0 + i at contraction kk .. kk+3.  A 16-lane group touches contraction
// rows kk..kk+3 (k & 3 = j) and two adjacent chunks; the XOR with 2(k & 3)
// spreads those eight 16-byte pieces over eight chunk slots, and bit 4 of
// the row (the next group's rows, 16 further) flips bit 3 of the slot, so
// 32 lanes read 256 distinct bytes.
constexpr int TR_ROWB = 512;
__device__ __forceinline__ int tr_perm(int k) { return (2 * (k & 3)) ^ (8 * ((k >> 4) & 1)); }
__device__ __forceinline__ int tr_off(int k, int c) { return k * TR_ROWB + ((c ^ tr_perm(k)) << 4); }

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s* lds_v4s_ptr;

// the fragment of frag() (lane group g: contraction 16g .. 16g+15 of the
// step, operand row row0 + lane%16) from an SRC_TR stage: four transposing
// loads of four contraction values each
__device__ __forceinline__ v8i frag_tr(const uint8_t* tile, int row0, int lane) {
  const int g = lane >> 4, j = (lane >> 2) & 3, q = lane & 3;
  const int c = (row0 >> 3) + (q >> 1);
  v8i f;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int k = 16 * g + 4 * h + j;
    const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4s_ptr)(tile + tr_off(k, c) + (q & 1) * 8));
    f[2 * h] = (int)(((uint32_t)(uint16_t)v[1] << 16) | (uint16_t)v[0]);
    f[2 * h + 1] = (int)(((uint32_t)(uint16_t)v[3] << 16) | (uint16_t)v[2]);
  }
  return f;
}

// acc += P . Q^T over one K step's fragment pair (64 bf16 or 32 fp32 values)
template <int EL>
__device__ __forceinline__ v4f mma_step(const v8i& p, const v8i& q, v4f acc) {
  if constexpr (EL == EL_BF16) {
    const v4i pl = {p[0], p[1], p[2], p[3]}, ph = {p[4], p[5], p[6], p[7]};
    const v4i ql = {q[0], q[1], q[2], q[3]}, qh = {q[4], q[5], q[6], q[7]};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, pl), __builtin_bit_cast(v8bf, ql), acc,
                                                  0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ph), __builtin_bit_cast(v8bf, qh), acc,
                                                  0, 0, 0);
  } else {
    // lane group g supplies contraction 8g + i to MFMA i
#pragma unroll
    for (int i = 0; i < 8; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__int_as_float(p[i]), __int_as_float(q[i]), acc, 0, 0, 0);
  }
  return acc;
}

struct Operand {
  const uint8_t* p;  // matrix or codes
  int64_t ld;        // row pitch of the stored matrix, in elements (codes: bytes)
  int64_t rows;      // DIRECT/CODES: rows of the matrix; TDIRECT/TCODES: stored columns (the operand's rows)
  int64_t kvalid;    // TDIRECT/TCODES: stored rows (contraction) holding data; zero past them
  const float* s;    // scales of a coded operand
  int64_t s_r, s_c;
  int r_shift, c_shift;
  int grid;          // GRID_INT (int8 codes, -128 = NaN) or GRID_E4M3
  int smode;         // TCODES scales: SC_SHARED or SC_CONTIG (set by the host)
  int64_t s_extent;  // scale elements addressed by the operand (max index + 1)
};

// How a TCODES operand's scales vary along the contraction rows of a wave
// (a template parameter of the kernel): one value for the wave's CPW rows
// (128-row blocks, tensor), or consecutive floats (per-token scales of 1x128
// tiles, per-row scales of a channel-scaled W^T), read as 16-byte loads.
constexpr int SC_SHARED = 0, SC_CONTIG = 1;

struct DqArgs {
  Operand a, b;
  int64_t M, N, Kc;  // Kc: contraction length, a multiple of the K step
  const void* bias;
  int bias_dtype;
  void* y;
  int y_dtype;
  int64_t ldy;
  int vec_out;
  // split-K tail (the blockwise GEMM's scheme): workgroups at or past
  // split_base take one of split_s K ranges of a tail tile; the last range to
  // finish sums the fp32 partials in range order and stores the tile
  int split_base, split_s;
  float* ws;
  uint32_t* ws_count;
  // grouped (per-expert) modes, the GRP template parameter; offsets int32
  // [n_experts + 1] into rows sorted by expert:
  //   GRP_ROWS: expert e owns the rows [offsets[e], offsets[e+1]) of A and of
  //     Y and multiplies its own B, at b.p + e*b_estride bytes with scales at
  //     b.s + e*bs_estride (the dgrad of every expert's Linear at once);
  //   GRP_K: the contraction of expert e runs over those rows of both
  //     (transposed) operands, and its Y, of M x N, lies at y + e*y_estride
  //     bytes (the wgrad of every expert's Linear at once).
  const int32_t* offsets;
  int n_experts;
  int64_t b_estride, bs_estride, y_estride;
  // IL kernels: the contraction is one half of a gate / up interleaved
  // operand (128-wide blocks alternating gate block t and up block t): logical
  // K step kt reads physical step 4*(kt/2) + kt%2 + 2*il_half of both operands
  int il_half;
  // add the bf16 output to what y holds: y = bf16(y + bf16(acc)), the sum of
  // two Linears' input gradients as autograd forms it
  int accum;
  // TDIRECT A (the wgrad's dY^T), ungrouped: the workgroups of the first
  // output column tile also store db[r] = the sum of A's row r over the
  // contraction (the column sums of dY: the bias gradient), in db_dtype
  void* db;
  int db_dtype;
};

constexpr int GRP_NONE = 0, GRP_ROWS = 1, GRP_K = 2;

// 4 codes (byte i = element i) times s in fp32: the reference's q * scale
template <int GRID>
__device__ __forceinline__ void decode4(uint32_t w, float s, float (&v)[4]) {
#pragma clang fp contract(off)
  if constexpr (GRID == GRID_E4M3) {
    const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    v[0] = lo[0] * s; v[1] = lo[1] * s; v[2] = hi[0] * s; v[3] = hi[1] * s;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = (int)(int8_t)(uint8_t)(w >> (8 * i));
      v[i] = c == -128 ? __uint_as_float(0x7FC00000u) : (float)c * s;
    }
  }
}

// two codes (bytes 2h, 2h+1 of w) times s
template <int GRID, int H>
__device__ __forceinline__ void decode2(uint32_t w, float s, float& v0, float& v1) {
#pragma clang fp contract(off)
  constexpr int h = H;
  if constexpr (GRID == GRID_E4M3) {
    const v2f t = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, H != 0);
    v0 = t[0] * s;
    v1 = t[1] * s;
  } else {
    const int c0 = (int)(int8_t)(uint8_t)(w >> (16 * h)), c1 = (int)(int8_t)(uint8_t)(w >> (16 * h + 8));
    v0 = c0 == -128 ? __uint_as_float(0x7FC00000u) : (float)c0 * s;
    v1 = c1 == -128 ? __uint_as_float(0x7FC00000u) : (float)c1 * s;
  }
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const v2bf p = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32, round to nearest even
  return __builtin_bit_cast(uint32_t, p);
}

// ---------------------------------------------------------------------------
// Register-staged operand loaders.  Each holds one K block's raw data and
// writes it decoded into a stage in two halves (two 16-byte chunks each).
// ---------------------------------------------------------------------------
template <int SRC, int EL, int GRID, int SCM>
struct Stager;

// DIRECT and TR: no registers (global -> LDS copies issued by the step)
template <int EL, int GRID, int SCM>
struct Stager<SRC_DIRECT, EL, GRID, SCM> {
  __device__ void init(const Operand&, int64_t, int, int) {}
  __device__ void load(const Operand&, int) {}
  template <int H>
  __device__ void decode_half(const Operand&, uint8_t*) {}
};
template <int EL, int GRID, int SCM>
struct Stager<SRC_TR, EL, GRID, SCM> : Stager<SRC_DIRECT, EL, GRID, SCM> {};

// CODES: thread t decodes row t/2, half t%2 of the K block
template <int EL, int GRID, int SCM>
struct Stager<SRC_CODES, EL, GRID, SCM> {
  static constexpr int span = ElemT<EL>::kstep / 2;  // codes per thread per K step: 32 or 16
  uint4 ra, rb;
  float sc;
  const uint8_t* rowp;
  int64_t srow;
  int br, bh;
  __device__ void init(const Operand& o, int64_t r0, int tid, int) {
    br = tid >> 1;
    bh = tid & 1;
    const int64_t r = min<int64_t>(r0 + br, o.rows - 1);  // rows past the end feed outputs never stored
    rowp = o.p + r * o.ld + bh * span;
    srow = (r >> o.r_shift) * o.s_r;
  }
  __device__ void load(const Operand& o, int kt) {
    const uint8_t* q = rowp + (int64_t)kt * ElemT<EL>::kstep;
    ra = *reinterpret_cast<const uint4*>(q);
    if constexpr (EL == EL_BF16) rb = *reinterpret_cast<const uint4*>(q + 16);
    const int64_t c0 = (int64_t)kt * ElemT<EL>::kstep + bh * span;
    sc = o.s[srow + (c0 >> o.c_shift) * o.s_c];
  }
  template <int H>
  __device__ void decode_half(const Operand& o, uint8_t* tile) {
    constexpr int h = H;
    const uint32_t w[8] = {ra.x, ra.y, ra.z, ra.w, rb.x, rb.y, rb.z, rb.w};
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * h + jj;  // chunk of this thread's span
      uint4 out;
      if constexpr (EL == EL_BF16) {
        float v[8];
        float t[4];
        decode4<GRID>(w[2 * j], sc, t);
        v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
        decode4<GRID>(w[2 * j + 1], sc, t);
        v[4] = t[0]; v[5] = t[1]; v[6] = t[2]; v[7] = t[3];
        out = make_uint4(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                         pack_bf16(v[6], v[7]));
      } else {
        float t[4];
        decode4<GRID>(w[j], sc, t);
        out = make_uint4(__float_as_uint(t[0]), __float_as_uint(t[1]), __float_as_uint(t[2]), __float_as_uint(t[3]));
      }
      *reinterpret_cast<uint4*>(tile + sw(br, bh * 4 + j)) = out;
    }
  }
};

// Buffer resource over the first kvalid stored rows of a transposed operand:
// reads at or past kvalid*ld*eb bytes return zero, which zero-fills the
// contraction past kvalid (and keeps the lanes past the last stored row in
// bounds).  Lanes whose operand row r lies past the operand's rows read
// whatever follows in memory: those values reach only output rows or columns
// that are never stored.  The entry points check (kvalid + 64) * ld * eb < 2^31.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t trows_rsrc(const Operand& o, int eb) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)o.p, (short)0, (int)(o.kvalid * o.ld * eb), 0x00020000);
}

// TDIRECT: wave w takes contraction rows [w*CPW, w*CPW + CPW) of the K step,
// lane l the operand rows 4l .. 4l+3 (one 8- or 16-byte load per row)
template <int EL, int GRID, int SCM>
struct Stager<SRC_TDIRECT, EL, GRID, SCM> {
  static constexpr int CPW = EL == EL_BF16 ? 8 : 4;
  uint32_t w[CPW][EL == EL_BF16 ? 2 : 4];
  __amdgpu_buffer_rsrc_t rs;
  uint32_t roff;   // byte offset of operand row 4l inside a stored row
  uint32_t rstep;  // bytes per stored row
  int cw, l;
  __device__ void init(const Operand& o, int64_t r0, int tid, int) {
    constexpr int eb = ElemT<EL>::bytes;
    cw = __builtin_amdgcn_readfirstlane(tid >> 6);
    l = tid & 63;
    rs = trows_rsrc(o, eb);
    roff = (uint32_t)((r0 + 4 * l) * eb);
    rstep = (uint32_t)(o.ld * eb);
  }
  __device__ void load(const Operand&, int kt) {
    const uint32_t c0 = (uint32_t)(kt * ElemT<EL>::kstep + cw * CPW);
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const uint32_t off = (c0 + j) * rstep + roff;
      if constexpr (EL == EL_BF16) {
        typedef unsigned v2u __attribute__((ext_vector_type(2)));
        const v2u t = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)off, 0, 0);
        w[j][0] = t[0]; w[j][1] = t[1];
      } else {
        typedef unsigned v4u __attribute__((ext_vector_type(4)));
        const v4u t = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0);
        w[j][0] = t[0]; w[j][1] = t[1]; w[j][2] = t[2]; w[j][3] = t[3];
      }
    }
  }
  template <int H>
  __device__ void decode_half(const Operand&, uint8_t* tile) {
    constexpr int h = H;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = 2 * h + ii;  // operand row 4l + i
      uint4 out;
      if constexpr (EL == EL_BF16) {
        // dword p = (element i of contraction row 2p, element i of row 2p+1)
        const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
        const int k = i >> 1;
        out = make_uint4(__builtin_amdgcn_perm(w[1][k], w[0][k], sel), __builtin_amdgcn_perm(w[3][k], w[2][k], sel),
                         __builtin_amdgcn_perm(w[5][k], w[4][k], sel), __builtin_amdgcn_perm(w[7][k], w[6][k], sel));
      } else {
        out = make_uint4(w[0][i], w[1][i], w[2][i], w[3][i]);
      }
      *reinterpret_cast<uint4*>(tile + sw(4 * l + i, cw)) = out;
    }
  }
  // bf16: adds the staged block's CPW contraction values of operand row
  // 4l + i to s[i] (an LDS slot), in row order, one row at a time
  __device__ void colsum(float* s) {
    if constexpr (EL == EL_BF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float t = s[i];
#pragma unroll
        for (int j = 0; j < CPW; ++j) t += bf16_bits_to_f32((w[j][i >> 1] >> (16 * (i & 1))) & 0xFFFFu);
        s[i] = t;
      }
    }
  }
};

// TCODES: as TDIRECT, with one code byte per element (one 4-byte load per
// contraction row) and a scale per contraction row: the scale of a lane's
// four rows is one value (r_shift >= 2 or s_r == 0)
template <int EL, int GRID, int SCM>
struct Stager<SRC_TCODES, EL, GRID, SCM> {
  static constexpr int CPW = EL == EL_BF16 ? 8 : 4;
  uint32_t w[CPW];
  float sc[CPW];  // per-row scales (SC_CONTIG, SC_GATHER)
  float sc1;      // the wave's one scale (SC_SHARED)
  __amdgpu_buffer_rsrc_t rs, rss;
  uint32_t roff, rstep, soff;
  int cw, l;
  __device__ void init(const Operand& o, int64_t r0, int tid, int) {
    cw = __builtin_amdgcn_readfirstlane(tid >> 6);
    l = tid & 63;
    const int64_t r = r0 + 4 * l;
    rs = trows_rsrc(o, 1);
    roff = (uint32_t)r;
    rstep = (uint32_t)o.ld;
    // scales through a resource bounded by their extent: indices past it read 0
    rss = __builtin_amdgcn_make_buffer_rsrc((void*)o.s, (short)0, (int)(o.s_extent * 4), 0x00020000);
    soff = (uint32_t)((min<int64_t>(r, o.rows - 1) >> o.r_shift) * o.s_r);
  }
  __device__ void load(const Operand& o, int kt) {
    const int cbase = kt * ElemT<EL>::kstep + cw * CPW;  // uniform over the wave
#pragma unroll
    for (int j = 0; j < CPW; ++j)
      w[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)((uint32_t)(cbase + j) * rstep + roff), 0, 0);
    if constexpr (SCM == SC_SHARED) {
      const int64_t c = min<int64_t>(cbase, o.kvalid - 1);
      sc1 = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(rss, (int)((soff + (uint32_t)((c >> o.c_shift) * o.s_c)) * 4), 0, 0));
    } else {
      // rows past kvalid hold zero codes, but the scale slots there are the
      // array's padding or the next rows' scales, which can be NaN or inf:
      // their scales are taken as zero so that 0 * scale adds nothing (cbase
      // is uniform over the wave, so only the last step's waves select)
#pragma unroll
      for (int k = 0; k < CPW / 4; ++k) {
        const uint4 v = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rss, (int)((soff + (uint32_t)cbase + 4 * k) * 4), 0, 0));
        sc[4 * k] = __uint_as_float(v.x); sc[4 * k + 1] = __uint_as_float(v.y);
        sc[4 * k + 2] = __uint_as_float(v.z); sc[4 * k + 3] = __uint_as_float(v.w);
      }
      if ((int64_t)(cbase + CPW) > o.kvalid) {
#pragma unroll
        for (int j = 0; j < CPW; ++j) sc[j] = (int64_t)(cbase + j) < o.kvalid ? sc[j] : 0.f;
      }
    }
  }
  template <int H>
  __device__ void decode_half(const Operand& o, uint8_t* tile) {
    constexpr int h = H;
    float v[CPW][2];
#pragma unroll
    for (int j = 0; j < CPW; ++j) decode2<GRID, H>(w[j], SCM == SC_SHARED ? sc1 : sc[j], v[j][0], v[j][1]);
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = 2 * h + ii;
      uint4 out;
      if constexpr (EL == EL_BF16) {
        out = make_uint4(pack_bf16(v[0][ii], v[1][ii]), pack_bf16(v[2][ii], v[3][ii]), pack_bf16(v[4][ii], v[5][ii]),
                         pack_bf16(v[6][ii], v[7][ii]));
      } else {
        out = make_uint4(__float_as_uint(v[0][ii]), __float_as_uint(v[1][ii]), __float_as_uint(v[2][ii]),
                         __float_as_uint(v[3][ii]));
      }
      *reinterpret_cast<uint4*>(tile + sw(4 * l + i, cw)) = out;
    }
  }
};

// PCODES: thread t decodes row t/2, half t%2 of the K block (as CODES), from
// a buffer resource over the whole weight: NF4 as 2-byte loads of four
// nibbles (the rows start at K/2-byte offsets, K % 4 == 0), e4m3 as 4-byte
// loads of four codes (K % 4 == 0).  The row's scale is loaded once.  Columns
// at or past K (kvalid) decode to 0: the loads there return the next row's
// codes, or zero past the buffer.
template <int EL, int GRID, int SCM>
struct Stager<SRC_PCODES, EL, GRID, SCM> {
  static constexpr int span = ElemT<EL>::kstep / 2;  // elements per thread per K step: 32 or 16
  static constexpr int NWD = span / 4;                 // words of four codes
  uint32_t w[NWD];
  float sc;
  __amdgpu_buffer_rsrc_t rs;
  uint32_t rowb;  // byte offset of the row
  int br, bh;
  int lim;        // elements of the loaded block inside K (0 .. span)
  const float* cb;  // NF4: the codebook in LDS, set by the kernel
  __device__ void init(const Operand& o, int64_t r0, int tid, int) {
    br = tid >> 1;
    bh = tid & 1;
    const int64_t r = min<int64_t>(r0 + br, o.rows - 1);  // rows past the end feed outputs never stored
    rs = __builtin_amdgcn_make_buffer_rsrc((void*)o.p, (short)0, (int)(o.rows * o.ld), 0x00020000);
    rowb = (uint32_t)(r * o.ld);
    sc = o.s[(r >> o.r_shift) * o.s_r];
  }
  __device__ void load(const Operand& o, int kt) {
    const uint32_t c0 = (uint32_t)(kt * ElemT<EL>::kstep + bh * span);
    lim = (int)max<int64_t>(0, min<int64_t>(o.kvalid - (int64_t)c0, span));
#pragma unroll
    for (int j = 0; j < NWD; ++j) {
      if constexpr (GRID == GRID_NF4)
        w[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)(rowb + ((c0 + 4 * j) >> 1)), 0, 0);
      else
        w[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(rowb + c0 + 4 * j), 0, 0);
    }
  }
  // the four values of word j (elements c0 + 4j .. c0 + 4j + 3)
  __device__ void value4(const Operand& o, int j, int lim, float (&v)[4]) {
#pragma clang fp contract(off)
    if constexpr (GRID == GRID_NF4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = cb[(w[j] >> (4 * i)) & 0xF] * sc;
    } else {
      decode4<GRID_E4M3>(w[j], sc, v);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = 4 * j + i < lim ? v[i] : 0.f;
  }
  template <int H>
  __device__ void decode_half(const Operand& o, uint8_t* tile) {
    constexpr int h = H;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * h + jj;  // chunk of this thread's span
      uint4 out;
      if constexpr (EL == EL_BF16) {
        float a[4], b[4];
        value4(o, 2 * j, lim, a);
        value4(o, 2 * j + 1, lim, b);
        out = make_uint4(pack_bf16(a[0], a[1]), pack_bf16(a[2], a[3]), pack_bf16(b[0], b[1]), pack_bf16(b[2], b[3]));
      } else {
        float a[4];
        value4(o, j, lim, a);
        out = make_uint4(__float_as_uint(a[0]), __float_as_uint(a[1]), __float_as_uint(a[2]), __float_as_uint(a[3]));
      }
      *reinterpret_cast<uint4*>(tile + sw(br, bh * 4 + j)) = out;
    }
  }
};

// TNF4: the TCODES walk over 4-bit codes.  The weight's nibbles run flat
// over its [kvalid, rows] storage (ld = bytes per stored row = rows / 2), so
// a lane's four operand rows of one contraction row are one 2-byte load.
// Value = codebook[nibble] * scale in fp32 (layers.py:172-184), the codebook
// read from LDS (16 floats, one per bank); rows past kvalid get scale 0 and
// so the value 0 (nibble 0 is the code value -1, not 0).
template <int EL, int GRID, int SCM>
struct Stager<SRC_TNF4, EL, GRID, SCM> {
  static constexpr int CPW = EL == EL_BF16 ? 8 : 4;
  uint32_t w[CPW];
  float sc[CPW];
  __amdgpu_buffer_rsrc_t rs, rss;
  uint32_t roff, rstep, soff;
  int cw, l;
  const float* cb;  // the codebook in LDS, set by the kernel
  __device__ void init(const Operand& o, int64_t r0, int tid, int) {
    cw = __builtin_amdgcn_readfirstlane(tid >> 6);
    l = tid & 63;
    const int64_t r = r0 + 4 * l;
    rs = trows_rsrc(o, 1);
    roff = (uint32_t)(r >> 1);
    rstep = (uint32_t)o.ld;
    rss = __builtin_amdgcn_make_buffer_rsrc((void*)o.s, (short)0, (int)(o.s_extent * 4), 0x00020000);
    soff = (uint32_t)((min<int64_t>(r, o.rows - 1) >> o.r_shift) * o.s_r);
  }
  __device__ void load(const Operand& o, int kt) {
    const int cbase = kt * ElemT<EL>::kstep + cw * CPW;  // uniform over the wave
#pragma unroll
    for (int j = 0; j < CPW; ++j)
      w[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)((uint32_t)(cbase + j) * rstep + roff), 0, 0);
    if constexpr (SCM == SC_SHARED) {
      const int64_t c = min<int64_t>(cbase, o.kvalid - 1);
      const float s1 = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(rss, (int)((soff + (uint32_t)((c >> o.c_shift) * o.s_c)) * 4), 0, 0));
#pragma unroll
      for (int j = 0; j < CPW; ++j) sc[j] = (int64_t)(cbase + j) < o.kvalid ? s1 : 0.f;
    } else {
#pragma unroll
      for (int k = 0; k < CPW / 4; ++k) {
        const uint4 v = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rss, (int)((soff + (uint32_t)cbase + 4 * k) * 4), 0, 0));
        const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sc[4 * k + i] = (int64_t)(cbase + 4 * k + i) < o.kvalid ? __uint_as_float(vv[i]) : 0.f;
      }
    }
  }
  template <int H>
  __device__ void decode_half(const Operand& o, uint8_t* tile) {
#pragma clang fp contract(off)
    constexpr int h = H;
    float v[CPW][2];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      v[j][0] = cb[(w[j] >> (8 * h)) & 0xF] * sc[j];
      v[j][1] = cb[(w[j] >> (8 * h + 4)) & 0xF] * sc[j];
    }
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = 2 * h + ii;
      uint4 out;
      if constexpr (EL == EL_BF16) {
        out = make_uint4(pack_bf16(v[0][ii], v[1][ii]), pack_bf16(v[2][ii], v[3][ii]), pack_bf16(v[4][ii], v[5][ii]),
                         pack_bf16(v[6][ii], v[7][ii]));
      } else {
        out = make_uint4(__float_as_uint(v[0][ii]), __float_as_uint(v[1][ii]), __float_as_uint(v[2][ii]),
                         __float_as_uint(v[3][ii]));
      }
      *reinterpret_cast<uint4*>(tile + sw(4 * l + i, cw)) = out;
    }
  }
};

// DIRECT copies: wave w moves the 8-row groups w, w+8, w+16, w+24 of the
// stage; lane i lands at byte 16*i of its group (row i/8, physical chunk i%8)
// and fetches logical chunk (i%8) ^ sw_perm(row), the same for all four
// groups since bit 3 of the rows is w & 1.  Rows past the matrix lie beyond
// the resource's num_records and read as zero.
struct Direct {
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off, grp;
  __device__ void init(const Operand& o, int64_t r0, int wave, int lane, int eb) {
    const int xr = wave * 8 + (lane >> 3);
    rs = __builtin_amdgcn_make_buffer_rsrc((void*)o.p, (short)0, (int)(o.rows * o.ld * eb), 0x00020000);
    off = (uint32_t)((r0 + xr) * o.ld * eb + ((lane & 7) ^ sw_perm(xr)) * 16);
    grp = (uint32_t)(64 * o.ld * eb);
  }
  __device__ void issue(uint8_t* stage, int kt, int wave, int j) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(stage + (wave + 8 * j) * 8 * ROWB), 16, off,
                                             (uint32_t)kt * ROWB + j * grp, 0, 0);
  }
};

// TR copies: copy j of wave w moves contraction rows R and R + 1 of the
// stage, R = 2(w & 3) + 16(w >> 2) + 8(j & 1) + 32(j >> 1), one 1 KiB LDS
// run: lane i lands at byte 16i of it (row R + i/32, chunk slot i%32) and
// fetches the chunk (i%32) ^ tr_perm(row), which is the same for the four
// copies (they differ in row bits 3 and 5, which tr_perm ignores).  Rows
// past kvalid read zero through the resource; columns past the operand's
// rows reach only outputs that are never stored.  The entry points check
// (kvalid + 64) * ld * 2 < 2^31.
struct TrCopy {
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off, rowb;
  __device__ static int row0(int wave, int j) {
    return 2 * (wave & 3) + 16 * (wave >> 2) + 8 * (j & 1) + 32 * (j >> 1);
  }
  __device__ void init(const Operand& o, int64_t r0, int wave, int lane) {
    const int R = row0(wave, 0) + (lane >> 5);
    const int c = (lane & 31) ^ tr_perm(R);
    rs = trows_rsrc(o, 2);
    rowb = (uint32_t)(o.ld * 2);
    off = (uint32_t)R * rowb + (uint32_t)((r0 + 8 * c) * 2);
  }
  __device__ void issue(uint8_t* stage, int kt, int wave, int j) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(stage + row0(wave, j) * TR_ROWB), 16, off,
                                             (uint32_t)(kt * 64 + 8 * (j & 1) + 32 * (j >> 1)) * rowb, 0, 0);
  }
};

template <int EL, int SA, int SB, int GRID, int SCM, int GRP = GRP_NONE, bool IL = false, bool DB = false>
__global__ void __launch_bounds__(NT, 1) gemm_dq_kernel(DqArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t la0[TILE];
  __shared__ __attribute__((aligned(16))) uint8_t lb0[TILE];
  __shared__ __attribute__((aligned(16))) uint8_t la1[TILE];
  __shared__ __attribute__((aligned(16))) uint8_t lb1[TILE];
  constexpr int EB = ElemT<EL>::bytes;
  constexpr int KSTEP = ElemT<EL>::kstep;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  // workgroup -> tile: each XCD walks a contiguous range of the whole tiles,
  // grouped raster of GROUP_M row tiles; the split tail's ranges keep their
  // tile
  constexpr int GROUP_M = 4;
  auto xcd_local = [](int p, int nwg) {
    const int xcd = p & 7, local = p >> 3;
    const int per = nwg >> 3, extra = nwg & 7;
    return xcd * per + min(xcd, extra) + local;
  };
  // tile l of a num_m x num_n raster of GROUP_M row tiles
  auto raster = [](int l, int num_m, int num_n, int64_t& m0, int64_t& n0) {
    const int group = l / (GROUP_M * num_n);
    const int first_m = group * GROUP_M;
    const int gsize = min(num_m - first_m, GROUP_M);
    const int in_group = l - group * GROUP_M * num_n;
    m0 = (int64_t)(first_m + in_group % gsize) * TM;
    n0 = (int64_t)(in_group / gsize) * TN;
  };
  const int num_n = (int)((g.N + TN - 1) / TN);
  const int num_m = (int)((g.M + TM - 1) / TM);
  SplitWork sw{(int)blockIdx.x, -1, 0};
  int64_t m0, n0;
  int nk = (int)(g.Kc / KSTEP);
  if constexpr (GRP == GRP_ROWS) {
    // experts in order, each one's row tiles in the raster of the dense case,
    // consecutive tiles on consecutive XCDs (not a contiguous range per XCD:
    // that gave the XCDs holding the small experts' ragged last row tiles
    // less work than the others); the grid is an upper bound on the tile
    // count (the offset table is read into LDS, free until the first copy)
    int32_t* tab = reinterpret_cast<int32_t*>(la0);
    for (int i = tid; i <= g.n_experts; i += NT) tab[i] = g.offsets[i];
    __syncthreads();
    const int pid = (int)blockIdx.x;
    int e = 0, before = 0, tiles_m = 0;
    int64_t lo = 0, hi = 0;
    for (; e < g.n_experts; ++e) {
      lo = tab[e];
      hi = tab[e + 1];
      tiles_m = (int)((hi - lo + TM - 1) / TM);
      if (pid < before + tiles_m * num_n) break;
      before += tiles_m * num_n;
    }
    __syncthreads();  // the table's LDS is a copy target from here on
    if (e >= g.n_experts) return;  // past the last expert's tiles
    raster(pid - before, tiles_m, num_n, m0, n0);
    m0 += lo;
    g.M = hi;  // rows at or past the expert's end are not stored
    g.b.p += (int64_t)e * g.b_estride;
    if constexpr (SB == SRC_TCODES) g.b.s += (int64_t)e * g.bs_estride;
  } else if constexpr (GRP == GRP_K) {
    // every expert has the num_m x num_n tiles of its own Y; its contraction
    // is its rows, so both operands start at row offsets[e] and hold
    // offsets[e+1] - offsets[e] valid rows (zero past them, through the
    // buffer resources); an expert without rows stores zeros.  A tile's work
    // is its expert's row count, which routing skews (Zipf at config 4: 263
    // to 4019 rows): the experts go out longest first, and consecutive tiles
    // go to consecutive XCDs (no contiguous per-XCD ranges, which would hand
    // one XCD all of the popular experts' tiles)
    const int per = num_m * num_n;
    const int q = (int)blockIdx.x / per;  // rank of the expert by row count
    int e = q;
    if (g.n_experts <= NT) {
      int32_t* tab = reinterpret_cast<int32_t*>(la0);
      for (int i = tid; i <= g.n_experts; i += NT) tab[i] = g.offsets[i];
      __syncthreads();
      int* who = reinterpret_cast<int*>(la0) + NT + 1;
      if (tid < g.n_experts) {
        const int ni = tab[tid + 1] - tab[tid];
        int rank = 0;
        for (int j = 0; j < g.n_experts; ++j) {
          const int nj = tab[j + 1] - tab[j];
          rank += (nj > ni || (nj == ni && j < tid)) ? 1 : 0;
        }
        who[rank] = tid;
      }
      __syncthreads();
      e = who[q];
      __syncthreads();  // the LDS is a copy target from here on
    }
    raster((int)blockIdx.x - q * per, num_m, num_n, m0, n0);
    const int64_t lo = g.offsets[e], rows_e = g.offsets[e + 1] - lo;
    g.a.p += lo * g.a.ld * EB;
    g.a.kvalid = rows_e;
    if constexpr (SB == SRC_TCODES) {
      g.b.p += lo * g.b.ld;
      g.b.s += lo;  // per-row scales, consecutive along the contraction
      g.b.s_extent -= lo;
    } else {
      g.b.p += lo * g.b.ld * EB;  // a dense operand: ld in elements
    }
    g.b.kvalid = rows_e;
    nk = max(1, (int)((rows_e + KSTEP - 1) / KSTEP));
    g.y = reinterpret_cast<uint8_t*>(g.y) + (int64_t)e * g.y_estride;
  } else {
    sw = split_work(blockIdx.x, g.split_base, g.split_s);
    int pid = sw.pid;
    if (sw.tail < 0) pid = xcd_local(pid, g.split_s > 1 ? g.split_base : num_m * num_n);
    raster(pid, num_m, num_n, m0, n0);
  }

  static_assert((SA != SRC_TR && SB != SRC_TR) || EL == EL_BF16, "transposing LDS loads take 16-bit values");
  Direct da, db;
  TrCopy ta_c, tb_c;
  if constexpr (SA == SRC_DIRECT) da.init(g.a, m0, wave, lane, EB);
  if constexpr (SB == SRC_DIRECT) db.init(g.b, n0, wave, lane, EB);
  if constexpr (SA == SRC_TR) ta_c.init(g.a, m0, wave, lane);
  if constexpr (SB == SRC_TR) tb_c.init(g.b, n0, wave, lane);
  Stager<SA, EL, GRID, SCM> sa;
  Stager<SB, EL, GRID, SCM> sb;
  sa.init(g.a, m0, tid, lane);
  sb.init(g.b, n0, tid, lane);
  if constexpr (SB == SRC_TNF4 || (SB == SRC_PCODES && GRID == GRID_NF4)) {
    __shared__ float nf4_tab[16];
    if (tid < 16) nf4_tab[tid] = kNF4v[tid];
    __syncthreads();
    sb.cb = nf4_tab;
  }

  // the bias gradient rides on the wgrad's dY stream: the tiles of the first
  // output column tile sum their A rows over the contraction (each staged
  // block once, in block order; the waves' sums added in wave order)
  const bool do_db = DB && n0 == 0;
  static_assert(!DB || (SA == SRC_TDIRECT && EL == EL_BF16 && GRP == GRP_NONE), "db rides on a bf16 dY^T stream");
  // each thread's running sums of its four operand rows live in LDS slots it
  // alone touches (registers here made the int-grid variants spill)
  // (the slot address is recomputed where it is used, from the scalar wave
  // index and the lane id, so that no register holds it through the loop)
  __shared__ float db_part[DB ? 8 * 256 : 1];
  auto db_slot = [&]() -> float* {
    const int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    return db_part + wave * 256 + 4 * ln;
  };
  if constexpr (DB) {
    if (do_db) {
      float* d = db_slot();
#pragma unroll
      for (int i = 0; i < 4; ++i) d[i] = 0.f;
    }
  }
  auto db_add = [&]() {
    if constexpr (DB) sa.colsum(db_slot());
  };

  // logical K step -> the step the loaders read (IL: one half of the
  // interleaved gate / up contraction)
  const int il_half = g.il_half;
  auto kmap = [il_half](int kt) { return IL ? ((kt >> 1) << 2) + (kt & 1) + 2 * il_half : kt; };
  // K steps [kb0, kb1) of this workgroup: all of them, or one split range
  const int kb0 = sw.tail >= 0 ? (int)((int64_t)sw.chunk * nk / g.split_s) : 0;
  const int kb1 = sw.tail >= 0 ? (int)((int64_t)(sw.chunk + 1) * nk / g.split_s) : nk;
  // the epilogue's arguments, kept in scalar registers through the K loop
  uintptr_t e_y = reinterpret_cast<uintptr_t>(g.y), e_bias = reinterpret_cast<uintptr_t>(g.bias);
  int64_t e_ldy = g.ldy, e_M = g.M, e_N = g.N;
  int e_misc = (g.vec_out ? 1 : 0) | (g.bias_dtype << 1) | (g.y_dtype << 4) | (g.accum ? 128 : 0);
  e_y = uniform64(e_y); e_bias = uniform64(e_bias);
  e_ldy = uniform64(e_ldy); e_M = uniform64(e_M); e_N = uniform64(e_N);
  e_misc = __builtin_amdgcn_readfirstlane(e_misc);
  asm volatile("" : "+s"(e_y), "+s"(e_bias), "+s"(e_ldy), "+s"(e_M), "+s"(e_N), "+s"(e_misc));

  v4f acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

  // prologue: block kb0 into stage 0, block kb0+1's raw data into registers
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (SA == SRC_DIRECT) da.issue(la0, kmap(kb0), wave, j);
    if constexpr (SB == SRC_DIRECT) db.issue(lb0, kmap(kb0), wave, j);
    if constexpr (SA == SRC_TR) ta_c.issue(la0, kmap(kb0), wave, j);
    if constexpr (SB == SRC_TR) tb_c.issue(lb0, kmap(kb0), wave, j);
  }
  sa.load(g.a, kmap(kb0));
  sb.load(g.b, kmap(kb0));
  sa.template decode_half<0>(g.a, la0);
  sb.template decode_half<0>(g.b, lb0);
  sa.template decode_half<1>(g.a, la0);
  sb.template decode_half<1>(g.b, lb0);
  if constexpr (DB) {
    if (do_db) db_add();
  }
  sa.load(g.a, kmap(min(kb0 + 1, kb1 - 1)));
  sb.load(g.b, kmap(min(kb0 + 1, kb1 - 1)));
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // one K block from stage BUF while stage BUF^1 receives block kt + 1.  The
  // DIRECT copies into the idle stage are unconditional (the last step reloads
  // its own block) so the step is one basic block.
  auto step = [&](auto bufc, int kt) {
    constexpr int BUF = decltype(bufc)::value;
    const uint8_t* ta = BUF ? la1 : la0;
    const uint8_t* tb = BUF ? lb1 : lb0;
    uint8_t* na = BUF ? la0 : la1;
    uint8_t* nb = BUF ? lb0 : lb1;
    const int kn = min(kt + 1, kb1 - 1);
    auto frag_a = [&](int row0) { return SA == SRC_TR ? frag_tr(ta, row0, lane) : frag(ta, row0, lane); };
    auto frag_b = [&](int row0) { return SB == SRC_TR ? frag_tr(tb, row0, lane) : frag(tb, row0, lane); };
    v8i bf[4];
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) bf[tn] = frag_b(wn * 64 + tn * 16);
    v8i af = frag_a(wm * 128);
#pragma unroll
    for (int tm = 0; tm < 8; ++tm) {
      v8i af_next;
      if (tm + 1 < 8) af_next = frag_a(wm * 128 + (tm + 1) * 16);
      if (tm < 4) {
        if constexpr (SA == SRC_DIRECT) da.issue(na, kmap(kn), wave, tm);
        if constexpr (SB == SRC_DIRECT) db.issue(nb, kmap(kn), wave, tm);
        if constexpr (SA == SRC_TR) ta_c.issue(na, kmap(kn), wave, tm);
        if constexpr (SB == SRC_TR) tb_c.issue(nb, kmap(kn), wave, tm);
      }
      if (tm == 4) {
        sa.template decode_half<0>(g.a, na);
        sb.template decode_half<0>(g.b, nb);
      }
      if (tm == 6) {
        sa.template decode_half<1>(g.a, na);
        sb.template decode_half<1>(g.b, nb);
      }
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) acc[tm][tn] = mma_step<EL>(bf[tn], af, acc[tm][tn]);
      asm volatile("" : "+v"(acc[tm][0]), "+v"(acc[tm][1]), "+v"(acc[tm][2]), "+v"(acc[tm][3])::"memory");
      if (tm + 1 < 8) af = af_next;
    }
    // the staged block kt+1 still sits in the A stager's registers, and the
    // fragments are dead: add it to the bias gradient (once: the last steps
    // reload the last block)
    if constexpr (DB) {
      if (do_db && kt + 1 < kb1) db_add();
    }
    // every copy of this step has landed (vmcnt(0)); then block kt+2's raw
    // data goes out and stays in flight across the barrier
    __builtin_amdgcn_s_waitcnt(0x0F70);
    sa.load(g.a, kmap(min(kt + 2, kb1 - 1)));
    sb.load(g.b, kmap(min(kt + 2, kb1 - 1)));
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the decode's LDS writes are done
    __syncthreads();
  };

  for (int kt = kb0; kt < kb1; kt += 2) {
    step(std::integral_constant<int, 0>(), kt);
    if (kt + 1 < kb1) step(std::integral_constant<int, 1>(), kt + 1);
  }
  // a split range: the last one to arrive sums all of them in range order
  // and stores the tile
  if (sw.tail >= 0 && !split_exchange(acc, g.ws, g.ws_count, sw.tail, g.split_s, sw.chunk, tid)) return;
  if constexpr (DB) {
    if (do_db) {  // uniform over the workgroup
      __syncthreads();
      const float* red = db_part;
      if (tid < 256 && m0 + tid < g.M) {
        float t = red[tid];
#pragma unroll
        for (int w8 = 1; w8 < 8; ++w8) t += red[w8 * 256 + tid];
        store_elem(g.db, g.db_dtype, m0 + tid, t);
      }
    }
  }

  // ---------------------------------------------------------------- epilogue
  int64_t m0e = uniform64(m0), n0e = uniform64(n0);
  int lane_e = lane;
  asm volatile("" : "+s"(m0e), "+s"(n0e), "+v"(lane_e));
  // lane_e holds rows m0 + wm*128 + tm*16 + lane_e%16, columns
  // n0 + wn*64 + tn*16 + 4*(lane_e/16) + r
  const int slab = wave >> 1;
  uint8_t* stage_w = (slab == 0 ? la0 : slab == 1 ? lb0 : slab == 2 ? la1 : lb1) + (wave & 1) * (TILE / 2);
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
        const int64_t n = min<int64_t>(n0e + wn * 64 + tn * 16 + (lane_e >> 4) * 4 + r, e_N - 1);
        bias[tn][r] = load_elem(reinterpret_cast<const void*>(e_bias), (e_misc >> 1) & 7, n);
      }
  }
  auto store_tile = [&](auto odtc, auto fullc) {
    constexpr int ODT = decltype(odtc)::value;
    constexpr bool FULL = decltype(fullc)::value;
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
          for (int r = 0; r < 4; ++r) v[r] = acc[tm][tn][r] + bias[tn][r];
          uint8_t* dst = stage_w + rloc * pitch + (tn * 16 + (lane_e >> 4) * 4) * esz;
          if constexpr (ODT == DT_F32) {
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
          } else if constexpr (ODT == DT_BF16) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
          } else {
            __half h[4] = {f32_to_f16(v[0]), f32_to_f16(v[1]), f32_to_f16(v[2]), f32_to_f16(v[3])};
            *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(h);
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's slice is written
      __builtin_amdgcn_wave_barrier();
      constexpr int cpr = 64 * esz / 16;  // 16-byte chunks per staged row
      constexpr int epc = 16 / esz;
#pragma unroll
      for (int j = 0; j < cpr / 2; ++j) {
        const int q = lane_e + 64 * j;
        const int row = q / cpr, c = q % cpr;
        const int64_t m = m0e + wm * 128 + part * EPI_ROWS + row;
        const int64_t n = n0e + wn * 64 + c * epc;
        const uint8_t* src = stage_w + row * pitch + c * 16;
        uint8_t* ydst = reinterpret_cast<uint8_t*>(e_y) + (m * e_ldy + n) * esz;
        if constexpr (ODT == DT_BF16) {
          if (e_misc & 128) {
            // y = bf16(y + bf16(acc)) (bf16 output only)
            if (!FULL && (m >= e_M || n >= e_N)) continue;
            if (FULL || ((e_misc & 1) && n + epc <= e_N)) {
              const uint4 o = *reinterpret_cast<const uint4*>(ydst);
              const uint4 a = *reinterpret_cast<const uint4*>(src);
              const uint32_t ow[4] = {o.x, o.y, o.z, o.w}, aw[4] = {a.x, a.y, a.z, a.w};
              uint32_t rw[4];
#pragma unroll
              for (int q = 0; q < 4; ++q)
                rw[q] = pack_bf16(bf16_bits_to_f32(ow[q] & 0xFFFFu) + bf16_bits_to_f32(aw[q] & 0xFFFFu),
                                  bf16_bits_to_f32(ow[q] >> 16) + bf16_bits_to_f32(aw[q] >> 16));
              *reinterpret_cast<uint4*>(ydst) = make_uint4(rw[0], rw[1], rw[2], rw[3]);
            } else {
              const int cnt = (int)min<int64_t>(epc, e_N - n);
#pragma nounroll
              for (int e = 0; e < cnt; ++e) {
                uint16_t* yp = reinterpret_cast<uint16_t*>(ydst) + e;
                const float a = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(src)[e]);
                *yp = f32_to_bf16_bits(bf16_bits_to_f32(*yp) + a);
              }
            }
            continue;
          }
        }
        if constexpr (FULL) {
          store16_nt(ydst, src);
          continue;
        }
        if (m >= e_M || n >= e_N) continue;
        if ((e_misc & 1) && n + epc <= e_N) {
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
  const bool full = (e_misc & 1) && m0e + TM <= e_M && n0e + TN <= e_N;
  const int odt = (e_misc >> 4) & 7;
  if (odt == DT_F32) {
    if (full) store_tile(std::integral_constant<int, DT_F32>(), std::true_type());
    else store_tile(std::integral_constant<int, DT_F32>(), std::false_type());
  } else if (odt == DT_F16) {
    if (full) store_tile(std::integral_constant<int, DT_F16>(), std::true_type());
    else store_tile(std::integral_constant<int, DT_F16>(), std::false_type());
  } else {
    if (full) store_tile(std::integral_constant<int, DT_BF16>(), std::true_type());
    else store_tile(std::integral_constant<int, DT_BF16>(), std::false_type());
  }
}

// ---------------------------------------------------------------------------
// Column sums db[n] = sum_m dY[m, n] in fp32 (the bias gradient of F.linear,
// te_backend.py:253-259), deterministic: pass 1 writes one fp32 partial per
// 256-row chunk and column, pass 2 adds the partials in chunk order.
// ---------------------------------------------------------------------------
constexpr int CS_ROWS = 256;  // rows per chunk
constexpr int CS_COLS = 512;  // columns per workgroup (64 lanes x 8)

template <int IN_DT>
__global__ void __launch_bounds__(256) colsum_partial_kernel(const void* x, int64_t M, int64_t N, int64_t ld,
                                                             float* part) {
  __shared__ float red[4][CS_COLS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n = (int64_t)blockIdx.x * CS_COLS + lane * 8;
  const int64_t chunk = blockIdx.y;
  const int64_t r_lo = chunk * CS_ROWS, r_hi = min<int64_t>(r_lo + CS_ROWS, M);
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  constexpr int esz = IN_DT == DT_F32 ? 4 : 2;
  const bool vec = n + 8 <= N && ((uintptr_t)x % 16 == 0) && ((ld * esz) % 16 == 0);
  int64_t r = r_lo + wave;
  if (vec && IN_DT != DT_F32) {
    // four of this wave's rows loaded before their sums, which stay in row
    // order (the same additions as one row at a time)
    for (; r + 12 < r_hi; r += 16) {
      uint4 a[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        a[u] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(x) + ((r + 4 * u) * ld + n) * esz);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t w[4] = {a[u].x, a[u].y, a[u].z, a[u].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          s[e] += IN_DT == DT_BF16 ? bf16_bits_to_f32(h) : __half2float(__ushort_as_half((unsigned short)h));
        }
      }
    }
  }
  for (; r < r_hi; r += 4) {
    const uint8_t* row = reinterpret_cast<const uint8_t*>(x) + (r * ld + n) * esz;
    if (vec) {
      if constexpr (IN_DT == DT_F32) {
        const float4 a = reinterpret_cast<const float4*>(row)[0];
        const float4 b = reinterpret_cast<const float4*>(row)[1];
        s[0] += a.x; s[1] += a.y; s[2] += a.z; s[3] += a.w;
        s[4] += b.x; s[5] += b.y; s[6] += b.z; s[7] += b.w;
      } else {
        const uint4 a = *reinterpret_cast<const uint4*>(row);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          s[e] += IN_DT == DT_BF16 ? bf16_bits_to_f32(h) : __half2float(__ushort_as_half((unsigned short)h));
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < N) s[e] += load_elem(x, IN_DT, r * ld + n + e);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[wave][lane * 8 + e] = s[e];
  __syncthreads();
  for (int c = tid; c < CS_COLS; c += 256) {
    const int64_t nn = (int64_t)blockIdx.x * CS_COLS + c;
    if (nn < N) part[chunk * N + nn] = ((red[0][c] + red[1][c]) + red[2][c]) + red[3][c];
  }
}

__global__ void __launch_bounds__(256) colsum_finish_kernel(const float* part, int64_t chunks, int64_t N, void* out,
                                                            int out_dtype) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float s = 0.f;
  for (int64_t c = 0; c < chunks; ++c) s += part[c * N + n];
  store_elem(out, out_dtype, n, s);
}

}  // namespace gdq
}  // namespace ntlb

using namespace ntlb;
using namespace ntlb::gdq;

namespace {

template <int EL, int SA, int SB, int GRID, int SCM = SC_SHARED>
void launch(const DqArgs& g, hipStream_t st) {
  const int64_t tiles = ((g.M + TM - 1) / TM) * ((g.N + TN - 1) / TN);
  const int64_t wgs = g.split_s > 1 ? (int64_t)g.split_base + (tiles - g.split_base) * g.split_s : tiles;
  // the db variant is built for e4m3 codes only: with the int grid's decode
  // it needs a few registers more than a wave of this kernel has
  if constexpr (SA == SRC_TDIRECT && SB == SRC_TCODES && EL == EL_BF16 && GRID == GRID_E4M3) {
    if (g.db) {
      gemm_dq_kernel<EL, SA, SB, GRID, SCM, GRP_NONE, false, true><<<dim3((unsigned)wgs), dim3(NT), 0, st>>>(g);
      return;
    }
  }
  gemm_dq_kernel<EL, SA, SB, GRID, SCM><<<dim3((unsigned)wgs), dim3(NT), 0, st>>>(g);
}

// a bf16 operand stored transposed takes the transposing LDS loads when its
// stored rows are whole 16-byte chunks (the copies move 16 bytes per lane);
// otherwise the register transpose, which needs 8-byte rows
static bool tr_ok(const Operand& o) { return aligned(o.p, 16) && (o.ld * 2) % 16 == 0; }

// the source combinations this library instantiates
int dispatch(int el, int sa, int sb, const DqArgs& g, hipStream_t st) {
  const int grid = (sa == SRC_CODES || sa == SRC_TCODES) ? g.a.grid : g.b.grid;  // PCODES: B's format
  const int scm = (sb == SRC_TCODES || sb == SRC_TNF4) ? g.b.smode : SC_SHARED;
  // bf16 operands stored transposed go through the transposing LDS loads,
  // except the wgrad that also sums its dY rows into db (that variant adds
  // up the values its register transpose holds)
  if (el == EL_BF16 && sa == SRC_TDIRECT && !g.db && tr_ok(g.a) && (sb != SRC_TDIRECT || tr_ok(g.b))) sa = SRC_TR;
  if (el == EL_BF16 && sb == SRC_TDIRECT && tr_ok(g.b) && sa != SRC_TDIRECT) sb = SRC_TR;
#define NTLB_DQ_CASE(E, A, B, G)                                \
  if (el == E && sa == A && sb == B && (grid == G || G < 0)) {  \
    launch<E, A, B, (G < 0 ? 0 : G)>(g, st);                    \
    return NTLB_OK;                                             \
  }
#define NTLB_DQ_CASE_SC(E, A, B, G, S)                          \
  if (el == E && sa == A && sb == B && grid == G && scm == S) { \
    launch<E, A, B, G, S>(g, st);                               \
    return NTLB_OK;                                             \
  }
  NTLB_DQ_CASE(EL_BF16, SRC_CODES, SRC_CODES, GRID_INT)
  NTLB_DQ_CASE(EL_BF16, SRC_CODES, SRC_CODES, GRID_E4M3)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_DIRECT, SRC_TCODES, GRID_INT, SC_SHARED)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_DIRECT, SRC_TCODES, GRID_E4M3, SC_SHARED)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_DIRECT, SRC_TCODES, GRID_INT, SC_CONTIG)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_DIRECT, SRC_TCODES, GRID_E4M3, SC_CONTIG)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_TR, SRC_TCODES, GRID_INT, SC_SHARED)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_TR, SRC_TCODES, GRID_E4M3, SC_SHARED)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_TR, SRC_TCODES, GRID_INT, SC_CONTIG)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_TR, SRC_TCODES, GRID_E4M3, SC_CONTIG)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_TDIRECT, SRC_TCODES, GRID_INT, SC_SHARED)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_TDIRECT, SRC_TCODES, GRID_E4M3, SC_SHARED)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_TDIRECT, SRC_TCODES, GRID_INT, SC_CONTIG)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_TDIRECT, SRC_TCODES, GRID_E4M3, SC_CONTIG)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_DIRECT, SRC_TNF4, GRID_E4M3, SC_SHARED)
  NTLB_DQ_CASE_SC(EL_BF16, SRC_DIRECT, SRC_TNF4, GRID_E4M3, SC_CONTIG)
  NTLB_DQ_CASE_SC(EL_F32, SRC_DIRECT, SRC_TNF4, GRID_E4M3, SC_SHARED)
  NTLB_DQ_CASE_SC(EL_F32, SRC_DIRECT, SRC_TNF4, GRID_E4M3, SC_CONTIG)
  NTLB_DQ_CASE_SC(EL_F32, SRC_DIRECT, SRC_TCODES, GRID_E4M3, SC_SHARED)
  NTLB_DQ_CASE_SC(EL_F32, SRC_DIRECT, SRC_TCODES, GRID_E4M3, SC_CONTIG)
  NTLB_DQ_CASE(EL_BF16, SRC_DIRECT, SRC_PCODES, GRID_NF4)
  NTLB_DQ_CASE(EL_BF16, SRC_DIRECT, SRC_PCODES, GRID_E4M3)
  NTLB_DQ_CASE(EL_F32, SRC_DIRECT, SRC_PCODES, GRID_NF4)
  NTLB_DQ_CASE(EL_F32, SRC_DIRECT, SRC_PCODES, GRID_E4M3)
  NTLB_DQ_CASE(EL_BF16, SRC_DIRECT, SRC_DIRECT, -1)
  NTLB_DQ_CASE(EL_BF16, SRC_DIRECT, SRC_TR, -1)
  NTLB_DQ_CASE(EL_BF16, SRC_TR, SRC_TR, -1)
  NTLB_DQ_CASE(EL_BF16, SRC_DIRECT, SRC_TDIRECT, -1)
  NTLB_DQ_CASE(EL_BF16, SRC_TDIRECT, SRC_TDIRECT, -1)
  NTLB_DQ_CASE(EL_F32, SRC_CODES, SRC_CODES, GRID_INT)
  NTLB_DQ_CASE(EL_F32, SRC_CODES, SRC_CODES, GRID_E4M3)
  NTLB_DQ_CASE(EL_F32, SRC_DIRECT, SRC_DIRECT, -1)
  NTLB_DQ_CASE(EL_F32, SRC_DIRECT, SRC_TDIRECT, -1)
  NTLB_DQ_CASE(EL_F32, SRC_TDIRECT, SRC_TDIRECT, -1)
#undef NTLB_DQ_CASE
#undef NTLB_DQ_CASE_SC
  return fail(NTLB_EUNSUPPORTED, "gemm_dq: operand sources (%d, %d) are not built for element type %d", sa, sb, el);
}

// the grouped GEMMs of the expert MLP backward: bf16 operands, the weights'
// 128x128 block scales (dgrad) or the activations' per-row 1x128 scales
// (wgrad)
template <int SA, int SB, int SCM, int GRP, bool IL = false>
void launch_grouped(const DqArgs& g, int64_t wgs, hipStream_t st) {
  const int grid = SB == SRC_TCODES ? g.b.grid : g.a.grid;
  if (grid == GRID_E4M3)
    gemm_dq_kernel<EL_BF16, SA, SB, GRID_E4M3, SCM, GRP, IL><<<dim3((unsigned)wgs), dim3(NT), 0, st>>>(g);
  else
    gemm_dq_kernel<EL_BF16, SA, SB, GRID_INT, SCM, GRP, IL><<<dim3((unsigned)wgs), dim3(NT), 0, st>>>(g);
}

// the grouped GEMMs over dense bf16 operands (the straight-through operands
// t + (t_dq - t) that stochastic rounding leaves apart from bf16(q * s))
template <int SA, int SB, int GRP, bool IL = false>
void launch_grouped_dense(const DqArgs& g, int64_t wgs, hipStream_t st) {
  gemm_dq_kernel<EL_BF16, SA, SB, GRID_E4M3, SC_SHARED, GRP, IL><<<dim3((unsigned)wgs), dim3(NT), 0, st>>>(g);
}

int elem_of(int op_dtype, const char* fn, int& el) {
  if (op_dtype == NTLB_BF16) el = EL_BF16;
  else if (op_dtype == NTLB_F32) el = EL_F32;
  else return fail(NTLB_EUNSUPPORTED, "%s: operand dtype must be bf16 or fp32", fn);
  return NTLB_OK;
}

// a coded operand in the scale convention of the blockwise GEMM:
// scale(row, k) = s[(row >> shift) * s_row + (k >> 7) * s_col]
int check_codes(const char* fn, const char* what, const uint8_t* codes, int64_t ldc, int64_t rows, int64_t Kp,
                const float* s, int shift, int grid) {
  if (!codes || !s) return fail(NTLB_EINVAL, "%s: NULL %s codes or scales", fn, what);
  if (grid != NTLB_GRID_INT && grid != NTLB_GRID_E4M3) return fail(NTLB_EINVAL, "%s: bad grid %d", fn, grid);
  if (ldc < Kp || ldc % 16 || !aligned(codes, 16))
    return fail(NTLB_EINVAL, "%s: %s codes need ld >= Kp, ld %% 16 == 0 and 16-byte alignment", fn, what);
  if (!(shift == 0 || shift == 7)) return fail(NTLB_EINVAL, "%s: %s scale shift must be 0 or 7", fn, what);
  // 32-bit buffer offsets, with a K step of zero-filled rows past the end
  if ((rows + 64) * ldc >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: %s codes exceed 2 GiB", fn, what);
  return NTLB_OK;
}

// the split-K tail's minimum K steps per range, as for the blockwise GEMM
// (a K step here is 128 bytes per row, the MFMA work of one of its blocks)
constexpr int DQ_SPLIT_MIN_STEPS = 9;

SplitPlan dq_plan(int64_t M, int64_t N, int64_t Kc, int el) {
  const int64_t tiles = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
  return split_plan(tiles, (int)(Kc / (el == EL_BF16 ? 64 : 32)), DQ_SPLIT_MIN_STEPS);
}

int finish(const char* fn, DqArgs& g, int el, int sa, int sb, int y_dtype, int64_t ldy, void* stream,
           void* workspace = nullptr, int64_t ws_bytes = 0) {
  if (!valid_dtype(y_dtype) || ldy < g.N) return fail(NTLB_EINVAL, "%s: bad output dtype or ld", fn);
  if (g.bias && !valid_dtype(g.bias_dtype)) return fail(NTLB_EINVAL, "%s: bad bias dtype", fn);
  const int64_t tiles = ((g.M + TM - 1) / TM) * ((g.N + TN - 1) / TN);
  if (tiles > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  g.split_base = (int)tiles; g.split_s = 1; g.ws = nullptr; g.ws_count = nullptr;
  if (workspace) {
    if (!aligned(workspace, 256)) return fail(NTLB_EINVAL, "%s: workspace must be 256-byte aligned", fn);
    const SplitPlan plan = dq_plan(g.M, g.N, g.Kc, el);
    if (plan.s > 1 && ws_bytes >= split_ws_bytes(plan)) {
      g.split_base = plan.base; g.split_s = plan.s;
      g.ws_count = reinterpret_cast<uint32_t*>(workspace);
      g.ws = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + split_count_bytes());
    }
  }
  g.y_dtype = y_dtype;
  g.ldy = ldy;
  g.vec_out = aligned(g.y, 16) && ((ldy * dtype_size(y_dtype)) % 16 == 0);
  int rc = dispatch(el, sa, sb, g, as_stream(stream));
  if (rc) return rc;
  return check_launch(fn);
}

// scale mode and extent of a transposed coded operand (scale of stored row c,
// operand row r: s[(r >> r_shift) * s_r + (c >> c_shift) * s_c])
int tcodes_scales(const char* fn, Operand& o) {
  if (o.s_c == 0 || o.c_shift >= 3) {
    o.smode = SC_SHARED;
  } else if (o.s_c == 1 && o.c_shift == 0 && aligned(o.s, 16) && o.s_r % 4 == 0) {
    o.smode = SC_CONTIG;
  } else {
    return fail(NTLB_EUNSUPPORTED,
                "%s: per-row scales of the coded operand must be contiguous along its rows (stride 1, 16-byte "
                "aligned, the other stride a multiple of 4: the tile-major 1x128 layout)", fn);
  }
  o.s_extent = ((o.rows - 1) >> o.r_shift) * o.s_r + ((o.kvalid - 1) >> o.c_shift) * o.s_c + 1;
  if (o.s_extent * 4 >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: scales exceed 2 GiB", fn);
  return NTLB_OK;
}

}  // namespace

extern "C" int ntlb_gemm_dq_forward(int op_dtype, int grid, const uint8_t* a, int64_t lda, const float* sa,
                                    int64_t sa_row, int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb,
                                    const float* sb, int64_t sb_row, int64_t sb_col, int b_shift, int64_t M, int64_t N,
                                    int64_t Kp, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                                    void* stream) {
  const char* fn = "ntlb_gemm_dq_forward";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (M < 0 || N < 0 || Kp < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (Kp % 128) return fail(NTLB_EINVAL, "%s: Kp %lld is not a multiple of 128", fn, (long long)Kp);
  if (M == 0 || N == 0) return NTLB_OK;
  if (Kp == 0) return fail(NTLB_EUNSUPPORTED, "%s: K == 0", fn);
  if (!y) return fail(NTLB_EINVAL, "%s: NULL output", fn);
  if (int rc = check_codes(fn, "A", a, lda, M, Kp, sa, a_shift, grid)) return rc;
  if (int rc = check_codes(fn, "B", b, ldb, N, Kp, sb, b_shift, grid)) return rc;
  DqArgs g{};
  g.a = Operand{a, lda, M, Kp, sa, sa_row, sa_col, a_shift, 7, grid, 0, 0};
  g.b = Operand{b, ldb, N, Kp, sb, sb_row, sb_col, b_shift, 7, grid, 0, 0};
  g.M = M; g.N = N; g.Kc = Kp;
  g.bias = bias; g.bias_dtype = bias_dtype; g.y = y;
  return finish(fn, g, el, SRC_CODES, SRC_CODES, y_dtype, ldy, stream);
}

extern "C" int64_t ntlb_gemm_dq_workspace_bytes(int op_dtype, int64_t M, int64_t N, int64_t Kc) {
  if (M <= 0 || N <= 0 || Kc <= 0) return 0;
  const int el = op_dtype == NTLB_F32 ? EL_F32 : EL_BF16;
  const int64_t kstep = el == EL_BF16 ? 64 : 32;
  const int64_t tiles = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
  if (tiles > 0x7FFFFFFF) return 0;
  return split_ws_bytes(dq_plan(M, N, (Kc + kstep - 1) / kstep * kstep, el));
}

extern "C" int ntlb_gemm_ste_dgrad_ws(int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N, int grid,
                                      const uint8_t* w, int64_t ldw, const float* sw, int64_t sw_row, int64_t sw_col,
                                      int w_shift, int64_t K, void* dx, int dx_dtype, int64_t lddx, void* workspace,
                                      int64_t ws_bytes, void* stream) {
  const char* fn = "ntlb_gemm_ste_dgrad";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (M < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (M == 0 || K == 0) return NTLB_OK;
  if (!dy || !dx) return fail(NTLB_EINVAL, "%s: NULL dY or dX", fn);
  if (el != EL_BF16) return fail(NTLB_EUNSUPPORTED, "%s: coded W needs bf16 operands", fn);
  if (N == 0) return fail(NTLB_EUNSUPPORTED, "%s: N == 0 (dX is zero)", fn);
  const int kstep = 64, eb = 2;
  const int64_t Nc = (N + kstep - 1) / kstep * kstep;  // the contraction, zero past N
  if (lddy < Nc || !aligned(dy, 16) || (lddy * eb) % 16)
    return fail(NTLB_EINVAL, "%s: dY needs ld >= N rounded up to %d (zero pad columns), 16-byte rows and alignment",
                fn, kstep);
  if ((M + 256) * lddy * eb >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: dY exceeds 2 GiB", fn);
  const int64_t Kp = (K + 127) / 128 * 128;
  if (int rc = check_codes(fn, "W", w, ldw, N, Kp, sw, w_shift, grid)) return rc;
  if (ldw % 4) return fail(NTLB_EINVAL, "%s: W ld must be a multiple of 4", fn);
  DqArgs g{};
  g.a = Operand{reinterpret_cast<const uint8_t*>(dy), lddy, M, Nc, nullptr, 0, 0, 0, 0, 0, 0, 0};
  // W^T as the B operand: element (r = k, c = n) of the codes [N, ldw]
  g.b = Operand{w, ldw, Kp, N, sw, sw_col, sw_row, 7, w_shift, grid, 0, 0};
  if (int rc = tcodes_scales(fn, g.b)) return rc;
  g.M = M; g.N = K; g.Kc = Nc;
  g.bias = nullptr; g.bias_dtype = 0; g.y = dx;
  return finish(fn, g, el, SRC_DIRECT, SRC_TCODES, dx_dtype, lddx, stream, workspace, ws_bytes);
}

extern "C" int ntlb_gemm_ste_dgrad(int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N, int grid,
                                   const uint8_t* w, int64_t ldw, const float* sw, int64_t sw_row, int64_t sw_col,
                                   int w_shift, int64_t K, void* dx, int dx_dtype, int64_t lddx, void* stream) {
  return ntlb_gemm_ste_dgrad_ws(op_dtype, dy, lddy, M, N, grid, w, ldw, sw, sw_row, sw_col, w_shift, K, dx, dx_dtype,
                                lddx, nullptr, 0, stream);
}

extern "C" int ntlb_gemm_lowbit_dgrad_ws(int fmt, int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N,
                                         const uint8_t* w, const float* w_scales, int64_t block, int64_t K, void* dx,
                                         int dx_dtype, int64_t lddx, void* workspace, int64_t ws_bytes,
                                         void* stream) {
  const char* fn = "ntlb_gemm_lowbit_dgrad";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (fmt != NTLB_LOWBIT_NF4 && fmt != NTLB_LOWBIT_FP8P)
    return fail(NTLB_EUNSUPPORTED, "%s: NF4 or persistent FP8 weights only (format %d)", fn, fmt);
  if (M < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (M == 0 || K == 0) return NTLB_OK;
  if (!dy || !dx || !w || !w_scales) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (N == 0) return fail(NTLB_EUNSUPPORTED, "%s: N == 0 (dX is zero)", fn);
  const bool per_row = block == K && N > 1;
  if (!(block == K || block == 0 || block == N * K))
    return fail(NTLB_EUNSUPPORTED, "%s: scales must be per weight row (block = K) or per tensor (0 or N*K)", fn);
  if (K % 4) return fail(NTLB_EUNSUPPORTED, "%s: K must be a multiple of 4", fn);
  const int kstep = el == EL_BF16 ? 64 : 32, eb = el == EL_BF16 ? 2 : 4;
  const int64_t Nc = (N + kstep - 1) / kstep * kstep;  // the contraction, zero past N
  if (lddy < Nc || !aligned(dy, 16) || (lddy * eb) % 16)
    return fail(NTLB_EINVAL, "%s: dY needs ld >= N rounded up to %d (zero pad columns), 16-byte rows and alignment",
                fn, kstep);
  if ((M + 256) * lddy * eb >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: dY exceeds 2 GiB", fn);
  // bytes per stored weight row: K nibbles or K e4m3 codes
  const int64_t ldw = fmt == NTLB_LOWBIT_NF4 ? K / 2 : K;
  if (!aligned(w, fmt == NTLB_LOWBIT_NF4 ? 2 : 4) || !aligned(w_scales, 16))
    return fail(NTLB_EINVAL, "%s: W needs 2-byte (NF4) or 4-byte (FP8) alignment, its scales 16-byte", fn);
  if ((N + 64) * ldw >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: W exceeds 2 GiB", fn);
  DqArgs g{};
  g.a = Operand{reinterpret_cast<const uint8_t*>(dy), lddy, M, Nc, nullptr, 0, 0, 0, 0, 0, 0, 0};
  // W^T as the B operand: element (r = k, c = n); one scale per stored row n
  // (contiguous along the contraction) or one for all
  g.b = Operand{w, ldw, K, N, w_scales, 0, per_row ? 1 : 0, 0, 0, GRID_E4M3, 0, 0};
  if (int rc = tcodes_scales(fn, g.b)) return rc;
  g.M = M; g.N = K; g.Kc = Nc;
  g.bias = nullptr; g.bias_dtype = 0; g.y = dx;
  return finish(fn, g, el, SRC_DIRECT, fmt == NTLB_LOWBIT_NF4 ? SRC_TNF4 : SRC_TCODES, dx_dtype, lddx, stream,
                workspace, ws_bytes);
}

extern "C" int ntlb_gemm_lowbit_dq_forward_ws(int fmt, int op_dtype, const void* x, int64_t ldx, int64_t M,
                                              const uint8_t* w, const float* w_scales, int64_t block, int64_t N,
                                              int64_t K, const void* bias, int bias_dtype, void* y, int y_dtype,
                                              int64_t ldy, void* workspace, int64_t ws_bytes, void* stream) {
  const char* fn = "ntlb_gemm_lowbit_dq_forward";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (fmt != NTLB_LOWBIT_NF4 && fmt != NTLB_LOWBIT_FP8P)
    return fail(NTLB_EUNSUPPORTED, "%s: NF4 or persistent FP8 weights only (format %d)", fn, fmt);
  if (M < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (M == 0 || N == 0) return NTLB_OK;
  if (K == 0) return fail(NTLB_EUNSUPPORTED, "%s: K == 0", fn);
  if (!x || !y || !w || !w_scales) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  const bool per_row = block == K && N > 1;
  if (!(block == K || block == 0 || block == N * K))
    return fail(NTLB_EUNSUPPORTED, "%s: scales must be per weight row (block = K) or per tensor (0 or N*K)", fn);
  if (K % 4) return fail(NTLB_EUNSUPPORTED, "%s: K must be a multiple of 4", fn);
  const int kstep = el == EL_BF16 ? 64 : 32, eb = el == EL_BF16 ? 2 : 4;
  const int64_t Kc = (K + kstep - 1) / kstep * kstep;  // the contraction, zero past K
  if (ldx < Kc || !aligned(x, 16) || (ldx * eb) % 16)
    return fail(NTLB_EINVAL, "%s: x needs ld >= K rounded up to %d (zero pad columns), 16-byte rows and alignment",
                fn, kstep);
  if ((M + 256) * ldx * eb >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: x exceeds 2 GiB", fn);
  const int64_t ldw = fmt == NTLB_LOWBIT_NF4 ? K / 2 : K;  // bytes per weight row
  if (!aligned(w, fmt == NTLB_LOWBIT_NF4 ? 2 : 4))
    return fail(NTLB_EINVAL, "%s: W needs 2-byte (NF4) or 4-byte (FP8) alignment", fn);
  if (N * ldw >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: W exceeds 2 GiB", fn);
  DqArgs g{};
  g.a = Operand{reinterpret_cast<const uint8_t*>(x), ldx, M, Kc, nullptr, 0, 0, 0, 0, 0, 0, 0};
  g.b = Operand{w, ldw, N, K, w_scales, per_row ? 1 : 0, 0, 0, 0,
                fmt == NTLB_LOWBIT_NF4 ? GRID_NF4 : GRID_E4M3, 0, 0};
  g.M = M; g.N = N; g.Kc = Kc;
  g.bias = bias; g.bias_dtype = bias_dtype; g.y = y;
  return finish(fn, g, el, SRC_DIRECT, SRC_PCODES, y_dtype, ldy, stream, workspace, ws_bytes);
}

extern "C" int ntlb_gemm_ste_wgrad_db(int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N, int grid,
                                      const uint8_t* x, int64_t ldx, const float* sx, int64_t sx_row, int64_t sx_col,
                                      int x_shift, int64_t K, void* dw, int dw_dtype, int64_t lddw, void* db,
                                      int db_dtype, void* stream) {
  const char* fn = "ntlb_gemm_ste_wgrad";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (M < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (N == 0 || K == 0) return NTLB_OK;
  if (!dy || !dw) return fail(NTLB_EINVAL, "%s: NULL dY or dW", fn);
  if (M == 0) return fail(NTLB_EUNSUPPORTED, "%s: M == 0 (dW is zero)", fn);
  if (el != EL_BF16) return fail(NTLB_EUNSUPPORTED, "%s: coded X needs bf16 operands", fn);
  if (lddy < N || !aligned(dy, 16) || lddy % 8)
    return fail(NTLB_EINVAL, "%s: dY needs ld >= N, ld %% 8 == 0 and 16-byte alignment", fn);
  if ((M + 64) * lddy * 2 >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: dY exceeds 2 GiB", fn);
  const int64_t Kp = (K + 127) / 128 * 128;
  if (int rc = check_codes(fn, "X", x, ldx, M, Kp, sx, x_shift, grid)) return rc;
  const int64_t Mc = (M + 63) / 64 * 64;  // contraction over the tokens, zero past M
  DqArgs g{};
  // dY^T as the A operand: element (r = n, c = m) at dy[m * lddy + n]
  g.a = Operand{reinterpret_cast<const uint8_t*>(dy), lddy, N, M, nullptr, 0, 0, 0, 0, 0, 0, 0};
  // X^T as the B operand: element (r = k, c = m) of the codes [M, ldx]
  g.b = Operand{x, ldx, Kp, M, sx, sx_col, sx_row, 7, x_shift, grid, 0, 0};
  if (int rc = tcodes_scales(fn, g.b)) return rc;
  g.M = N; g.N = K; g.Kc = Mc;
  g.bias = nullptr; g.bias_dtype = 0; g.y = dw;
  if (db && !valid_dtype(db_dtype)) return fail(NTLB_EINVAL, "%s: bad db dtype", fn);
  if (db && grid != NTLB_GRID_E4M3) return fail(NTLB_EUNSUPPORTED, "%s: db rides on the e4m3 kernel only", fn);
  g.db = db; g.db_dtype = db_dtype;
  return finish(fn, g, el, SRC_TDIRECT, SRC_TCODES, dw_dtype, lddw, stream);
}

extern "C" int ntlb_gemm_ste_wgrad(int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N, int grid,
                                   const uint8_t* x, int64_t ldx, const float* sx, int64_t sx_row, int64_t sx_col,
                                   int x_shift, int64_t K, void* dw, int dw_dtype, int64_t lddw, void* stream) {
  return ntlb_gemm_ste_wgrad_db(op_dtype, dy, lddy, M, N, grid, x, ldx, sx, sx_row, sx_col, x_shift, K, dw, dw_dtype,
                                lddw, nullptr, 0, stream);
}

// offset table of rows sorted by expert, as the grouped kernels read it
static int check_offsets(const char* fn, const int32_t* offsets, int n_experts) {
  if (!offsets) return fail(NTLB_EINVAL, "%s: NULL offsets", fn);
  if (n_experts < 1 || n_experts >= TILE / 4) return fail(NTLB_EINVAL, "%s: n_experts must be in [1, %d)", fn, TILE / 4);
  return NTLB_OK;
}

extern "C" int ntlb_gemm_grouped_ste_dgrad(int op_dtype, const void* dy, int64_t lddy, int64_t R, int64_t N,
                                           const int32_t* offsets, int n_experts, int grid, const uint8_t* w,
                                           int64_t ldw, int64_t w_estride, const float* sw, int64_t sw_row,
                                           int64_t sw_col, int w_shift, int64_t sw_estride, int64_t K, void* dx,
                                           int dx_dtype, int64_t lddx, void* stream) {
  const char* fn = "ntlb_gemm_grouped_ste_dgrad";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (el != EL_BF16) return fail(NTLB_EUNSUPPORTED, "%s: coded W needs bf16 operands", fn);
  if (R < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (R == 0 || K == 0) return NTLB_OK;
  if (N == 0) return fail(NTLB_EUNSUPPORTED, "%s: N == 0 (dX is zero)", fn);
  if (!dy || !dx) return fail(NTLB_EINVAL, "%s: NULL dY or dX", fn);
  if (int rc = check_offsets(fn, offsets, n_experts)) return rc;
  const int kstep = 64, eb = 2;
  const int64_t Nc = (N + kstep - 1) / kstep * kstep;
  if (lddy < Nc || !aligned(dy, 16) || (lddy * eb) % 16)
    return fail(NTLB_EINVAL, "%s: dY needs ld >= N rounded up to %d (zero pad columns), 16-byte rows and alignment",
                fn, kstep);
  if ((R + 256) * lddy * eb >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: dY exceeds 2 GiB", fn);
  const int64_t Kp = (K + 127) / 128 * 128;
  if (int rc = check_codes(fn, "W", w, ldw, N, Kp, sw, w_shift, grid)) return rc;
  if (ldw % 4 || w_estride < N * ldw || w_estride % 16) return fail(NTLB_EINVAL, "%s: bad W ld or expert stride", fn);
  if (!valid_dtype(dx_dtype) || lddx < K) return fail(NTLB_EINVAL, "%s: bad dX dtype or ld", fn);
  DqArgs g{};
  g.a = Operand{reinterpret_cast<const uint8_t*>(dy), lddy, R, Nc, nullptr, 0, 0, 0, 0, 0, 0, 0};
  // W_e^T as the B operand: element (r = k, c = n) of expert e's codes [N, ldw]
  g.b = Operand{w, ldw, Kp, N, sw, sw_col, sw_row, 7, w_shift, grid, 0, 0};
  if (int rc = tcodes_scales(fn, g.b)) return rc;
  if (g.b.smode != SC_SHARED) return fail(NTLB_EUNSUPPORTED, "%s: W needs block or tensor scales", fn);
  g.M = R; g.N = K; g.Kc = Nc;
  g.y = dx; g.y_dtype = dx_dtype; g.ldy = lddx;
  g.vec_out = aligned(dx, 16) && ((lddx * dtype_size(dx_dtype)) % 16 == 0);
  g.offsets = offsets; g.n_experts = n_experts;
  g.b_estride = w_estride; g.bs_estride = sw_estride;
  const int64_t num_n = (K + TN - 1) / TN;
  const int64_t wgs = ((R + TM - 1) / TM + n_experts) * num_n;  // at least every expert's row tiles
  if (wgs > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  launch_grouped<SRC_DIRECT, SRC_TCODES, SC_SHARED, GRP_ROWS>(g, wgs, as_stream(stream));
  return check_launch(fn);
}

extern "C" int ntlb_gemm_grouped_ste_dgrad_gate_up(int op_dtype, const void* dgu, int64_t lddgu, int64_t R,
                                                   int64_t I, const int32_t* offsets, int n_experts, int grid,
                                                   const uint8_t* w, int64_t ldw, int64_t w_estride, const float* sw,
                                                   int64_t sw_row, int64_t sw_col, int64_t sw_estride, int64_t K,
                                                   void* dx, int64_t lddx, void* stream) {
  const char* fn = "ntlb_gemm_grouped_ste_dgrad_gate_up";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (el != EL_BF16) return fail(NTLB_EUNSUPPORTED, "%s: coded W needs bf16 operands", fn);
  if (R < 0 || I < 0 || K < 0 || I % 128) return fail(NTLB_EINVAL, "%s: bad shape (I %% 128 == 0)", fn);
  if (R == 0 || K == 0) return NTLB_OK;
  if (I == 0) return fail(NTLB_EUNSUPPORTED, "%s: I == 0 (dX is zero)", fn);
  if (!dgu || !dx) return fail(NTLB_EINVAL, "%s: NULL dY or dX", fn);
  if (int rc = check_offsets(fn, offsets, n_experts)) return rc;
  const int64_t N = 2 * I, eb = 2;
  if (lddgu < N || !aligned(dgu, 16) || (lddgu * eb) % 16)
    return fail(NTLB_EINVAL, "%s: d_gate_up needs ld >= 2I, 16-byte rows and alignment", fn);
  if ((R + 256) * lddgu * eb >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: dY exceeds 2 GiB", fn);
  const int64_t Kp = (K + 127) / 128 * 128;
  if (int rc = check_codes(fn, "W", w, ldw, N, Kp, sw, 7, grid)) return rc;
  if (ldw % 4 || w_estride < N * ldw || w_estride % 16) return fail(NTLB_EINVAL, "%s: bad W ld or expert stride", fn);
  if (lddx < K) return fail(NTLB_EINVAL, "%s: bad dX ld", fn);
  DqArgs g{};
  g.a = Operand{reinterpret_cast<const uint8_t*>(dgu), lddgu, R, N, nullptr, 0, 0, 0, 0, 0, 0, 0};
  g.b = Operand{w, ldw, Kp, N, sw, sw_col, sw_row, 7, 7, grid, 0, 0};
  if (int rc = tcodes_scales(fn, g.b)) return rc;
  if (g.b.smode != SC_SHARED) return fail(NTLB_EUNSUPPORTED, "%s: W needs block scales", fn);
  g.M = R; g.N = K; g.Kc = I;  // one half of the interleaved contraction per launch
  g.y = dx; g.y_dtype = DT_BF16; g.ldy = lddx;
  g.vec_out = aligned(dx, 16) && ((lddx * 2) % 16 == 0);
  g.offsets = offsets; g.n_experts = n_experts;
  g.b_estride = w_estride; g.bs_estride = sw_estride;
  const int64_t num_n = (K + TN - 1) / TN;
  const int64_t wgs = ((R + TM - 1) / TM + n_experts) * num_n;
  if (wgs > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  hipStream_t st = as_stream(stream);
  // the gate Linear's input gradient, then the up Linear's added to it in bf16
  g.il_half = 0; g.accum = 0;
  launch_grouped<SRC_DIRECT, SRC_TCODES, SC_SHARED, GRP_ROWS, true>(g, wgs, st);
  g.il_half = 1; g.accum = 1;
  launch_grouped<SRC_DIRECT, SRC_TCODES, SC_SHARED, GRP_ROWS, true>(g, wgs, st);
  return check_launch(fn);
}

extern "C" int ntlb_gemm_grouped_ste_wgrad(int op_dtype, const void* dy, int64_t lddy, int64_t R, int64_t N,
                                           const int32_t* offsets, int n_experts, int grid, const uint8_t* x,
                                           int64_t ldx, const float* sx, int64_t sx_row, int64_t sx_col, int x_shift,
                                           int64_t K, void* dw, int dw_dtype, int64_t lddw, int64_t dw_estride,
                                           void* stream) {
  const char* fn = "ntlb_gemm_grouped_ste_wgrad";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (el != EL_BF16) return fail(NTLB_EUNSUPPORTED, "%s: coded X needs bf16 operands", fn);
  if (R < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (N == 0 || K == 0) return NTLB_OK;
  if (!dy || !dw) return fail(NTLB_EINVAL, "%s: NULL dY or dW", fn);
  if (int rc = check_offsets(fn, offsets, n_experts)) return rc;
  if (lddy < N || !aligned(dy, 16) || lddy % 8)
    return fail(NTLB_EINVAL, "%s: dY needs ld >= N, ld %% 8 == 0 and 16-byte alignment", fn);
  if ((R + 64) * lddy * 2 >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: dY exceeds 2 GiB", fn);
  const int64_t Kp = (K + 127) / 128 * 128;
  if (int rc = check_codes(fn, "X", x, ldx, R, Kp, sx, x_shift, grid)) return rc;
  if (!valid_dtype(dw_dtype) || lddw < K) return fail(NTLB_EINVAL, "%s: bad dW dtype or ld", fn);
  if (dw_estride < N * lddw * dtype_size(dw_dtype)) return fail(NTLB_EINVAL, "%s: dW expert stride too small", fn);
  DqArgs g{};
  // dY^T as the A operand: element (r = n, c = m) at dy[m * lddy + n]; the
  // kernel moves both operands to the expert's first row
  g.a = Operand{reinterpret_cast<const uint8_t*>(dy), lddy, N, R, nullptr, 0, 0, 0, 0, 0, 0, 0};
  // X^T as the B operand: element (r = k, c = m) of the codes [R, ldx]
  g.b = Operand{x, ldx, Kp, R, sx, sx_col, sx_row, 7, x_shift, grid, 0, 0};
  if (int rc = tcodes_scales(fn, g.b)) return rc;
  if (g.b.smode != SC_CONTIG) return fail(NTLB_EUNSUPPORTED, "%s: X needs per-row (1x128) scales", fn);
  g.M = N; g.N = K; g.Kc = (R + 63) / 64 * 64;
  g.y = dw; g.y_dtype = dw_dtype; g.ldy = lddw;
  g.vec_out = aligned(dw, 16) && ((lddw * dtype_size(dw_dtype)) % 16 == 0) && dw_estride % 16 == 0;
  g.offsets = offsets; g.n_experts = n_experts;
  g.y_estride = dw_estride;
  const int64_t wgs = ((N + TM - 1) / TM) * ((K + TN - 1) / TN) * n_experts;
  if (wgs > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  if (tr_ok(g.a))
    launch_grouped<SRC_TR, SRC_TCODES, SC_CONTIG, GRP_K>(g, wgs, as_stream(stream));
  else
    launch_grouped<SRC_TDIRECT, SRC_TCODES, SC_CONTIG, GRP_K>(g, wgs, as_stream(stream));
  return check_launch(fn);
}

// a dense bf16 operand read transposed: 8-byte loads of four operand rows
static int check_tdense(const char* fn, const char* what, const void* p, int64_t ld, int64_t rows, int64_t kvalid) {
  if (!p) return fail(NTLB_EINVAL, "%s: NULL %s", fn, what);
  if (ld < rows || ld % 4 || !aligned(p, 16))
    return fail(NTLB_EINVAL, "%s: %s needs ld >= %lld, ld %% 4 == 0 and 16-byte alignment", fn, what, (long long)rows);
  if ((kvalid + 64) * ld * 2 >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: %s exceeds 2 GiB", fn, what);
  return NTLB_OK;
}

extern "C" int ntlb_gemm_grouped_dgrad_dense(int op_dtype, const void* dy, int64_t lddy, int64_t R, int64_t N,
                                             const int32_t* offsets, int n_experts, const void* w, int64_t ldw,
                                             int64_t w_estride, int64_t K, void* dx, int dx_dtype, int64_t lddx,
                                             void* stream) {
  const char* fn = "ntlb_gemm_grouped_dgrad_dense";
  if (op_dtype != NTLB_BF16) return fail(NTLB_EUNSUPPORTED, "%s: bf16 operands only", fn);
  if (R < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (R == 0 || K == 0) return NTLB_OK;
  if (N == 0) return fail(NTLB_EUNSUPPORTED, "%s: N == 0 (dX is zero)", fn);
  if (!dy || !dx) return fail(NTLB_EINVAL, "%s: NULL dY or dX", fn);
  if (int rc = check_offsets(fn, offsets, n_experts)) return rc;
  const int64_t Nc = (N + 63) / 64 * 64;
  if (lddy < Nc || !aligned(dy, 16) || (lddy * 2) % 16)
    return fail(NTLB_EINVAL, "%s: dY needs ld >= N rounded up to 64 (zero pad columns), 16-byte rows and alignment",
                fn);
  if ((R + 256) * lddy * 2 >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: dY exceeds 2 GiB", fn);
  if (int rc = check_tdense(fn, "W", w, ldw, K, N)) return rc;
  if (w_estride < N * ldw || w_estride % 8) return fail(NTLB_EINVAL, "%s: bad W expert stride", fn);
  if (!valid_dtype(dx_dtype) || lddx < K) return fail(NTLB_EINVAL, "%s: bad dX dtype or ld", fn);
  DqArgs g{};
  g.a = Operand{reinterpret_cast<const uint8_t*>(dy), lddy, R, Nc, nullptr, 0, 0, 0, 0, 0, 0, 0};
  // W_e^T as the B operand: element (r = k, c = n) at w_e[n * ldw + k]
  g.b = Operand{reinterpret_cast<const uint8_t*>(w), ldw, K, N, nullptr, 0, 0, 0, 0, 0, 0, 0};
  g.M = R; g.N = K; g.Kc = Nc;
  g.y = dx; g.y_dtype = dx_dtype; g.ldy = lddx;
  g.vec_out = aligned(dx, 16) && ((lddx * dtype_size(dx_dtype)) % 16 == 0);
  g.offsets = offsets; g.n_experts = n_experts;
  g.b_estride = w_estride * 2;
  const int64_t num_n = (K + TN - 1) / TN;
  const int64_t wgs = ((R + TM - 1) / TM + n_experts) * num_n;
  if (wgs > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  if (tr_ok(g.b))
    launch_grouped_dense<SRC_DIRECT, SRC_TR, GRP_ROWS>(g, wgs, as_stream(stream));
  else
    launch_grouped_dense<SRC_DIRECT, SRC_TDIRECT, GRP_ROWS>(g, wgs, as_stream(stream));
  return check_launch(fn);
}

extern "C" int ntlb_gemm_grouped_dgrad_dense_gate_up(int op_dtype, const void* dgu, int64_t lddgu, int64_t R,
                                                     int64_t I, const int32_t* offsets, int n_experts, const void* w,
                                                     int64_t ldw, int64_t w_estride, int64_t K, void* dx,
                                                     int64_t lddx, void* stream) {
  const char* fn = "ntlb_gemm_grouped_dgrad_dense_gate_up";
  if (op_dtype != NTLB_BF16) return fail(NTLB_EUNSUPPORTED, "%s: bf16 operands only", fn);
  if (R < 0 || I < 0 || K < 0 || I % 128) return fail(NTLB_EINVAL, "%s: bad shape (I %% 128 == 0)", fn);
  if (R == 0 || K == 0) return NTLB_OK;
  if (I == 0) return fail(NTLB_EUNSUPPORTED, "%s: I == 0 (dX is zero)", fn);
  if (!dgu || !dx) return fail(NTLB_EINVAL, "%s: NULL dY or dX", fn);
  if (int rc = check_offsets(fn, offsets, n_experts)) return rc;
  const int64_t N = 2 * I;
  if (lddgu < N || !aligned(dgu, 16) || (lddgu * 2) % 16)
    return fail(NTLB_EINVAL, "%s: d_gate_up needs ld >= 2I, 16-byte rows and alignment", fn);
  if ((R + 256) * lddgu * 2 >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: dY exceeds 2 GiB", fn);
  if (int rc = check_tdense(fn, "W", w, ldw, K, N)) return rc;
  if (w_estride < N * ldw || w_estride % 8) return fail(NTLB_EINVAL, "%s: bad W expert stride", fn);
  if (lddx < K) return fail(NTLB_EINVAL, "%s: bad dX ld", fn);
  DqArgs g{};
  g.a = Operand{reinterpret_cast<const uint8_t*>(dgu), lddgu, R, N, nullptr, 0, 0, 0, 0, 0, 0, 0};
  g.b = Operand{reinterpret_cast<const uint8_t*>(w), ldw, K, N, nullptr, 0, 0, 0, 0, 0, 0, 0};
  g.M = R; g.N = K; g.Kc = I;  // one half of the interleaved contraction per launch
  g.y = dx; g.y_dtype = DT_BF16; g.ldy = lddx;
  g.vec_out = aligned(dx, 16) && ((lddx * 2) % 16 == 0);
  g.offsets = offsets; g.n_experts = n_experts;
  g.b_estride = w_estride * 2;
  const int64_t num_n = (K + TN - 1) / TN;
  const int64_t wgs = ((R + TM - 1) / TM + n_experts) * num_n;
  if (wgs > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  hipStream_t st = as_stream(stream);
  const bool tr = tr_ok(g.b);
  for (int half = 0; half < 2; ++half) {
    g.il_half = half; g.accum = half;
    if (tr)
      launch_grouped_dense<SRC_DIRECT, SRC_TR, GRP_ROWS, true>(g, wgs, st);
    else
      launch_grouped_dense<SRC_DIRECT, SRC_TDIRECT, GRP_ROWS, true>(g, wgs, st);
  }
  return check_launch(fn);
}

extern "C" int ntlb_gemm_grouped_wgrad_dense(int op_dtype, const void* dy, int64_t lddy, int64_t R, int64_t N,
                                             const int32_t* offsets, int n_experts, const void* x, int64_t ldx,
                                             int64_t K, void* dw, int dw_dtype, int64_t lddw, int64_t dw_estride,
                                             void* stream) {
  const char* fn = "ntlb_gemm_grouped_wgrad_dense";
  if (op_dtype != NTLB_BF16) return fail(NTLB_EUNSUPPORTED, "%s: bf16 operands only", fn);
  if (R < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (N == 0 || K == 0) return NTLB_OK;
  if (!dy || !dw) return fail(NTLB_EINVAL, "%s: NULL dY or dW", fn);
  if (int rc = check_offsets(fn, offsets, n_experts)) return rc;
  if (int rc = check_tdense(fn, "dY", dy, lddy, N, R)) return rc;
  if (int rc = check_tdense(fn, "X", x, ldx, K, R)) return rc;
  if (!valid_dtype(dw_dtype) || lddw < K) return fail(NTLB_EINVAL, "%s: bad dW dtype or ld", fn);
  if (dw_estride < N * lddw * dtype_size(dw_dtype)) return fail(NTLB_EINVAL, "%s: dW expert stride too small", fn);
  DqArgs g{};
  // dY^T and X^T as the operands: (r = n, c = m) at dy[m * lddy + n], (r = k, c = m) at x[m * ldx + k]; the
  // kernel moves both to the expert's first row
  g.a = Operand{reinterpret_cast<const uint8_t*>(dy), lddy, N, R, nullptr, 0, 0, 0, 0, 0, 0, 0};
  g.b = Operand{reinterpret_cast<const uint8_t*>(x), ldx, K, R, nullptr, 0, 0, 0, 0, 0, 0, 0};
  g.M = N; g.N = K; g.Kc = (R + 63) / 64 * 64;
  g.y = dw; g.y_dtype = dw_dtype; g.ldy = lddw;
  g.vec_out = aligned(dw, 16) && ((lddw * dtype_size(dw_dtype)) % 16 == 0) && dw_estride % 16 == 0;
  g.offsets = offsets; g.n_experts = n_experts;
  g.y_estride = dw_estride;
  const int64_t wgs = ((N + TM - 1) / TM) * ((K + TN - 1) / TN) * n_experts;
  if (wgs > 0x7FFFFFFF) return fail(NTLB_EINVAL, "%s: too many tiles", fn);
  if (tr_ok(g.a) && tr_ok(g.b))
    launch_grouped_dense<SRC_TR, SRC_TR, GRP_K>(g, wgs, as_stream(stream));
  else
    launch_grouped_dense<SRC_TDIRECT, SRC_TDIRECT, GRP_K>(g, wgs, as_stream(stream));
  return check_launch(fn);
}

extern "C" int ntlb_gemm_dense(int op_dtype, const void* a, int64_t lda, int a_trans, const void* b, int64_t ldb,
                               int b_trans, int64_t M, int64_t N, int64_t K, const void* bias, int bias_dtype, void* y,
                               int y_dtype, int64_t ldy, void* stream) {
  const char* fn = "ntlb_gemm_dense";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (M < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (M == 0 || N == 0) return NTLB_OK;
  if (!a || !b || !y) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  if (a_trans) return fail(NTLB_EUNSUPPORTED, "%s: A must be [M, K] row-major (a_trans = 0)", fn);
  const int kstep = el == EL_BF16 ? 64 : 32;
  const int eb = el == EL_BF16 ? 2 : 4;
  if (K == 0 || K % kstep) return fail(NTLB_EUNSUPPORTED, "%s: K must be a positive multiple of %d", fn, kstep);
  if (lda < K || !aligned(a, 16) || (lda * eb) % 16) return fail(NTLB_EINVAL, "%s: A needs ld >= K, 16-byte rows", fn);
  if ((M + 256) * lda * eb >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: A exceeds 2 GiB", fn);
  DqArgs g{};
  g.a = Operand{reinterpret_cast<const uint8_t*>(a), lda, M, K, nullptr, 0, 0, 0, 0, 0, 0, 0};
  int sb;
  if (b_trans) {
    // B stored [K, N]: element (r = n, c = k) at b[k * ldb + n]
    if (ldb < N || !aligned(b, 16) || (ldb * eb) % 16) return fail(NTLB_EINVAL, "%s: B^T needs ld >= N, 16-byte rows", fn);
    if ((K + 64) * ldb * eb >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: B exceeds 2 GiB", fn);
    g.b = Operand{reinterpret_cast<const uint8_t*>(b), ldb, N, K, nullptr, 0, 0, 0, 0, 0, 0, 0};
    sb = SRC_TDIRECT;
  } else {
    if (ldb < K || !aligned(b, 16) || (ldb * eb) % 16) return fail(NTLB_EINVAL, "%s: B needs ld >= K, 16-byte rows", fn);
    if ((N + 256) * ldb * eb >= (int64_t)0x7FFFFFFF) return fail(NTLB_EUNSUPPORTED, "%s: B exceeds 2 GiB", fn);
    g.b = Operand{reinterpret_cast<const uint8_t*>(b), ldb, N, K, nullptr, 0, 0, 0, 0, 0, 0, 0};
    sb = SRC_DIRECT;
  }
  g.M = M; g.N = N; g.Kc = K;
  g.bias = bias; g.bias_dtype = bias_dtype; g.y = y;
  return finish(fn, g, el, SRC_DIRECT, sb, y_dtype, ldy, stream);
}

extern "C" int ntlb_gemm_dense_tn(int op_dtype, const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M,
                                  int64_t N, int64_t K, void* y, int y_dtype, int64_t ldy, void* stream) {
  const char* fn = "ntlb_gemm_dense_tn";
  int el;
  if (int rc = elem_of(op_dtype, fn, el)) return rc;
  if (M < 0 || N < 0 || K < 0) return fail(NTLB_EINVAL, "%s: negative shape", fn);
  if (M == 0 || N == 0) return NTLB_OK;
  if (!a || !b || !y) return fail(NTLB_EINVAL, "%s: NULL pointer", fn);
  const int eb = el == EL_BF16 ? 2 : 4;
  if (lda < M || ldb < N || !aligned(a, 16) || !aligned(b, 16) || (lda * eb) % 16 || (ldb * eb) % 16)
    return fail(NTLB_EINVAL, "%s: A^T and B^T need ld >= M / N and 16-byte rows", fn);
  if ((K + 64) * lda * eb >= (int64_t)0x7FFFFFFF || (K + 64) * ldb * eb >= (int64_t)0x7FFFFFFF)
    return fail(NTLB_EUNSUPPORTED, "%s: an operand exceeds 2 GiB", fn);
  const int kstep = el == EL_BF16 ? 64 : 32;
  DqArgs g{};
  // Y[M,N] = A^T B with A stored [K, M] and B stored [K, N]: both operands transposed
  g.a = Operand{reinterpret_cast<const uint8_t*>(a), lda, M, K, nullptr, 0, 0, 0, 0, 0, 0, 0};
  g.b = Operand{reinterpret_cast<const uint8_t*>(b), ldb, N, K, nullptr, 0, 0, 0, 0, 0, 0, 0};
  g.M = M; g.N = N; g.Kc = (K + kstep - 1) / kstep * kstep;
  g.bias = nullptr; g.bias_dtype = 0; g.y = y;
  if (K == 0) return fail(NTLB_EUNSUPPORTED, "%s: K == 0", fn);
  return finish(fn, g, el, SRC_TDIRECT, SRC_TDIRECT, y_dtype, ldy, stream);
}

extern "C" int64_t ntlb_colsum_workspace_bytes(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return 0;
  return (M + CS_ROWS - 1) / CS_ROWS * N * 4;
}

extern "C" int ntlb_colsum(const void* x, int x_dtype, int64_t M, int64_t N, int64_t ldx, float* workspace,
                           int64_t ws_bytes, void* out, int out_dtype, void* stream) {
  const char* fn = "ntlb_colsum";
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype)) return fail(NTLB_EINVAL, "%s: bad dtype", fn);
  if (M < 0 || N < 0 || ldx < N) return fail(NTLB_EINVAL, "%s: bad shape", fn);
  if (N == 0) return NTLB_OK;
  if (!out) return fail(NTLB_EINVAL, "%s: NULL output", fn);
  hipStream_t st = as_stream(stream);
  const int64_t chunks = (M + CS_ROWS - 1) / CS_ROWS;
  if (M > 0) {
    if (!x || !workspace) return fail(NTLB_EINVAL, "%s: NULL input or workspace", fn);
    if (ws_bytes < ntlb_colsum_workspace_bytes(M, N)) return fail(NTLB_EINVAL, "%s: workspace too small", fn);
    const int64_t gx = (N + CS_COLS - 1) / CS_COLS;
    if (gx > 0x7FFFFFFF || chunks > 65535) return fail(NTLB_EUNSUPPORTED, "%s: too large", fn);
    dim3 grd((unsigned)gx, (unsigned)chunks);
    if (x_dtype == NTLB_BF16)
      colsum_partial_kernel<DT_BF16><<<grd, 256, 0, st>>>(x, M, N, ldx, workspace);
    else if (x_dtype == NTLB_F32)
      colsum_partial_kernel<DT_F32><<<grd, 256, 0, st>>>(x, M, N, ldx, workspace);
    else
      colsum_partial_kernel<DT_F16><<<grd, 256, 0, st>>>(x, M, N, ldx, workspace);
  }
  colsum_finish_kernel<<<(unsigned)((N + 255) / 256), 256, 0, st>>>(workspace, chunks, N, out, out_dtype);
  return check_launch(fn);
}
