/*
 * CPU oracle for the nano-train low-bit linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or as the timed CPU baseline.  The product path (nano-train_amd/) never
 * links, imports or calls it.
 *
 * Each function restates, in plain C with IEEE fp32 arithmetic (built with
 * -ffp-contract=off, no fast-math), one piece of the reference's emulated
 * path.  Citations are to lastweek/nano-train:
 *
 *   te_backend.py  = src/runtime/te_backend.py
 *   moe.py         = src/models/moe.py
 *   layers.py      = src/layers.py
 *
 * Rounding of values to integers follows torch.round (round half to even,
 * te_backend.py:71), i.e. rintf() under the default rounding mode.
 *
 * Code formats (the byte that the kernels write per element):
 *   GRID_INT  : int8 two's complement of q, |q| <= qmax (qmax = 2^(bits-1)-1,
 *               te_backend.py:98).  A NaN q (NaN input) is encoded as -128,
 *               which the clamp to +-qmax never produces.
 *   GRID_E4M3 : OCP float8 e4m3fn bit pattern of q (DeepSeek-V3 recipe:
 *               scale = amax/448).  No reference function; semantics are the
 *               clamp-then-cast of layers.py:115-116 applied per tile.
 *
 * Stochastic-rounding bit contract (replaces torch.rand_like,
 * te_backend.py:62 / moe.py:73, which is unseeded): element e of a call with
 * (seed, offset) draws r = Philox4x32-10(counter = {lo(e/4), hi(e/4),
 * lo(offset), hi(offset)}, key = {lo(seed), hi(seed)})[e % 4] and uses
 * u = (r >> 8) * 2^-24 in [0, 1).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define GRID_INT 0
#define GRID_E4M3 1
#define ROUND_NEAREST 0
#define ROUND_STOCHASTIC 1
/* scale rules: how an amax becomes a scale */
#define SCALE_AFTER_DIVIDE 0 /* te_backend.py:74-79,99-100: safe(amax/qmax) */
#define SCALE_BEFORE_DIVIDE 1 /* moe.py:94-98, te_backend.py:49-53 */

/* ------------------------------------------------------------------ */
/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11, "Parallel random    */
/* numbers: as easy as 1, 2, 3"), restated from the paper.               */
/* ------------------------------------------------------------------ */
void ntlo_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint32_t k0 = key_in[0], k1 = key_in[1];
  for (int round = 0; round < 10; ++round) {
    uint64_t p0 = (uint64_t)M0 * c0;
    uint64_t p1 = (uint64_t)M1 * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += W0;
    k1 += W1;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

uint32_t ntlo_sr_bits(uint64_t seed, uint64_t offset, uint64_t e) {
  uint32_t ctr[4], key[2], out[4];
  uint64_t g = e >> 2;
  ctr[0] = (uint32_t)g;
  ctr[1] = (uint32_t)(g >> 32);
  ctr[2] = (uint32_t)offset;
  ctr[3] = (uint32_t)(offset >> 32);
  key[0] = (uint32_t)seed;
  key[1] = (uint32_t)(seed >> 32);
  ntlo_philox4x32_10(ctr, key, out);
  return out[e & 3];
}

static float sr_uniform(uint32_t r) { return (float)(r >> 8) * 0x1p-24f; }

/* ------------------------------------------------------------------ */
/* OCP e4m3fn conversions                                              */
/* ------------------------------------------------------------------ */
/* Round-to-nearest-even fp32 -> e4m3fn, non-saturating: 464 is the tie
 * between 448 and the NaN pattern and goes to 448 (even), anything larger
 * gives NaN, as torch's float8_e4m3fn cast does; NaN keeps its sign bit. */
uint8_t ntlo_e4m3_from_f32(float v) {
  uint32_t bits;
  memcpy(&bits, &v, 4);
  uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
  float a = fabsf(v);
  if (isnan(v)) return (uint8_t)(sign | 0x7Fu);
  if (a > 464.0f) return (uint8_t)(sign | 0x7Fu);
  if (a < 0x1p-6f) {
    /* subnormal range: multiples of 2^-9; a*2^9 is exact */
    float m = rintf(a * 512.0f); /* 0..8; 8 == smallest normal (code 0x08) */
    return (uint8_t)(sign | (uint8_t)m);
  }
  int e;
  float f = frexpf(a, &e);          /* a = f * 2^e, f in [0.5, 1) */
  float m = rintf(f * 16.0f);       /* 8..16: 1.mmm with 3 mantissa bits */
  int exp_field = e - 1 + 7;        /* unbiased exponent e-1 */
  if (m >= 16.0f) {
    m = 8.0f;
    exp_field += 1;
  }
  int mant = (int)m - 8;
  uint8_t code = (uint8_t)((exp_field << 3) | mant); /* a <= 464 keeps code <= 0x7E */
  return (uint8_t)(sign | code);
}

float ntlo_e4m3_to_f32(uint8_t c) {
  int sign = c & 0x80;
  int ef = (c >> 3) & 0xF;
  int mant = c & 7;
  float v;
  if (ef == 0xF && mant == 7) return sign ? -NAN : NAN;
  if (ef == 0)
    v = ldexpf((float)mant, -9);
  else
    v = ldexpf((float)(8 + mant), ef - 10);
  return sign ? -v : v;
}

/* Stochastic rounding onto the e4m3 grid, the integer form: with |v| in
 * [8, 16) units of its e4m3 spacing, the 20 bits of |v| just below the
 * spacing (truncated) plus the top 20 bits of the contract word r carry into
 * the code: |v| rounds away from zero iff frac20 + (r >> 12) >= 2^20.  In the
 * subnormal range (spacing 2^-9) frac20 is the 20 bits of |v| * 512 just
 * below the integer part.  The sign of v is kept; inputs are already clamped
 * to [-448, 448] (at 448 frac20 is 0). */
static uint8_t e4m3_stochastic(float v, uint32_t r) {
  if (isnan(v)) return ntlo_e4m3_from_f32(v);
  uint32_t bits;
  memcpy(&bits, &v, 4);
  uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
  uint32_t ab = bits & 0x7FFFFFFFu;
  if (ab >= 0x43E00000u) return (uint8_t)(sign | 0x7E); /* >= 448 */
  uint32_t e8 = ab >> 23, trunc, f20;
  if (e8 >= 121u) {
    trunc = ((e8 - 120u) << 3) + ((ab >> 20) & 7u);
    f20 = ab & 0xFFFFFu;
  } else {
    uint64_t m = (ab & 0x7FFFFFu) | (e8 ? 0x800000u : 0u);
    uint32_t sh = 141u - (e8 ? e8 : 1u); /* |v| * 512 = m / 2^sh */
    trunc = sh < 64u ? (uint32_t)(m >> sh) : 0u;
    f20 = sh - 20u < 64u ? (uint32_t)((m >> (sh - 20u)) & 0xFFFFFu) : 0u;
  }
  uint32_t c = trunc + ((f20 + (r >> 12)) >> 20);
  if (c > 0x7Eu) c = 0x7Eu;
  return (uint8_t)(sign | c);
}

/* ------------------------------------------------------------------ */
/* scale and element quantization                                      */
/* ------------------------------------------------------------------ */
/* torch.amax over |x| propagates NaN (probed); comparisons skip it. */
static float amax_accum(float m, float x) {
  if (isnan(m)) return m;
  float a = fabsf(x);
  if (isnan(a)) return a;
  return a > m ? a : m;
}

static float scale_from_amax(float amax, float qmaxf, int rule) {
  if (rule == SCALE_BEFORE_DIVIDE) {
    /* moe.py:94-98: if not finite(amax) or amax <= 0: 1.0 else amax/qmax */
    if (!isfinite(amax) || amax <= 0.0f) return 1.0f;
    return amax / qmaxf;
  }
  /* te_backend.py:99-100 then _safe_scale (:74-79) */
  float s = amax / qmaxf;
  if (isfinite(s) && s > 0.0f) return s;
  return 1.0f;
}

static float grid_qmax(int grid, int qmax) { return grid == GRID_E4M3 ? 448.0f : (float)qmax; }

/* Quantize one element with scale s.  Returns q (as the reference holds it,
 * a float) and writes the code byte.  te_backend.py:101-106 / moe.py:99-105. */
static float quant_one(float x, float s, int grid, int qmax, int rounding, uint32_t r, uint8_t* code) {
  float v = x / s;
  if (grid == GRID_INT) {
    float q;
    if (rounding == ROUND_STOCHASTIC) {
      float u = sr_uniform(r);
      q = (v >= 0.0f) ? floorf(v + u) : ceilf(v - u);
    } else {
      q = rintf(v);
    }
    float qm = (float)qmax;
    if (q < -qm) q = -qm;
    if (q > qm) q = qm;
    *code = isnan(q) ? (uint8_t)0x80 : (uint8_t)(int8_t)q;
    return q;
  }
  /* e4m3: clamp to the finite range first (layers.py:115), then cast */
  if (v < -448.0f) v = -448.0f;
  if (v > 448.0f) v = 448.0f;
  uint8_t c = (rounding == ROUND_STOCHASTIC) ? e4m3_stochastic(v, r) : ntlo_e4m3_from_f32(v);
  *code = c;
  return ntlo_e4m3_to_f32(c);
}

float ntlo_code_value(uint8_t code, int grid) {
  if (grid == GRID_E4M3) return ntlo_e4m3_to_f32(code);
  if (code == 0x80) return NAN;
  return (float)(int8_t)code;
}

/* ------------------------------------------------------------------ */
/* Grouped quantization: the common form of every granularity.        */
/*                                                                      */
/* x is a row-major [R, K] fp32 matrix.  Element (i, k) shares its scale */
/* with every element of the group (i / gr, k / gc); scales is          */
/* [ceil(R/gr), ceil(K/gc)].  Out-of-range elements of a partial group   */
/* count as zeros (the F.pad of te_backend.py:94-95, :134-135).          */
/*   tile_1x128     gr = 1,   gc = 128   (te_backend.py:82-110)          */
/*   block_128x128  gr = 128, gc = 128   (te_backend.py:113-149)         */
/*   128x1          gr = 128, gc = 1     (benchmark c3 recipe)           */
/*   tensor         gr = R,   gc = K     (te_backend.py:165-173)         */
/*   channel ax -1  gr = R,   gc = 1     (te_backend.py:175-185)         */
/*   channel ax 0   gr = 1,   gc = K                                     */
/*   comm strip     gr = R,   gc = 128   (moe.py:123-140)                */
/* codes: [R, ldc] bytes, ldc >= K (entries k >= K are written 0).       */
/* q_out / dq: [R, K] floats (q and q*scale in fp32), may be NULL.       */
/* SR bits are drawn for the source element index i*K + k.               */
/* ------------------------------------------------------------------ */
/* Element (i, k) of x draws the stochastic-rounding bits of source index
 * e_base + i * e_row + k (e_row = 0 means K): a slice of a larger [R', K']
 * matrix -- rows [r0, r1) with e_base = r0 * K', or columns [c0, c1) with
 * e_base = c0 and e_row = K' -- then gets the bits of its place in that
 * matrix, and groups that do not cross the slice's edge give that matrix's
 * codes. */
int ntlo_quant_grouped_at(const float* x, int64_t R, int64_t K, int64_t gr, int64_t gc, int grid, int qmax,
                          int rounding, int scale_rule, uint64_t seed, uint64_t offset, uint8_t* codes,
                          int64_t ldc, float* scales, float* q_out, float* dq, uint64_t e_base, uint64_t e_row) {
  if (e_row == 0) e_row = (uint64_t)K;
  if (R < 0 || K < 0 || gr <= 0 || gc <= 0 || ldc < K) return -1;
  int64_t nsr = (R + gr - 1) / gr, nsc = (K + gc - 1) / gc;
  float qmaxf = grid_qmax(grid, qmax);
  for (int64_t bi = 0; bi < nsr; ++bi) {
    for (int64_t bk = 0; bk < nsc; ++bk) {
      float m = 0.0f;
      for (int64_t i = bi * gr; i < (bi + 1) * gr && i < R; ++i)
        for (int64_t k = bk * gc; k < (bk + 1) * gc && k < K; ++k) m = amax_accum(m, x[i * K + k]);
      scales[bi * nsc + bk] = scale_from_amax(m, qmaxf, scale_rule);
    }
  }
  for (int64_t i = 0; i < R; ++i) {
    for (int64_t k = 0; k < ldc; ++k) {
      if (k >= K) {
        codes[i * ldc + k] = 0;
        continue;
      }
      float s = scales[(i / gr) * nsc + (k / gc)];
      uint32_t r = rounding == ROUND_STOCHASTIC ? ntlo_sr_bits(seed, offset, e_base + (uint64_t)i * e_row + (uint64_t)k)
                                                : 0u;
      uint8_t c;
      float q = quant_one(x[i * K + k], s, grid, qmax, rounding, r, &c);
      codes[i * ldc + k] = c;
      if (q_out) q_out[i * K + k] = q;
      if (dq) dq[i * K + k] = q * s;
    }
  }
  return 0;
}

int ntlo_quant_grouped(const float* x, int64_t R, int64_t K, int64_t gr, int64_t gc, int grid, int qmax,
                       int rounding, int scale_rule, uint64_t seed, uint64_t offset, uint8_t* codes,
                       int64_t ldc, float* scales, float* q_out, float* dq) {
  return ntlo_quant_grouped_at(x, R, K, gr, gc, grid, qmax, rounding, scale_rule, seed, offset, codes, ldc, scales,
                               q_out, dq, 0, 0);
}

/* Comm-quant 'channel' granularity loops over columns with one scale per
 * column taken over all rows (moe.py:112-121); it is the grouped form with
 * gr = R, gc = 1 and the before-divide scale rule. */

/* ------------------------------------------------------------------ */
/* Persistent NF4 (layers.py:60-184)                                   */
/* ------------------------------------------------------------------ */
static const float NF4_CODEBOOK[16] = {
    -1.0f,        -0.6961928f,  -0.52507305f, -0.3949175f, -0.28444138f, -0.18477343f,
    -0.09105004f, 0.0f,         0.0795803f,   0.1609302f,  0.2461123f,   0.33791524f,
    0.44070983f,  0.562617f,    0.72295684f,  1.0f};

float ntlo_nf4_codebook(int i) { return NF4_CODEBOOK[i & 15]; }

/* One scale per run of `block` consecutive elements of the flat tensor:
 * block = K for per_channel on a 2-D [N, K] weight, block = numel for
 * per_tensor (layers.py:86-101), block = 64 for the 64-element recipe.
 * scale = amax (not divided), non-finite or <= 0 -> 1.0 (layers.py:98-100).
 * idx = argmin_i |clamp(w/s, -1, 1) - cb_i| with the first minimum winning
 * and an all-NaN row giving 0 (torch.argmin, layers.py:165-166). */
int ntlo_nf4_quant(const float* w, int64_t n, int64_t block, uint8_t* packed, float* scales) {
  if (n < 0 || block <= 0) return -1;
  int64_t nb = (n + block - 1) / block;
  for (int64_t b = 0; b < nb; ++b) {
    float m = 0.0f;
    for (int64_t i = b * block; i < (b + 1) * block && i < n; ++i) m = amax_accum(m, w[i]);
    scales[b] = (isfinite(m) && m > 0.0f) ? m : 1.0f;
  }
  int64_t np = (n + 1) / 2;
  memset(packed, 0, (size_t)np);
  for (int64_t i = 0; i < n; ++i) {
    float c = w[i] / scales[i / block];
    if (c < -1.0f) c = -1.0f;
    if (c > 1.0f) c = 1.0f;
    int best = 0;
    float bd = fabsf(c - NF4_CODEBOOK[0]);
    if (!isnan(bd)) {
      for (int j = 1; j < 16; ++j) {
        float d = fabsf(c - NF4_CODEBOOK[j]);
        if (d < bd) {
          bd = d;
          best = j;
        }
      }
    }
    if (i & 1)
      packed[i >> 1] |= (uint8_t)(best << 4);
    else
      packed[i >> 1] |= (uint8_t)best;
  }
  return 0;
}

/* codebook[idx] * scale in fp32 (layers.py:172-184, before the dtype cast) */
int ntlo_nf4_dequant(const uint8_t* packed, const float* scales, int64_t n, int64_t block, float* out) {
  if (n < 0 || block <= 0) return -1;
  for (int64_t i = 0; i < n; ++i) {
    uint8_t byte = packed[i >> 1];
    int idx = (i & 1) ? (byte >> 4) : (byte & 15);
    out[i] = NF4_CODEBOOK[idx] * scales[i / block];
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* MXFP4: OCP Microscaling v1.0, e2m1 elements, e8m0 shared scale per  */
/* 32 elements.  No reference function (benchmark c5).                  */
/*   X = 2^(floor(log2 amax) - 2), exponent clamped to [-127, 127],     */
/*   stored biased by 127; a block whose amax is NaN or inf stores the  */
/*   NaN scale 0xFF and zero codes; an all-zero block stores 2^-127.    */
/*   elements: v = w / X, round to nearest even onto                   */
/*   {0, .5, 1, 1.5, 2, 3, 4, 6}, saturating at 6, sign kept.          */
/* ------------------------------------------------------------------ */
static const float E2M1_VALUES[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

uint8_t ntlo_e2m1_from_f32(float v) {
  uint32_t bits;
  memcpy(&bits, &v, 4);
  uint8_t sign = (uint8_t)((bits >> 28) & 0x8u);
  float a = fabsf(v);
  if (isnan(a)) return 0;
  int best = 0;
  for (int j = 1; j < 8; ++j) {
    float lo = E2M1_VALUES[j - 1], hi = E2M1_VALUES[j];
    float mid = 0.5f * (lo + hi);
    if (a > mid || (a == mid && (j % 2) == 0)) best = j;
  }
  return (uint8_t)(sign | best);
}

float ntlo_e2m1_to_f32(uint8_t c) {
  float v = E2M1_VALUES[c & 7];
  return (c & 8) ? -v : v;
}

int ntlo_mxfp4_quant(const float* w, int64_t n, uint8_t* packed, uint8_t* scales) {
  if (n < 0) return -1;
  const int64_t B = 32;
  int64_t nb = (n + B - 1) / B;
  memset(packed, 0, (size_t)((n + 1) / 2));
  for (int64_t b = 0; b < nb; ++b) {
    float m = 0.0f;
    for (int64_t i = b * B; i < (b + 1) * B && i < n; ++i) m = amax_accum(m, w[i]);
    if (!isfinite(m)) {
      scales[b] = 0xFF;
      continue;
    }
    int e;
    if (m == 0.0f) {
      e = -127;
    } else {
      int fe;
      frexpf(m, &fe); /* m in [2^(fe-1), 2^fe) */
      e = (fe - 1) - 2;
      if (e < -127) e = -127;
      if (e > 127) e = 127;
    }
    scales[b] = (uint8_t)(e + 127);
    for (int64_t i = b * B; i < (b + 1) * B && i < n; ++i) {
      float v = ldexpf(w[i], -e);
      uint8_t c = ntlo_e2m1_from_f32(v);
      if (i & 1)
        packed[i >> 1] |= (uint8_t)(c << 4);
      else
        packed[i >> 1] |= c;
    }
  }
  return 0;
}

int ntlo_mxfp4_dequant(const uint8_t* packed, const uint8_t* scales, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint8_t byte = packed[i >> 1];
    uint8_t c = (i & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15);
    uint8_t sb = scales[i / 32];
    if (sb == 0xFF) {
      out[i] = NAN;
      continue;
    }
    out[i] = ldexpf(ntlo_e2m1_to_f32(c), (int)sb - 127);
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* Persistent FP8 (layers.py:86-127): scale = amax per row (per_channel) */
/* or global (per_tensor), no /448; code = e4m3(clamp(w/s, +-448)).      */
/* ------------------------------------------------------------------ */
int ntlo_fp8_persistent_quant(const float* w, int64_t n, int64_t block, uint8_t* codes, float* scales) {
  if (n < 0 || block <= 0) return -1;
  int64_t nb = (n + block - 1) / block;
  for (int64_t b = 0; b < nb; ++b) {
    float m = 0.0f;
    for (int64_t i = b * block; i < (b + 1) * block && i < n; ++i) m = amax_accum(m, w[i]);
    scales[b] = (isfinite(m) && m > 0.0f) ? m : 1.0f;
  }
  for (int64_t i = 0; i < n; ++i) {
    float v = w[i] / scales[i / block];
    if (v < -448.0f) v = -448.0f;
    if (v > 448.0f) v = 448.0f;
    codes[i] = ntlo_e4m3_from_f32(v);
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* array helpers for the Python wrapper                                */
/* ------------------------------------------------------------------ */
void ntlo_sr_bits_fill(uint64_t seed, uint64_t offset, uint64_t start, int64_t n, uint32_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = ntlo_sr_bits(seed, offset, start + (uint64_t)i);
}

void ntlo_e4m3_encode_array(const float* v, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = ntlo_e4m3_from_f32(v[i]);
}

void ntlo_e4m3_sr_encode_array(const float* v, const uint32_t* r, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    float x = v[i];
    if (x < -448.0f) x = -448.0f;
    if (x > 448.0f) x = 448.0f;
    out[i] = e4m3_stochastic(x, r[i]);
  }
}

void ntlo_code_decode_array(const uint8_t* c, int64_t n, int grid, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = ntlo_code_value(c[i], grid);
}

void ntlo_e2m1_encode_array(const float* v, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = ntlo_e2m1_from_f32(v[i]);
}
