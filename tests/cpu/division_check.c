/*
 * Exhaustive check of the quantizers' fast division (ntlb_quant8.h,
 * fast_div_ok / quant8_tile_rs): with r = RN(1/s), y = RN(x*r),
 * e = RN(fma(-y, s, x)) and q = RN(fma(e, r, y)), q equals RN(x/s).
 *
 * Scaling x or s by a power of two scales every step exactly while nothing
 * underflows or overflows, so covering every pair of significands (x and s
 * in [1, 2): 2^23 x 2^23 = 2^46 pairs) covers every normal case.  Each s
 * takes the 2^23 values of x eight at a time in AVX2 (IEEE single precision,
 * round to nearest even, FMA), against the hardware division.
 *
 *   division_check LO HI THREADS   checks s significands [LO, HI)
 *
 * prints the count of mismatching pairs (with the first few) and exits 1 if
 * there are any.  The whole range (0 8388608) takes about 4.5 CPU hours.
 */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

typedef struct {
  uint32_t lo, hi;
  uint64_t bad, done;
} job_t;

static void* run(void* p) {
  job_t* j = (job_t*)p;
  const __m256i idx = _mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7);
  for (uint32_t sm = j->lo; sm < j->hi; ++sm) {
    const float s = u2f((127u << 23) | sm);
    const float r = 1.0f / s;
    const __m256 vs = _mm256_set1_ps(s), vr = _mm256_set1_ps(r);
    __m256i acc = _mm256_setzero_si256();
    for (uint32_t xm = 0; xm < (1u << 23); xm += 8) {
      const __m256 x = _mm256_castsi256_ps(_mm256_add_epi32(_mm256_set1_epi32((int)((127u << 23) | xm)), idx));
      const __m256 y = _mm256_mul_ps(x, vr);
      const __m256 e = _mm256_fnmadd_ps(y, vs, x);
      const __m256 q = _mm256_fmadd_ps(e, vr, y);
      const __m256 d = _mm256_div_ps(x, vs);
      acc = _mm256_or_si256(acc, _mm256_xor_si256(_mm256_castps_si256(q), _mm256_castps_si256(d)));
    }
    if (!_mm256_testz_si256(acc, acc)) {
      for (uint32_t xm = 0; xm < (1u << 23); ++xm) {
        const float x = u2f((127u << 23) | xm);
        const float y = x * r, e = fmaf(-y, s, x), q = fmaf(e, r, y);
        if (f2u(q) != f2u(x / s)) {
          if (j->bad < 10) printf("mismatch s=%a x=%a q=%a x/s=%a\n", s, x, q, x / s);
          j->bad++;
        }
      }
    }
    j->done++;
  }
  return NULL;
}

int main(int argc, char** argv) {
  if (argc != 4) {
    fprintf(stderr, "usage: %s LO HI THREADS\n", argv[0]);
    return 2;
  }
  const uint32_t lo = (uint32_t)strtoul(argv[1], 0, 0), hi = (uint32_t)strtoul(argv[2], 0, 0);
  int nt = atoi(argv[3]);
  if (hi > (1u << 23) || lo > hi || nt < 1) return 2;
  if (nt > 64) nt = 64;
  pthread_t th[64];
  job_t jobs[64];
  const uint32_t step = (hi - lo + (uint32_t)nt - 1) / (uint32_t)nt;
  for (int t = 0; t < nt; ++t) {
    jobs[t].lo = lo + (uint32_t)t * step < hi ? lo + (uint32_t)t * step : hi;
    jobs[t].hi = jobs[t].lo + step < hi ? jobs[t].lo + step : hi;
    jobs[t].bad = jobs[t].done = 0;
    pthread_create(&th[t], 0, run, &jobs[t]);
  }
  uint64_t bad = 0, done = 0;
  for (int t = 0; t < nt; ++t) {
    pthread_join(th[t], 0);
    bad += jobs[t].bad;
    done += jobs[t].done;
  }
  printf("s significands [%u, %u): %llu checked, %llu mismatching pairs\n", lo, hi, (unsigned long long)done,
         (unsigned long long)bad);
  return bad != 0;
}
