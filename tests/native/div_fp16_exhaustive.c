/* Exhaustive check of the reciprocal-with-correction quotient used by the
 * baseline-format kernels (div_fp16_divisor in stepquant_hip.hip):
 *   inv = RN(1 / d), q0 = RN(x * inv), r = RN(fma(-q0, d, x)), q1 = RN(fma(r, inv, q0))
 * equals the IEEE quotient RN(x / d) for every x in [1, 2) (all 2^23
 * significands) and every d in [1, 2) with a 10-bit fraction (the fp16
 * significands).  In the normal range exponents only scale the operands and
 * the result, so this covers every normal x and fp16-representable d.
 * Prints the number of mismatches (0 expected) and exits non-zero on any. */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

typedef struct { int d0, d1; long bad; } job_t;

static void *run(void *p) {
  job_t *j = (job_t *)p;
  for (int m = j->d0; m < j->d1; m++) {
    const float d = f_of(0x3f800000u | ((uint32_t)m << 13));
    volatile float one = 1.0f;
    const float inv = one / d;
    for (uint32_t xm = 0; xm < (1u << 23); xm++) {
      const float x = f_of(0x3f800000u | xm);
      const float q0 = x * inv;
      const float r = fmaf(-q0, d, x);
      const float q1 = fmaf(r, inv, q0);
      if (u_of(q1) != u_of(x / d)) j->bad++;
    }
  }
  return 0;
}

int main(void) {
  enum { NT = 8 };
  pthread_t t[NT];
  job_t j[NT];
  for (int i = 0; i < NT; i++) {
    j[i].d0 = 1024 / NT * i;
    j[i].d1 = 1024 / NT * (i + 1);
    j[i].bad = 0;
    pthread_create(&t[i], 0, run, &j[i]);
  }
  long bad = 0;
  for (int i = 0; i < NT; i++) {
    pthread_join(t[i], 0);
    bad += j[i].bad;
  }
  printf("mismatches: %ld\n", bad);
  return bad != 0;
}
