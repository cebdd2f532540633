/*
 * Exhaustive check of the transcoding kernel's division (test infrastructure).
 *
 * The reference's INT8 demote (kv_memory_manager.py:245-247) computes, per
 * element x of a float16 page with absmax m (a float16 value):
 *     s    = float32(m / 127)                         (m > 0)
 *     code = clamp(rint(float16(float32(x) / s)), -128, 127)
 * with IEEE float32 division. The kernel replaces the per-element division by
 *     r  = 1 / s                                       (once per page, IEEE)
 *     q0 = x * r;  e = fma(-q0, s, x);  q = fma(e, r, q0)
 * (Markstein's correction). This program checks, for every positive finite
 * float16 m and every float16 x with |x| <= m (every page element that can
 * occur), that both give the same code: exit status 0 and a count on success,
 * 1 and the first counterexample found otherwise. float16 conversions use the
 * F16C instructions (round to nearest even).
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math -mf16c -mfma -fopenmp -o check demote_division_check.c -lm
 * (-DPLANT_NO_CORRECTION drops the correction step: the check must then fail.)
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }

static inline int code_of(float q) {
  float r = rintf(_cvtsh_ss(_cvtss_sh(q, _MM_FROUND_TO_NEAREST_INT)));
  if (r != r) return 0;
  if (r < -128.f) r = -128.f;
  if (r > 127.f) r = 127.f;
  return (int)r;
}

int main(void) {
  unsigned long long n = 0;
  int bad_m = -1, bad_x = -1;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : n)
  for (int mh = 1; mh < 0x7c00; ++mh) {                   /* positive finite float16 m */
    const float m = h2f((uint16_t)mh);
    const float s = (float)((double)m / 127.0);           /* the reference's float scale, as float32 */
    const float r = 1.0f / s;
    for (int xh = 0; xh < 0x10000; ++xh) {
      if ((xh & 0x7fff) > mh) continue;                   /* |x| <= m */
      const float x = h2f((uint16_t)xh);
      const float q0 = x * r;
      const float e = fmaf(-q0, s, x);
#ifdef PLANT_NO_CORRECTION
      const float q = q0 + 0.0f * e;                      /* planted mistake: the bare product */
#else
      const float q = fmaf(e, r, q0);
#endif
      if (code_of(x / s) != code_of(q)) {
#pragma omp critical
        { bad_m = mh; bad_x = xh; }
      }
      ++n;
    }
  }
  if (bad_m >= 0) {
    const float m = h2f((uint16_t)bad_m), s = (float)((double)m / 127.0), x = h2f((uint16_t)bad_x);
    printf("MISMATCH m=0x%04x x=0x%04x quotient=%.9g\n", bad_m, bad_x, x / s);
    return 1;
  }
  printf("OK %llu pairs\n", n);
  return 0;
}
