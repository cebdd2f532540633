/* Exhaustive host check of the quantiser's division: for every finite float16
 * numerator x and every positive finite float16 scale s,
 *     e = fma(-q0, s, x),  q = (e == 0 ? q0 : fma(e, r, q0)),
 *     r = RN(1 / s),  q0 = RN(x * r)
 * gives fl16(q) == fl16(RN(x / s)), the float32 quotient the reference rounds
 * to float16, bit for bit (signed zeros included: e == 0 means q0 * s == x
 * exactly, so q0 is the quotient). Prints the number of (x, s) pairs checked and of mismatches.
 * With the argument "uncorrected" it checks q = q0 instead (expected to fail:
 * the check can tell a wrong quotient).
 * Build: clang -O2 -ffp-contract=off -fopenmp (a host compiler with _Float16). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float h2f(uint16_t h) {
  _Float16 v;
  memcpy(&v, &h, 2);
  return (float)v;
}

static uint16_t f2h(float f) {
  _Float16 v = (_Float16)f;
  uint16_t h;
  memcpy(&h, &v, 2);
  return h;
}

int main(int argc, char** argv) {
  const int uncorrected = argc > 1 && strcmp(argv[1], "uncorrected") == 0;
  long long checked = 0, bad = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : checked, bad)
  for (int sb = 1; sb < 0x7C00; ++sb) {
    const float s = h2f((uint16_t)sb);
    const float r = 1.0f / s;
    for (int xb = 0; xb < 0x10000; ++xb) {
      if ((xb & 0x7C00) == 0x7C00) continue;            /* inf / NaN numerators */
      const float x = h2f((uint16_t)xb);
      const float q0 = x * r;
      const float e = fmaf(-q0, s, x);
      const float q = (uncorrected || e == 0.0f) ? q0 : fmaf(e, r, q0);
      const float ref = x / s;
      checked++;
      if (f2h(q) != f2h(ref)) {
        bad++;
        if (bad < 5 && !uncorrected) printf("mismatch x=%a s=%a fast=%a ref=%a\n", x, s, q, ref);
      }
    }
  }
  printf("checked %lld mismatches %lld\n", checked, bad);
  return bad != 0;
}
