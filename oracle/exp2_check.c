/*
 * Exhaustive check: orc_exp2f (the oracle's restatement of glibc's exp2f
 * algorithm) against the host libm exp2f on every float in [-151, 129],
 * which covers every input whose result is neither 0 nor +inf, and a sweep
 * of the special values outside it.  TEST INFRASTRUCTURE ONLY.
 * Prints "checked=N mismatches=M" and exits 0 iff M == 0.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "ref_qwen3.h"

static float asf(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t asu(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

int main(void) {
  long long checked = 0, bad = 0;
#pragma omp parallel for reduction(+ : checked, bad) schedule(static)
  for (long long hi = 0; hi < 65536; ++hi) {
    for (uint32_t lo = 0; lo < 65536; ++lo) {
      const uint32_t u = ((uint32_t)hi << 16) | lo;
      const float x = asf(u);
      const int inside = (x > -151.0f && x < 129.0f);
      /* outside the window only sample every 4096th pattern (+ specials) */
      if (!inside && (lo & 0xFFF) != 0 && !isnan(x) && !isinf(x)) continue;
      const float a = orc_exp2f(x), b = exp2f(x);
      ++checked;
      if (asu(a) != asu(b) && !(isnan(a) && isnan(b))) {
        ++bad;
        if (bad < 4) fprintf(stderr, "x=%a orc=%a libm=%a\n", x, a, b);
      }
    }
  }
  printf("checked=%lld mismatches=%lld\n", checked, bad);
  return bad == 0 ? 0 : 1;
}
