/* Exhaustive check of the quotient the 16-bit e4m3 row quantiser uses in place of a division
 * (flide_amd/csrc/rowwise.hip, div_markstein): for every finite row maximum amax of a 16-bit format
 * and every x of that format with |x| <= amax, with s = max(amax, 1e-12) * (1/448) as the quantiser
 * makes it,
 *     q0 = x * (1/s),  q1 = fma(fma(q0, s, -x), -(1/s), q0)
 * must equal the correctly rounded x / s bit for bit wherever |x / s| > 2^-11, and have its sign below
 * that (where both encode to +-0 in e4m3, whose smallest step is 2^-9).
 * Usage: division_check bf16|f16   prints "<pairs> <mismatches> <tiny differences>", exit 1 on a mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bf16(uint32_t h) {
  uint32_t u = h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float from_f16(uint32_t h) {
  const uint32_t e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 1024), (int)e - 25);
  return (h & 0x8000) ? -v : v;
}

static uint32_t bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

int main(int argc, char** argv) {
  const int f16 = argc > 1 && strcmp(argv[1], "f16") == 0;
  long long pairs = 0, bad = 0, tiny = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, bad, tiny)
  for (uint32_t a = 0; a < 0x8000; ++a) {
    const float amax = f16 ? from_f16(a) : from_bf16(a);
    if (!isfinite(amax)) continue;
    const float s = fmaxf(amax, 1e-12f) * (1.0f / 448.0f);
    const float rinv = 1.0f / s, nrinv = -rinv;
    for (uint32_t h = 0; h < 0x10000; ++h) {
      const float x = f16 ? from_f16(h) : from_bf16(h);
      if (!(fabsf(x) <= amax)) continue;
      ++pairs;
      const float d = x / s;
      const float q0 = x * rinv;
      const float q1 = fmaf(fmaf(q0, s, -x), nrinv, q0);
      if (bits(q1) == bits(d)) continue;
      if ((fabsf(d) > 0x1p-11f || fabsf(q1) > 0x1p-11f) || signbit(d) != signbit(q1)) {
        if (bad < 5) printf("mismatch amax %a x %a: %a vs %a\n", amax, x, q1, d);
        ++bad;
      } else {
        ++tiny;
      }
    }
  }
  printf("%lld %lld %lld\n", pairs, bad, tiny);
  return bad != 0;
}
