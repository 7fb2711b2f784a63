/* Checks Markstein's FMA division, q = fma(a - q0 b, r, q0) with r = RN(1/b)
 * and q0 = RN(a r), against IEEE float division: for each divisor given on
 * the command line and `nrand` random divisor significands, every dividend of
 * the binade [1, 2) (the exponents scale away while the quotient stays
 * normal).  Prints the number of checks and mismatches; exit status 1 on any
 * mismatch.  Built and run by tests/test_markstein_division.py. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bits2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static uint64_t check(float b, uint64_t* n) {
  volatile float one = 1.0f;
  const float r = one / b;
  uint64_t bad = 0;
  for (uint32_t u = 0x3F800000u; u < 0x40000000u; ++u) {
    const float a = bits2f(u);
    const float q0 = a * r;
    const float q = fmaf(fmaf(-q0, b, a), r, q0);
    bad += f2bits(q) != f2bits(a / b);
    ++*n;
  }
  return bad;
}

int main(int argc, char** argv) {
  const int nrand = atoi(argv[1]);
  uint64_t n = 0, bad = 0, s = 0x9E3779B97F4A7C15ull;
  for (int i = 2; i < argc; ++i) bad += check(strtof(argv[i], NULL), &n);
  for (int k = 0; k < nrand; ++k) {
    s ^= s << 13; s ^= s >> 7; s ^= s << 17;
    bad += check(ldexpf(bits2f(0x3F800000u | (uint32_t)(s & 0x7FFFFF)), (int)(s >> 40) % 30 - 15), &n);
  }
  printf("%llu checks, %llu mismatches\n", (unsigned long long)n, (unsigned long long)bad);
  return bad != 0;
}
