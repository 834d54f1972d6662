/* Exhaustive check of the fp8 quantiser's corrected quotient.
 *
 * For every positive finite bf16 frame maximum m >= 2^-96 and every bf16 value
 * x with |x| <= m, with sc = fl(m / 448) and r = fl(1 / sc):
 *   q  = fl(x * r)
 *   ne = fma(q, sc, -x)          (minus the residual x - q * sc)
 *   q1 = fma(-ne, r, q)
 * must give the same OCP e4m3fn code (after clamping to +-448, round to
 * nearest even) as the IEEE quotient fl(x / sc).  Build with
 * -ffp-contract=off so that the compiler adds no contractions.
 *
 * Output: "pairs N bits_differ D codes_differ C" and exit status C != 0.
 * With an argument "encode" it prints the e4m3 code of each float read from
 * stdin (one per line), for checking the encoder against a library cast.
 */
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

static uint32_t bits_of(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* OCP e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits; subnormals
 * k * 2^-9; largest finite 448.  Values are clamped to +-448 first. */
static unsigned e4m3_code(float v) {
  const unsigned s = signbit(v) ? 0x80u : 0u;
  float a = fabsf(v);
  if (a > 448.0f) a = 448.0f;
  if (a < 0.015625f) return s | (unsigned)rintf(a * 512.0f); /* exact scaling, RNE */
  int e;
  frexpf(a, &e);
  e -= 1;                                   /* a in [2^e, 2^(e+1)) */
  const int k = (int)rintf(ldexpf(a, 3 - e)); /* in [8, 16], RNE */
  return s | (unsigned)(((e + 7) << 3) + (k - 8));
}

int main(int argc, char** argv) {
  if (argc > 1 && strcmp(argv[1], "encode") == 0) {
    float v;
    while (scanf("%f", &v) == 1) printf("%u\n", e4m3_code(v));
    return 0;
  }
  long long pairs = 0, bits_differ = 0, codes_differ = 0;
  const uint32_t first = 0x0F80; /* bf16 bits of 2^-96 */
  for (uint32_t hm = first; hm < 0x7F80; ++hm) {
    const float m = from_bf16(hm);
    const float sc = m / 448.0f;
    const float r = 1.0f / sc;
    long long lp = 0, lb = 0, lc = 0;
    /* x = +-(magnitude bits 0 .. hm): every bf16 value with |x| <= m */
#pragma omp parallel for reduction(+ : lp, lb, lc)
    for (uint32_t i = 0; i <= 2 * hm + 1; ++i) {
      const float x = from_bf16((i >> 1) | ((i & 1u) << 15));
      const float exact = x / sc;
      const float q = x * r;
      const float ne = fmaf(q, sc, -x);
      const float q1 = fmaf(-ne, r, q);
      lp++;
      if (bits_of(q1) != bits_of(exact)) {
        lb++;
        if (e4m3_code(q1) != e4m3_code(exact)) lc++;
      }
    }
    pairs += lp;
    bits_differ += lb;
    codes_differ += lc;
  }
  printf("pairs %lld bits_differ %lld codes_differ %lld\n", pairs, bits_differ, codes_differ);
  return codes_differ != 0;
}
