/* Exhaustive checks of two fp32 identities the GPU kernels rely on (CPU only).
 *
 * round:    trunc(x + copysign(0.5 - 2^-25, x)) == roundf(x) for every float
 *           with |x| < 2^23 (k_q8_fast's round-half-away).
 * quotient: for every bf16 m > 0 and bf16 s >= 2^-23 with m/s <= 256,
 *           ceil(fmaf(m, H, m * L)) == ceil(65536 * RN(m/s)) with
 *           hi = RN(1/s), lo = fmaf(-s, hi, 1) * hi, H = 65536 hi, L = 65536 lo
 *           (k_rows_fast's INT8 stochastic-rounding quotient) for s <= 2^100,
 *           and the three-instruction form above; the one exception allowed
 *           is RN(m/s) underflowing to zero.
 * Usage: identities round|quotient ; exit status 0 when the identity holds. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf(uint32_t h) { uint32_t u = h << 16; float f; memcpy(&f, &u, 4); return f; }

static int check_round(void) {
  const float c = 0.49999997f;
  uint64_t n = 0, bad = 0;
  for (uint64_t u = 0; u <= 0xFFFFFFFFull; ++u) {
    uint32_t b = (uint32_t)u;
    float x;
    memcpy(&x, &b, 4);
    if (!(fabsf(x) < 8388608.0f)) continue;
    volatile float s = x + copysignf(c, x);
    if (truncf(s) != roundf(x)) ++bad;
    ++n;
  }
  printf("round: %llu floats, %llu mismatches\n", (unsigned long long)n, (unsigned long long)bad);
  return bad != 0;
}

static int check_quotient(void) {
  uint64_t n = 0, bad = 0, under = 0;
  for (uint32_t hs = 0x3400; hs < 0x7f80; ++hs) {
    const float s = bf(hs);
    const float hi = 1.0f / s;
    const float lo = fmaf(-s, hi, 1.0f) * hi;
    const float H = hi * 65536.0f, L = lo * 65536.0f;
    for (uint32_t hm = 1; hm < 0x7f80; ++hm) {
      const float m = bf(hm);
      const float y = m / s;
      if (y > 256.0f) break;
      float got;
      if (s <= 0x1p100f) {
        got = fmaf(m, H, m * L);
      } else {
        const float q0 = m * H;
        const float e = fmaf(-q0, s * (1.0f / 65536.0f), m);
        got = fmaf(e, H, q0);
      }
      ++n;
      if ((double)ceilf(got) != ceil(65536.0 * (double)y)) {
        if (y == 0.0f) ++under;
        else ++bad;
      }
    }
  }
  printf("quotient: %llu pairs, %llu mismatches, %llu with RN(m/s) underflowing to 0\n", (unsigned long long)n,
         (unsigned long long)bad, (unsigned long long)under);
  return bad != 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && strcmp(argv[1], "round") == 0) return check_round();
  if (argc > 1 && strcmp(argv[1], "quotient") == 0) return check_quotient();
  fprintf(stderr, "usage: identities round|quotient\n");
  return 2;
}
