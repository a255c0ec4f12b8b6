/* Exhaustive checks of fp32 identities the GPU kernels rely on (CPU only).
 *
 * round:    trunc(x + copysign(0.5 - 2^-25, x)) == roundf(x) for every float
 *           with |x| < 2^23 (k_q8_fast's round-half-away).
 * quotient: with r = RN(1/s), q0 = RN(v r), e = fma(q0, s, -v),
 *           q1 = fma(-e, r, q0) is the IEEE quotient RN(v / s), sign of a
 *           zero included, for every bf16 (quotient_bf16) or fp16
 *           (quotient_f16) v and s > 0 whose magnitudes and quotient lie in
 *           [2^-100, 2^100] or v = +-0 (lm_device.h div_rn).
 * Usage: identities round|quotient_bf16|quotient_f16 ; exit status 0 when
 * the identity holds. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>


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

static float from_bits16(uint32_t h, int f16) {
  uint32_t b;
  if (!f16) {
    b = h << 16;
  } else {  /* fp16 -> fp32, exact */
    uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31) b = sign | 0x7f800000u | (m << 13);
    else if (e != 0) b = sign | ((e + 112u) << 23) | (m << 13);
    else if (m == 0) b = sign;
    else {
      float x = ldexpf((float)m, -24);
      memcpy(&b, &x, 4);
      b |= sign;
    }
  }
  float x;
  memcpy(&x, &b, 4);
  return x;
}
static int in_domain(float x) {
  const float a = fabsf(x);
  return a >= 0x1p-100f && a <= 0x1p100f;
}
static int check_quotient(int f16) {
  uint64_t n = 0, bad = 0;
  for (uint32_t hs = 1; hs < 0x7fffu; ++hs) {
    const float s = from_bits16(hs, f16);
    if (!isfinite(s) || !in_domain(s)) continue;
    const float r = 1.0f / s;
    for (uint32_t hv = 0; hv < 0x10000u; ++hv) {
      const float v = from_bits16(hv, f16);
      if (!isfinite(v)) continue;
      const int zero = v == 0.0f;
      if (!zero && !in_domain(v)) continue;
      const float want = v / s;
      if (!zero && !in_domain(want)) continue;
      volatile float q0 = v * r;
      volatile float e = fmaf(q0, s, -v);
      const float q1 = fmaf(-e, r, q0);
      uint32_t a, b;
      memcpy(&a, &q1, 4);
      memcpy(&b, &want, 4);
      bad += a != b;
      ++n;
    }
  }
  printf("quotient_%s: %llu pairs, %llu mismatches\n", f16 ? "f16" : "bf16", (unsigned long long)n,
         (unsigned long long)bad);
  return bad != 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && strcmp(argv[1], "round") == 0) return check_round();
  if (argc > 1 && strcmp(argv[1], "quotient_bf16") == 0) return check_quotient(0);
  if (argc > 1 && strcmp(argv[1], "quotient_f16") == 0) return check_quotient(1);
  fprintf(stderr, "usage: identities round|quotient_bf16|quotient_f16\n");
  return 2;
}
