/* Exhaustive check of an fp32 identity a GPU kernel relies on (CPU only).
 *
 * round:    trunc(x + copysign(0.5 - 2^-25, x)) == roundf(x) for every float
 *           with |x| < 2^23 (k_q8_fast's round-half-away).
 * Usage: identities round ; exit status 0 when the identity holds. */
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

int main(int argc, char** argv) {
  if (argc > 1 && strcmp(argv[1], "round") == 0) return check_round();
  fprintf(stderr, "usage: identities round\n");
  return 2;
}
