/*
 * lm_oracle.c -- CPU restatement of piper-offload's LoRA-merge hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * kernels: it is loaded by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py, never by the product path.
 *
 * Every function restates the arithmetic of the reference's fused Triton
 * path (the only in-tree statement of TorchAO's rounding sequence); the
 * citations below use the shorthand P/ = /root/reference/src/piper_offload/.
 *
 * Numeric conventions shared with the HIP kernels:
 *   - the LoRA delta of one element is an fp32 sum over k = 0..r-1 in
 *     ascending order, one fmaf per term (P/_triton_int8_lora.py:51-66 uses
 *     tl.dot with fp32 accumulation; its order is hardware-defined, so this
 *     is a canonical restatement -- see the tolerance contract in tests/);
 *   - merged = round_cd(fmaf(delta, strength, base))
 *     (P/_triton_int8_lora.py:89-93);
 *   - stochastic rounding draws u = k * 2^-16 with k a 16-bit half of word
 *     (idx & 7) >> 1 of Philox4x32-7(ctr = (idx >> 3, 0, 0), key = seed)
 *     (the high half for even idx; words 1 and 3 complemented), or the
 *     Triton tl.rand stream (P/_triton_stochastic_quantization.py:19-22) in
 *     compatibility mode.
 *
 * Build: oracle/Makefile (gcc -O2 -mfma -ffp-contract=off -fopenmp).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* dtype ids (must match include/lora_merge.h)                          */
/* ------------------------------------------------------------------ */
enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_E4M3 = 3, DT_E5M2 = 4, DT_E2M1 = 5, DT_E8M0 = 6, DT_I8 = 7, DT_U8 = 8 };
enum { SR_OFF = 0, SR_PHILOX8 = 1, SR_TRITON = 2 };
enum { MX_FLOOR = 0, MX_RCEIL = 1, MX_CEIL = 2, MX_EVEN = 3 };

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fp32 -> bf16 round-to-nearest-even (NaN stays NaN). */
static inline uint16_t bf16_bits(float x) {
  uint32_t u = f2u(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static inline float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }
static inline float bf16r(float x) { return bf16_to_f32(bf16_bits(x)); }

/* fp32 -> fp16 RNE with subnormals and overflow to inf. */
static uint16_t f16_bits(float x) {
  uint32_t u = f2u(x);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;
  if (a >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                         /* below 2^-14: subnormal */
    float q = fabsf(x) * 16777216.0f;            /* / 2^-24, exact scaling */
    return sign | (uint16_t)nearbyintf(q);
  }
  uint32_t e = (a >> 23) - 127 + 15;
  uint32_t m = a & 0x7fffffu;
  uint32_t r = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1;
  return sign | (uint16_t)r;
}
static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 31, m = h & 1023;
  if (e == 0) { float v = ldexpf((float)m, -24); return (h & 0x8000u) ? -v : v; }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}
static inline float f16r(float x) { return f16_to_f32(f16_bits(x)); }

static inline float round_dt(int dt, float x) {
  if (dt == DT_BF16) return bf16r(x);
  if (dt == DT_F16) return f16r(x);
  return x;
}
static inline float load_dt(int dt, const void* p, int64_t i) {
  if (dt == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  if (dt == DT_F16) return f16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}
static inline void store_dt(int dt, void* p, int64_t i, float v) {
  if (dt == DT_BF16) ((uint16_t*)p)[i] = bf16_bits(v);
  else if (dt == DT_F16) ((uint16_t*)p)[i] = f16_bits(v);
  else ((float*)p)[i] = v;
}

/* ---- OCP 8-bit floats ------------------------------------------------ */
/* decode e4m3fn: bias 7, 0x7f/0xff NaN, no inf. */
static float e4m3_to_f32(uint8_t c) {
  int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7) v = NAN;
  else if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + m / 8.0f, e - 7);
  return s ? -v : v;
}
/* decode e5m2: bias 15, IEEE-like inf/NaN. */
static float e5m2_to_f32(uint8_t c) {
  int s = c >> 7, e = (c >> 2) & 31, m = c & 3;
  float v;
  if (e == 31) v = m ? NAN : INFINITY;
  else if (e == 0) v = ldexpf((float)m, -16);
  else v = ldexpf(1.0f + m / 4.0f, e - 15);
  return s ? -v : v;
}
/* Generic RNE magnitude encode for a minifloat with mbits mantissa bits,
 * exponent bias `bias`, smallest normal exponent 1-bias. Returns the code of
 * |x| (no sign); caller guarantees |x| is within the finite range. */
static uint8_t minifloat_mag_rne(float a, int mbits, int bias) {
  if (a == 0.0f) return 0;
  float min_normal = ldexpf(1.0f, 1 - bias);
  int steps = 1 << mbits;
  if (a < min_normal) {
    float q = ldexpf(a, bias - 1 + mbits); /* a / subnormal step, exact */
    return (uint8_t)nearbyintf(q);         /* == steps -> smallest normal */
  }
  int e2;
  (void)frexpf(a, &e2);
  int E = e2 - 1; /* a in [2^E, 2^(E+1)) */
  float q = ldexpf(a, -E) * (float)steps - (float)steps;
  int m = (int)nearbyintf(q);
  int biased = E + bias;
  if (m == steps) { biased += 1; m = 0; }
  return (uint8_t)((biased << mbits) | m);
}
static uint8_t f32_to_e4m3(float x) { /* RNE, caller clamps to +-448 */
  uint8_t sign = (uint8_t)((f2u(x) >> 24) & 0x80);
  if (isnan(x)) return 0x7f | sign;
  float a = fabsf(x);
  if (a >= 464.0f) return 0x7f | sign;
  return sign | minifloat_mag_rne(a, 3, 7);
}
static uint8_t f32_to_e5m2(float x) { /* RNE, caller clamps to +-57344 */
  uint8_t sign = (uint8_t)((f2u(x) >> 24) & 0x80);
  if (isnan(x)) return 0x7e | sign;
  float a = fabsf(x);
  if (a >= 61440.0f) return 0x7c | sign;
  return sign | minifloat_mag_rne(a, 2, 15);
}
static inline float fp8_decode(int fmt, uint8_t c) { return fmt == DT_E4M3 ? e4m3_to_f32(c) : e5m2_to_f32(c); }
static inline uint8_t fp8_encode(int fmt, float x) { return fmt == DT_E4M3 ? f32_to_e4m3(x) : f32_to_e5m2(x); }

/* ---- E2M1 ------------------------------------------------------------ */
static const float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
/* P/_triton_nvfp4_lora.py:24-52 */
static inline float e2m1_to_f32(uint8_t c) { float v = kE2M1[c & 7]; return (c & 8) ? -v : v; }
/* P/_triton_nvfp4_lora.py:55-85 (thresholds encode RNE with ties to even) */
static inline uint8_t f32_to_e2m1(float x) {
  float m = fabsf(x);
  int c = m <= 0.25f ? 0 : m < 0.75f ? 1 : m <= 1.25f ? 2 : m < 1.75f ? 3 : m <= 2.5f ? 4 : m < 3.5f ? 5 : m <= 5.0f ? 6 : 7;
  return (uint8_t)(c | ((f2u(x) >> 31) << 3));
}

/* ---- E8M0 (P/_triton_mx_lora.py:30-37) -------------------------------- */
static inline float e8m0_to_f32(uint8_t c) {
  if (c == 255) return NAN;
  if (c == 0) return u2f(0x00400000u); /* 2^-127, an fp32 subnormal */
  return u2f((uint32_t)c << 23);
}

/* ------------------------------------------------------------------ */
/* Philox4x32 (Random123; triton/language/random.py philox_impl)         */
/* ------------------------------------------------------------------ */
static void philox4x32(uint32_t c[4], uint32_t k0, uint32_t k1, int rounds) {
  for (int r = 0; r < rounds; ++r) {
    uint32_t c0 = c[0], c2 = c[2];
    uint64_t pb = (uint64_t)0xCD9E8D57u * c2, pa = (uint64_t)0xD2511F53u * c0;
    c[0] = (uint32_t)(pb >> 32) ^ c[1] ^ k0;
    c[2] = (uint32_t)(pa >> 32) ^ c[3] ^ k1;
    c[1] = (uint32_t)pb;
    c[3] = (uint32_t)pa;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}
EXPORT void lmo_philox4x32(const uint32_t* ctr, uint32_t k0, uint32_t k1, int rounds, uint32_t* out) {
  uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
  philox4x32(c, k0, k1, rounds);
  memcpy(out, c, 16);
}

/* Rounds of the SR_PHILOX8 stream: Random123's Philox4x32-7 (published
 * known answers in tests/golden/kat.json; the HIP kernels' SR_ROUNDS). */
#define SR_PHILOX_ROUNDS 7
EXPORT int lmo_sr_rounds(void) { return SR_PHILOX_ROUNDS; }

/* 16-bit Philox draw h of the element at offset idx (SR_PHILOX8 layout):
 * word k = (idx & 7) >> 1 of Philox4x32-7(counter idx >> 3, key seed),
 * complemented for odd k (words 1 and 3); its high half for even idx, its
 * low half for odd idx. */
static inline uint32_t sr_h16(uint64_t seed, uint64_t idx) {
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  uint64_t g = idx >> 3;
  uint32_t c[4] = {(uint32_t)g, (uint32_t)(g >> 32), 0, 0};
  philox4x32(c, k0, k1, SR_PHILOX_ROUNDS);
  int j = (int)(idx & 7);
  uint32_t w = ((j >> 1) & 1) ? ~c[j >> 1] : c[j >> 1];
  return (j & 1) ? (w & 0xffffu) : (w >> 16);
}

/* Uniform for the element at logical offset idx.
 * SR_PHILOX8: one Philox call per 8 consecutive offsets, 16 bits each.
 * SR_TRITON : triton tl.rand(seed, idx) (uint_to_uniform_float of word 0). */
static inline float sr_uniform(int mode, uint64_t seed, uint64_t idx) {
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  if (mode == SR_TRITON) {
    uint32_t c[4] = {(uint32_t)idx, (uint32_t)(idx >> 32), 0, 0};
    philox4x32(c, k0, k1, 10);
    int32_t x = (int32_t)c[0];
    if (x < 0) x = -x - 1;
    return (float)x * (float)4.6566127342e-10;
  }
  return (float)sr_h16(seed, idx) * (1.0f / 65536.0f);
}
EXPORT void lmo_uniforms(int mode, uint64_t seed, uint64_t start, int64_t n, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = sr_uniform(mode, seed, start + (uint64_t)i);
}

/* ---- stochastic selections (P/_triton_stochastic_quantization.py) ---- */
/* :25-40 */
static inline int sr_int(float x, int det, float u, int qmin, int qmax) {
  int interior = (x > (float)qmin) && (x < (float)qmax);
  float safe = interior ? x : 0.0f;
  float lower = floorf(safe);
  float p = safe - lower;
  float rounded = lower + ((u < p) ? 1.0f : 0.0f);
  return (interior && p > 0.0f) ? (int)rounded : det;
}

/* Integer stochastic rounding (INT8, Q8_0) in the form the HIP kernels run on
 * gfx950's v_cvt_sr_f16_f32 (the selection rule of
 * P/_triton_stochastic_quantization.py:25-40, u < p):
 *   t = clamp(RN(v * rcp + (1536 + zp)), 1536 + qmin, 1536 + qmax)
 *   code = floor(t) - 1536 + [u < frac(t)],  u = (h >> 3) * 2^-13.
 * rcp = RN(1 / s).  t lies in [1024, 2048), where fp32 keeps 13 fraction bits,
 * so frac(t) is p = frac(v / s + zp) rounded to 13 bits and u is the draw
 * truncated to 13 bits.  Exact integers and clamped values keep their code.
 * The clamp is v_med3_f32's: a NaN t gives 1536 + qmin.  (The instruction's
 * rule, measured on MI355X over every 13-bit fraction and 13-bit random
 * field: round up iff (R >> 19) + frac * 2^13 >= 2^13; the kernels pass
 * R = (65535 - h) << 16, i.e. R >> 19 = 8191 - (h >> 3).) */
static inline int sr_int13(float v, float rcp, float zp, int qmin, int qmax, uint32_t h) {
  float lo = 1536.0f + (float)qmin, hi = 1536.0f + (float)qmax;
  float t = fmaf(v, rcp, 1536.0f + zp);
  t = isnan(t) ? lo : fminf(fmaxf(t, lo), hi);
  float fl = floorf(t);
  uint32_t frac13 = (uint32_t)((t - fl) * 8192.0f);
  return (int)fl - 1536 + (((h >> 3) < frac13) ? 1 : 0);
}
EXPORT void lmo_sr_int13(const float* v, const float* rcp, const float* zp, const uint32_t* h, int64_t n, int qmin,
                         int qmax, int32_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = sr_int13(v[i], rcp[i], zp[i], qmin, qmax, h[i]);
}
EXPORT void lmo_sr_h16(uint64_t seed, uint64_t start, int64_t n, uint32_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = sr_h16(seed, start + (uint64_t)i);
}
/* The up-probability p = (|x| - lo) / (hi - lo) of the 4- and 8-bit float
 * formats is exact in fp32 (the grid steps are powers of two).  It is used
 * truncated to W fraction bits, W = 23 - (target mantissa bits): 22 for e2m1,
 * 20 for e4m3, 21 for e5m2.  That is the precision of gfx950's stochastic
 * conversions (v_cvt_scalef32_sr_*), which the GPU kernels use; it changes p
 * only below 2^-W, i.e. in the formats' subnormal range. */
static inline float sr_trunc(float p, int w) { return ldexpf(floorf(ldexpf(p, w)), -w); }

/* :110-130 */
static inline uint8_t sr_e2m1(float v, uint8_t det, float u) {
  float mag = fabsf(v);
  int nc = det & 7;
  float nearest = kE2M1[nc];
  int rd = nearest > mag;
  int lo = rd ? nc - 1 : nc, hi = rd ? nc : nc + 1;
  float lov = kE2M1[lo & 7], hiv = kE2M1[hi & 7];
  float p = (hiv > lov) ? (mag - lov) / (hiv - lov) : 0.0f;
  int mc = (u < sr_trunc(p, 22)) ? hi : lo;
  int sign = (int)((f2u(v) >> 28) & 8);
  uint8_t chosen = (uint8_t)(mc | sign);
  int interior = (mag > 0.0f) && (mag < 6.0f) && (p > 0.0f);
  return interior ? chosen : det;
}
/* :133-177, returns the chosen 8-bit code */
static inline uint8_t sr_fp8(int fmt, float v, float u, float limit) {
  float mag = fabsf(v);
  uint8_t det = fp8_encode(fmt, mag);
  float detv = fp8_decode(fmt, det);
  int rd = detv > mag;
  uint8_t lo = rd ? (uint8_t)(det - 1) : det, hi = rd ? det : (uint8_t)(det + 1);
  float lov = fp8_decode(fmt, lo), hiv = fp8_decode(fmt, hi);
  float p = (hiv > lov) ? (mag - lov) / (hiv - lov) : 0.0f;
  uint8_t mb = (u < sr_trunc(p, fmt == DT_E4M3 ? 20 : 21)) ? hi : lo;
  uint8_t sign = (uint8_t)((f2u(v) >> 24) & 0x80);
  int interior = (mag < limit) && (p > 0.0f);
  return interior ? (uint8_t)(mb | sign) : (uint8_t)(det | sign);
}

/* ------------------------------------------------------------------ */
/* LoRA delta and dense merge                                           */
/* ------------------------------------------------------------------ */
/* B [M, r] row stride ldb, A [r, N] row stride lda, both in factor dtype fdt. */
static inline float lora_delta(const void* b, int64_t ldb, const void* a, int64_t lda, int fdt, int r, int64_t row,
                               int64_t col) {
  float acc = 0.0f;
  for (int k = 0; k < r; ++k) acc = fmaf(load_dt(fdt, b, row * ldb + k), load_dt(fdt, a, (int64_t)k * lda + col), acc);
  return acc;
}

/* merged = round_cd(fmaf(delta, strength, base)); keep_zero_update reproduces
 * the NVFP4 rule merged = (update == 0 ? base : ...) (P/_triton_nvfp4_lora.py:183-186).
 * base and out are bf16/fp16/fp32 arrays in dtype cd, [M, N] contiguous. */
EXPORT void lmo_merge_dense(const void* base, void* out, int cd, int64_t M, int64_t N, const void* b, int64_t ldb,
                            const void* a, int64_t lda, int fdt, int r, float strength, int keep_zero_update) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t j = 0; j < N; ++j) {
      float bv = load_dt(cd, base, i * N + j);
      float d = r > 0 ? lora_delta(b, ldb, a, lda, fdt, r, i, j) : 0.0f;
      float m;
      if (keep_zero_update && d * strength == 0.0f) m = bv;
      else m = round_dt(cd, fmaf(d, strength, bv));
      store_dt(cd, out, i * N + j, m);
    }
}

/* ------------------------------------------------------------------ */
/* INT8 (TorchAO Int8Tensor; P/_triton_int8_lora.py)                    */
/* ------------------------------------------------------------------ */
/* dequant: P/_triton_int8_lora.py:68-87.  group = elements per qparam
 * (N for per-row, M*N per-tensor, a divisor of N per-group). */
EXPORT void lmo_int8_dequant(const int8_t* q, const void* scale, int scale_dt, const int8_t* zp, int64_t M, int64_t N,
                             int64_t group, int cd, void* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t j = 0; j < N; ++j) {
      int64_t f = i * N + j, qi = f / group;
      float z = zp ? (float)zp[qi] : 0.0f;
      float base = round_dt(cd, (float)q[f] - z);
      base = round_dt(cd, base * load_dt(scale_dt, scale, qi));
      store_dt(cd, out, f, base);
    }
}

/* requant of a dense tensor (values in dtype cd): P/_triton_int8_lora.py:98-236 */
EXPORT void lmo_int8_requant(const void* dense, int cd, int64_t M, int64_t N, int64_t group, int scale_dt, int asymmetric,
                             int reduce_range, int sr_mode, uint64_t seed, int8_t* q_out, void* scale_out,
                             int8_t* zp_out) {
  int qmin = reduce_range ? -64 : -128, qmax = reduce_range ? 63 : 127;
  int64_t numel = M * N, nq = numel / group;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t g = 0; g < nq; ++g) {
    float mn = 0.0f, mx = 0.0f;
    for (int64_t f = g * group; f < (g + 1) * group; ++f) {
      float v = load_dt(cd, dense, f);
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
    mn = round_dt(cd, mn);
    mx = round_dt(cd, mx);
    float scale;
    if (asymmetric) {
      float range = round_dt(cd, mx - mn);
      scale = range / (float)(qmax - qmin);
    } else {
      scale = fmaxf(-mn, mx) / ((float)(qmax - qmin) / 2.0f);
    }
    scale = round_dt(cd, scale);
    scale = fmaxf(scale, 1.1920928955078125e-07f);
    scale = round_dt(cd, scale);
    int zp = 0;
    if (asymmetric) {
      float ratio = round_dt(cd, mn / scale);
      zp = qmin - (int)nearbyintf(ratio);
      zp = zp < qmin ? qmin : (zp > qmax ? qmax : zp);
    }
    store_dt(scale_dt, scale_out, g, scale);
    if (zp_out) zp_out[g] = (int8_t)zp;
    float s = load_dt(scale_dt, scale_out, g); /* quantize reads the stored qparam */
    float inv = round_dt(scale_dt, 1.0f / s);
    for (int64_t f = g * group; f < (g + 1) * group; ++f) {
      float v = load_dt(cd, dense, f);
      float scaled = round_dt(scale_dt, v * inv);
      int qv = isnan(scaled) ? 0 : (int)nearbyintf(scaled);
      qv += zp;
      if (sr_mode == SR_PHILOX8) {
        qv = sr_int13(v, 1.0f / s, (float)zp, qmin, qmax, sr_h16(seed, (uint64_t)f));
      } else if (sr_mode != SR_OFF) {
        float x = v / s + (float)zp;
        qv = sr_int(x, qv, sr_uniform(sr_mode, seed, (uint64_t)f), qmin, qmax);
      }
      q_out[f] = (int8_t)(qv < qmin ? qmin : (qv > qmax ? qmax : qv));
    }
  }
}

/* ------------------------------------------------------------------ */
/* Scaled FP8 (TorchAO Float8Tensor; P/_triton_float8_lora.py)          */
/* ------------------------------------------------------------------ */
/* dequant P/_triton_float8_lora.py:72-85; scale fp32 per group (N = per-row). */
EXPORT void lmo_fp8_dequant(const uint8_t* q, int fmt, const float* scale, int64_t M, int64_t N, int64_t group, int cd,
                            void* out) {
#pragma omp parallel for schedule(static)
  for (int64_t f = 0; f < M * N; ++f) store_dt(cd, out, f, round_dt(cd, fp8_decode(fmt, q[f]) * scale[f / group]));
}
/* requant: scale = round_cd(amax/limit), 0 -> 2^-23 (:249-271); quantize
 * dense/scale clamped to +-limit, optional SR, RNE cast (:275-308). */
EXPORT void lmo_fp8_requant(const void* dense, int cd, int64_t M, int64_t N, int64_t group, int fmt, int sr_mode,
                            uint64_t seed, uint8_t* q_out, float* scale_out) {
  float limit = fmt == DT_E4M3 ? 448.0f : 57344.0f;
  int64_t nq = (M * N) / group;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t g = 0; g < nq; ++g) {
    float amax = 0.0f;
    for (int64_t f = g * group; f < (g + 1) * group; ++f) amax = fmaxf(amax, fabsf(load_dt(cd, dense, f)));
    float scale = round_dt(cd, amax / limit);
    if (scale == 0.0f) scale = 1.1920928955078125e-07f;
    scale_out[g] = scale;
    for (int64_t f = g * group; f < (g + 1) * group; ++f) {
      float x = load_dt(cd, dense, f) / scale;
      x = fminf(fmaxf(x, -limit), limit);
      if (sr_mode != SR_OFF) q_out[f] = sr_fp8(fmt, x, sr_uniform(sr_mode, seed, (uint64_t)f), limit);
      else q_out[f] = fp8_encode(fmt, x);
    }
  }
}

/* ------------------------------------------------------------------ */
/* NVFP4 (TorchAO NVFP4Tensor; P/_triton_nvfp4_lora.py)                 */
/* ------------------------------------------------------------------ */
/* P/_triton_nvfp4_lora.py:88-104 */
EXPORT int64_t lmo_blocked_scale_offset(int64_t row, int64_t scale_col, int64_t scale_cols, int swizzled) {
  if (!swizzled) return row * scale_cols + scale_col;
  int64_t ncb = (scale_cols + 3) / 4;
  int64_t rb = row / 128, rib = row % 128, cb = scale_col / 4, cib = scale_col % 4;
  return (rb * ncb + cb) * 512 + (rib % 32) * 16 + (rib / 32) * 4 + cib;
}

/* dequant P/_triton_nvfp4_lora.py:133-163. pts = per-tensor scale or NULL. */
EXPORT void lmo_nvfp4_dequant(const uint8_t* q, const uint8_t* scale, const float* pts, int64_t M, int64_t N, int swizzled,
                              int cd, void* out) {
  int64_t sc = N / 16;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t j = 0; j < N; ++j) {
      uint8_t byte = q[i * (N / 2) + j / 2];
      uint8_t code = (j & 1) ? (byte >> 4) : (byte & 15);
      float bs = e4m3_to_f32(scale[lmo_blocked_scale_offset(i, j / 16, sc, swizzled)]);
      if (cd == DT_BF16) bs = bf16r(bs);
      if (pts) {
        bs = bs * pts[0];
        if (cd == DT_BF16) bs = bf16r(bs);
      }
      float base = e2m1_to_f32(code) * bs;
      if (cd == DT_BF16) base = bf16r(base);
      store_dt(cd, out, i * N + j, base);
    }
}

/* requant of merged dense (P/_triton_nvfp4_lora.py:251-367).
 * two_level: recompute g' = max(amax/2688, 2^-23) into *pts_out.
 * scale_out must be pre-zeroed by the caller for swizzled padding. */
EXPORT void lmo_nvfp4_requant(const void* dense, int cd, int64_t M, int64_t N, int swizzled, int two_level, int sr_mode,
                              uint64_t seed, uint8_t* q_out, uint8_t* scale_out, float* pts_out) {
  int64_t sc = N / 16;
  float g = 1.0f;
  if (two_level) {
    float amax = 0.0f;
    for (int64_t f = 0; f < M * N; ++f) amax = fmaxf(amax, fabsf(load_dt(cd, dense, f)));
    g = fmaxf(amax / 2688.0f, 1.1920928955078125e-07f);
    *pts_out = g;
  }
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t b = 0; b < sc; ++b) {
      float v[16], bmax = 0.0f;
      for (int t = 0; t < 16; ++t) {
        v[t] = load_dt(cd, dense, i * N + b * 16 + t);
        bmax = fmaxf(bmax, fabsf(v[t]));
      }
      float bscale = bmax / 6.0f;
      float fs = two_level ? bscale / g : bscale;
      fs = fminf(fmaxf(fs, 0.015625f), 448.0f);
      uint8_t sc8 = f32_to_e4m3(fs);
      fs = e4m3_to_f32(sc8);
      scale_out[lmo_blocked_scale_offset(i, b, sc, swizzled)] = sc8;
      float recip = two_level ? (1.0f / g) / fs : 0.0f;
      uint8_t codes[16];
      for (int t = 0; t < 16; ++t) {
        float nrm = two_level ? v[t] * recip : v[t] / fs;
        nrm = fminf(fmaxf(nrm, -6.0f), 6.0f);
        uint8_t c = f32_to_e2m1(nrm);
        if (sr_mode != SR_OFF) c = sr_e2m1(nrm, c, sr_uniform(sr_mode, seed, (uint64_t)(i * N + b * 16 + t)));
        codes[t] = c;
      }
      for (int t = 0; t < 8; ++t) q_out[i * (N / 2) + b * 8 + t] = (uint8_t)(codes[2 * t] | (codes[2 * t + 1] << 4));
    }
}

/* ------------------------------------------------------------------ */
/* MX (TorchAO MXTensor; P/_triton_mx_lora.py)                          */
/* ------------------------------------------------------------------ */
static void mx_params(int fmt, int* emax, float* maxpos, int* mbits) {
  if (fmt == DT_E4M3) { *emax = 8; *maxpos = 448.0f; *mbits = 3; }
  else if (fmt == DT_E5M2) { *emax = 15; *maxpos = 57344.0f; *mbits = 2; }
  else { *emax = 2; *maxpos = 6.0f; *mbits = 1; }
}
/* P/_triton_mx_lora.py:97-112 (scale tile 128 rows x 4 scale columns) */
static inline int64_t mx_scale_offset(int64_t row, int64_t blk, int64_t nblk, int swizzled) {
  return lmo_blocked_scale_offset(row, blk, nblk, swizzled);
}
/* exact ceil(log2(x)) for finite x > 0 */
static int ceil_log2_exact(float x) {
  int e;
  float m = frexpf(x, &e); /* x = m * 2^e, m in [0.5, 1) */
  return (m == 0.5f) ? e - 1 : e;
}
/* P/_triton_mx_lora.py:115-159; returns code, writes inverse scale */
static uint8_t mx_scale(float max_abs, int mode, int emax, float maxpos, int mbits, float* inv) {
  if (mode == MX_RCEIL) {
    float descale = max_abs / maxpos;
    float unb;
    if (isnan(descale)) { *inv = NAN; return 255; }
    if (descale == 0.0f) unb = -127.0f;
    else if (isinf(descale)) unb = 127.0f;
    else unb = (float)ceil_log2_exact(descale);
    unb = fminf(fmaxf(unb, -127.0f), 127.0f);
    uint8_t enc = (uint8_t)(unb + 127.0f);
    *inv = enc == 0 ? 1.0f : ldexpf(1.0f, -(int)unb);
    return enc;
  }
  uint32_t bits = f2u(max_abs);
  if (mode == MX_EVEN) {
    uint32_t bias = mbits == 3 ? 524288u : (mbits == 2 ? 1048576u : 2097152u);
    bits = (bits + bias) & 0xff800000u;
  }
  int ex = (int)((bits >> 23) & 255) - 127;
  if (mode == MX_CEIL) ex += (bits & 0x7fffffu) > 0;
  int unb = ex - emax;
  unb = unb < -127 ? -127 : (unb > 128 ? 128 : unb);
  uint8_t enc = (uint8_t)(unb + 127);
  if (isnan(max_abs)) enc = 255;
  float scale = u2f((uint32_t)enc << 23);
  scale = fmaxf(scale, 1.1754943508222875e-38f);
  *inv = 1.0f / scale;
  return enc;
}
/* dequant P/_triton_mx_lora.py:209-242 */
EXPORT void lmo_mx_dequant(const uint8_t* q, const uint8_t* scale, int fmt, int64_t M, int64_t N, int swizzled, int cd,
                           void* out) {
  int64_t nblk = N / 32;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t j = 0; j < N; ++j) {
      float lp;
      if (fmt == DT_E2M1) {
        uint8_t byte = q[i * (N / 2) + j / 2];
        lp = e2m1_to_f32((j & 1) ? (byte >> 4) : (byte & 15));
      } else {
        lp = fp8_decode(fmt, q[i * N + j]);
      }
      float s = e8m0_to_f32(scale[mx_scale_offset(i, j / 32, nblk, swizzled)]);
      float base = (cd == DT_BF16) ? bf16r(bf16r(lp) * bf16r(s)) : lp * s;
      store_dt(cd, out, i * N + j, base);
    }
}
/* requant P/_triton_mx_lora.py:248-295 (writes qdata + scale). */
EXPORT void lmo_mx_requant(const void* dense, int cd, int64_t M, int64_t N, int fmt, int mode, int swizzled, int sr_mode,
                           uint64_t seed, uint8_t* q_out, uint8_t* scale_out) {
  int emax, mbits;
  float maxpos;
  mx_params(fmt, &emax, &maxpos, &mbits);
  int64_t nblk = N / 32;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t b = 0; b < nblk; ++b) {
      float v[32], amax = 0.0f;
      for (int t = 0; t < 32; ++t) {
        v[t] = load_dt(cd, dense, i * N + b * 32 + t);
        amax = fmaxf(amax, fabsf(v[t]));
      }
      float inv;
      uint8_t enc = mx_scale(amax, mode, emax, maxpos, mbits, &inv);
      scale_out[mx_scale_offset(i, b, nblk, swizzled)] = enc;
      uint8_t codes[32];
      for (int t = 0; t < 32; ++t) {
        float nrm = v[t] * inv;
        nrm = fminf(fmaxf(nrm, -maxpos), maxpos);
        uint64_t idx = (uint64_t)(i * N + b * 32 + t);
        if (fmt == DT_E2M1) {
          uint8_t c = f32_to_e2m1(nrm);
          if (sr_mode != SR_OFF) c = sr_e2m1(nrm, c, sr_uniform(sr_mode, seed, idx));
          codes[t] = c;
        } else {
          uint8_t c = (sr_mode != SR_OFF) ? sr_fp8(fmt, nrm, sr_uniform(sr_mode, seed, idx), maxpos) : fp8_encode(fmt, nrm);
          q_out[i * N + b * 32 + t] = c;
        }
      }
      if (fmt == DT_E2M1)
        for (int t = 0; t < 16; ++t) q_out[i * (N / 2) + b * 16 + t] = (uint8_t)(codes[2 * t] | (codes[2 * t + 1] << 4));
    }
}

/* ------------------------------------------------------------------ */
/* GGUF Q8_0                                                            */
/* ------------------------------------------------------------------ */
/* dequant: P/gguf_dequant.py:57-61 with dtype bf16: out = bf16(bf16(d) * q) */
EXPORT void lmo_q8_0_dequant(const uint8_t* packed, int64_t M, int64_t N, int cd, void* out) {
  int64_t nb = N / 32, rowbytes = nb * 34;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = packed + i * rowbytes + b * 34;
      uint16_t dh;
      memcpy(&dh, blk, 2);
      float d = round_dt(cd, f16_to_f32(dh));
      for (int t = 0; t < 32; ++t) store_dt(cd, out, i * N + b * 32 + t, round_dt(cd, d * (float)(int8_t)blk[2 + t]));
    }
}
/* requant: ggml quantize_row_q8_0_ref (MIT): d = amax/127, id = d ? 1/d : 0,
 * q = roundf(x*id) (half away from zero), store fp16(d). SR (an extension: the
 * reference routes GGUF only) is the integer rule sr_int13 with rcp = id. */
EXPORT void lmo_q8_0_requant(const void* dense, int cd, int64_t M, int64_t N, int sr_mode, uint64_t seed,
                             uint8_t* packed_out) {
  int64_t nb = N / 32, rowbytes = nb * 34;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t b = 0; b < nb; ++b) {
      float v[32], amax = 0.0f;
      for (int t = 0; t < 32; ++t) {
        v[t] = load_dt(cd, dense, i * N + b * 32 + t);
        amax = fmaxf(amax, fabsf(v[t]));
      }
      float d = amax / 127.0f;
      float id = d != 0.0f ? 1.0f / d : 0.0f;
      uint8_t* blk = packed_out + i * rowbytes + b * 34;
      uint16_t dh = f16_bits(d);
      memcpy(blk, &dh, 2);
      for (int t = 0; t < 32; ++t) {
        float x = v[t] * id;
        int qv = (int)roundf(x);
        if (sr_mode == SR_PHILOX8) qv = sr_int13(v[t], id, 0.0f, -127, 127, sr_h16(seed, (uint64_t)(i * N + b * 32 + t)));
        else if (sr_mode != SR_OFF)
          qv = sr_int(x, qv, sr_uniform(sr_mode, seed, (uint64_t)(i * N + b * 32 + t)), -127, 127);
        blk[2 + t] = (uint8_t)(int8_t)qv;
      }
    }
}

/* ------------------------------------------------------------------ */
/* small codec entry points (for exhaustive tests)                      */
/* ------------------------------------------------------------------ */
/* ------------------------------------------------------------------ */
/* GGUF dequantize, every type P/gguf_dequant.py:278-294 dispatches      */
/* ------------------------------------------------------------------ */
/* The reference evaluates each type as a short sequence of torch ops in the
 * output dtype `dt` (P/gguf_dequant.py:303-331): every op computes in fp32
 * and rounds to `dt` (round_dt), fp16 block scales are first converted to
 * `dt`, and integer codes are exact in every dt.  Byte offsets are the ggml
 * block structs (block_q4_0 ... block_iq4_xs); the element order is the one
 * the reference's reshapes produce, cited per type. */
enum {
  GG_F32 = 0, GG_F16 = 1, GG_Q4_0 = 2, GG_Q4_1 = 3, GG_Q5_0 = 6, GG_Q5_1 = 7, GG_Q8_0 = 8, GG_Q2_K = 10,
  GG_Q3_K = 11, GG_Q4_K = 12, GG_Q5_K = 13, GG_Q6_K = 14, GG_IQ4_NL = 20, GG_IQ4_XS = 23, GG_BF16 = 30
};
static const int8_t kIQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

static inline float gg_f16(const uint8_t* p) { return f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* P/gguf_dequant.py:44-49 (_get_scale_min): 6-bit scale and min of sub-block j */
static void gg_scale_min(const uint8_t* s, int j, int* sc, int* mn) {
  if (j < 4) {
    *sc = s[j] & 0x3F;
    *mn = s[4 + j] & 0x3F;
  } else {
    *sc = (s[8 + j - 4] & 0x0F) | ((s[j - 4] >> 2) & 0x30);
    *mn = (s[8 + j - 4] >> 4) | ((s[4 + j - 4] >> 2) & 0x30);
  }
}

/* block size and bytes per block (ggml GGML_QUANT_SIZES); 0 if unsupported */
EXPORT int lmo_gguf_sizes(int type, int* block, int* bytes) {
  int b = 0, t = 0;
  switch (type) {
    case GG_F32: b = 1; t = 4; break;
    case GG_F16: b = 1; t = 2; break;
    case GG_BF16: b = 1; t = 2; break;
    case GG_Q4_0: b = 32; t = 18; break;
    case GG_Q4_1: b = 32; t = 20; break;
    case GG_Q5_0: b = 32; t = 22; break;
    case GG_Q5_1: b = 32; t = 24; break;
    case GG_Q8_0: b = 32; t = 34; break;
    case GG_IQ4_NL: b = 32; t = 18; break;
    case GG_Q2_K: b = 256; t = 84; break;
    case GG_Q3_K: b = 256; t = 110; break;
    case GG_Q4_K: b = 256; t = 144; break;
    case GG_Q5_K: b = 256; t = 176; break;
    case GG_Q6_K: b = 256; t = 210; break;
    case GG_IQ4_XS: b = 256; t = 136; break;
    default: return 0;
  }
  if (block) *block = b;
  if (bytes) *bytes = t;
  return 1;
}

static void gg_block(int type, const uint8_t* b, int dt, float* y) {
  switch (type) {
    case GG_F32: { /* :222-223, then .to(dtype) at :328-330 */
      float v;
      memcpy(&v, b, 4);
      y[0] = round_dt(dt, v);
      break;
    }
    case GG_F16: y[0] = round_dt(dt, gg_f16(b)); break;                               /* :218-219 */
    case GG_BF16: y[0] = round_dt(dt, bf16_to_f32((uint16_t)(b[0] | (b[1] << 8)))); break; /* :214-215 */
    case GG_Q8_0: { /* :57-61 */
      const float d = round_dt(dt, gg_f16(b));
      for (int e = 0; e < 32; ++e) y[e] = round_dt(dt, d * (float)(int8_t)b[2 + e]);
      break;
    }
    case GG_Q4_0:   /* :107-115: element e < 16 is the low nibble of qs[e], e >= 16 the high nibble of qs[e-16] */
    case GG_IQ4_NL: { /* :226-242: the same nibbles index the IQ4_NL table */
      const float d = round_dt(dt, gg_f16(b));
      for (int e = 0; e < 32; ++e) {
        const int nib = (b[2 + (e & 15)] >> (e < 16 ? 0 : 4)) & 15;
        y[e] = round_dt(dt, d * (float)(type == GG_Q4_0 ? nib - 8 : kIQ4NL[nib]));
      }
      break;
    }
    case GG_Q4_1: { /* :95-104: (d * q) + m */
      const float d = round_dt(dt, gg_f16(b)), m = round_dt(dt, gg_f16(b + 2));
      for (int e = 0; e < 32; ++e) {
        const int nib = (b[4 + (e & 15)] >> (e < 16 ? 0 : 4)) & 15;
        y[e] = round_dt(dt, round_dt(dt, d * (float)nib) + m);
      }
      break;
    }
    case GG_Q5_0:   /* :80-92: bit e of the little-endian qh word is bit 4 of element e; q - 16 */
    case GG_Q5_1: { /* :64-77: (d * q) + m */
      const int q1 = type == GG_Q5_1;
      const float d = round_dt(dt, gg_f16(b)), m = q1 ? round_dt(dt, gg_f16(b + 2)) : 0.0f;
      const uint8_t* qhp = b + (q1 ? 4 : 2);
      const uint8_t* qs = b + (q1 ? 8 : 6);
      const uint32_t qh = (uint32_t)qhp[0] | ((uint32_t)qhp[1] << 8) | ((uint32_t)qhp[2] << 16) | ((uint32_t)qhp[3] << 24);
      for (int e = 0; e < 32; ++e) {
        const int q = ((qs[e & 15] >> (e < 16 ? 0 : 4)) & 15) | (int)(((qh >> e) & 1u) << 4);
        y[e] = q1 ? round_dt(dt, round_dt(dt, d * (float)q) + m) : round_dt(dt, d * (float)(q - 16));
      }
      break;
    }
    case GG_Q2_K: { /* :200-211: scales[16] | qs[64] | d | dmin; dl*q - ml per 16 elements */
      const float d = round_dt(dt, gg_f16(b + 80)), dmin = round_dt(dt, gg_f16(b + 82));
      for (int e = 0; e < 256; ++e) {
        const int sc = b[e >> 4];
        const float dl = round_dt(dt, d * (float)(sc & 15)), ml = round_dt(dt, dmin * (float)(sc >> 4));
        const int q = (b[16 + 32 * (e >> 7) + (e & 31)] >> (2 * ((e & 127) >> 5))) & 3;
        y[e] = round_dt(dt, round_dt(dt, dl * (float)q) - ml);
      }
      break;
    }
    case GG_Q3_K: { /* :172-197: hmask[32] | qs[64] | scales[12] | d */
      const float d = round_dt(dt, gg_f16(b + 108));
      const uint8_t *hm = b, *qs = b + 32, *sc = b + 96;
      for (int e = 0; e < 256; ++e) {
        const int i = e >> 4;
        const int lo = i < 8 ? (sc[i] & 15) : (sc[i - 8] >> 4);
        const int hi = (sc[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
        const float dl = round_dt(dt, d * (float)((lo | (hi << 4)) - 32));
        const int ql = (qs[32 * (e >> 7) + (e & 31)] >> (2 * ((e & 127) >> 5))) & 3;
        const int hbit = (hm[e & 31] >> (e >> 5)) & 1;
        y[e] = round_dt(dt, dl * (float)(ql - (hbit ? 0 : 4)));
      }
      break;
    }
    case GG_Q4_K:   /* :157-169: d | dmin | scales[12] | qs[128] */
    case GG_Q5_K: { /* :137-154: d | dmin | scales[12] | qh[32] | qs[128] */
      const int q5 = type == GG_Q5_K;
      const float d = round_dt(dt, gg_f16(b)), dmin = round_dt(dt, gg_f16(b + 2));
      const uint8_t* qh = b + 16;
      const uint8_t* qs = b + (q5 ? 48 : 16);
      for (int e = 0; e < 256; ++e) {
        const int j = e >> 5;
        int sc, mn;
        gg_scale_min(b + 4, j, &sc, &mn);
        const float ds = round_dt(dt, d * (float)sc), dm = round_dt(dt, dmin * (float)mn);
        int q = (qs[32 * (j >> 1) + (e & 31)] >> (4 * (j & 1))) & 15;
        if (q5) q |= ((qh[e & 31] >> j) & 1) << 4;
        y[e] = round_dt(dt, round_dt(dt, ds * (float)q) - dm);
      }
      break;
    }
    case GG_Q6_K: { /* :118-134: ql[128] | qh[64] | scales[16] (int8) | d */
      const float d = round_dt(dt, gg_f16(b + 208));
      for (int e = 0; e < 256; ++e) {
        const int h = e >> 7, r = e & 127;
        const float ds = round_dt(dt, d * (float)(int8_t)b[192 + (e >> 4)]);
        const int lo = (b[64 * h + (r & 63)] >> (4 * (r >> 6))) & 15;
        const int hi = (b[128 + 32 * h + (r & 31)] >> (2 * (r >> 5))) & 3;
        y[e] = round_dt(dt, ds * (float)((lo | (hi << 4)) - 32));
      }
      break;
    }
    case GG_IQ4_XS: { /* :245-274: d | scales_h (u16) | scales_l[4] | qs[128] */
      const float d = round_dt(dt, gg_f16(b));
      const int sh = b[2] | (b[3] << 8);
      for (int e = 0; e < 256; ++e) {
        const int j = e >> 5, p = e & 31;
        const int ls = (((b[4 + (j >> 1)] >> (4 * (j & 1))) & 15) | (((sh >> (2 * j)) & 3) << 4)) - 32;
        const float dl = round_dt(dt, d * (float)ls);
        const int nib = (b[8 + 16 * j + (p & 15)] >> (p < 16 ? 0 : 4)) & 15;
        y[e] = round_dt(dt, dl * (float)kIQ4NL[nib]);
      }
      break;
    }
  }
}

/* P/gguf_dequant.py:303-331 over `nblocks` consecutive blocks; returns 0 for
 * a type the reference does not dispatch */
EXPORT int lmo_gguf_dequant(const uint8_t* packed, int type, int64_t nblocks, int dt, void* out) {
  int bs, ts;
  if (!lmo_gguf_sizes(type, &bs, &ts)) return 0;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < nblocks; ++i) {
    float y[256];
    gg_block(type, packed + i * ts, dt, y);
    for (int e = 0; e < bs; ++e) store_dt(dt, out, i * bs + e, y[e]);
  }
  return 1;
}

EXPORT void lmo_f32_to_bf16(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = bf16_bits(x[i]);
}
EXPORT void lmo_f32_to_f16(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f16_bits(x[i]);
}
EXPORT void lmo_f16_to_f32(const uint16_t* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(x[i]);
}
EXPORT void lmo_f32_to_fp8(int fmt, const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = fp8_encode(fmt, x[i]);
}
EXPORT void lmo_fp8_to_f32(int fmt, const uint8_t* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = fp8_decode(fmt, x[i]);
}
EXPORT void lmo_f32_to_e2m1(const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_e2m1(x[i]);
}
EXPORT void lmo_e8m0_to_f32(const uint8_t* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = e8m0_to_f32(x[i]);
}
EXPORT void lmo_mx_scale(const float* amax, int64_t n, int fmt, int mode, uint8_t* codes, float* inv) {
  int emax, mbits;
  float maxpos;
  mx_params(fmt, &emax, &maxpos, &mbits);
  for (int64_t i = 0; i < n; ++i) codes[i] = mx_scale(amax[i], mode, emax, maxpos, mbits, &inv[i]);
}
EXPORT void lmo_sr_int(const float* x, const int32_t* det, const float* u, int64_t n, int qmin, int qmax, int32_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = sr_int(x[i], det[i], u[i], qmin, qmax);
}
EXPORT void lmo_sr_e2m1(const float* x, const uint8_t* det, const float* u, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = sr_e2m1(x[i], det[i], u[i]);
}
EXPORT void lmo_sr_fp8(int fmt, const float* x, const float* u, int64_t n, float limit, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = sr_fp8(fmt, x[i], u[i], limit);
}
EXPORT int lmo_version(void) { return 1; }

/* ------------------------------------------------------------------ */
/* Routed LoRA residual (P/lora.py:801-829, _routed_residual)           */
/* ------------------------------------------------------------------ */
/* out = dt(y + total), total = part_0, dt(total + part_i) for i > 0 in order,
 *   part_i = dt(dt(dt(dt(x A_i^T) s_i) B_i^T)), + dt(bias_i s_i) then dt when
 *   a bias is present,
 * the reference's torch expression ((x @ a.T) * s) @ b.T (+ bias * s) with
 * every op's result in the output dtype dt (bf16/fp16) and each matmul an
 * fp32 sum in ascending k (fmaf per term).  x [T, K], y/out [T, N],
 * a_i [r_i, K], b_i [N, r_i], bias_i [N] or NULL, all in dt. */
EXPORT void lmo_routed_residual(const void* x, const void* y, void* out, int64_t T, int64_t K, int64_t N, int dt,
                                int nf, const void* const* a, const void* const* b, const void* const* bias,
                                const float* s, const int32_t* rank) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    float* total = (float*)malloc(sizeof(float) * (size_t)N);
    float ps[64];
    for (int i = 0; i < nf; ++i) {
      for (int r = 0; r < rank[i]; ++r) {
        float acc = 0.0f;
        for (int64_t k = 0; k < K; ++k) acc = fmaf(load_dt(dt, x, t * K + k), load_dt(dt, a[i], (int64_t)r * K + k), acc);
        ps[r] = round_dt(dt, round_dt(dt, acc) * s[i]);
      }
      for (int64_t n = 0; n < N; ++n) {
        float acc = 0.0f;
        for (int r = 0; r < rank[i]; ++r) acc = fmaf(ps[r], load_dt(dt, b[i], n * rank[i] + r), acc);
        float part = round_dt(dt, acc);
        if (bias[i]) part = round_dt(dt, part + round_dt(dt, load_dt(dt, bias[i], n) * s[i]));
        total[n] = i == 0 ? part : round_dt(dt, total[n] + part);
      }
    }
    for (int64_t n = 0; n < N; ++n) store_dt(dt, out, t * N + n, round_dt(dt, load_dt(dt, y, t * N + n) + total[n]));
    free(total);
  }
}
