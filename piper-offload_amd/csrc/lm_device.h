// lm_device.h -- gfx950 device building blocks for the LoRA-merge kernels.
//
// Numerics follow the reference's fused Triton path (P/ = the reference's
// src/piper_offload/):
//   * bf16 rounding uses v_cvt_pk_bf16_f32 (RNE);
//   * fp8 e4m3fn / e5m2 encodes use v_cvt_pk_{fp8,bf8}_f32 (RNE, the values
//     are clamped to the finite range first, P/_triton_float8_lora.py:295-299);
//   * e2m1 encodes use v_cvt_scalef32_pk_fp4_f32 with scale 1.0, which is
//     round-to-nearest-even and therefore identical to the threshold chain of
//     P/_triton_nvfp4_lora.py:55-85;
//   * the per-element quotient v / s (FP8 and single-level NVFP4
//     quantization) is the IEEE-correct quotient computed as q0 = v*r,
//     e = fma(q0, s, -v), q1 = fma(-e, r, q0) with r = RN(1/s); this equals
//     RN(v/s), the sign of a zero included, for all bf16 and fp16 operands
//     whose magnitudes and quotient lie in [2^-100, 2^100] and for v = +-0
//     (exhaustively checked on the CPU: tests/arith/identities.c).  The
//     residual is taken negated so that v = -0 gives e = +0 and q1 =
//     -0 * r + -0 = -0; the form with e = fma(-q0, s, v) loses that sign.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DEV __device__ __forceinline__
// global (HBM) address space: global_load/store with immediate offsets.
// Vector accesses through it use clang vector types (HIP's uint2/uint4
// classes cannot be copied from another address space).
#define LM_GLOBAL __attribute__((address_space(1)))
typedef uint32_t lm_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t lm_u32x4 __attribute__((ext_vector_type(4)));

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef _Float16 v4f16 __attribute__((ext_vector_type(4)));
typedef float v4f32 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));
typedef _Float16 v8f16 __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf16 __attribute__((ext_vector_type(8)));

namespace lm {

enum : int { F32 = 0, BF16 = 1, F16 = 2, E4M3 = 3, E5M2 = 4, E2M1 = 5, E8M0 = 6 };
enum : int { MX_FLOOR = 0, MX_RCEIL = 1, MX_CEIL = 2, MX_EVEN = 3 };

constexpr float kEps = 1.1920928955078125e-07f;  // torch.finfo(float32).eps

DEV uint32_t f2u(float x) { return __float_as_uint(x); }
DEV float u2f(uint32_t x) { return __uint_as_float(x); }

typedef float v2f32 __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf16 __attribute__((ext_vector_type(2)));

DEV uint16_t bf16_bits(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
DEV float bf16_val(uint32_t h) { return u2f(h << 16); }
// RNE bf16 of (a, b) packed low/high: one v_cvt_pk_bf16_f32
DEV uint32_t pack_bf16x2(float a, float b) {
  const v2f32 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2bf16));
}
// bf16-rounded x as an fp32 value: v_cvt_pk_bf16_f32 with x in the high half
DEV float bf16r(float x) { return u2f(pack_bf16x2(0.0f, x)); }
DEV uint16_t f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
DEV float f16_val(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
DEV float f16r(float x) { return f16_val(f16_bits(x)); }

// ---- cross-lane reductions, VALU only (no LDS crossbar) -------------------
// All 64 lanes must be active.  Within a 16-lane row: DPP (quad_perm xor 1,
// xor 2; row_half_mirror; row_mirror).  Across rows: the gfx950 lane swaps.
// v_permlane16_swap(x, x) returns x with odd rows exchanged for even rows in
// one output and the other way round in the second, so one of the two
// outputs holds x[l] and the other x[l ^ 16]; v_permlane32_swap likewise
// for l ^ 32.
DEV float lanes_max16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(f2u(x), f2u(x), false, false);
  return __builtin_fmaxf(u2f(r[0]), u2f(r[1]));
}
DEV float lanes_min16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(f2u(x), f2u(x), false, false);
  return __builtin_fminf(u2f(r[0]), u2f(r[1]));
}
DEV float lanes_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(f2u(x), f2u(x), false, false);
  return __builtin_fmaxf(u2f(r[0]), u2f(r[1]));
}
DEV float lanes_min32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(f2u(x), f2u(x), false, false);
  return __builtin_fminf(u2f(r[0]), u2f(r[1]));
}
template <int CTRL>
DEV float dpp_f32(float x) {
  return u2f((uint32_t)__builtin_amdgcn_update_dpp((int)f2u(x), (int)f2u(x), CTRL, 0xf, 0xf, false));
}
// max over all 64 lanes: after xor 1 and xor 2 a quad is uniform, so the
// half-row mirror (lane i <-> 7 - i) pairs quad 0 with quad 1 and the row
// mirror (i <-> 15 - i) pairs the two halves
DEV float row_max16(float x) {  // max over each 16-lane row
  x = __builtin_fmaxf(x, dpp_f32<0xB1>(x));   // quad_perm [1, 0, 3, 2]
  x = __builtin_fmaxf(x, dpp_f32<0x4E>(x));   // quad_perm [2, 3, 0, 1]
  x = __builtin_fmaxf(x, dpp_f32<0x141>(x));  // row_half_mirror
  return __builtin_fmaxf(x, dpp_f32<0x140>(x));  // row_mirror
}
DEV float wave_max(float x) { return lanes_max32(lanes_max16(row_max16(x))); }

template <int DT>
DEV float round_dt(float x) {
  if constexpr (DT == BF16) return bf16r(x);
  else if constexpr (DT == F16) return f16r(x);
  else return x;
}
template <int DT>
DEV uint16_t bits_dt(float x) {
  if constexpr (DT == F16) return f16_bits(x);
  else return bf16_bits(x);
}
template <int DT>
DEV float val_dt(uint32_t h) {
  if constexpr (DT == F16) return f16_val(h);
  else return bf16_val(h);
}
// load one element of a runtime-dtype scalar array (f32 / bf16 / f16)
DEV float load_scalar(const void* p, int64_t i, int dt) {
  if (dt == BF16) return bf16_val(((const uint16_t*)p)[i]);
  if (dt == F16) return f16_val(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}
DEV void store_scalar(void* p, int64_t i, int dt, float v) {
  if (dt == BF16) ((uint16_t*)p)[i] = bf16_bits(v);
  else if (dt == F16) ((uint16_t*)p)[i] = f16_bits(v);
  else ((float*)p)[i] = v;
}
DEV float round_runtime(float x, int dt) {
  if (dt == BF16) return bf16r(x);
  if (dt == F16) return f16r(x);
  return x;
}

// RN(v / s) given r = RN(1/s); see header comment for the validity domain.
DEV float div_rn(float v, float s, float r) {
  const float q0 = v * r;
  const float e = __builtin_fmaf(q0, s, -v);  // -(v - q0 s), exact
  return __builtin_fmaf(-e, r, q0);
}

// A 16-byte global store whose data registers stay unwritten for two wait
// states after it.  On gfx950 a VALU write to a data register of a 16-byte
// store in the very next instruction corrupts what the store writes (the
// last lanes of each row of 16), and the compiler does not pad it; the
// s_nop takes the data registers as inputs, so nothing can overwrite them
// before it.
DEV void store_b128_guarded(LM_GLOBAL lm_u32x4* p, lm_u32x4 v) {
  *p = v;
  asm volatile("s_nop 1" ::"v"(v) : "memory");
}

// ---- 8-bit floats -----------------------------------------------------
template <int FMT>
DEV float fp8_decode(uint32_t word, int byte) {
  if constexpr (FMT == E4M3) {
    switch (byte) {
      case 0: return __builtin_amdgcn_cvt_f32_fp8(word, 0);
      case 1: return __builtin_amdgcn_cvt_f32_fp8(word, 1);
      case 2: return __builtin_amdgcn_cvt_f32_fp8(word, 2);
      default: return __builtin_amdgcn_cvt_f32_fp8(word, 3);
    }
  } else {
    switch (byte) {
      case 0: return __builtin_amdgcn_cvt_f32_bf8(word, 0);
      case 1: return __builtin_amdgcn_cvt_f32_bf8(word, 1);
      case 2: return __builtin_amdgcn_cvt_f32_bf8(word, 2);
      default: return __builtin_amdgcn_cvt_f32_bf8(word, 3);
    }
  }
}
// bytes 2 HI and 2 HI + 1 of a word as fp32, in one v_cvt_pk_f32_fp8 / _bf8
// (the same exact conversion as fp8_decode)
template <int FMT, bool HI>
DEV v2f32 fp8_decode_pair(uint32_t word) {
  if constexpr (FMT == E4M3) return __builtin_amdgcn_cvt_pk_f32_fp8(word, HI);
  else return __builtin_amdgcn_cvt_pk_f32_bf8(word, HI);
}
// pack 4 values (already clamped to the finite range) to 4 fp8 codes, RNE
template <int FMT>
DEV uint32_t fp8_pack4(float a, float b, float c, float d) {
  if constexpr (FMT == E4M3) {
    uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  } else {
    uint32_t w = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
    return __builtin_amdgcn_cvt_pk_bf8_f32(c, d, w, true);
  }
}
template <int FMT>
DEV uint32_t fp8_encode1(float a) {
  if constexpr (FMT == E4M3) return __builtin_amdgcn_cvt_pk_fp8_f32(a, a, 0, false) & 0xffu;
  else return __builtin_amdgcn_cvt_pk_bf8_f32(a, a, 0, false) & 0xffu;
}
template <int FMT>
DEV float fp8_value(uint32_t code) {  // decode one code held in the low byte
  return fp8_decode<FMT>(code, 0);
}

// ---- e2m1 ---------------------------------------------------------------
DEV float e2m1_mag(uint32_t m) {  // m in 0..7 -> 0,0.5,1,1.5,2,3,4,6
  uint32_t bits = m == 0 ? 0u : (m == 1 ? 0x3f000000u : ((((m >> 1) + 126u) << 23) | ((m & 1u) << 22)));
  return u2f(bits);
}
DEV float e2m1_value(uint32_t code) {
  float v = e2m1_mag(code & 7u);
  return (code & 8u) ? -v : v;
}
// two values -> two e2m1 codes in the low byte (first value in the low nibble)
DEV uint32_t e2m1_pack2(float a, float b) {
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, a, b, 1.0f, 0) & 0xffu;
}

// ---- e8m0 (P/_triton_mx_lora.py:30-37) -------------------------------
DEV float e8m0_value(uint32_t c) {
  if (c == 255u) return __builtin_nanf("");
  if (c == 0u) return u2f(0x00400000u);
  return u2f(c << 23);
}

// ---- Philox4x32-7: the stochastic-rounding stream ----------------------
// Random123's Philox4x32 (the round function of
// triton.language.random.philox_impl) with 7 rounds, the smallest count its
// authors report free of TestU01 BigCrush failures (Salmon et al., SC'11,
// "Parallel random numbers: as easy as 1, 2, 3"); Random123 publishes
// known-answer vectors for it.  Triton's default is 10 rounds.
constexpr int SR_ROUNDS = 7;
DEV void philox_sr(uint64_t ctr, uint64_t seed, uint32_t (&c)[4]) {
  c[0] = (uint32_t)ctr;
  c[1] = (uint32_t)(ctr >> 32);
  c[2] = 0;
  c[3] = 0;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  // One round: both halves of each 32x32 product come from one v_mad_u64_u32
  // and each output word is one v_bitop3_b32 (0x96 = a ^ b ^ c).
#pragma unroll
  for (int r = 0; r < SR_ROUNDS; ++r) {
    const uint64_t pb = (uint64_t)c[2] * 0xCD9E8D57u;
    const uint64_t pa = (uint64_t)c[0] * 0xD2511F53u;
    c[0] = __builtin_amdgcn_bitop3_b32((uint32_t)(pb >> 32), c[1], k0, 0x96);
    c[2] = __builtin_amdgcn_bitop3_b32((uint32_t)(pa >> 32), c[3], k1, 0x96);
    c[1] = (uint32_t)pb;
    c[3] = (uint32_t)pa;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}
// philox_sr of the counter (lo, hi) with output words 0 and 2
// complemented: the last round's three-way XOR of those words becomes an
// XNOR (v_bitop3_b32 0x69), so the complement costs nothing.  The stochastic
// rounding rules below consume 65535 - h = ~h (16 bits), i.e. complemented
// words.
DEV void philox_sr_n02(uint32_t lo, uint32_t hi, uint64_t seed, uint32_t (&c)[4]) {
  c[0] = lo;
  c[1] = hi;
  c[2] = 0;
  c[3] = 0;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < SR_ROUNDS; ++r) {
    const uint64_t pb = (uint64_t)c[2] * 0xCD9E8D57u;
    const uint64_t pa = (uint64_t)c[0] * 0xD2511F53u;
    if (r == 0) {
      // c[2] = 0 makes the first word seed-only when the high counter word is
      // wave-uniform: plain C keeps it (and the next round's product with it)
      // on the scalar unit, where the builtin would move it to a VGPR
      c[0] = (uint32_t)(pb >> 32) ^ c[1] ^ k0;
      c[2] = __builtin_amdgcn_bitop3_b32((uint32_t)(pa >> 32), c[3], k1, 0x96);
    } else if (r < SR_ROUNDS - 1) {
      c[0] = __builtin_amdgcn_bitop3_b32((uint32_t)(pb >> 32), c[1], k0, 0x96);
      c[2] = __builtin_amdgcn_bitop3_b32((uint32_t)(pa >> 32), c[3], k1, 0x96);
    } else {
      c[0] = __builtin_amdgcn_bitop3_b32((uint32_t)(pb >> 32), c[1], k0, 0x69);
      c[2] = __builtin_amdgcn_bitop3_b32((uint32_t)(pa >> 32), c[3], k1, 0x69);
    }
    c[1] = (uint32_t)pb;
    c[3] = (uint32_t)pa;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}
// philox_sr_n02 of the counter (lo, 0): with the high word zero the first
// round's word 0 is the key itself, so round 2's A product and round 3's
// word 3 are wave-uniform.  Written out, the compiler keeps them (and their
// XOR with the round keys) on the scalar unit: three fewer VALU operations
// per call, and no per-call v_mul_hi_u32 / v_mul_lo_u32 of the seed.
DEV void philox_sr_n02_lo(uint32_t lo, uint64_t seed, uint32_t (&c)[4]) {
  constexpr uint32_t MA = 0xD2511F53u, MB = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  // round 1 of (lo, 0, 0, 0): the B product is 0
  uint64_t pa = (uint64_t)lo * MA;
  uint64_t pb;
  c[0] = k0;
  c[1] = 0u;
  c[2] = (uint32_t)(pa >> 32) ^ k1;
  c[3] = (uint32_t)pa;
  k0 += W0;
  k1 += W1;
  // round 2: c[0] and c[1] are uniform
  pb = (uint64_t)c[2] * MB;
  pa = (uint64_t)c[0] * MA;
  c[0] = (uint32_t)(pb >> 32) ^ k0;
  c[2] = c[3] ^ ((uint32_t)(pa >> 32) ^ k1);
  c[1] = (uint32_t)pb;
  c[3] = (uint32_t)pa;
  k0 += W0;
  k1 += W1;
  // round 3: c[3] is uniform
  pb = (uint64_t)c[2] * MB;
  pa = (uint64_t)c[0] * MA;
  c[0] = __builtin_amdgcn_bitop3_b32((uint32_t)(pb >> 32), c[1], k0, 0x96);
  c[2] = (uint32_t)(pa >> 32) ^ (c[3] ^ k1);
  c[1] = (uint32_t)pb;
  c[3] = (uint32_t)pa;
  k0 += W0;
  k1 += W1;
#pragma unroll
  for (int r = 3; r < SR_ROUNDS; ++r) {
    pb = (uint64_t)c[2] * MB;
    pa = (uint64_t)c[0] * MA;
    const int op = r < SR_ROUNDS - 1 ? 0x96 : 0x69;  // XNOR in the last round
    if (op == 0x96) {
      c[0] = __builtin_amdgcn_bitop3_b32((uint32_t)(pb >> 32), c[1], k0, 0x96);
      c[2] = __builtin_amdgcn_bitop3_b32((uint32_t)(pa >> 32), c[3], k1, 0x96);
    } else {
      c[0] = __builtin_amdgcn_bitop3_b32((uint32_t)(pb >> 32), c[1], k0, 0x69);
      c[2] = __builtin_amdgcn_bitop3_b32((uint32_t)(pa >> 32), c[3], k1, 0x69);
    }
    c[1] = (uint32_t)pb;
    c[3] = (uint32_t)pa;
    k0 += W0;
    k1 += W1;
  }
}
// The stream: element idx draws the 16-bit h from word k = (idx & 7) >> 1 of
// philox_sr(counter idx >> 3), complemented when k is odd (words 1 and 3):
// the high half for even idx, the low half for odd idx.  The rounding rules consume 65535 - h = ~h: words 0
// and 2 come out of philox_sr_n02 complemented, and the complements of
// words 1 and 3 are their raw values, so ~h costs no instruction.
// The 8 words ~h of the 16 offsets 8 ctr .. 8 ctr + 15 for an even 32-bit
// counter ctr (offsets below 2^35): the second block's counter is ctr | 1,
// and the high counter word is 0.
DEV void sr_nwords16_even(uint64_t seed, uint32_t ctr, uint32_t (&nw)[8]) {
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    uint32_t c[4];
    philox_sr_n02_lo(ctr | (uint32_t)gi, seed, c);
    nw[4 * gi + 0] = c[0];
    nw[4 * gi + 1] = c[1];
    nw[4 * gi + 2] = c[2];
    nw[4 * gi + 3] = c[3];
  }
}
// The SPAN/2 words ~h of offsets idx0 .. idx0+SPAN-1 when idx0 % SPAN == 0
// (SPAN a multiple of 8): the SPAN/8 counters are (idx0 >> 3) | gi with no
// carry.
template <int SPAN>
DEV void sr_nwords_aligned(uint64_t seed, uint64_t idx0, uint32_t (&nw)[SPAN / 2]) {
  const uint64_t ctr = idx0 >> 3;
  const uint32_t lo = (uint32_t)ctr, hi = (uint32_t)(ctr >> 32);
#pragma unroll
  for (int gi = 0; gi < SPAN / 8; ++gi) {
    uint32_t c[4];
    philox_sr_n02(lo | (uint32_t)gi, hi, seed, c);
    nw[4 * gi + 0] = c[0];
    nw[4 * gi + 1] = c[1];
    nw[4 * gi + 2] = c[2];
    nw[4 * gi + 3] = c[3];
  }
}
// the same for idx0 < 2^35, whose counters fit the low word
// (philox_sr_n02_lo); the fast block-format kernels require M N <= 2^35
template <int SPAN>
DEV void sr_nwords_aligned_lo(uint64_t seed, uint32_t ctr, uint32_t (&nw)[SPAN / 2]) {
#pragma unroll
  for (int gi = 0; gi < SPAN / 8; ++gi) {
    uint32_t c[4];
    philox_sr_n02_lo(ctr | (uint32_t)gi, seed, c);
    nw[4 * gi + 0] = c[0];
    nw[4 * gi + 1] = c[1];
    nw[4 * gi + 2] = c[2];
    nw[4 * gi + 3] = c[3];
  }
}
// 16-bit uniform integers h for offsets idx0 .. idx0+SPAN-1 (u = h * 2^-16)
DEV uint32_t sr_h_of(const uint32_t (&c)[4], int j) {
  const uint32_t w = ((j >> 1) & 1) ? ~c[j >> 1] : c[j >> 1];
  return (j & 1) ? (w & 0xffffu) : (w >> 16);
}
template <int SPAN>
DEV void sr_bits(uint64_t seed, uint64_t idx0, uint32_t (&h)[SPAN]) {
  if ((idx0 & 7u) == 0) {
#pragma unroll
    for (int gi = 0; gi < SPAN / 8; ++gi) {
      uint32_t c[4];
      philox_sr((idx0 >> 3) + gi, seed, c);
#pragma unroll
      for (int j = 0; j < 8; ++j) h[gi * 8 + j] = sr_h_of(c, j);
    }
  } else {
    for (int j = 0; j < SPAN; ++j) {
      uint64_t idx = idx0 + j;
      uint32_t c[4];
      philox_sr(idx >> 3, seed, c);
      h[j] = sr_h_of(c, (int)(idx & 7));
    }
  }
}
// u < p with u = h * 2^-16 (exact: both sides scaled by 2^16)

// ---- stochastic selections (P/_triton_stochastic_quantization.py) --------
// ---- stochastic 4- and 8-bit float conversions (gfx950 hardware) ----------
// v_cvt_scalef32_sr_{pk_fp4,fp8,bf8}_f32 (scale 1.0) round x onto the target
// grid with a 32-bit random operand R: with W = 23 - (target mantissa bits)
// (22 e2m1, 20 e4m3, 21 e5m2) and F = floor(p * 2^W), p = (|x| - lo) / (hi - lo)
// the position of |x| between its grid neighbours, x rounds away from zero iff
// (R >> (32 - W)) + F >= 2^W.  The second element of the fp4 pair uses R << 1.
// Beyond the range e2m1 saturates to +-6 and fp8 becomes NaN (callers clamp).
// (Measured on MI355X: every one of 5e5 random values x seeds, all binades,
// subnormals, signed zeros, saturation.)
// For a 16-bit draw h, R = ((65535 - h) << 16) | 0xffff makes the rule
//   up <=> F > h * 2^(W-16) <=> h * 2^-16 < trunc_W(p),
// the reference's u < p with p truncated to W fraction bits
// (P/_triton_stochastic_quantization.py:110-177).
// The builtin of the fp4 form does not tie its byte-select destination to the
// previous value, so the conversions are written as asm with a "+v" operand.
// nw = ~h of two elements: the even one in the high half, the odd one in
// the low half
DEV uint32_t sr_seed_hi(uint32_t nw) { return nw | 0xffffu; }          // the even element's R
DEV uint32_t sr_seed_lo(uint32_t nw) { return (nw << 16) | 0xffffu; }  // the odd element's R
// the odd element's R as the second operand of an fp4 pair conversion, which
// rounds it with R << 1: (nw << 15) | 0x7fff, one v_lshl_or_b32
DEV uint32_t sr_seed_lo_second(uint32_t nw) { return (nw << 15) | 0x7fffu; }
DEV uint32_t sr_seed(uint32_t h) { return ((65535u - h) << 16) | 0xffffu; }

// byte SEL of `old` := e2m1(a) | e2m1(b) << 4 (a with seed R, b with R << 1)
template <int SEL>
DEV uint32_t cvt_sr_fp4(uint32_t old, float a, float b, uint32_t seed) {
  const v2f32 v = {a, b};
  if constexpr (SEL == 0) asm("v_cvt_scalef32_sr_pk_fp4_f32 %0, %1, %2, 1.0" : "+v"(old) : "v"(v), "v"(seed));
  else if constexpr (SEL == 1)
    asm("v_cvt_scalef32_sr_pk_fp4_f32 %0, %1, %2, 1.0 op_sel:[0,0,1,0]" : "+v"(old) : "v"(v), "v"(seed));
  else if constexpr (SEL == 2)
    asm("v_cvt_scalef32_sr_pk_fp4_f32 %0, %1, %2, 1.0 op_sel:[0,0,0,1]" : "+v"(old) : "v"(v), "v"(seed));
  else asm("v_cvt_scalef32_sr_pk_fp4_f32 %0, %1, %2, 1.0 op_sel:[0,0,1,1]" : "+v"(old) : "v"(v), "v"(seed));
  return old;
}
// byte SEL of `old` := fp8 (FMT e4m3 or e5m2) of x with seed R
template <int FMT, int SEL>
DEV uint32_t cvt_sr_fp8(uint32_t old, float x, uint32_t seed) {
#define LM_SR8(OP, SELS) asm(OP " %0, %1, %2, 1.0" SELS : "+v"(old) : "v"(x), "v"(seed))
  if constexpr (FMT == E4M3) {
    if constexpr (SEL == 0) LM_SR8("v_cvt_scalef32_sr_fp8_f32", "");
    else if constexpr (SEL == 1) LM_SR8("v_cvt_scalef32_sr_fp8_f32", " op_sel:[0,0,1,0]");
    else if constexpr (SEL == 2) LM_SR8("v_cvt_scalef32_sr_fp8_f32", " op_sel:[0,0,0,1]");
    else LM_SR8("v_cvt_scalef32_sr_fp8_f32", " op_sel:[0,0,1,1]");
  } else {
    if constexpr (SEL == 0) LM_SR8("v_cvt_scalef32_sr_bf8_f32", "");
    else if constexpr (SEL == 1) LM_SR8("v_cvt_scalef32_sr_bf8_f32", " op_sel:[0,0,1,0]");
    else if constexpr (SEL == 2) LM_SR8("v_cvt_scalef32_sr_bf8_f32", " op_sel:[0,0,0,1]");
    else LM_SR8("v_cvt_scalef32_sr_bf8_f32", " op_sel:[0,0,1,1]");
  }
#undef LM_SR8
  return old;
}
// Eight e2m1 codes of x[0..7], element 2k drawn from the high half of nw[k]
// and 2k+1 from its low half.  Two conversions of the same pair (x[2k],
// x[2k+1]) give independent draws: `ev` rounds the first element with the
// even element's R and keeps the low nibbles; `od` passes the odd element's
// R shifted right by one, so that the instruction's R << 1 for the second
// element is that R, and keeps the high nibbles.
DEV uint32_t sr_e2m1_nword(const float* x, const uint32_t* nw) {
  // every byte of ev and od is written below: no initial value is needed
  uint32_t ev, od;
  asm("" : "=v"(ev), "=v"(od));
  ev = cvt_sr_fp4<0>(ev, x[0], x[1], sr_seed_hi(nw[0]));
  od = cvt_sr_fp4<0>(od, x[0], x[1], sr_seed_lo_second(nw[0]));
  ev = cvt_sr_fp4<1>(ev, x[2], x[3], sr_seed_hi(nw[1]));
  od = cvt_sr_fp4<1>(od, x[2], x[3], sr_seed_lo_second(nw[1]));
  ev = cvt_sr_fp4<2>(ev, x[4], x[5], sr_seed_hi(nw[2]));
  od = cvt_sr_fp4<2>(od, x[4], x[5], sr_seed_lo_second(nw[2]));
  ev = cvt_sr_fp4<3>(ev, x[6], x[7], sr_seed_hi(nw[3]));
  od = cvt_sr_fp4<3>(od, x[6], x[7], sr_seed_lo_second(nw[3]));
  return (ev & 0x0f0f0f0fu) | (od & 0xf0f0f0f0u);
}
// Four fp8 codes of x[0..3] (clamped by the caller), element 2k drawn from
// the high half of nw[k] and 2k + 1 from its low half
template <int FMT>
DEV uint32_t sr_fp8_nword(const float* x, const uint32_t* nw) {
  uint32_t r;  // every byte is written below
  asm("" : "=v"(r));
  const uint32_t n0 = nw[0], n1 = nw[1];
  r = cvt_sr_fp8<FMT, 0>(r, x[0], sr_seed_hi(n0));
  r = cvt_sr_fp8<FMT, 1>(r, x[1], sr_seed_lo(n0));
  r = cvt_sr_fp8<FMT, 2>(r, x[2], sr_seed_hi(n1));
  r = cvt_sr_fp8<FMT, 3>(r, x[3], sr_seed_lo(n1));
  return r;
}
// single elements (generic kernels): det is the RTN code, which the hardware
// reproduces for exact, zero, saturated and non-finite inputs
DEV uint32_t sr_e2m1(float v, uint32_t /*det*/, uint32_t h) { return cvt_sr_fp4<0>(0u, v, 0.0f, sr_seed(h)) & 15u; }
// v already clamped to +-limit by the caller
template <int FMT>
DEV uint32_t sr_fp8(float v, uint32_t h, float /*limit*/) { return cvt_sr_fp8<FMT, 0>(0u, v, sr_seed(h)) & 0xffu; }


// ---- packed helpers for the fast paths -----------------------------------
// Inline asm and the MFMA wait states.  gfx950 needs software wait states
// between an MFMA and a VALU instruction that reads or overwrites its
// destination, or overwrites its accumulator input, while it is in flight.
// The compiler pads only the instructions it emits itself, never inline asm.
// So every asm helper below (a) takes no MFMA result as an input (callers pass
// values of ordinary arithmetic) and (b) writes only a register tied to one
// of its inputs ("+v"): that register holds a live value the compiler itself
// produced, so it is never the destination or accumulator input of an MFMA
// in flight.  An untied output may be allocated over the accumulator input
// of an MFMA just issued, and an asm v_min3_f32 that read MFMA results saw
// stale registers depending on timing.  The compiled kernels are checked for
// both by csrc/check_asm_hazards.py (make check-asm).
//
// the wave's index in its workgroup, as a wave-uniform (scalar) value: from
// threadIdx.x alone the compiler treats it as per-lane, and every address
// derived from it (tile offsets) then costs 64-bit VALU adds per tile
DEV int wave_index() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }
// The dispatcher places workgroup b of a launch on XCD b % 8.  xcd_unit maps
// it to a unit index so that each XCD takes one contiguous eighth of the n
// units, and operands that neighbouring units share (a grouped item's A^T)
// stay in that XCD's L2 instead of being fetched into all eight.  It is a
// bijection on [0, n) whatever the placement: XCD x's workgroups b = 8 k + x
// get units x q + min(x, r) + k, q = n / 8, r = n % 8.
DEV int64_t xcd_unit(int64_t b, int64_t n) {
  const int64_t q = n >> 3, r = n & 7, x = b & 7, k = b >> 3;
  return x * q + (x < r ? x : r) + k;
}

// max(acc, |a|, |b|) in one v_max3_f32 (IEEE maxNum: a NaN operand is
// ignored, as fmaxf does).  Written as asm because the builtin form makes the
// compiler add canonicalizing maxima of loop-carried values (+2-4% VALU
// instructions in the per-row kernels).
DEV float max3_abs(float acc, float a, float b) {
  asm("v_max3_f32 %0, %0, |%1|, |%2|" : "+v"(acc) : "v"(a), "v"(b));
  return acc;
}
// min(acc, |a|, |b|) in one v_min3_f32
DEV float min3_abs(float acc, float a, float b) {
  asm("v_min3_f32 %0, %0, |%1|, |%2|" : "+v"(acc) : "v"(a), "v"(b));
  return acc;
}
// two fp32 -> packed bf16 pair (RNE, v_cvt_pk_bf16_f32); low half = a
DEV float bf16_lo(uint32_t w) { return u2f(w << 16); }
DEV float bf16_hi(uint32_t w) { return u2f(w & 0xffff0000u); }
// per-halfword unsigned max (v_pk_max_u16)
DEV uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  us2 x = __builtin_bit_cast(us2, a), y = __builtin_bit_cast(us2, b);
  us2 r = __builtin_elementwise_max(x, y);
  return __builtin_bit_cast(uint32_t, r);
}
// low bytes of four 32-bit words -> one word (byte k from w_k)
DEV uint32_t pack_low_bytes(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  uint32_t lo = __builtin_amdgcn_perm(w1, w0, 0x0c0c0400u);
  uint32_t hi = __builtin_amdgcn_perm(w3, w2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// ---- integer stochastic rounding on gfx950's v_cvt_sr_f16_f32 -------------
// INT8 and Q8_0 codes round v / s + zp stochastically (the selection of
// P/_triton_stochastic_quantization.py:25-40, u < p) through the hardware's
// stochastic conversion to f16.  The caller forms
//   t = med3(fma(v, RN(1/s), 1536 + zp), 1536 + qmin, 1536 + qmax):
// fp32 in [1024, 2048) keeps 13 fraction bits and f16 has spacing 1 there, so
// the conversion picks floor(t) or floor(t) + 1.  Its rule, measured on
// MI355X over every 13-bit fraction and every 13-bit random field: round up
// iff (R >> 19) + frac(t) 2^13 >= 2^13.  With R = (65535 - h) << 16, h the
// element's 16-bit Philox draw, that is u < frac(t) with u = (h >> 3) 2^-13.
// The code is floor(t) + up - 1536, whose two's-complement low byte is the
// low byte of the f16 result (f16 bits of 1536 + c are 0x6600 + c).
typedef _Float16 lm_v2f16 __attribute__((ext_vector_type(2)));
// two codes: t0 with random operand r0 in byte 0, t1 with r1 in byte 2 (the
// conversions overwrite both halves of `old`, which only gives a register)
DEV uint32_t sr_i8_pair(uint32_t old, float t0, float t1, uint32_t r0, uint32_t r1) {
  lm_v2f16 o = __builtin_bit_cast(lm_v2f16, old);
  o = __builtin_amdgcn_cvt_sr_f16_f32(o, t0, r0, false);
  o = __builtin_amdgcn_cvt_sr_f16_f32(o, t1, r1, true);
  return __builtin_bit_cast(uint32_t, o);
}
// the four codes of two pairs (bytes 0 and 2 of each) as one word
DEV uint32_t pack_sr_i8(uint32_t p01, uint32_t p23) { return __builtin_amdgcn_perm(p23, p01, 0x06040200u); }
// t of the rule above
DEV float sr_i8_t(float v, float rcp, float base, float lo, float hi) {
  return __builtin_amdgcn_fmed3f(__builtin_fmaf(v, rcp, base), lo, hi);
}

// ---- blocked (swizzled) scale offsets: P/_triton_nvfp4_lora.py:88-104,
//      P/_triton_mx_lora.py:97-112 --------------------------------------
DEV int64_t blocked_offset(int64_t row, int64_t scol, int64_t scols, bool swz) {
  if (!swz) return row * scols + scol;
  int64_t ncb = (scols + 3) >> 2;
  int64_t rb = row >> 7, rib = row & 127, cb = scol >> 2, cib = scol & 3;
  return (rb * ncb + cb) * 512 + (rib & 31) * 16 + (rib >> 5) * 4 + cib;
}

// ---- MX scale (P/_triton_mx_lora.py:115-159) -----------------------------
DEV uint32_t mx_scale(float max_abs, int mode, int emax, float maxpos, int mbits, float& inv) {
  if (mode == MX_RCEIL) {
    float descale = max_abs / maxpos;
    if (descale != descale) {
      inv = __builtin_nanf("");
      return 255u;
    }
    int unb;
    if (descale == 0.0f) unb = -127;
    else if (__builtin_isinf(descale)) unb = 127;
    else {
      int e;
      float m = __builtin_frexpf(descale, &e);
      unb = (m == 0.5f) ? e - 1 : e;  // exact ceil(log2(descale))
    }
    unb = unb < -127 ? -127 : (unb > 127 ? 127 : unb);
    uint32_t enc = (uint32_t)(unb + 127);
    inv = enc == 0 ? 1.0f : __builtin_ldexpf(1.0f, -unb);
    return enc;
  }
  uint32_t bits = f2u(max_abs);
  if (mode == MX_EVEN) {
    uint32_t bias = mbits == 3 ? 524288u : (mbits == 2 ? 1048576u : 2097152u);
    bits = (bits + bias) & 0xff800000u;
  }
  int ex = (int)((bits >> 23) & 255u) - 127;
  if (mode == MX_CEIL) ex += (bits & 0x7fffffu) > 0 ? 1 : 0;
  int unb = ex - emax;
  unb = unb < -127 ? -127 : (unb > 128 ? 128 : unb);
  uint32_t enc = (uint32_t)(unb + 127);
  if (max_abs != max_abs) enc = 255u;
  float scale = u2f(enc << 23);
  scale = __builtin_fmaxf(scale, 1.1754943508222875e-38f);
  inv = 1.0f / scale;
  return enc;
}

// ---- MFMA tile engine ---------------------------------------------------
// Layout of the prepared factors (written by the prep kernel):
//   At[col][g][kc][i] = A[kc*16 + 4g + i][col]   (zero for k >= rank)
//   Bp[row][g][kc][i] = B[row][kc*16 + 4g + i]
// A wavefront owns 16 weight rows; lane l holds row (l & 15) and, inside a
// macro tile of 4*SPAN columns, the SPAN consecutive columns starting at
// SPAN*(l >> 4).  The MFMA computes D^T (positions x rows): position p of
// MFMA t maps to column SPAN*(p >> 2) + 4t + (p & 3), so the four fp32
// results of MFMA t in lane l are columns SPAN*(l>>4) + 4t + 0..3.
// Rank above 16: chunks kc = 2h and 2h + 1 go to one 16x16x32 MFMA, which
// gfx950 issues at the rate of one 16x16x16 (twice the work per cycle).  Its
// lane group g supplies k slots 8g..8g+7; the operand words hold
// k = 32h + 4g + 0..3 and 32h + 16 + 4g + 0..3 there, for A and B alike, so
// the slot-to-k map is the same on both sides and the sum covers the 32 k
// of the pair.
template <int NKC, bool F16>
DEV v4f32 mfma_chain(const v4i16 (&a)[NKC], const v4i16 (&b)[NKC]) {
  v4f32 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (NKC == 1) {
    if constexpr (F16)
      acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4f16, a[0]), __builtin_bit_cast(v4f16, b[0]), acc,
                                                  0, 0, 0);
    else
      acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a[0], b[0], acc, 0, 0, 0);
  } else {
#pragma unroll
    for (int h = 0; h < NKC / 2; ++h) {
      const v8i16 av = __builtin_shufflevector(a[2 * h], a[2 * h + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      const v8i16 bv = __builtin_shufflevector(b[2 * h], b[2 * h + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      if constexpr (F16)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8f16, av), __builtin_bit_cast(v8f16, bv), acc,
                                                     0, 0, 0);
      else
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf16, av), __builtin_bit_cast(v8bf16, bv),
                                                      acc, 0, 0, 0);
    }
  }
  return acc;
}

template <int NKC>
DEV void load_kchunks(const uint16_t* __restrict__ p, v4i16 (&out)[NKC]) {
  if constexpr (NKC == 1) {
    uint2 w = *(const uint2*)p;
    out[0] = __builtin_bit_cast(v4i16, w);
  } else {
#pragma unroll
    for (int h = 0; h < NKC / 2; ++h) {
      uint4 w = *(const uint4*)(p + 8 * h);
      uint2 lo = make_uint2(w.x, w.y), hi = make_uint2(w.z, w.w);
      out[2 * h] = __builtin_bit_cast(v4i16, lo);
      out[2 * h + 1] = __builtin_bit_cast(v4i16, hi);
    }
  }
}

// delta for the lane's SPAN columns of the macro tile starting at mt_col0
template <int SPAN, int NKC, bool F16>
DEV void tile_delta(const uint16_t* __restrict__ at, int64_t mt_col0, int lane, const v4i16 (&bop)[NKC],
                    float (&d)[SPAN]) {
  constexpr int T = SPAN / 4;
  constexpr int RPAD = NKC * 16;
  const int p = lane & 15, g = lane >> 4;
  const int64_t colbase = mt_col0 + SPAN * (p >> 2) + (p & 3);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    v4i16 aop[NKC];
    load_kchunks<NKC>(at + (colbase + 4 * t) * RPAD + g * (NKC * 4), aop);
    v4f32 acc = mfma_chain<NKC, F16>(aop, bop);
    d[4 * t + 0] = acc[0];
    d[4 * t + 1] = acc[1];
    d[4 * t + 2] = acc[2];
    d[4 * t + 3] = acc[3];
  }
}

// load_kchunks from a global-address-space pointer (global_load with an
// immediate offset instead of flat loads with 64-bit address arithmetic)
template <int NKC>
DEV void load_kchunks_g(const LM_GLOBAL uint16_t* p, v4i16 (&out)[NKC]) {
  if constexpr (NKC == 1) {
    const lm_u32x2 w = *(const LM_GLOBAL lm_u32x2*)p;
    out[0] = __builtin_bit_cast(v4i16, w);
  } else {
#pragma unroll
    for (int h = 0; h < NKC / 2; ++h) {
      const lm_u32x4 w = *(const LM_GLOBAL lm_u32x4*)(p + 8 * h);
      const lm_u32x2 lo = {w.x, w.y}, hi = {w.z, w.w};
      out[2 * h] = __builtin_bit_cast(v4i16, lo);
      out[2 * h + 1] = __builtin_bit_cast(v4i16, hi);
    }
  }
}

template <int NKC>
DEV void load_bop(const uint16_t* __restrict__ bp, int64_t row, int lane, v4i16 (&bop)[NKC]) {
  load_kchunks<NKC>(bp + row * (NKC * 16) + (lane >> 4) * (NKC * 4), bop);
}
// the same through a global-address-space pointer: kernels whose pointers
// come from a descriptor table in memory would otherwise use flat accesses,
// for which the compiler waits for every outstanding load
template <int NKC>
DEV void load_bop_g(const uint16_t* bp, int64_t row, int lane, v4i16 (&bop)[NKC]) {
  load_kchunks_g<NKC>((const LM_GLOBAL uint16_t*)bp + row * (NKC * 16) + (lane >> 4) * (NKC * 4), bop);
}

}  // namespace lm
