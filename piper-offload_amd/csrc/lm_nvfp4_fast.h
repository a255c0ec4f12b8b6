// lm_nvfp4_fast.h -- NVFP4 merge kernels for the production layout: bf16
// factors, N % 128 == 0, one or two scale levels, plain or 128x4-swizzled
// block scales.  P/ = the reference's src/piper_offload/.
//
// Work decomposition: a 512-thread workgroup owns 16 rows (and, for single
// tensors, a chunk of 16 macro tiles); wave w walks the 128-column macro tiles
// w, w + 8, ... of its range, so at any time the workgroup streams 8
// consecutive tiles (512 contiguous bytes) of each of its rows.
// (Measured on MI355X with copy kernels of the same footprint: ~5.3 TB/s for
// NVFP4 row lengths, against ~3.7 TB/s for 128-row workgroups whose waves
// share one tile.)  A lane holds row (lane & 15) and the 32 consecutive
// columns 32*(lane >> 4) .. +31 of a macro tile: two NVFP4 blocks, i.e. one
// 16-byte code load and one 2-byte scale load, so block reductions never
// leave the lane.  The delta of a macro tile is 8 x NKC
// v_mfma_f32_16x16x16_bf16 (tile_delta's SPAN = 32 orientation), with the
// A^T fragments read through per-lane pointers.
//
// Two-level tensors take two passes (P/_triton_nvfp4_lora.py:437-512, 327-366):
//   k_nv_amax  -- max |merged| over the tensor into red[0] (float bits, so
//                 atomicMax on uint orders them); the reference reduces
//                 bf16(merged), and since RNE is monotone the max of the
//                 rounded values is the rounded max of the unrounded ones;
//   k_nv_quant -- g = max(amax / 2688, eps); per block s = e4m3(clamp(
//                 (bmax / 6) / g, 2^-6, 448)); codes = e2m1(merged * ((1/g)/s));
//   The amax pass copies the input g into red[1] and the quant pass reads
//   that copy, so the quant pass's first workgroup can write the output g
//   even where it aliases the input.  For a round-to-nearest stack both
//   passes run in one launch (k_nv_fused_stack).
// Single-level tensors skip the amax pass and divide by the block scale.
#pragma once
#include "lm_impl.h"

struct NvArgs {
  const uint8_t* q;        // [M, N/2] e2m1 pairs, even column in the low nibble
  const uint8_t* scale;    // e4m3 block-16 scales (plain [M, N/16] or swizzled)
  const float* gin;        // input per-tensor scale; nullptr = single level
  uint8_t* q_out;
  uint8_t* scale_out;
  float* gout;             // output per-tensor scale (two-level)
  const uint16_t* at;
  const uint16_t* bp;
  uint32_t* red;           // red[0]: max |merged| bits (cleared by the prep kernel)
  int64_t M, N;
  float strength;
  int swizzled;
  uint64_t seed;
};
struct NvStackItem {
  NvArgs a;
  int64_t tile_begin;  // prefix of 16-row groups (quant launches)
  int64_t pair_begin;  // prefix of 32-row units (amax launch)
};

constexpr int NV_NW = 8;

// decode the two e2m1 codes of byte `b` of w to fp32 (low nibble -> .x).
// The conversion's own scale operand stays 1.0: with a general bf16 block
// scale it does not give the exact product (measured: the NVFP4 parity tests
// fail), so the block scale is a separate multiply.
DEV v2f32 e2m1_pair(uint32_t w, int b) {
  switch (b) {
    case 0: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
    case 1: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
    case 2: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
    default: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
  }
}

template <int NKC>
struct NvTileIn {
  uint4 codes;
  uint32_t sc;  // the lane's two block-scale bytes
  v4i16 aop[8][NKC];
};

// Per-lane base pointers; every per-tile address is base + mt * stride, and
// the A^T fragments of a tile use immediate offsets.  Scales: mt advances the
// scale column by 8, which is 8 bytes in the plain layout and 2 col-blocks =
// 1024 bytes in the 128x4 swizzle (P/_triton_nvfp4_lora.py:88-104).
template <int NKC>
// (global-address-space pointers: the stack kernels read them from a
// descriptor table, and flat accesses would make every wait a full one)
struct NvLane {
  const LM_GLOBAL uint8_t* q;
  const LM_GLOBAL uint8_t* sc;
  const LM_GLOBAL uint16_t* at;
  int64_t sc_stride;
};

template <int NKC>
DEV NvLane<NKC> nv_lane(const NvArgs& a, int64_t rowc, int lane) {
  constexpr int RPAD = NKC * 16;
  const int p = lane & 15, g = lane >> 4;
  NvLane<NKC> l;
  l.q = (const LM_GLOBAL uint8_t*)a.q + rowc * (a.N >> 1) + 16 * g;
  l.sc = (const LM_GLOBAL uint8_t*)a.scale + blocked_offset(rowc, 2 * g, a.N >> 4, a.swizzled);
  l.sc_stride = a.swizzled ? 1024 : 8;
  l.at = (const LM_GLOBAL uint16_t*)a.at + (int64_t)(32 * (p >> 2) + (p & 3)) * RPAD + g * (NKC * 4);
  return l;
}

template <int NKC>
DEV void nv_load_tile(const NvLane<NKC>& l, int mt, NvTileIn<NKC>& t) {
  constexpr int RPAD = NKC * 16;
  const lm_u32x4 c = *(const LM_GLOBAL lm_u32x4*)(l.q + (int64_t)mt * 64);
  t.codes = make_uint4(c.x, c.y, c.z, c.w);
  // the lane's scale column is even: both blocks' scales are adjacent bytes
  t.sc = *(const LM_GLOBAL uint16_t*)(l.sc + (int64_t)mt * l.sc_stride);
  const LM_GLOBAL uint16_t* at = l.at + (int64_t)mt * (128 * RPAD);
#pragma unroll
  for (int k = 0; k < 8; ++k) load_kchunks_g<NKC>(at + 4 * k * RPAD, t.aop[k]);
}

// merged values of the lane's 32 columns, for max |merged| (the reference's
// "update == 0 keeps the base" rule only changes the sign of a zero, so the
// amax pass does not need it)
template <int NKC, bool TWO>
DEV void nv_merged_parts(const uint4& codes, uint32_t sc, const v4i16 (&aop)[8][NKC], const v4i16 (&bop)[NKC],
                         float strength, float gin, float (&m)[32]) {
  float d[32];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const v4f32 acc = mfma_chain<NKC, false>(aop[k], bop);
    d[4 * k + 0] = acc[0];
    d[4 * k + 1] = acc[1];
    d[4 * k + 2] = acc[2];
    d[4 * k + 3] = acc[3];
  }
  float bs[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const float v = fp8_decode<E4M3>(sc, b);  // e4m3 is exact in bf16
    bs[b] = TWO ? bf16r(v * gin) : v;
  }
  const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const v2f32 pr = e2m1_pair(w[q >> 2], q & 3);
#pragma unroll
    for (int e = 0; e < 2; ++e) m[2 * q + e] = __builtin_fmaf(d[2 * q + e], strength, bf16r(pr[e] * bs[q >> 3]));
  }
}
template <int NKC, bool TWO>
DEV void nv_merged(const NvTileIn<NKC>& in, const v4i16 (&bop)[NKC], float strength, float gin, float (&m)[32]) {
  nv_merged_parts<NKC, TWO>(in.codes, in.sc, in.aop, bop, strength, gin, m);
}

// Merged values of block B (the lane's columns 16B .. 16B+15) of a tile: the
// same arithmetic as nv_merged, one 16-element block at a time so that the
// quantizer keeps half as many values live.
template <int NKC, bool TWO, int B>
DEV void nv_merged_block(const NvTileIn<NKC>& in, const v4i16 (&bop)[NKC], float strength, float gin,
                         float (&m)[16]) {
  float d[16];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const v4f32 acc = mfma_chain<NKC, false>(in.aop[4 * B + k], bop);
    d[4 * k + 0] = acc[0];
    d[4 * k + 1] = acc[1];
    d[4 * k + 2] = acc[2];
    d[4 * k + 3] = acc[3];
  }
  const float v = fp8_decode<E4M3>(in.sc, B);  // e4m3 is exact in bf16
  const float bs = TWO ? bf16r(v * gin) : v;
  const uint32_t w[2] = {B == 0 ? in.codes.x : in.codes.z, B == 0 ? in.codes.y : in.codes.w};
  float base[16];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const v2f32 pr = e2m1_pair(w[q >> 2], q & 3);
    base[2 * q] = bf16r(pr[0] * bs);
    base[2 * q + 1] = bf16r(pr[1] * bs);
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) m[j] = __builtin_fmaf(d[j], strength, base[j]);
  // "update == 0 keeps the base" (P/_triton_nvfp4_lora.py:183-186).  Where
  // d * strength == 0 the fma gives base + (+-0), which is the base itself
  // unless the base is a zero, and then the fma's result is a zero too.  So
  // the rule can change a value only where that value is +-0: a block whose
  // merged values are all non-zero is final, and a block with a zero re-applies
  // the rule element by element.
  float mmin = __builtin_fabsf(m[0]);
#pragma unroll
  for (int j = 1; j < 15; j += 2) mmin = min3_abs(mmin, m[j], m[j + 1]);
  mmin = __builtin_fminf(mmin, __builtin_fabsf(m[15]));
  if (mmin == 0.0f) {
#pragma unroll
    for (int j = 0; j < 16; ++j) m[j] = (d[j] * strength == 0.0f) ? base[j] : m[j];
  }
}

// RN(a / b) from y = RN(1 / b): q0 = RN(a y), r = a - b q0 (exact by fma),
// RN(q0 + r y).  Correctly rounded when a, b and the quotient are normal
// with room for the residual (Markstein); checked against IEEE division on
// 4e8 random binary32 pairs within 2^+-60 of 1, the range of NVFP4 scales.
DEV float div_markstein(float a, float b, float y) {
  const float q0 = a * y;
  return __builtin_fmaf(__builtin_fmaf(-q0, b, a), y, q0);
}

// RN(1 / (1 + k/8)), k = 0..7: the reciprocal mantissas of e4m3 values
static __device__ __constant__ const float kRcpE4M3[8] = {1.0f / 1.0f, 1.0f / 1.125f, 1.0f / 1.25f, 1.0f / 1.375f,
                                                   1.0f / 1.5f, 1.0f / 1.625f, 1.0f / 1.75f, 1.0f / 1.875f};

// Quantize block B of a tile into two code words and one scale byte
// (P/_triton_nvfp4_lora.py:316-366).
template <bool TWO, bool SR, int B>
DEV void nv_quant_block(const NvArgs& a, int64_t row, int mt, int lane, float gq, float inv_g, const float* rtab,
                        const float (&m)[16], uint32_t (&words)[4], uint32_t& scb) {
  uint32_t nw[8];  // complemented Philox words
  if constexpr (SR)
    sr_nwords_aligned_lo<16>(a.seed, (uint32_t)((row * a.N + (int64_t)mt * 128 + 32 * (lane >> 4) + 16 * B) >> 3), nw);
  // bmax over the bf16-rounded values = bf16(max |m|) (rounding is monotone)
  float mb[16];
  float bmax = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; j += 2) {
    mb[j] = bf16r(m[j]);
    mb[j + 1] = bf16r(m[j + 1]);
    bmax = max3_abs(bmax, m[j], m[j + 1]);
  }
  bmax = bf16r(bmax);
  // bmax is a bf16 value and 6 is exact in bf16: div_rn is the IEEE quotient
  float fs = div_rn(bmax, 6.0f, 1.0f / 6.0f);
  if constexpr (TWO) fs = div_markstein(fs, gq, inv_g);
  fs = __builtin_fminf(__builtin_fmaxf(fs, 0.015625f), 448.0f);
  const uint32_t s8 = fp8_encode1<E4M3>(fs);
  fs = fp8_value<E4M3>(s8);
  scb |= s8 << (8 * B);
  const uint32_t fb = f2u(fs);
  const float rfs = __builtin_ldexpf(rtab[(fb >> 20) & 7u], 127 - (int)((fb >> 23) & 255u));  // RN(1/fs)
  const float recip = TWO ? div_markstein(inv_g, fs, rfs) : 0.0f;
  float x[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) x[j] = TWO ? mb[j] * recip : div_rn(mb[j], fs, rfs);
  // the e2m1 conversions saturate to +-6 (checked on gfx950)
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if constexpr (SR) {
      words[2 * B + k] = sr_e2m1_nword(x + 8 * k, nw + 4 * k);
    } else {
      // dst_sel k writes byte k and keeps the others (checked on gfx950)
      uint32_t wd = 0u;
      wd = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(wd, x[8 * k + 0], x[8 * k + 1], 1.0f, 0);
      wd = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(wd, x[8 * k + 2], x[8 * k + 3], 1.0f, 1);
      wd = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(wd, x[8 * k + 4], x[8 * k + 5], 1.0f, 2);
      wd = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(wd, x[8 * k + 6], x[8 * k + 7], 1.0f, 3);
      words[2 * B + k] = wd;
    }
  }
}

// merge + quantize one tile, block by block, then one 16-byte code store and
// one 2-byte scale store
template <int NKC, bool TWO, bool SR>
DEV void nv_quant_tile(const NvArgs& a, const NvTileIn<NKC>& in, const v4i16 (&bop)[NKC], float gin, int64_t row,
                       int mt, int lane, float gq, float inv_g, const float* rtab, LM_GLOBAL uint8_t* qo,
                       LM_GLOBAL uint8_t* so,
                       int64_t so_stride) {
  uint32_t words[4];
  uint32_t scb = 0;
  {
    float m[16];
    nv_merged_block<NKC, TWO, 0>(in, bop, a.strength, gin, m);
    nv_quant_block<TWO, SR, 0>(a, row, mt, lane, gq, inv_g, rtab, m, words, scb);
  }
  {
    float m[16];
    nv_merged_block<NKC, TWO, 1>(in, bop, a.strength, gin, m);
    nv_quant_block<TWO, SR, 1>(a, row, mt, lane, gq, inv_g, rtab, m, words, scb);
  }
  *(LM_GLOBAL lm_u32x4*)(qo + (int64_t)mt * 64) = lm_u32x4{words[0], words[1], words[2], words[3]};
  *(LM_GLOBAL uint16_t*)(so + (int64_t)mt * so_stride) = (uint16_t)scb;
}

// ---- pass bodies -------------------------------------------------------------
// Rows past M load row M-1 (valid memory) and store nothing.
// Tiles [t0, t1) of rows row0 .. row0+15 (the stack passes whole rows).
// The amax pass keeps no register cache, so a wave merges 32 rows (two
// 16-row groups) per macro tile: both groups' MFMAs share the tile's A^T
// fragments, which halves the operand loads (L2) per element.  The pass is
// bound by the texture-address unit (TA_BUSY ~85%, VALU ~63%) through its
// code and scale loads, whose every instruction touches 16 rows: four
// groups per wave, sharing the A^T loads further, measured the same.  Rows
// row0 .. row0 + 31; the second group exists when row0 + 16 < M.
// the copy of the input per-tensor scale in red[1]: a plain store when the
// quant pass is a later launch, a device-scope atomic exchange when it runs in
// the same launch (k_nv_fused_stack)
DEV void nv_keep_gin(uint32_t* red, float gin, bool fused) {
  if (fused) __hip_atomic_exchange(red + 1, f2u(gin), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else ((LM_GLOBAL uint32_t*)red)[1] = f2u(gin);
}
template <int NKC>
struct NvAmaxIn {
  uint4 codes[2];
  uint32_t sc[2];
  v4i16 aop[8][NKC];
};
template <int NKC>
DEV void nv_amax_load(const NvLane<NKC>& l0, const NvLane<NKC>& l1, int mt, NvAmaxIn<NKC>& t) {
  constexpr int RPAD = NKC * 16;
  const lm_u32x4 c0 = *(const LM_GLOBAL lm_u32x4*)(l0.q + (int64_t)mt * 64);
  const lm_u32x4 c1 = *(const LM_GLOBAL lm_u32x4*)(l1.q + (int64_t)mt * 64);
  t.codes[0] = make_uint4(c0.x, c0.y, c0.z, c0.w);
  t.codes[1] = make_uint4(c1.x, c1.y, c1.z, c1.w);
  t.sc[0] = *(const LM_GLOBAL uint16_t*)(l0.sc + (int64_t)mt * l0.sc_stride);
  t.sc[1] = *(const LM_GLOBAL uint16_t*)(l1.sc + (int64_t)mt * l1.sc_stride);
  const LM_GLOBAL uint16_t* at = l0.at + (int64_t)mt * (128 * RPAD);
#pragma unroll
  for (int k = 0; k < 8; ++k) load_kchunks_g<NKC>(at + 4 * k * RPAD, t.aop[k]);
}
template <int NKC>
DEV void nv_amax_body_direct(const NvArgs& a, int64_t row0, int t0, int t1, bool fused) {
  __shared__ float sh[NV_NW];
  const int lane = threadIdx.x & 63, wave = wave_index(), rl = lane & 15;
  const int64_t r0 = row0 + rl, r1 = row0 + 16 + rl;
  const bool rok0 = r0 < a.M, rok1 = r1 < a.M;
  const bool second = row0 + 16 < a.M;  // wave-uniform
  const int ntiles = t1;
  const float gin = *(const LM_GLOBAL float*)a.gin;
  // the quant pass reads this copy: the per-tensor scale output may alias gin
  if (row0 == 0 && t0 == 0 && threadIdx.x == 0) nv_keep_gin(a.red, gin, fused);
  const float strength = a.strength;
  // rows past M read row M - 1 (valid memory) and are left out of the max
  const NvLane<NKC> l0 = nv_lane<NKC>(a, rok0 ? r0 : a.M - 1, lane);
  const NvLane<NKC> l1 = nv_lane<NKC>(a, rok1 ? r1 : a.M - 1, lane);
  v4i16 bop0[NKC], bop1[NKC];
  load_bop_g<NKC>(a.bp, r0, lane, bop0);  // Bp holds ceil(M/16)*16 rows
  if (second) {
    load_bop_g<NKC>(a.bp, r1, lane, bop1);
  } else {
#pragma unroll
    for (int k = 0; k < NKC; ++k) bop1[k] = (v4i16){0, 0, 0, 0};
  }
  float mx0 = 0.0f, mx1 = 0.0f;
  if (t0 + wave < ntiles) {
    NvAmaxIn<NKC> cur;
    nv_amax_load<NKC>(l0, l1, t0 + wave, cur);
    for (int mt = t0 + wave; mt < ntiles; mt += NV_NW) {
      NvAmaxIn<NKC> nxt;
      nv_amax_load<NKC>(l0, l1, mt + NV_NW < ntiles ? mt + NV_NW : mt, nxt);
      float m[32];
      nv_merged_parts<NKC, true>(cur.codes[0], cur.sc[0], cur.aop, bop0, strength, gin, m);
#pragma unroll
      for (int j = 0; j < 32; j += 2) mx0 = max3_abs(mx0, m[j], m[j + 1]);
      if (second) {
        nv_merged_parts<NKC, true>(cur.codes[1], cur.sc[1], cur.aop, bop1, strength, gin, m);
#pragma unroll
        for (int j = 0; j < 32; j += 2) mx1 = max3_abs(mx1, m[j], m[j + 1]);
      }
      cur = nxt;
    }
  }
  float mx = __builtin_fmaxf(rok0 ? mx0 : 0.0f, rok1 ? mx1 : 0.0f);
  mx = wave_max(mx);
  if (lane == 0) sh[wave] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = sh[0];
#pragma unroll
    for (int w = 1; w < NV_NW; ++w) r = __builtin_fmaxf(r, sh[w]);
    atomicMax(a.red, f2u(bf16r(r)));
  }
}

// Plain (unswizzled) scales: the workgroup stages each step's codes and
// scales through LDS.  A step is the 8 consecutive macro tiles its waves
// take (wave w: tile ts + w) of the 32 rows.  The codes arrive as 512-byte
// row segments (two rows per wave instruction) and the scales as 64-byte row
// segments, one instruction for the whole step.  Loaded per lane, every
// code and scale instruction touched 16 rows, which kept the
// texture-address unit busy.  The next step's bytes are requested into
// registers while the current one is merged.  Row pitches are padded (528
// and 68 bytes) so that the lanes' LDS reads of one row group do not share
// banks.
constexpr int NV_CPITCH = 528, NV_SPITCH = 68;
template <int NKC>
DEV void nv_amax_body_lds(const NvArgs& a, int64_t row0, int t0, int t1, bool fused) {
  constexpr int RPAD = NKC * 16;
  __shared__ float sh[NV_NW];
  // two buffers: step s reads buffer s & 1 while the next step's bytes go to
  // the other one, so a step needs one barrier
  __shared__ __attribute__((aligned(16))) uint8_t lcodes[2][32 * NV_CPITCH];
  __shared__ __attribute__((aligned(16))) uint8_t lsc[2][32 * NV_SPITCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(), rl = lane & 15, g = lane >> 4;
  const int ntiles = t1;
  const int steps = (ntiles - t0 + NV_NW - 1) / NV_NW;  // workgroup-uniform
  const int64_t half = a.N >> 1, scols = a.N >> 4;
  const float gin = *(const LM_GLOBAL float*)a.gin;
  // the quant pass reads this copy: the per-tensor scale output may alias gin
  if (row0 == 0 && t0 == 0 && threadIdx.x == 0) nv_keep_gin(a.red, gin, fused);
  const float strength = a.strength;
  const bool second = row0 + 16 < a.M;  // workgroup-uniform
  // staging: thread tid loads code chunks q = tid, tid + 512 (row q >> 5,
  // 16-byte chunk q & 31 of the row's 512-byte step segment); threads 0..255
  // load the scales of row tid >> 3, tile tid & 7 (8 bytes)
  const LM_GLOBAL uint8_t* qb = (const LM_GLOBAL uint8_t*)a.q;
  const LM_GLOBAL uint8_t* sb = (const LM_GLOBAL uint8_t*)a.scale;
  auto rowc = [&](int r) { const int64_t row = row0 + r; return row < a.M ? row : a.M - 1; };
  lm_u32x4 sc0, sc1;
  lm_u32x2 ss;
  auto stage = [&](int ts) {
    const int qa = tid, qq = tid + 512;
    const int ta = ts + ((qa & 31) >> 2), tq = ts + ((qq & 31) >> 2);
    const int tca = ta < ntiles ? ta : ntiles - 1, tcq = tq < ntiles ? tq : ntiles - 1;
    sc0 = *(const LM_GLOBAL lm_u32x4*)(qb + rowc(qa >> 5) * half + (int64_t)tca * 64 + (qa & 3) * 16);
    sc1 = *(const LM_GLOBAL lm_u32x4*)(qb + rowc(qq >> 5) * half + (int64_t)tcq * 64 + (qq & 3) * 16);
    if (tid < 256) {
      const int tt = ts + (tid & 7), tc = tt < ntiles ? tt : ntiles - 1;
      ss = *(const LM_GLOBAL lm_u32x2*)(sb + rowc(tid >> 3) * scols + (int64_t)tc * 8);
    }
  };
  auto publish = [&](int b) {
    *(lm_u32x4*)(lcodes[b] + (tid >> 5) * NV_CPITCH + (tid & 31) * 16) = sc0;
    *(lm_u32x4*)(lcodes[b] + ((tid + 512) >> 5) * NV_CPITCH + (tid & 31) * 16) = sc1;
    if (tid < 256) {
      uint32_t* d = (uint32_t*)(lsc[b] + (tid >> 3) * NV_SPITCH + (tid & 7) * 8);
      d[0] = ss.x;
      d[1] = ss.y;
    }
  };
  // per wave: its tile's A^T fragments (from L2), one step ahead
  const int p = lane & 15;
  const LM_GLOBAL uint16_t* atl = (const LM_GLOBAL uint16_t*)a.at + (int64_t)(32 * (p >> 2) + (p & 3)) * RPAD + g * (NKC * 4);
  auto load_aop = [&](int ts, v4i16 (&aop)[8][NKC]) {
    const int mt = ts + wave, mtc = mt < ntiles ? mt : ntiles - 1;
    const LM_GLOBAL uint16_t* at = atl + (int64_t)mtc * (128 * RPAD);
#pragma unroll
    for (int k = 0; k < 8; ++k) load_kchunks_g<NKC>(at + 4 * k * RPAD, aop[k]);
  };
  v4i16 bop0[NKC], bop1[NKC];
  load_bop_g<NKC>(a.bp, row0 + rl, lane, bop0);  // Bp holds ceil(M/16)*16 rows
  if (second) {
    load_bop_g<NKC>(a.bp, row0 + 16 + rl, lane, bop1);
  } else {
#pragma unroll
    for (int k = 0; k < NKC; ++k) bop1[k] = (v4i16){0, 0, 0, 0};
  }
  float mx0 = 0.0f, mx1 = 0.0f;
  v4i16 aop[8][NKC];
  stage(t0);
  load_aop(t0, aop);
  publish(0);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    const uint8_t* lc = lcodes[s & 1];
    const uint8_t* ls = lsc[s & 1];
    const int ts = t0 + s * NV_NW;
    if (s + 1 < steps) stage(ts + NV_NW);
    v4i16 nxt[8][NKC];
    load_aop(ts + NV_NW, nxt);
    if (ts + wave < ntiles) {
      const int cofs = wave * 64 + 16 * g, sofs = wave * 8 + 2 * g;
      float m[32];
      {
        const lm_u32x4 c = *(const lm_u32x4*)(lc + rl * NV_CPITCH + cofs);
        const uint32_t scv = *(const uint16_t*)(ls + rl * NV_SPITCH + sofs);
        nv_merged_parts<NKC, true>(make_uint4(c.x, c.y, c.z, c.w), scv, aop, bop0, strength, gin, m);
#pragma unroll
        for (int j = 0; j < 32; j += 2) mx0 = max3_abs(mx0, m[j], m[j + 1]);
      }
      if (second) {
        const lm_u32x4 c = *(const lm_u32x4*)(lc + (16 + rl) * NV_CPITCH + cofs);
        const uint32_t scv = *(const uint16_t*)(ls + (16 + rl) * NV_SPITCH + sofs);
        nv_merged_parts<NKC, true>(make_uint4(c.x, c.y, c.z, c.w), scv, aop, bop1, strength, gin, m);
#pragma unroll
        for (int j = 0; j < 32; j += 2) mx1 = max3_abs(mx1, m[j], m[j + 1]);
      }
    }
    // the other buffer was last read in step s - 1, before the barrier that
    // ended it; after this one, step s + 1 may read it
    if (s + 1 < steps) publish((s + 1) & 1);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int c = 0; c < NKC; ++c) aop[k][c] = nxt[k][c];
  }
  const bool rok0 = row0 + rl < a.M, rok1 = row0 + 16 + rl < a.M;
  float mx = __builtin_fmaxf(rok0 ? mx0 : 0.0f, rok1 ? mx1 : 0.0f);
  mx = wave_max(mx);
  if (lane == 0) sh[wave] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = sh[0];
#pragma unroll
    for (int w = 1; w < NV_NW; ++w) r = __builtin_fmaxf(r, sh[w]);
    atomicMax(a.red, f2u(bf16r(r)));
  }
}
// (the staged loads need 16-byte aligned codes and 8-byte aligned scales)
// fused: the amax pass runs in the same launch as the quant pass
// (k_nv_fused_stack), which reads the copy of gin as an atomic
template <int NKC>
DEV void nv_amax_body(const NvArgs& a, int64_t row0, int t0, int t1, bool fused = false) {
  if (a.swizzled || (((uintptr_t)a.q) & 15) != 0 || (((uintptr_t)a.scale) & 7) != 0)
    nv_amax_body_direct<NKC>(a, row0, t0, t1, fused);
  else
    nv_amax_body_lds<NKC>(a, row0, t0, t1, fused);
}

// amax_bits, gin_bits: red[0] and red[1] as the amax pass left them (the
// max |merged| and the copy of the input per-tensor scale); two-level only
template <int NKC, bool TWO, bool SR>
DEV void nv_quant_body(const NvArgs& a, int64_t row0, int t0, int t1, const float* rtab, uint32_t amax_bits,
                       uint32_t gin_bits) {
  const int lane = threadIdx.x & 63, wave = wave_index(), rl = lane & 15;
  const int64_t row = row0 + rl;
  const bool rok = row < a.M;
  const int64_t rowc = rok ? row : a.M - 1;
  const int ntiles = t1;
  // the input per-tensor scale from the amax pass's copy; the output one is
  // written here, by one thread, since it may alias the input
  const float gin = TWO ? u2f(gin_bits) : 1.0f;
  float gq = 1.0f, inv_g = 1.0f;
  if constexpr (TWO) {
    gq = __builtin_fmaxf(u2f(amax_bits) / 2688.0f, kEps);
    inv_g = 1.0f / gq;
    if (row0 == 0 && t0 == 0 && threadIdx.x == 0 && a.gout != nullptr) *(LM_GLOBAL float*)a.gout = gq;
  }
  const NvLane<NKC> l = nv_lane<NKC>(a, rowc, lane);
  LM_GLOBAL uint8_t* qo = (LM_GLOBAL uint8_t*)a.q_out + rowc * (a.N >> 1) + 16 * (lane >> 4);
  LM_GLOBAL uint8_t* so = (LM_GLOBAL uint8_t*)a.scale_out + blocked_offset(rowc, 2 * (lane >> 4), a.N >> 4, a.swizzled);
  v4i16 bop[NKC];
  load_bop_g<NKC>(a.bp, row, lane, bop);
  if (t0 + wave >= ntiles) return;
  NvTileIn<NKC> cur;
  nv_load_tile<NKC>(l, t0 + wave, cur);
  for (int mt = t0 + wave; mt < ntiles; mt += NV_NW) {
    NvTileIn<NKC> nxt;
    nv_load_tile<NKC>(l, mt + NV_NW < ntiles ? mt + NV_NW : mt, nxt);
    if (rok) nv_quant_tile<NKC, TWO, SR>(a, cur, bop, gin, row, mt, lane, gq, inv_g, rtab, qo, so, l.sc_stride);
    cur = nxt;
  }
}

template <bool PAIRS = false>
DEV int nv_find(const NvStackItem* __restrict__ items, int count, int64_t t) {
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((PAIRS ? items[mid].pair_begin : items[mid].tile_begin) <= t) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// ---- kernels: single tensor (args by value) and grouped (descriptor table) ---
// One workgroup per 16 rows (tile_begin counts 16-row groups).
__host__ __device__ static inline int64_t nv_units(int64_t M, int64_t /*N*/) { return (M + 15) / 16; }
// the amax pass: one workgroup per 32 rows
__host__ __device__ static inline int64_t nv_pairs(int64_t M) { return (M + 31) / 32; }

// Single tensors: blocks are independent once the global scale is known, so a
// workgroup owns 16 rows x NV_CHUNK macro tiles (blockIdx.y picks the chunk).
// 32 tiles keep 4096-column rows whole: for [14336, 4096] that measured
// 0.0519 ms per step (RTN) against 0.0546 with chunks of 16 tiles (1792
// workgroups instead of 896), and 0.069 with chunks of 8; stochastic
// rounding 0.0612 against 0.0618.
constexpr int NV_CHUNK = 4 * NV_NW;
DEV int nv_chunk_end(const NvArgs& a) {
  const int t1 = ((int)blockIdx.y + 1) * NV_CHUNK, nt = (int)(a.N >> 7);
  return t1 < nt ? t1 : nt;
}
template <int NKC>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_amax(NvArgs a) {
  nv_amax_body<NKC>(a, (int64_t)blockIdx.x * 32, (int)blockIdx.y * NV_CHUNK, nv_chunk_end(a));
}
template <int NKC, bool SR, bool TWO>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_quant(NvArgs a) {
  __shared__ float rtab[8];
  if (threadIdx.x < 8) rtab[threadIdx.x] = kRcpE4M3[threadIdx.x];
  __syncthreads();
  const LM_GLOBAL uint32_t* red = (const LM_GLOBAL uint32_t*)a.red;
  nv_quant_body<NKC, TWO, SR>(a, (int64_t)blockIdx.x * 16, (int)blockIdx.y * NV_CHUNK, nv_chunk_end(a), rtab,
                              TWO ? red[0] : 0u, TWO ? red[1] : 0u);
}
template <int NKC>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_amax_stack(const NvStackItem* __restrict__ items, int count) {
  const int i = nv_find<true>(items, count, blockIdx.x);
  const NvArgs a = items[i].a;
  if (a.gin == nullptr) return;  // single-level item: no global scale to find
  nv_amax_body<NKC>(a, ((int64_t)blockIdx.x - items[i].pair_begin) * 32, 0, (int)(a.N >> 7));
}
// TWO: every item of the launch is two-level (the host splits a mixed stack)
template <int NKC, bool SR, bool TWO>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_quant_stack(const NvStackItem* __restrict__ items, int count) {
  __shared__ float rtab[8];
  if (threadIdx.x < 8) rtab[threadIdx.x] = kRcpE4M3[threadIdx.x];
  __syncthreads();
  const int i = nv_find(items, count, blockIdx.x);
  const NvArgs& a = items[i].a;
  const LM_GLOBAL uint32_t* red = (const LM_GLOBAL uint32_t*)a.red;
  nv_quant_body<NKC, TWO, SR>(a, ((int64_t)blockIdx.x - items[i].tile_begin) * 16, 0, (int)(a.N >> 7), rtab,
                              TWO ? red[0] : 0u, TWO ? red[1] : 0u);
}
// ---- grouped two-level stack in one launch ------------------------------------
// The amax and quant passes of a round-to-nearest stack in one grid (the
// host keeps two launches for stochastic rounding, where they measured
// faster).  A workgroup takes the next ticket from a counter, so tickets are
// handed out in order to running workgroups.  The tickets run through
// segments, each covering all amax units (32 rows) or all quant units (16
// rows) of one item.  An item's quant segment is placed at least
// NV_LOOKAHEAD tickets after its last amax unit.  A quant unit waits until
// the item's amax units have all published (red[2] counts them), which by
// then they normally have.
//   - Waiting cannot deadlock: every ticket before a quant unit's was taken
//     by a running workgroup, and amax units wait on nothing.  The wait is
//     bounded all the same (NV_SPIN_LIMIT polls); a unit that gives up sets
//     the stack workspace's status word (lm_stack_status_offset) and stores
//     nothing.
//   - The texture-address-bound amax units and the quant units share the CUs
//     instead of running one launch after the other.
//   - An item's codes and scales are read twice within about NV_LOOKAHEAD
//     units of work (~40 MB of 4096-column rows), so the second read can hit
//     the 256 MB Infinity Cache.  (Measured per step on the 8B-shaped stack:
//     4.35-4.37 ms at 512 tickets, 4.42 at 1024, 4.45 at 2048, 4.84 at 4096;
//     4.84 at 256 and 5.45 at 128, where quant units wait; two launches
//     4.76.  FETCH_SIZE, which counts L2 misses whether or not the Infinity
//     Cache holds the line, reads the same as with two launches.)
// Items must not share buffers (an item may be in place): a quant unit may
// run while other items' amax units still read.
struct NvSeg {
  int32_t item;          // descriptor index
  int32_t quant;         // 0: amax units, 1: quant units
  int64_t ticket_begin;  // first ticket of the segment
};
constexpr int64_t NV_LOOKAHEAD = 512;
constexpr uint32_t NV_SPIN_LIMIT = 1u << 20;  // polls of up to ~3 us: a few seconds
// The fused launch's bounded wait: a quant unit polls at most spin_limit
// times for need + extra_need finished amax units (extra_need is 0 except
// under lm_debug_stack_wait, which lets a test make every wait give up while
// each wave still ends normally).  A unit that gives up stores nothing and
// sets bit 0 of the caller-visible status word.
struct NvWait {
  uint32_t* status;      // sticky status word of the stack workspace
  uint32_t spin_limit;
  uint32_t extra_need;
};

// rank 16: both passes fit 128 VGPRs, two workgroups per CU
template <int NKC>
constexpr int nv_fused_min_waves() { return NKC == 1 ? 4 : 1; }
template <int NKC>
__global__ __launch_bounds__(NV_NW * 64, nv_fused_min_waves<NKC>()) void k_nv_fused_stack(const NvStackItem* __restrict__ items,
                                                                  const NvSeg* __restrict__ segs, int nseg,
                                                                  uint32_t* ctl, NvWait wt) {
  __shared__ float rtab[8];
  // [0] the ticket (read by every thread after the first barrier), [1] [2]
  // the amax words, [3] the quant unit's go / give-up flag: separate slots, so
  // no thread can read a ticket that the flag has overwritten
  __shared__ uint32_t sh_w[4];
  if (threadIdx.x < 8) rtab[threadIdx.x] = kRcpE4M3[threadIdx.x];
  if (threadIdx.x == 0) sh_w[0] = atomicAdd(ctl, 1u);
  __syncthreads();
  const int64_t t = sh_w[0];
  int lo = 0, hi = nseg - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (segs[mid].ticket_begin <= t) lo = mid;
    else hi = mid - 1;
  }
  const NvSeg sg = segs[lo];
  const NvArgs& a = items[sg.item].a;
  const int64_t unit = t - sg.ticket_begin;
  uint32_t* red = a.red;
  if (!sg.quant) {
    nv_amax_body<NKC>(a, unit * 32, 0, (int)(a.N >> 7), true);
    // Thread 0 made this unit's atomicMax (and unit 0's exchange of the gin
    // copy), both device-scope atomics; once they are acknowledged, count the
    // unit.  Everything a quant unit reads from red is an atomic, so no
    // cache write-back or invalidation is needed (agent-scope release and
    // acquire fences write back / invalidate the whole L2 of an XCD, which
    // slowed the launch by a third).
    if (threadIdx.x == 0) {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // (flat atomics count in both)
      __hip_atomic_fetch_add(red + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  if (threadIdx.x == 0) {
    const uint32_t need = (uint32_t)nv_pairs(a.M) + wt.extra_need;
    uint32_t polls = 0;
    uint32_t done = __hip_atomic_load(red + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while (done < need && polls < wt.spin_limit) {
      // back off: many waiting workgroups polling one counter slow every
      // other access (small stacks, where most quant units do wait)
      const uint32_t reps = polls < 16 ? 1u : (polls < 64 ? 4u : 16u);
      for (uint32_t k = 0; k < reps; ++k) __builtin_amdgcn_s_sleep(8);
      ++polls;
      done = __hip_atomic_load(red + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const bool ok = done >= need;
    if (!ok) __hip_atomic_fetch_or(wt.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh_w[3] = ok ? 1u : 0u;
    sh_w[1] = __hip_atomic_load(red + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh_w[2] = __hip_atomic_load(red + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (sh_w[3] == 0u) return;
  nv_quant_body<NKC, true, false>(a, unit * 16, 0, (int)(a.N >> 7), rtab, sh_w[1], sh_w[2]);
}

// Ticket order of the fused launch over the `n` two-level descriptors h[0,n):
// amax segments in item order, each item's quant segment as soon as
// NV_LOOKAHEAD tickets have followed its last amax unit (or no amax is left).
// Returns the number of tickets; segs holds 2 n entries.
static inline int64_t nv_schedule(const NvStackItem* h, int n, NvSeg* segs, int64_t* a_end) {
  int64_t ticket = 0;
  int ia = 0, iq = 0, k = 0;
  while (iq < n) {
    if (ia < n && (ia <= iq || ticket - a_end[iq] < NV_LOOKAHEAD)) {
      segs[k++] = NvSeg{ia, 0, ticket};
      ticket += nv_pairs(h[ia].a.M);
      a_end[ia++] = ticket;
    } else {
      segs[k++] = NvSeg{iq, 1, ticket};
      ticket += nv_units(h[iq].a.M, h[iq].a.N);
      ++iq;
    }
  }
  return ticket;
}

// bf16 factors, a rank bucket, whole macro tiles
// (M N <= 2^35: the stochastic-rounding counters, offset / 8, fit 32 bits)
static inline bool nv_fast_ok(int cd, int nkc, int64_t M, int64_t N) {
  return cd == LM_BF16 && nkc > 0 && (N % 128) == 0 && M * N <= (int64_t(1) << 35);
}

// single tensor: amax (two-level), then quant on `st`
static int nv_fast_run(const NvArgs& a, int nkc, bool sr, hipStream_t st) {
  const dim3 grid((unsigned)nv_units(a.M, a.N), (unsigned)(((a.N >> 7) + NV_CHUNK - 1) / NV_CHUNK)), block(NV_NW * 64);
  if (a.gin) {
    TimedLaunch timed("nvfp4", st);
    const dim3 agrid((unsigned)nv_pairs(a.M), grid.y);
    NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_nv_amax<NKC_>), agrid, block, 0, st, a));
    LAUNCH_CHECK();
  }
  {
    TimedLaunch timed("nvfp4", st);
#define NQ1(SR_, TWO_) NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_nv_quant<NKC_, SR_, TWO_>), grid, block, 0, st, a))
    if (a.gin) { if (sr) { NQ1(true, true); } else { NQ1(false, true); } }
    else { if (sr) { NQ1(true, false); } else { NQ1(false, false); } }
#undef NQ1
    LAUNCH_CHECK();
  }
  return LM_OK;
}
