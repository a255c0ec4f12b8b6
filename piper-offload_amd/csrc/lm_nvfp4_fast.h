// lm_nvfp4_fast.h -- NVFP4 merge kernels for the production layout: bf16
// factors, N % 128 == 0, one or two scale levels, plain or 128x4-swizzled
// block scales.  P/ = the reference's src/piper_offload/.
//
// Work decomposition: a 512-thread quant workgroup owns 32 rows, two 16-row
// groups (and, for single tensors, a chunk of 32 macro tiles); wave w walks
// the 128-column macro tiles w, w + 8, ... of its range for both groups, so
// at any time the workgroup streams 8 consecutive tiles (512 contiguous
// bytes) of each of its rows.
// (Measured on MI355X with copy kernels of the same footprint: ~5.3 TB/s for
// NVFP4 row lengths, against ~3.7 TB/s for 128-row workgroups whose waves
// share one tile.)  A lane holds row (lane & 15) and the 32 consecutive
// columns 32*(lane >> 4) .. +31 of a macro tile: two NVFP4 blocks, i.e. one
// 16-byte code load and one 2-byte scale read (from LDS where a stack's
// scales are staged there, below), so block reductions never leave the
// lane.  The delta of a macro tile is 8 x NKC
// v_mfma_f32_16x16x16_bf16 (tile_delta's SPAN = 32 orientation), with the
// A^T fragments read through per-lane pointers.
//
// Two-level tensors take two passes (P/_triton_nvfp4_lora.py:437-512, 327-366):
//   amax  -- max |bf16(merged)| over the tensor into red[0] (float bits, so
//            atomicMax on uint orders them), found without merging every
//            tile (the pruned amax below: bound with seed, refine); the
//            reference reduces bf16(merged), and since RNE is monotone the
//            max of the rounded values is the rounded max of the unrounded
//            ones;
//   k_nv_quant -- g = max(amax / 2688, eps); per block s = e4m3(clamp(
//                 (bmax / 6) / g, 2^-6, 448)); codes = e2m1(merged * ((1/g)/s));
//   The amax pass copies the input g into red[1] and the quant pass reads
//   that copy, so the quant pass's first workgroup can write the output g
//   even where it aliases the input.
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
  const float* nrm;        // ||B_i|| (Mpad rows), then ||A_j|| (Npad columns): the pruned amax
  float* ub;               // per-tile bounds: the pruned amax
  int64_t M, N;
  float strength;
  int swizzled;
  uint64_t seed;
};
struct NvStackItem {
  NvArgs a;
  int64_t tile_begin;    // prefix of 32-row units (quant launches)
  int64_t bound_begin;   // prefix of 128-row chunks (pruned amax: bound launch)
  int64_t refine_begin;  // prefix of 512-tile chunks (pruned amax: refine launch)
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

// Per-lane addresses: a wave-uniform base (scalar registers) plus a 32-bit
// lane offset, so the loads and stores take the base as an SGPR pair and the
// per-tile offset needs one 32-bit add (nv_fast_ok bounds N so that a 16-row
// group's codes and an item's scales and A^T fit 32-bit offsets).  Every
// per-tile offset is lane offset + mt * stride, and the A^T fragments of a
// tile use immediate offsets.  Scales: mt advances the scale column by 8,
// which is 8 bytes in the plain layout and 2 col-blocks = 1024 bytes in the
// 128x4 swizzle (P/_triton_nvfp4_lora.py:88-104).  The output codes and
// scales share the input's layout, so the stores reuse q_off and sc_off.
// (global-address-space pointers: the stack kernels read them from a
// descriptor table, and flat accesses would make every wait a full one)
template <int NKC>
struct NvLane {
  const LM_GLOBAL uint8_t* q;   // codes of the 16-row group's first row
  const LM_GLOBAL uint8_t* sc;  // the item's scales
  const LM_GLOBAL uint8_t* at;  // the item's A^T (bytes)
  uint32_t q_off, sc_off, at_off, sc_stride;
  uint32_t lsc_off;             // the lane's scale pair in the staged block (tile t0)
};

// Block scales staged in LDS (stacks in the plain layout whose rows have at
// most NV_LSC_TILES macro tiles): the quant workgroup reads its 32 rows'
// scale bytes of tiles [t0, t1) with 8-byte loads that cover whole lines,
// each lane reads and writes its 2 bytes per tile in LDS, and the workgroup
// writes the block back after its last tile.  Per tile and row group that
// takes the 2-byte scale load and store off the texture-address unit, which
// bounds round-to-nearest, and the partial-line scale traffic off HBM.  A
// row's bytes sit NV_LSC_STRIDE apart: 8 * 129, so the 16 rows a load reads
// fall in distinct banks.
constexpr int NV_LSC_TILES = 128;
constexpr int NV_LSC_STRIDE = 8 * (NV_LSC_TILES + 1);

// row0: the 16-row group's first row (wave-uniform); rowc: the lane's row,
// clamped to M - 1
template <int NKC>
DEV NvLane<NKC> nv_lane(const NvArgs& a, int64_t row0, int64_t rowc, int lane) {
  constexpr int RPAD = NKC * 16;
  const int p = lane & 15, g = lane >> 4;
  NvLane<NKC> l;
  l.q = (const LM_GLOBAL uint8_t*)a.q + row0 * (a.N >> 1);
  l.q_off = (uint32_t)((rowc - row0) * (a.N >> 1)) + 16u * (uint32_t)g;
  l.sc = (const LM_GLOBAL uint8_t*)a.scale;
  l.sc_off = (uint32_t)blocked_offset(rowc, 2 * g, a.N >> 4, a.swizzled);
  l.sc_stride = a.swizzled ? 1024u : 8u;
  l.at = (const LM_GLOBAL uint8_t*)a.at;
  // rank 16: the AT_NV16 order, 16 bytes per lane and fragment pair
  l.at_off = NKC == 1 ? 16u * (uint32_t)lane : 2u * ((uint32_t)(32 * (p >> 2) + (p & 3)) * RPAD + (uint32_t)g * (NKC * 4));
  l.lsc_off = 0u;
  return l;
}

template <int NKC, bool LSC = false>
DEV void nv_load_codes(const NvLane<NKC>& l, int mt, NvTileIn<NKC>& t, const uint8_t* lsc = nullptr, int t0 = 0) {
  const lm_u32x4 c = *(const LM_GLOBAL lm_u32x4*)(l.q + (l.q_off + (uint32_t)mt * 64u));
  t.codes = make_uint4(c.x, c.y, c.z, c.w);
  // the lane's scale column is even: both blocks' scales are adjacent bytes
  if constexpr (LSC) t.sc = *(const uint16_t*)(lsc + (l.lsc_off + 8u * (uint32_t)(mt - t0)));
  else t.sc = *(const LM_GLOBAL uint16_t*)(l.sc + (l.sc_off + (uint32_t)mt * l.sc_stride));
}
template <int NKC>
DEV void nv_load_aop(const NvLane<NKC>& l, int mt, NvTileIn<NKC>& t) {
  constexpr int RPAD = NKC * 16;
  if constexpr (NKC == 1) {
    // AT_NV16: four 16-byte loads, each 1 KiB contiguous across the wave
    // (eight 8-byte loads, one per MFMA, kept the texture-address unit busy)
    const LM_GLOBAL uint8_t* at = l.at + (l.at_off + (uint32_t)mt * (256u * RPAD));
#pragma unroll
    for (int kp = 0; kp < 4; ++kp) {
      const lm_u32x4 w = *(const LM_GLOBAL lm_u32x4*)(at + 1024 * kp);
      t.aop[2 * kp][0] = __builtin_bit_cast(v4i16, lm_u32x2{w.x, w.y});
      t.aop[2 * kp + 1][0] = __builtin_bit_cast(v4i16, lm_u32x2{w.z, w.w});
    }
  } else {
    const LM_GLOBAL uint16_t* at = (const LM_GLOBAL uint16_t*)(l.at + (l.at_off + (uint32_t)mt * (256u * RPAD)));
#pragma unroll
    for (int k = 0; k < 8; ++k) load_kchunks_g<NKC>(at + 4 * k * RPAD, t.aop[k]);
  }
}
template <int NKC>
DEV void nv_load_tile(const NvLane<NKC>& l, int mt, NvTileIn<NKC>& t) {
  nv_load_codes<NKC>(l, mt, t);
  nv_load_aop<NKC>(l, mt, t);
}

// merged values of the lane's 32 columns, for max |merged| (the reference's
// "update == 0 keeps the base" rule only changes the sign of a zero, so the
// amax does not need it)
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
// one 2-byte scale store (qo, so: the outputs' bases, at the lane offsets of
// l), by lanes whose row is < M.  Every lane runs the merge: an MFMA reads
// its operands from all 64 lanes whatever the exec mask, so the operand
// loads must not be skipped for the rows past M (a load under a lane
// condition leaves those lanes' registers stale).
template <int NKC, bool TWO, bool SR, bool LSC = false>
DEV void nv_quant_tile(const NvArgs& a, const NvTileIn<NKC>& in, const v4i16 (&bop)[NKC], float gin, int64_t row,
                       int mt, int lane, float gq, float inv_g, const float* rtab, LM_GLOBAL uint8_t* qo,
                       LM_GLOBAL uint8_t* so, const NvLane<NKC>& l, bool rok, uint8_t* lsc = nullptr, int t0 = 0) {
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
  // (the staged slot was read for this tile only, by this lane; rows past M
  // are not written back)
  if constexpr (LSC) *(uint16_t*)(lsc + (l.lsc_off + 8u * (uint32_t)(mt - t0))) = (uint16_t)scb;
  if (rok) {
    *(LM_GLOBAL lm_u32x4*)(qo + (l.q_off + (uint32_t)mt * 64u)) = lm_u32x4{words[0], words[1], words[2], words[3]};
    if constexpr (!LSC) *(LM_GLOBAL uint16_t*)(so + (l.sc_off + (uint32_t)mt * l.sc_stride)) = (uint16_t)scb;
  }
}

// the staged block: rows row0 .. row0 + 31 (rows past M repeat row M - 1),
// tiles [t0, t1), 8 bytes each; wave w moves rows w, w + 8, ...
DEV void nv_lsc_load(const NvArgs& a, int64_t row0, int t0, int t1, uint8_t* lsc) {
  const int lane = threadIdx.x & 63, wave = wave_index();
  const LM_GLOBAL uint8_t* sb = (const LM_GLOBAL uint8_t*)a.scale + 8 * t0;
  const int64_t scols = a.N >> 4;
#pragma unroll
  for (int i = 0; i < 32 / NV_NW; ++i) {
    const int r = wave + NV_NW * i;
    const int64_t rr = row0 + r < a.M ? row0 + r : a.M - 1;
    for (int c = lane; c < t1 - t0; c += 64)
      *(lm_u32x2*)(lsc + r * NV_LSC_STRIDE + 8 * c) = *(const LM_GLOBAL lm_u32x2*)(sb + (rr * scols + 8 * c));
  }
}
DEV void nv_lsc_store(const NvArgs& a, int64_t row0, int t0, int t1, const uint8_t* lsc) {
  const int lane = threadIdx.x & 63, wave = wave_index();
  LM_GLOBAL uint8_t* sb = (LM_GLOBAL uint8_t*)a.scale_out + 8 * t0;
  const int64_t scols = a.N >> 4;
#pragma unroll
  for (int i = 0; i < 32 / NV_NW; ++i) {
    const int r = wave + NV_NW * i;
    if (row0 + r >= a.M) break;  // wave-uniform
    for (int c = lane; c < t1 - t0; c += 64)
      *(LM_GLOBAL lm_u32x2*)(sb + ((row0 + r) * scols + 8 * c)) = *(const lm_u32x2*)(lsc + r * NV_LSC_STRIDE + 8 * c);
  }
}

// ---- pass bodies -------------------------------------------------------------
// Rows past M load row M-1 (valid memory) and store nothing.
// Tiles [t0, t1) of rows row0 .. row0+15 (the stack passes whole rows).
// the copy of the input per-tensor scale in red[1], which the quant pass reads
DEV void nv_keep_gin(uint32_t* red, float gin) { ((LM_GLOBAL uint32_t*)red)[1] = f2u(gin); }

// amax_bits, gin_bits: red[0] and red[1] as the amax pass left them (the
// max |merged| and the copy of the input per-tensor scale); two-level only
template <int NKC, bool TWO, bool SR, bool LSC = false>
DEV void nv_quant_body(const NvArgs& a, int64_t row0, int t0, int t1, const float* rtab, uint32_t amax_bits,
                       uint32_t gin_bits) {
  __shared__ __attribute__((aligned(16))) uint8_t lsc[LSC ? 32 * NV_LSC_STRIDE : 16];
  if constexpr (LSC) {
    nv_lsc_load(a, row0, t0, t1, lsc);
    __syncthreads();
  }
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
  // Two 16-row groups per wave (rows row0 .. row0 + 31): each tile's A^T
  // fragments are loaded once for both.  The quant pass was bound by the
  // texture-address unit (TA_BUSY 0.83 of cycles, round to nearest), and
  // the fragments were most of its address work.
  // The second group exists when row0 + 16 < M; its lane offsets are taken
  // from its own first row, so they are only formed (and its loads issued)
  // when it exists: with row0 + 16 >= M the clamped row M - 1 would lie
  // before that row and the 32-bit offset would wrap.
  const int64_t rowB = row0 + 16 + rl;
  const bool rokB = rowB < a.M;
  const int64_t rowcB = rokB ? rowB : a.M - 1;
  const bool hasB = row0 + 16 < a.M;  // wave-uniform
  NvLane<NKC> l = nv_lane<NKC>(a, row0, rowc, lane);
  NvLane<NKC> lB = nv_lane<NKC>(a, hasB ? row0 + 16 : row0, hasB ? rowcB : rowc, lane);
  l.lsc_off = (uint32_t)(rl * NV_LSC_STRIDE + 2 * (lane >> 4));
  lB.lsc_off = l.lsc_off + 16u * NV_LSC_STRIDE;
  LM_GLOBAL uint8_t* qo = (LM_GLOBAL uint8_t*)a.q_out + row0 * (a.N >> 1);
  LM_GLOBAL uint8_t* qoB = (LM_GLOBAL uint8_t*)a.q_out + (row0 + 16) * (a.N >> 1);
  LM_GLOBAL uint8_t* so = (LM_GLOBAL uint8_t*)a.scale_out;
  v4i16 bop[NKC], bopB[NKC];
  load_bop_g<NKC>(a.bp, row, lane, bop);
  load_bop_g<NKC>(a.bp, rowcB, lane, bopB);  // Bp holds ceil(M/16)*16 rows
  // (with LSC every wave reaches the write-back barrier, tiles or not)
  if (t0 + wave < ntiles) {
    // The next tile's codes and scales (HBM) are requested before the current
    // tile is merged; its A^T fragments (L2) at the top of its own iteration.
    // Prefetching the fragments too held 16 more VGPRs (103 against 87 for
    // round-to-nearest, one row group): 8B-shaped stack 3.72 -> 3.53 ms per
    // step without it (round-to-nearest), 4.06 -> 3.92 (stochastic).
    NvTileIn<NKC> cur, curB;
    nv_load_codes<NKC, LSC>(l, t0 + wave, cur, lsc, t0);
    if (hasB) nv_load_codes<NKC, LSC>(lB, t0 + wave, curB, lsc, t0);
    for (int mt = t0 + wave; mt < ntiles; mt += NV_NW) {
      nv_load_aop<NKC>(l, mt, cur);  // the fragments depend on the lane and tile only
      NvTileIn<NKC> nxt, nxtB;
      const int mn = mt + NV_NW < ntiles ? mt + NV_NW : mt;
      nv_load_codes<NKC, LSC>(l, mn, nxt, lsc, t0);
      if (hasB) nv_load_codes<NKC, LSC>(lB, mn, nxtB, lsc, t0);
      nv_quant_tile<NKC, TWO, SR, LSC>(a, cur, bop, gin, row, mt, lane, gq, inv_g, rtab, qo, so, l, rok, lsc, t0);
      if (hasB) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
          for (int c = 0; c < NKC; ++c) curB.aop[k][c] = cur.aop[k][c];
        nv_quant_tile<NKC, TWO, SR, LSC>(a, curB, bopB, gin, rowB, mt, lane, gq, inv_g, rtab, qoB, so, lB, rokB, lsc,
                                         t0);
      }
      cur.codes = nxt.codes;
      cur.sc = nxt.sc;
      curB.codes = nxtB.codes;
      curB.sc = nxtB.sc;
    }
  }
  if constexpr (LSC) {
    __syncthreads();
    nv_lsc_store(a, row0, t0, t1, lsc);
  }
}

// the item of launch unit t: the last item whose prefix (of the launch's
// kind of unit) is <= t
enum : int { NV_TILES = 0, NV_BOUND = 1, NV_REFINE = 2 };
template <int KIND = NV_TILES>
DEV int nv_find(const NvStackItem* __restrict__ items, int count, int64_t t) {
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    const NvStackItem& m = items[mid];
    const int64_t b = KIND == NV_BOUND ? m.bound_begin : KIND == NV_REFINE ? m.refine_begin : m.tile_begin;
    if (b <= t) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// ---- kernels: single tensor (args by value) and grouped (descriptor table) ---
// One quant workgroup per 32 rows (tile_begin counts 32-row units).
__host__ __device__ static inline int64_t nv_units(int64_t M, int64_t /*N*/) { return (M + 31) / 32; }

// Single tensors: blocks are independent once the global scale is known, so a
// workgroup owns 32 rows x NV_CHUNK macro tiles (blockIdx.y picks the chunk).
// With 16-row workgroups, 32 tiles (whole 4096-column rows) measured 0.0519
// ms per step (RTN, [14336, 4096]) against 0.0546 with chunks of 16 tiles
// (1792 workgroups instead of 896), and 0.069 with chunks of 8; stochastic
// rounding 0.0612 against 0.0618.
constexpr int NV_CHUNK = 4 * NV_NW;
DEV int nv_chunk_end(const NvArgs& a) {
  const int t1 = ((int)blockIdx.y + 1) * NV_CHUNK, nt = (int)(a.N >> 7);
  return t1 < nt ? t1 : nt;
}
// (single tensors read the scales from global memory: with 4 tiles per wave
// the staging measured slower, [14336, 4096] stochastic 0.0503 -> 0.0515 ms)
template <int NKC, bool SR, bool TWO>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_quant(NvArgs a) {
  __shared__ float rtab[8];
  if (threadIdx.x < 8) rtab[threadIdx.x] = kRcpE4M3[threadIdx.x];
  __syncthreads();
  const LM_GLOBAL uint32_t* red = (const LM_GLOBAL uint32_t*)a.red;
  nv_quant_body<NKC, TWO, SR>(a, (int64_t)blockIdx.x * 32, (int)blockIdx.y * NV_CHUNK, nv_chunk_end(a), rtab,
                              TWO ? red[0] : 0u, TWO ? red[1] : 0u);
}
// TWO: every item of the launch is two-level (the host splits a mixed stack);
// LSC: block scales staged in LDS, every item's rows have at most
// NV_LSC_TILES macro tiles (the staging's barrier also covers rtab)
template <int NKC, bool SR, bool TWO, bool LSC>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_quant_stack(const NvStackItem* __restrict__ items, int count) {
  __shared__ float rtab[8];
  if (threadIdx.x < 8) rtab[threadIdx.x] = kRcpE4M3[threadIdx.x];
  if constexpr (!LSC) __syncthreads();
  const int64_t t = xcd_unit(blockIdx.x, gridDim.x);
  const int i = nv_find(items, count, t);
  const NvArgs& a = items[i].a;
  const LM_GLOBAL uint32_t* red = (const LM_GLOBAL uint32_t*)a.red;
  nv_quant_body<NKC, TWO, SR, LSC>(a, (t - items[i].tile_begin) * 32, 0, (int)(a.N >> 7), rtab,
                                   TWO ? red[0] : 0u, TWO ? red[1] : 0u);
}
// ---- the pruned per-tensor amax (two-level) ---------------------------------
// max |merged| over a tensor without merging every element.  For element
// (i, j) of a block b, with bs_b = bf16(e4m3(s_b) g) its dequant scale:
//   |base| = |bf16(e2m1 * bs_b)| <= bf16(6 bs_b)           (|e2m1| <= 6, RNE monotone)
//   |delta| <= sum_k |B_ik A_kj| <= ||B_i|| ||A_j||          (Cauchy-Schwarz; the
//              MFMA's fp32 sum of exact bf16 products adds < r 2^-23 relative)
//   |merged| = |bf16(fma(delta, strength, base))| <= (|base| + |delta| |strength|)(1 + 2^-8)
// so one bound per 16-row x 128-column tile needs only the tile's 128 scale
// bytes, its rows' and columns' norms (prep) and the input global scale:
//   ub = (bf16(6 bf16(e4m3(maxcode) |g|)) + max||B_i|| max||A_j|| |strength| (1 + 2^-10)) (1 + 2^-6)
// (generous margins, plus 2^-120 for subnormal results; a NaN scale code or a
// non-finite bound gives +inf).  Two launches then find the exact maximum:
//   bound  -- every tile's ub; then (seed) each 128-row chunk's tile with the
//             largest ub merged exactly by the chunk's wave 0: atomicMax
//             into red[0];
//   refine -- every tile whose ub >= red[0] (as read) merged exactly.
// Skipping is exact: red[0] only ever holds the exact maximum of some merged
// tile, so a tile with ub < red[0] <= amax holds no element that could raise
// it.  With weights ~N(0, s) the bound sits a fraction of s above the stored
// block maximum; on the 8B-shaped stack about 0.5% of the tiles are merged.
constexpr int NV_BOUND_ROWS = 8 * 16;     // rows per bound chunk (one 16-row group per wave)
constexpr int NV_REFINE_TILES = 8 * 64;   // tiles per refine workgroup (64 per wave)
constexpr int NV_BOUND_MAX_TILES = 1024;  // tile columns whose norms a bound workgroup keeps in LDS at a time
__host__ __device__ static inline int64_t nv_tcols(int64_t N) { return N >> 7; }
__host__ __device__ static inline int64_t nv_bound_units(int64_t M) { return (M + NV_BOUND_ROWS - 1) / NV_BOUND_ROWS; }
__host__ __device__ static inline int64_t nv_tile_count(int64_t M, int64_t N) { return ((M + 15) / 16) * nv_tcols(N); }
__host__ __device__ static inline int64_t nv_refine_units(int64_t M, int64_t N) {
  return (nv_tile_count(M, N) + NV_REFINE_TILES - 1) / NV_REFINE_TILES;
}

DEV float nv_tile_bound(uint32_t maxcode, bool nan, float bnmax, float anmax, float gin, float strength) {
  const float bs = bf16r(fp8_value<E4M3>(maxcode) * __builtin_fabsf(gin));
  const float base = bf16r(6.0f * bs);
  const float d = bnmax * anmax * __builtin_fabsf(strength) * (1.0f + 0x1p-10f);
  const float ub = (base + d) * (1.0f + 0x1p-6f) + 0x1p-120f;
  return (nan || !(ub <= 3.0e38f)) ? __builtin_inff() : ub;
}

// bound: one workgroup per 128-row chunk, wave w its 16-row group; lane l
// owns tile columns l, l + 64, ...: it reads the 8 scale bytes of each of the
// 16 rows (one 8-byte load per row; a wave's loads cover 512 contiguous bytes
// of a row in the plain layout) and keeps their largest magnitude code, so the
// bound needs no cross-lane work.  Rows past M repeat the last row, so all 16
// loads are unconditional and in flight together.  A NaN code (0x7f) is the largest
// magnitude, so the maximum also flags it.
DEV uint32_t nv_code_max4(uint32_t m, uint32_t w) {
  // per-byte maximum of m (bytes <= 0x7f) and w's magnitude codes: for 7-bit
  // bytes (x | 0x80) - y keeps bit 7 set exactly where x >= y, with no borrow
  // between bytes
  const uint32_t x = w & 0x7f7f7f7fu;
  const uint32_t ge = ((x | 0x80808080u) - m) & 0x80808080u;
  const uint32_t sel = (ge << 1) - (ge >> 7);  // 0xff in the bytes where x >= m
  return (x & sel) | (m & ~sel);
}
// returns the chunk's tile with the largest bound (the same in every thread)
DEV int64_t nv_bound_body(const NvArgs& a, int64_t chunk) {
  __shared__ float sh_an[NV_BOUND_MAX_TILES];  // max ||A_j|| per tile column
  __shared__ float sh_best[NV_NW];
  __shared__ int sh_mt[NV_NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
  const int ntn = (int)nv_tcols(a.N);
  const int64_t mpad = (a.M + 15) / 16 * 16;  // (the host's mpad_of)
  const float gin = *(const LM_GLOBAL float*)a.gin;
  // the quant pass reads this copy: the per-tensor scale output may alias gin
  if (chunk == 0 && tid == 0) nv_keep_gin(a.red, gin);
  const LM_GLOBAL float* an = (const LM_GLOBAL float*)a.nrm + mpad;
  const int64_t row0 = chunk * NV_BOUND_ROWS + 16 * wave;
  const int nrows = a.M - row0 < 16 ? (int)(a.M - row0) : 16;  // <= 0: the wave has no rows
  const float bnmax = wave_max(lane < nrows ? ((const LM_GLOBAL float*)a.nrm)[row0 + lane] : 0.0f);
  const int64_t scols = a.N >> 4;
  LM_GLOBAL float* ubp = (LM_GLOBAL float*)a.ub + (row0 >> 4) * ntn;
  float best = -1.0f;
  int best_mt = 0;
  // strips of NV_BOUND_MAX_TILES tile columns, whose column norms the workgroup keeps in LDS
  for (int s0 = 0; s0 < ntn; s0 += NV_BOUND_MAX_TILES) {
    const int s1 = ntn - s0 < NV_BOUND_MAX_TILES ? ntn : s0 + NV_BOUND_MAX_TILES;
    if (s0 > 0) __syncthreads();  // the previous strip's norms are no longer read
    // column norms: tile column t is threads 16 t' .. 16 t' + 15 of a pass, 8 columns each
    for (int t0 = s0; t0 < s1; t0 += NV_NW * 64 / 16) {
      const int t = t0 + (tid >> 4);
      float m = 0.0f;
      if (t < s1) {
        const lm_u32x4 v0 = *(const LM_GLOBAL lm_u32x4*)(an + (int64_t)t * 128 + (tid & 15) * 8);
        const lm_u32x4 v1 = *(const LM_GLOBAL lm_u32x4*)(an + (int64_t)t * 128 + (tid & 15) * 8 + 4);
        m = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(u2f(v0.x), u2f(v0.y)), __builtin_fmaxf(u2f(v0.z), u2f(v0.w))),
                            __builtin_fmaxf(__builtin_fmaxf(u2f(v1.x), u2f(v1.y)), __builtin_fmaxf(u2f(v1.z), u2f(v1.w))));
      }
      m = row_max16(m);
      if (t < s1 && (tid & 15) == 0) sh_an[t - s0] = m;
    }
    __syncthreads();
    for (int mt = s0 + lane; nrows > 0 && mt < s1; mt += 64) {
      // 32-bit offsets from the scale base (an item's scales are < 2^31
      // bytes): a wave-uniform row part plus the lane's column part, so the
      // loads take the base in scalar registers and one VGPR of offset
      uint32_t cm = 0u;
      const LM_GLOBAL uint8_t* sb = (const LM_GLOBAL uint8_t*)a.scale;
      if (!a.swizzled) {
        const uint32_t off = (uint32_t)mt * 8u;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t ro = (uint32_t)((row0 + (r < nrows ? r : nrows - 1)) * scols);
          const lm_u32x2 w = *(const LM_GLOBAL lm_u32x2*)(sb + (ro + off));
          cm = nv_code_max4(nv_code_max4(cm, w.x), w.y);
        }
      } else {
        // 128x4 swizzle: the scale columns 4 c .. 4 c + 3 of a row are 4
        // consecutive bytes and column block c + 1 starts 512 bytes later, so
        // the lane's 8 columns are words at row part + 1024 mt and + 512
        const uint32_t off = (uint32_t)mt * 1024u;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t ro = (uint32_t)blocked_offset(row0 + (r < nrows ? r : nrows - 1), 0, scols, true);
          const uint32_t w0 = *(const LM_GLOBAL uint32_t*)(sb + (ro + off));
          const uint32_t w1 = *(const LM_GLOBAL uint32_t*)(sb + (ro + off + 512u));
          cm = nv_code_max4(nv_code_max4(cm, w0), w1);
        }
      }
      const uint32_t c2 = (cm & 0xffu) > ((cm >> 8) & 0xffu) ? (cm & 0xffu) : ((cm >> 8) & 0xffu);
      const uint32_t c3 = ((cm >> 16) & 0xffu) > (cm >> 24) ? ((cm >> 16) & 0xffu) : (cm >> 24);
      const uint32_t cmax = c2 > c3 ? c2 : c3;
      const float ub = nv_tile_bound(cmax, cmax == 0x7fu, bnmax, sh_an[mt - s0], gin, a.strength);
      ubp[mt] = ub;
      if (ub > best) {
        best = ub;
        best_mt = mt;
      }
    }
  }
  if (nrows > 0) {  // wave-uniform
    // the wave's best tile: the largest bound, the lowest lane among equals
    const float wb = wave_max(best);
    const uint64_t who = __ballot(best == wb);
    const int src = (int)__builtin_ctzll(who);
    best_mt = __builtin_amdgcn_readlane(best_mt, src);
    best = wb;
  }
  if (lane == 0) {
    sh_best[wave] = best;
    sh_mt[wave] = best_mt;
  }
  __syncthreads();
  // the chunk's best tile, as its index in the item's tile grid: the largest
  // bound, the lowest wave among equals (every thread reads the same slots)
  int w = 0;
  for (int k = 1; k < NV_NW; ++k)
    if (sh_best[k] > sh_best[w]) w = k;
  return ((chunk * NV_BOUND_ROWS + 16 * w) >> 4) * ntn + sh_mt[w];
}

// max |bf16(merged)| over tile `tile` (16 rows x 128 columns), by one wave,
// with the quant pass's merge arithmetic (rows past M left out)
template <int NKC>
DEV float nv_tile_exact(const NvArgs& a, int64_t tile, float gin) {
  const int lane = threadIdx.x & 63;
  const int ntn = (int)nv_tcols(a.N);
  const int64_t row0 = (tile / ntn) * 16, row = row0 + (lane & 15);
  const int mt = (int)(tile % ntn);
  const bool rok = row < a.M;
  const NvLane<NKC> l = nv_lane<NKC>(a, row0, rok ? row : a.M - 1, lane);
  v4i16 bop[NKC];
  load_bop_g<NKC>(a.bp, row, lane, bop);  // Bp holds ceil(M/16)*16 rows
  NvTileIn<NKC> t;
  nv_load_tile<NKC>(l, mt, t);
  float m[32];
  nv_merged<NKC, true>(t, bop, a.strength, gin, m);
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j += 2) mx = max3_abs(mx, m[j], m[j + 1]);
  return bf16r(wave_max(rok ? mx : 0.0f));
}

// bound + seed: the chunk's bounds, then wave 0 merges the chunk's best tile
// exactly and folds its maximum into red[0] (red[0] then only ever holds the
// exact maximum of some merged tile)
template <int NKC>
DEV void nv_bound_seed(const NvArgs& a, int64_t chunk) {
  const int64_t best = nv_bound_body(a, chunk);
  if (wave_index() != 0) return;  // wave-uniform; no barrier follows
  const float mx = nv_tile_exact<NKC>(a, best, *(const LM_GLOBAL float*)a.gin);
  if ((threadIdx.x & 63) == 0) atomicMax(a.red, f2u(mx));
}

// refine: wave w of chunk c checks tiles 512 c + 64 w + lane against the
// current lower bound and merges, one at a time, those that reach it
template <int NKC>
DEV void nv_refine_body(const NvArgs& a, int64_t chunk) {
  const int lane = threadIdx.x & 63, wave = wave_index();
  const int64_t ntiles = nv_tile_count(a.M, a.N);
  const int64_t t = chunk * NV_REFINE_TILES + 64 * wave + lane;
  const float ub = t < ntiles ? ((const LM_GLOBAL float*)a.ub)[t] : -1.0f;
  const float lb = u2f(__hip_atomic_load(a.red, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  uint64_t todo = __ballot(ub >= lb);
  if (todo == 0) return;
  const float gin = *(const LM_GLOBAL float*)a.gin;
  float mx = 0.0f;
  while (todo) {
    const int k = __builtin_ctzll(todo);
    todo &= todo - 1;
    mx = __builtin_fmaxf(mx, nv_tile_exact<NKC>(a, chunk * NV_REFINE_TILES + 64 * wave + k, gin));
  }
  if (lane == 0) atomicMax(a.red, f2u(mx));
}

template <int NKC>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_bound(NvArgs a) { nv_bound_seed<NKC>(a, blockIdx.x); }
template <int NKC>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_refine(NvArgs a) { nv_refine_body<NKC>(a, blockIdx.x); }
// stacks: the bound launch counts 128-row chunks of the two-level items
// (bound_begin), the refine launch 512-tile chunks (refine_begin)
template <int NKC>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_bound_stack(const NvStackItem* __restrict__ items, int count) {
  const int i = nv_find<NV_BOUND>(items, count, blockIdx.x);
  nv_bound_seed<NKC>(items[i].a, (int64_t)blockIdx.x - items[i].bound_begin);
}
template <int NKC>
__global__ __launch_bounds__(NV_NW * 64) void k_nv_refine_stack(const NvStackItem* __restrict__ items, int count) {
  const int i = nv_find<NV_REFINE>(items, count, blockIdx.x);
  nv_refine_body<NKC>(items[i].a, (int64_t)blockIdx.x - items[i].refine_begin);
}

// bf16 factors, a rank bucket, whole macro tiles
// (M N <= 2^35: the stochastic-rounding counters, offset / 8, fit 32 bits;
// M N / 16 < 2^31 and N <= 2^22: scale, A^T and 16-row code offsets fit 32 bits)
static inline bool nv_fast_ok(int cd, int nkc, int64_t M, int64_t N) {
  return cd == LM_BF16 && nkc > 0 && (N % 128) == 0 && M * N <= (int64_t(1) << 35) && N <= (int64_t(1) << 22);
}

// single tensor: the pruned amax (two-level; prep gave it the factors' norms),
// then quant on `st`
static int nv_fast_run(const NvArgs& a, int nkc, bool sr, hipStream_t st) {
  const dim3 grid((unsigned)nv_units(a.M, a.N), (unsigned)(((a.N >> 7) + NV_CHUNK - 1) / NV_CHUNK)), block(NV_NW * 64);
  if (a.gin) {
    if (a.nrm == nullptr || a.ub == nullptr) return fail(LM_EINVAL, "nvfp4 two-level merge without its norm workspace");
    TimedLaunch timed("nvfp4", st);
    const int64_t chunks = nv_bound_units(a.M);
    NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_nv_bound<NKC_>), dim3((unsigned)chunks), block, 0, st, a));
    NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_nv_refine<NKC_>), dim3((unsigned)nv_refine_units(a.M, a.N)),
                                                   block, 0, st, a));
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
