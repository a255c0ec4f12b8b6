// lm_mx_fast.h -- in-place MX merge (MXFP4 / MXFP8 e4m3 / e5m2 elements,
// e8m0 block-32 scales, plain or 128x4-swizzled) for bf16 factors and
// N % 128 == 0.  P/ = the reference's src/piper_offload/.
//
// Same decomposition as the NVFP4 quant pass: a 512-thread workgroup owns 32
// rows (two 16-row groups; 16 rows with stochastic rounding) and a chunk of
// MX_CHUNK macro tiles (blockIdx.y), wave w walks the 128-column macro tiles
// chunk + w, chunk + w + 8, ... for its groups, which share each tile's A^T
// fragments (at rank 16 four 16-byte loads in the AT_NV16 order), and a
// lane holds row (lane & 15) of
// its group and the 32 columns 32*(lane >> 4) .. +31 of a macro tile --
// exactly one MX block, so the block max, the shared exponent and the codes
// never leave the lane (P/_triton_mx_lora.py:333-425 does one
// pass: merge, block amax, scale, encode, all in place).
//
// Arithmetic (P/_triton_mx_lora.py:209-295, bf16 compute):
//   base   = bf16(bf16(code) * bf16(2^e))  -- an e2m1 value times a power of
//            two is exact in fp32 and in bf16, so this is one multiply; fp8
//            elements can fall below bf16's subnormal range and keep the
//            rounding;
//   merged = bf16(fma(delta, strength, base));
//   scale  = mx_scale(max |merged|, mode); codes = enc(clamp(merged * 1/scale)),
//   stochastic codes by the hardware conversions (lm_device.h).
#pragma once
#include "lm_nvfp4_fast.h"

struct MxArgs {
  uint8_t* q;       // MXFP4: [M, N/2] e2m1 pairs; MXFP8: [M, N] codes (in place)
  uint8_t* scale;   // e8m0 block-32 scales (in place)
  const uint16_t* at;
  const uint16_t* bp;
  int64_t M, N;
  float strength;
  int swizzled;
  int mode;         // MX_FLOOR / MX_RCEIL / MX_CEIL / MX_EVEN
  uint64_t seed;
};

template <int ELEM>
struct MxTraits {
  static constexpr int emax = ELEM == E2M1 ? 2 : (ELEM == E4M3 ? 8 : 15);
  static constexpr float maxpos = ELEM == E2M1 ? 6.0f : (ELEM == E4M3 ? 448.0f : 57344.0f);
  static constexpr int mbits = ELEM == E2M1 ? 1 : (ELEM == E4M3 ? 3 : 2);
  static constexpr int lane_bytes = ELEM == E2M1 ? 16 : 32;  // code bytes of one lane's block
};

template <int ELEM, int NKC>
struct MxTileIn {
  uint4 codes[MxTraits<ELEM>::lane_bytes / 16];
  uint32_t sc;
  v4i16 aop[8][NKC];
};

// A lane's addresses: wave-uniform bases plus 32-bit lane offsets (codes
// relative to the 16-row group's first row, scales and A^T to the item).
// Per-tile strides: codes advance 64 (fp4) / 128 (fp8) bytes per macro tile;
// the scale column advances by 4: 4 bytes plain, one 512-byte col-block
// swizzled.
template <int ELEM, int NKC>
struct MxLane {
  LM_GLOBAL uint8_t* q;         // codes of the group's first row (in place: read and written)
  LM_GLOBAL uint8_t* sc;        // the item's scales (in place)
  const LM_GLOBAL uint8_t* at;  // the item's A^T (bytes)
  uint32_t q_off, sc_off, at_off, sc_stride;
};

// row0: the 16-row group's first row (wave-uniform, < M); rowc: the lane's
// row clamped to M - 1 (>= row0)
template <int ELEM, int NKC>
DEV MxLane<ELEM, NKC> mx_lane(const MxArgs& a, int64_t row0, int64_t rowc, int lane) {
  constexpr int RPAD = NKC * 16;
  constexpr int LB = MxTraits<ELEM>::lane_bytes;
  const int p = lane & 15, g = lane >> 4;
  const int64_t rowbytes = ELEM == E2M1 ? (a.N >> 1) : a.N;
  MxLane<ELEM, NKC> l;
  l.q = (LM_GLOBAL uint8_t*)a.q + row0 * rowbytes;
  l.q_off = (uint32_t)((rowc - row0) * rowbytes) + (uint32_t)(LB * g);
  l.sc = (LM_GLOBAL uint8_t*)a.scale;
  l.sc_off = (uint32_t)blocked_offset(rowc, g, a.N >> 5, a.swizzled);
  l.sc_stride = a.swizzled ? 512u : 4u;
  l.at = (const LM_GLOBAL uint8_t*)a.at;
  l.at_off = NKC == 1 ? 16u * (uint32_t)lane : 2u * ((uint32_t)(32 * (p >> 2) + (p & 3)) * RPAD + (uint32_t)g * (NKC * 4));
  return l;
}

template <int ELEM, int NKC>
DEV void mx_load_codes(const MxLane<ELEM, NKC>& l, int mt, MxTileIn<ELEM, NKC>& t) {
  constexpr int LB = MxTraits<ELEM>::lane_bytes;
  const LM_GLOBAL uint8_t* q = l.q + (l.q_off + (uint32_t)mt * (4u * LB));
#pragma unroll
  for (int i = 0; i < LB / 16; ++i) {
    const lm_u32x4 c = *(const LM_GLOBAL lm_u32x4*)(q + 16 * i);
    t.codes[i] = make_uint4(c.x, c.y, c.z, c.w);
  }
  t.sc = l.sc[l.sc_off + (uint32_t)mt * l.sc_stride];
}
template <int ELEM, int NKC>
DEV void mx_load_aop(const MxLane<ELEM, NKC>& l, int mt, MxTileIn<ELEM, NKC>& t) {
  constexpr int RPAD = NKC * 16;
  if constexpr (NKC == 1) {  // AT_NV16
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

template <int ELEM, int NKC, bool SR>
DEV void mx_tile(const MxArgs& a, const MxTileIn<ELEM, NKC>& in, const v4i16 (&bop)[NKC], int64_t row, int mt,
                 int lane, uint8_t* qo, uint8_t* so, bool rok) {
  constexpr float L = MxTraits<ELEM>::maxpos;
  float d[32];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const v4f32 acc = mfma_chain<NKC, false>(in.aop[k], bop);
    d[4 * k + 0] = acc[0];
    d[4 * k + 1] = acc[1];
    d[4 * k + 2] = acc[2];
    d[4 * k + 3] = acc[3];
  }
  const float s = e8m0_value(in.sc);
  float m[32];
  float amax = 0.0f;
  if constexpr (ELEM == E2M1) {
    const uint32_t w[4] = {in.codes[0].x, in.codes[0].y, in.codes[0].z, in.codes[0].w};
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const v2f32 pr = e2m1_pair(w[q >> 2], q & 3);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int j = 2 * q + e;
        m[j] = bf16r(__builtin_fmaf(d[j], a.strength, pr[e] * s));
        amax = __builtin_fmaxf(amax, __builtin_fabsf(m[j]));
      }
    }
  } else {
    const uint32_t w[8] = {in.codes[0].x, in.codes[0].y, in.codes[0].z, in.codes[0].w,
                           in.codes[1].x, in.codes[1].y, in.codes[1].z, in.codes[1].w};
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const float base = bf16r(fp8_decode<ELEM>(w[j >> 2], j & 3) * s);
      m[j] = bf16r(__builtin_fmaf(d[j], a.strength, base));
      amax = __builtin_fmaxf(amax, __builtin_fabsf(m[j]));
    }
  }
  float inv;
  const uint32_t enc = mx_scale(amax, a.mode, MxTraits<ELEM>::emax, L, MxTraits<ELEM>::mbits, inv);
  uint32_t nw[16];  // complemented Philox words
  if constexpr (SR) sr_nwords_aligned_lo<32>(a.seed, (uint32_t)((row * a.N + (int64_t)mt * 128 + 32 * (lane >> 4)) >> 3), nw);
  float x[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    // the e2m1 conversions saturate by themselves; fp8 ones need the clamp
    x[j] = ELEM == E2M1 ? m[j] * inv : __builtin_amdgcn_fmed3f(m[j] * inv, -L, L);
  }
  if constexpr (ELEM == E2M1) {
    uint32_t words[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (SR) {
        words[k] = sr_e2m1_nword(x + 8 * k, nw + 4 * k);
      } else {
        uint32_t wd = 0u;
        wd = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(wd, x[8 * k + 0], x[8 * k + 1], 1.0f, 0);
        wd = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(wd, x[8 * k + 2], x[8 * k + 3], 1.0f, 1);
        wd = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(wd, x[8 * k + 4], x[8 * k + 5], 1.0f, 2);
        wd = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(wd, x[8 * k + 6], x[8 * k + 7], 1.0f, 3);
        words[k] = wd;
      }
    }
    if (rok) *(uint4*)(qo + (int64_t)mt * 64) = make_uint4(words[0], words[1], words[2], words[3]);
  } else {
    uint32_t wv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (SR) wv[i] = sr_fp8_nword<ELEM>(x + 4 * i, nw + 2 * i);
      else wv[i] = fp8_pack4<ELEM>(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
    }
    if (rok) {
      uint4* dst = (uint4*)(qo + (int64_t)mt * 128);
      dst[0] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
      dst[1] = make_uint4(wv[4], wv[5], wv[6], wv[7]);
    }
  }
  if (rok) so[0] = (uint8_t)enc;
}

// Chunks of 16 tiles: for MXFP4 [14336, 4096] with 16-row workgroups, whole
// 32-tile rows measured 0.0398 ms per step (stochastic) against 0.0379
// (round-to-nearest 0.0326 against 0.0330).
constexpr int MX_CHUNK = 2 * NV_NW;
// Rows per workgroup: round to nearest takes two 16-row groups per wave
// (MXFP4 [14336, 4096]: 0.0325-0.0368 -> 0.028 ms per step, where the
// A^T address work bound it); stochastic rounding keeps one, since it is
// VALU-bound and the second group's registers cost it 2%.
template <bool SR>
constexpr int mx_rows_per_wg() { return SR ? 16 : 32; }
template <int ELEM, int NKC, bool SR>
__global__ __launch_bounds__(NV_NW * 64) void k_mx_fast(MxArgs a) {
  // (the per-lane wave index: wave_index() measured 2.7% slower here)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, rl = lane & 15;
  const int64_t row0 = (int64_t)blockIdx.x * mx_rows_per_wg<SR>();
  const int64_t row = row0 + rl, rowB = row0 + 16 + rl;
  const bool rok = row < a.M, rokB = rowB < a.M;
  const int64_t rowc = rok ? row : a.M - 1, rowcB = rokB ? rowB : a.M - 1;  // in-bounds loads; results dropped
  // the second group exists when row0 + 16 < M; its offsets are relative to
  // its first row, so they are formed (and its loads issued) only then
  const bool hasB = mx_rows_per_wg<SR>() == 32 && row0 + 16 < a.M;  // wave-uniform
  const int t0 = (int)blockIdx.y * MX_CHUNK;  // this workgroup's chunk of macro tiles
  const int ntiles = (int)((a.N >> 7) < t0 + MX_CHUNK ? (a.N >> 7) : t0 + MX_CHUNK);
  const MxLane<ELEM, NKC> l = mx_lane<ELEM, NKC>(a, row0, rowc, lane);
  const MxLane<ELEM, NKC> lB = mx_lane<ELEM, NKC>(a, hasB ? row0 + 16 : row0, hasB ? rowcB : rowc, lane);
  v4i16 bop[NKC], bopB[NKC];
  load_bop<NKC>(a.bp, row, lane, bop);  // Bp holds ceil(M/16)*16 rows
  load_bop<NKC>(a.bp, rowcB, lane, bopB);
  if (t0 + wave >= ntiles) return;
  // the next tile's codes and scales are requested before the current tile
  // is merged; its A^T fragments at the top of its own iteration
  MxTileIn<ELEM, NKC> cur, curB;
  mx_load_codes<ELEM, NKC>(l, t0 + wave, cur);
  if (hasB) mx_load_codes<ELEM, NKC>(lB, t0 + wave, curB);
  constexpr int LB = MxTraits<ELEM>::lane_bytes;
  for (int mt = t0 + wave; mt < ntiles; mt += NV_NW) {
    mx_load_aop<ELEM, NKC>(l, mt, cur);
    MxTileIn<ELEM, NKC> nxt, nxtB;
    const int mn = mt + NV_NW < ntiles ? mt + NV_NW : mt;
    mx_load_codes<ELEM, NKC>(l, mn, nxt);
    if (hasB) mx_load_codes<ELEM, NKC>(lB, mn, nxtB);
    // every lane merges (the MFMAs read all lanes' operands); rows past M store nothing
    mx_tile<ELEM, NKC, SR>(a, cur, bop, row, mt, lane, (uint8_t*)(l.q + l.q_off),
                           (uint8_t*)(l.sc + (l.sc_off + (uint32_t)mt * l.sc_stride)), rok);
    if (hasB) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int c = 0; c < NKC; ++c) curB.aop[k][c] = cur.aop[k][c];
      mx_tile<ELEM, NKC, SR>(a, curB, bopB, rowB, mt, lane, (uint8_t*)(lB.q + lB.q_off),
                             (uint8_t*)(lB.sc + (lB.sc_off + (uint32_t)mt * lB.sc_stride)), rokB);
    }
#pragma unroll
    for (int i = 0; i < LB / 16; ++i) {
      cur.codes[i] = nxt.codes[i];
      curB.codes[i] = nxtB.codes[i];
    }
    cur.sc = nxt.sc;
    curB.sc = nxtB.sc;
  }
}

// (M N <= 2^35: the stochastic-rounding counters, offset / 8, fit 32 bits;
// M N / 32 < 2^31 and N <= 2^22: scale, A^T and 16-row code offsets fit 32 bits)
static inline bool mx_fast_ok(int cd, int nkc, int64_t M, int64_t N) {
  return cd == LM_BF16 && nkc > 0 && (N % 128) == 0 && M * N <= (int64_t(1) << 35) && N <= (int64_t(1) << 22);
}

static int mx_fast_run(const MxArgs& a, int elem, int nkc, bool sr, hipStream_t st) {
  const int rows = sr ? mx_rows_per_wg<true>() : mx_rows_per_wg<false>();
  const dim3 grid((unsigned)((a.M + rows - 1) / rows), (unsigned)(((a.N >> 7) + MX_CHUNK - 1) / MX_CHUNK)),
      block(NV_NW * 64);
  TimedLaunch timed("mx", st);
#define MXL(E_, SR_) NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_mx_fast<E_, NKC_, SR_>), grid, block, 0, st, a))
  if (elem == LM_E2M1) { if (sr) { MXL(E2M1, true); } else { MXL(E2M1, false); } }
  else if (elem == LM_E4M3) { if (sr) { MXL(E4M3, true); } else { MXL(E4M3, false); } }
  else { if (sr) { MXL(E5M2, true); } else { MXL(E5M2, false); } }
#undef MXL
  LAUNCH_CHECK();
  return LM_OK;
}
