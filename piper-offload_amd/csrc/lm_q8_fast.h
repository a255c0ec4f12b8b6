// lm_q8_fast.h -- GGUF Q8_0 merge for bf16 factors and N % 128 == 0 (the
// production layout; config 4 is [13824, 5120]).  A Q8_0 block is 34 bytes,
// [fp16 d][32 x int8], 32 logical columns (P/gguf_dequant.py:57-61).
//
// A wave works on one 16-row x 128-column macro tile at a time (see
// k_q8_fast for how waves pick tiles), and a lane holds row (lane & 15) and
// the 32 columns 32*(lane >> 4) .. +31 of it -- exactly one Q8_0 block, so
// the block max, the new d and the codes never leave the lane.  The tile's
// bytes are 16 row segments of 136 bytes (rows are rowbytes apart, segments
// 8-byte aligned).  The wave reads them as 272 consecutive 8-byte chunks
// (17 per row, a few cache lines per instruction), stages them in its own
// LDS slot, and each lane reads its block from there through a dword-aligned
// 36-byte window (blocks start at even offsets).  The new blocks go back into
// the slot and out in the same chunks, so every byte is written once and the
// merge may run in place.
//
// Arithmetic (bf16 compute, as the generic block kernel):
//   base   = bf16(bf16(d) * q)                   (P/gguf_dequant.py:57-61)
//   merged = bf16(fma(delta, strength, base))
//   requant (ggml quantize_row_q8_0_ref): d' = amax / 127, id = d' ? 1/d' : 0,
//   q' = round-half-away(merged * id) or the stochastic choice, store fp16(d').
#pragma once
#include <atomic>

#include "lm_impl.h"

struct Q8Args {
  const uint8_t* q;  // [M, N/32*34] Q8_0 blocks in
  uint8_t* q_out;    // the same layout out (may alias q)
  const uint16_t* at;
  const uint16_t* bp;
  int64_t M, N;
  float strength;
  uint64_t seed;
};

// An item's bytes as the wave loads them: chunk c = lane + 64 i (i < 5) is
// bytes 8 (c % 17) .. + 7 of row c / 17 of the item's 16 x 136-byte segment
// (rows of the tile are rowbytes apart in memory); chunks 272.. do not exist.
struct Q8Raw {
  lm_u32x2 c[5];
};
constexpr int Q8_CHUNKS = 16 * 17;
constexpr int Q8_SLOT = 64 * 5 * 8;  // LDS bytes per wave: 320 chunks (272 used)
template <int NKC>
struct Q8Ops {
  v4i16 aop[8][NKC];
  v4i16 bop[NKC];
};

// A lane's addresses within one item: the item's row group and tile are
// wave-uniform (scalar bases); the lane parts are 32-bit offsets.
struct Q8Lane {
  uint32_t aoff;  // A^T operand offset (elements) within a tile
  uint32_t boff;  // Bp operand offset (elements) within a row group
};

// chunk offsets of the lane within a row group; rows at or past M read row
// M - 1 (their bytes are never stored)
DEV void q8_chunk_offsets(int lane, int rows_left, int64_t rowbytes, uint32_t (&off)[5]) {
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int c = lane + 64 * i < Q8_CHUNKS ? lane + 64 * i : 0;
    const int r = c / 17;
    const int rc = r < rows_left ? r : rows_left - 1;
    off[i] = (uint32_t)rc * (uint32_t)rowbytes + (uint32_t)(c - 17 * r) * 8u;
  }
}

DEV void q8_load_raw(const Q8Args& a, const uint32_t (&off)[5], int64_t rg, int mt, int64_t rowbytes, Q8Raw& t) {
  const LM_GLOBAL uint8_t* p = (const LM_GLOBAL uint8_t*)a.q + rg * 16 * rowbytes + (uint32_t)(mt * 136);
#pragma unroll
  for (int i = 0; i < 5; ++i) t.c[i] = *(const LM_GLOBAL lm_u32x2*)(p + off[i]);
}
template <int NKC>
DEV void q8_load_ops(const Q8Args& a, const Q8Lane& L, int64_t rg, int mt, Q8Ops<NKC>& t) {
  constexpr int RPAD = NKC * 16;
  const LM_GLOBAL uint16_t* at = (const LM_GLOBAL uint16_t*)a.at + (uint32_t)(mt * (128 * RPAD)) + L.aoff;
#pragma unroll
  for (int k = 0; k < 8; ++k) load_kchunks_g<NKC>(at + 4 * k * RPAD, t.aop[k]);
  load_kchunks_g<NKC>((const LM_GLOBAL uint16_t*)a.bp + rg * (16 * RPAD) + L.boff, t.bop);
}

// roundf(x) (half away from zero) for |x| < 2^23 in two instructions: adding
// 0.5 - 2^-25 with x's sign rounds every tie up to the next integer and never
// carries a non-tie across one, so truncation finishes it (checked against
// roundf for every float below 2^23).  Contraction stays off so that the add
// is not fused with the multiply producing x.
DEV int round_half_away(float x) {
#pragma clang fp contract(off)
  return (int)(x + __builtin_copysignf(0.49999997f, x));
}

// One item: the lane's block (row `row`, columns 128 mt + 32 g ..) merged,
// requantized and stored at `wout` (the window base of the output).
//
// Stochastic rounding of x = RN(m id) with the reference's rule (floor(x) or
// floor(x) + 1, up iff h 2^-16 < frac(x); x itself when it is an integer or
// outside (-127, 127), where the round-half-away code is +-127 since
// |x| <= 127 (1 + 2^-22)): with Y = 65536 x clamped to [-127, 127] 65536
// (exact: a power-of-two scaling of |x| < 2^7) and T = ceil(Y), the code is
// (T + 65535 - h) >> 16, whose low byte is bits 16..23 of T + 65535 - h.
template <int NKC, bool SR>
DEV void q8_tile(const Q8Args& a, const Q8Raw& raw, const Q8Ops<NKC>& in, uint8_t* slot, int sh, int64_t row,
                 int mt, int lane, int rows_left, const uint32_t (&off)[5], LM_GLOBAL uint8_t* p) {
  float d[32];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const v4f32 acc = mfma_chain<NKC, false>(in.aop[k], in.bop);
    d[4 * k + 0] = acc[0];
    d[4 * k + 1] = acc[1];
    d[4 * k + 2] = acc[2];
    d[4 * k + 3] = acc[3];
  }
  // stage the item's bytes in the wave's LDS slot (chunk c at byte 8 c, so
  // row r of the segment starts at byte 136 r), then read the lane's block
  // through its dword-aligned 36-byte window: [d lo][d hi][q0..q31] from byte sh
#pragma unroll
  for (int i = 0; i < 5; ++i) *(lm_u32x2*)(slot + 8 * (lane + 64 * i)) = raw.c[i];
  const int bofs = 136 * (lane & 15) + 34 * (lane >> 4);  // the block's first byte in the slot
  const uint32_t* wsrc = (const uint32_t*)(slot + bofs - sh);
  uint32_t win[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) win[k] = wsrc[k];
  uint32_t blk[9];
#pragma unroll
  for (int k = 0; k < 8; ++k) blk[k] = __builtin_amdgcn_alignbyte(win[k + 1], win[k], sh);
  blk[8] = win[8] >> (8 * sh);
  const float dd = bf16r(f16_val(blk[0] & 0xffffu));
  float m[32];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j += 2) {
    const int b0 = j + 2, b1 = j + 3;
    const float base0 = bf16r(dd * (float)(int8_t)(blk[b0 >> 2] >> (8 * (b0 & 3))));
    const float base1 = bf16r(dd * (float)(int8_t)(blk[b1 >> 2] >> (8 * (b1 & 3))));
    m[j] = bf16r(__builtin_fmaf(d[j], a.strength, base0));
    m[j + 1] = bf16r(__builtin_fmaf(d[j + 1], a.strength, base1));
    amax = max3_abs(amax, m[j], m[j + 1]);
  }
  const float dq = amax / 127.0f;
  const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
  uint32_t ob[9];
  ob[0] = (uint32_t)f16_bits(dq);
  if constexpr (SR) {
    uint32_t nw[16];  // 65535 - h of element j in nw[j >> 1]: even j high half, odd j low half
    sr_nwords_aligned_lo<32>(a.seed, (uint32_t)((row * a.N + (int64_t)mt * 128 + 32 * (lane >> 4)) >> 3), nw);
    // integer stochastic rounding on the 13-bit grid (sr_i8_pair); pair i
    // holds codes 2i and 2i + 1 in bytes 0 and 2
    uint32_t pr[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      pr[i] = sr_i8_pair(nw[i], sr_i8_t(m[2 * i], id, 1536.0f, 1409.0f, 1663.0f),
                         sr_i8_t(m[2 * i + 1], id, 1536.0f, 1409.0f, 1663.0f), nw[i], nw[i] << 16);
    // code j is byte 2 + j of the block: word (j + 2) >> 2
    ob[0] |= __builtin_amdgcn_perm(pr[0], pr[0], 0x06040c0cu);
#pragma unroll
    for (int k = 1; k < 8; ++k) ob[k] = pack_sr_i8(pr[2 * k - 1], pr[2 * k]);
    ob[8] = __builtin_amdgcn_perm(pr[15], pr[15], 0x0c0c0200u);
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int q = round_half_away(m[j] * id);
      const int bi = j + 2;
      if ((bi & 3) == 0) ob[bi >> 2] = 0u;
      ob[bi >> 2] |= ((uint32_t)q & 0xffu) << (8 * (bi & 3));
    }
  }
  // the new block back into the slot, then the segment out in chunks
  if (sh == 0) {
    uint32_t* d32 = (uint32_t*)(slot + bofs);
#pragma unroll
    for (int k = 0; k < 8; ++k) d32[k] = ob[k];
    *(uint16_t*)(slot + bofs + 32) = (uint16_t)ob[8];
  } else {  // the block starts 2 bytes into a dword: one short, then 8 aligned dwords
    *(uint16_t*)(slot + bofs) = (uint16_t)ob[0];
    uint32_t* d32 = (uint32_t*)(slot + bofs + 2);
#pragma unroll
    for (int k = 0; k < 8; ++k) d32[k] = __builtin_amdgcn_alignbyte(ob[k + 1], ob[k], 2);
  }
  (void)row;
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int c = lane + 64 * i;
    if (c < Q8_CHUNKS && (rows_left == 16 || c / 17 < rows_left))
      *(LM_GLOBAL lm_u32x2*)(p + off[i]) = *(const lm_u32x2*)(slot + 8 * c);
  }
}

constexpr int Q8_NW = 4;

// Wave-persistent: the grid holds exactly the workgroups that fit on the GPU
// at once, and every wave walks the work items item = gwave, gwave + waves,
// ... where item = row_group * ntiles + tile (one 16-row x 128-column tile).
// Single tensors are too small to amortise a wave's launch over a few tiles
// (a [13824, 5120] tensor is 34560 tiles), so waves stay resident and the last
// round is at most one tile per wave.  Blocks are independent, so no two
// waves need each other's results.  The item's row group and tile are
// wave-uniform and advance by the fixed stride without a division; two
// register sets alternate so that the next item's loads are in flight while
// the current one is merged (loads complete in order, so the wait for the
// current item never waits for the next).  A lane's block starts 2 (g & 1)
// bytes past a dword boundary in every item (rows are 136 k bytes long), so
// its window shift is fixed.
// the second bound is waves per SIMD: rank 16 fits 128 VGPRs (4 waves).
// Five waves (96 VGPRs) spill and run slower.
template <int NKC, bool SR>
constexpr int q8_min_waves() { return NKC == 1 ? 4 : 1; }

template <int NKC, bool SR>
__global__ __launch_bounds__(Q8_NW * 64, (q8_min_waves<NKC, SR>())) void k_q8_fast(Q8Args a) {
  const int lane = threadIdx.x & 63, rl = lane & 15, g = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int RPAD = NKC * 16;
  const int ntiles = (int)(a.N >> 7);
  const int64_t nrg = (a.M + 15) / 16;
  const int64_t stride = (int64_t)gridDim.x * Q8_NW;
  const int64_t item0 = (int64_t)blockIdx.x * Q8_NW + wv;
  if (item0 >= nrg * ntiles) return;
  int64_t rg = item0 / ntiles;
  int mt = (int)(item0 - rg * ntiles);
  const int64_t srg = stride / ntiles;
  const int smt = (int)(stride - srg * ntiles);
  auto advance = [&](int64_t& r, int& t) {
    t += smt;
    r += srg;
    if (t >= ntiles) {
      t -= ntiles;
      ++r;
    }
  };
  const int64_t rowbytes = a.N / 32 * 34;
  const int sh = 2 * (g & 1);
  const int p = lane & 15;
  __shared__ __attribute__((aligned(16))) uint8_t q8_lds[Q8_NW * Q8_SLOT];
  uint8_t* slot = q8_lds + wv * Q8_SLOT;  // the wave's own: no barriers
  Q8Lane L;
  L.aoff = (uint32_t)((32 * (p >> 2) + (p & 3)) * RPAD + g * (NKC * 4));
  L.boff = (uint32_t)(rl * RPAD + g * (NKC * 4));
  uint32_t off_full[5];
  q8_chunk_offsets(lane, 16, rowbytes, off_full);
  // chunk offsets of row group r (only the last one can be short)
  auto offsets = [&](int64_t r, uint32_t (&off)[5]) {
    const int64_t left = a.M - r * 16;
    if (left >= 16) {
#pragma unroll
      for (int i = 0; i < 5; ++i) off[i] = off_full[i];
    } else {
      q8_chunk_offsets(lane, (int)left, rowbytes, off);
    }
  };
  auto load_raw = [&](int64_t r, int tile, Q8Raw& t) {
    uint32_t off[5];
    offsets(r, off);
    q8_load_raw(a, off, r, tile, rowbytes, t);
  };
  auto run = [&](const Q8Raw& w, const Q8Ops<NKC>& t, int64_t r, int tile) {
    uint32_t off[5];
    offsets(r, off);
    LM_GLOBAL uint8_t* out = (LM_GLOBAL uint8_t*)a.q_out + r * 16 * rowbytes + (uint32_t)(tile * 136);
    const int64_t left = a.M - r * 16;
    q8_tile<NKC, SR>(a, w, t, slot, sh, r * 16 + rl, tile, lane, left < 16 ? (int)left : 16, off, out);
  };
  // the MFMA operands (L2-resident) are requested at the start of their own
  // item, then the next item's bytes, into alternating registers (loads
  // complete in order: waiting for the operands never waits for the next item)
  Q8Raw w0, w1;
  int64_t rg1 = rg;
  int mt1 = mt;
  advance(rg1, mt1);
  load_raw(rg, mt, w0);
#define Q8_STEP(WC, WN)                                   \
  {                                                       \
    Q8Ops<NKC> ops;                                       \
    q8_load_ops<NKC>(a, L, rg, mt, ops);                  \
    if (rg1 < nrg) load_raw(rg1, mt1, WN);                \
    run(WC, ops, rg, mt);                                 \
    if (rg1 >= nrg) break;                                \
    rg = rg1;                                             \
    mt = mt1;                                             \
    advance(rg1, mt1);                                    \
  }
  for (;;) {
    Q8_STEP(w0, w1)
    Q8_STEP(w1, w0)
  }
#undef Q8_STEP
}

// workgroups resident at once on the current device for a kernel (cached per
// device; callers on several host threads may race to fill an entry, which
// the atomic makes benign: they store the same value)
template <int NKC, bool SR>
static unsigned q8_resident_grid() {
  static std::atomic<unsigned> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1024;
  unsigned v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_q8_fast<NKC, SR>, Q8_NW * 64, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 ||
        cus <= 0)
      return 1024;
    v = (unsigned)(per_cu * cus);
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// (M N <= 2^35: the stochastic-rounding counters, offset / 8, fit 32 bits)
static inline bool q8_fast_ok(int cd, int nkc, int64_t M, int64_t N) {
  return cd == LM_BF16 && nkc > 0 && (N % 128) == 0 && M * N <= (int64_t(1) << 35);
}

static int q8_fast_run(const Q8Args& a, int nkc, bool sr, hipStream_t st) {
  const int64_t nitems = ((a.M + 15) / 16) * (a.N >> 7);
  const dim3 block(Q8_NW * 64);
  TimedLaunch timed("q8", st);
#define Q8L(SR_)                                                                                           \
  NKC_SWITCH(nkc_bucket(nkc), {                                                                            \
    const int64_t need = (nitems + Q8_NW - 1) / Q8_NW;                                                     \
    const unsigned res = q8_resident_grid<NKC_, SR_>();                                                    \
    hipLaunchKernelGGL((k_q8_fast<NKC_, SR_>), dim3((unsigned)(need < res ? need : res)), block, 0, st, a); \
  })
  if (sr) { Q8L(true); } else { Q8L(false); }
#undef Q8L
  LAUNCH_CHECK();
  return LM_OK;
}
