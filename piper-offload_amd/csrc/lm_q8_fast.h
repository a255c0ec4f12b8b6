// lm_q8_fast.h -- GGUF Q8_0 merge for bf16 factors and N % 128 == 0 (the
// production layout; config 4 is [13824, 5120]).  A Q8_0 block is 34 bytes,
// [fp16 d][32 x int8], 32 logical columns (P/gguf_dequant.py:57-61).
//
// A wave works on one 16-row x 128-column macro tile at a time (see
// k_q8_fast for how waves pick tiles), and a lane holds row (lane & 15) and
// the 32 columns 32*(lane >> 4) .. +31 of it -- exactly one Q8_0 block, so the block max, the new d and the codes never
// leave the lane.  Blocks start at even byte offsets; a lane reads its block
// through a dword-aligned 36-byte window (two 16-byte loads and one 4- or
// 2-byte load, never past the block's last byte) and writes it back as eight
// dword-aligned dwords plus one 2-byte store.  Every block is read and
// written by one lane, so the merge may run in place.
//
// Arithmetic (bf16 compute, as the generic block kernel):
//   base   = bf16(bf16(d) * q)                   (P/gguf_dequant.py:57-61)
//   merged = bf16(fma(delta, strength, base))
//   requant (ggml quantize_row_q8_0_ref): d' = amax / 127, id = d' ? 1/d' : 0,
//   q' = round-half-away(merged * id) or the stochastic choice, store fp16(d').
#pragma once
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

template <int NKC>
struct Q8TileIn {
  uint32_t win[9];
  v4i16 aop[8][NKC];
};

template <int NKC>
DEV void q8_load_tile(const uint8_t* wbase, int sh, const uint16_t* at, int mt, Q8TileIn<NKC>& t) {
  constexpr int RPAD = NKC * 16;
  typedef uint32_t u4a4 __attribute__((ext_vector_type(4), aligned(4)));
  const uint8_t* p = wbase + (int64_t)mt * 136;  // 4 blocks per macro tile
  const u4a4 v0 = *(const u4a4*)p, v1 = *(const u4a4*)(p + 16);
  t.win[0] = v0[0];
  t.win[1] = v0[1];
  t.win[2] = v0[2];
  t.win[3] = v0[3];
  t.win[4] = v1[0];
  t.win[5] = v1[1];
  t.win[6] = v1[2];
  t.win[7] = v1[3];
  // sh == 0: the block ends at byte 34 of the window
  t.win[8] = sh ? *(const uint32_t*)(p + 32) : (uint32_t)*(const uint16_t*)(p + 32);
  const uint16_t* a = at + (int64_t)mt * (128 * RPAD);
#pragma unroll
  for (int k = 0; k < 8; ++k) load_kchunks<NKC>(a + 4 * k * RPAD, t.aop[k]);
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

template <int NKC, bool SR>
DEV void q8_tile(const Q8Args& a, const Q8TileIn<NKC>& in, const v4i16 (&bop)[NKC], int sh, int64_t row, int mt,
                 int lane, uint8_t* wout) {
  float d[32];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const v4f32 acc = mfma_chain<NKC, false>(in.aop[k], bop);
    d[4 * k + 0] = acc[0];
    d[4 * k + 1] = acc[1];
    d[4 * k + 2] = acc[2];
    d[4 * k + 3] = acc[3];
  }
  // the block's 34 bytes from byte sh of the window: [d lo][d hi][q0..q31]
  uint32_t blk[9];
#pragma unroll
  for (int k = 0; k < 8; ++k) blk[k] = __builtin_amdgcn_alignbyte(in.win[k + 1], in.win[k], sh);
  blk[8] = in.win[8] >> (8 * sh);
  const float dd = bf16r(f16_val(blk[0] & 0xffffu));
  float m[32];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const int bi = j + 2;
    const float base = bf16r(dd * (float)(int8_t)(blk[bi >> 2] >> (8 * (bi & 3))));
    m[j] = bf16r(__builtin_fmaf(d[j], a.strength, base));
    amax = __builtin_fmaxf(amax, __builtin_fabsf(m[j]));
  }
  const float dq = amax / 127.0f;
  const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
  uint32_t rw[16];  // element j's 16-bit draw is half (j & 1) of rw[j >> 1]
  if constexpr (SR) sr_words_aligned<32>(a.seed, (uint64_t)(row * a.N + (int64_t)mt * 128 + 32 * (lane >> 4)), rw);
  uint32_t ob[9];
  ob[0] = (uint32_t)f16_bits(dq);
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const float x = m[j] * id;
    int q = round_half_away(x);
    if constexpr (SR) q = sr_int(x, q, (j & 1) ? (rw[j >> 1] >> 16) : (rw[j >> 1] & 0xffffu), -127.0f, 127.0f);
    const int bi = j + 2;
    if ((bi & 3) == 0) ob[bi >> 2] = 0u;
    ob[bi >> 2] |= ((uint32_t)q & 0xffu) << (8 * (bi & 3));
  }
  typedef uint32_t u4a4 __attribute__((ext_vector_type(4), aligned(4)));
  uint8_t* p = wout + (int64_t)mt * 136;
  if (sh == 0) {
    *(u4a4*)p = (u4a4){ob[0], ob[1], ob[2], ob[3]};
    *(u4a4*)(p + 16) = (u4a4){ob[4], ob[5], ob[6], ob[7]};
    *(uint16_t*)(p + 32) = (uint16_t)ob[8];
  } else {  // the block starts 2 bytes into the window: one short, then 8 aligned dwords
    *(uint16_t*)(p + 2) = (uint16_t)ob[0];
    uint32_t s[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) s[k] = __builtin_amdgcn_alignbyte(ob[k + 1], ob[k], 2);
    *(u4a4*)(p + 4) = (u4a4){s[0], s[1], s[2], s[3]};
    *(u4a4*)(p + 20) = (u4a4){s[4], s[5], s[6], s[7]};
  }
}

constexpr int Q8_NW = 4;

// Wave-persistent: the grid holds exactly the workgroups that fit on the GPU
// at once, and every wave walks the work items item = gwave, gwave + waves,
// ... where item = row_group * ntiles + tile (one 16-row x 128-column tile).
// Single tensors are too small to amortise a wave's launch over a few tiles
// (a [13824, 5120] tensor is 34560 tiles), so waves stay resident, prefetch
// their next item and the last round is at most one tile per wave.  Blocks are
// independent, so no two waves need each other's results.  A lane's block
// starts 2 * (g & 1) bytes past a dword boundary in every item (rows are
// 136k bytes long), so its window shift is fixed.
template <int NKC, bool SR>
__global__ __launch_bounds__(Q8_NW * 64) void k_q8_fast(Q8Args a) {
  const int lane = threadIdx.x & 63, rl = lane & 15, g = lane >> 4;
  constexpr int RPAD = NKC * 16;
  const int ntiles = (int)(a.N >> 7);
  const int64_t nitems = ((a.M + 15) / 16) * (int64_t)ntiles;
  const int64_t stride = (int64_t)gridDim.x * Q8_NW;
  int64_t item = (int64_t)blockIdx.x * Q8_NW + (threadIdx.x >> 6);
  if (item >= nitems) return;
  const int64_t rowbytes = a.N / 32 * 34;
  const int sh = 2 * (g & 1);
  const int p = lane & 15;
  const uint16_t* at = a.at + (int64_t)(32 * (p >> 2) + (p & 3)) * RPAD + g * (NKC * 4);
  // per item: the lane's row, its clamp (loads stay in bounds; rows past M store nothing) and window base
  auto locate = [&](int64_t it, int64_t& row, int& mt, int64_t& wofs) {
    const int64_t rg = it / ntiles;
    mt = (int)(it - rg * ntiles);
    row = rg * 16 + rl;
    const int64_t rowc = row < a.M ? row : a.M - 1;
    wofs = rowc * rowbytes + (int64_t)g * 34 - sh;
  };
  int64_t row, nrow;
  int mt, nmt;
  int64_t wofs, nwofs;
  locate(item, row, mt, wofs);
  Q8TileIn<NKC> cur;
  v4i16 bop[NKC];
  q8_load_tile<NKC>(a.q + wofs, sh, at, mt, cur);
  load_bop<NKC>(a.bp, row, lane, bop);  // Bp holds ceil(M/16)*16 rows
  for (;;) {
    const int64_t next = item + stride;
    const bool more = next < nitems;
    locate(more ? next : item, nrow, nmt, nwofs);
    Q8TileIn<NKC> nxt;
    v4i16 nbop[NKC];
    q8_load_tile<NKC>(a.q + nwofs, sh, at, nmt, nxt);
    load_bop<NKC>(a.bp, nrow, lane, nbop);
    if (row < a.M) q8_tile<NKC, SR>(a, cur, bop, sh, row, mt, lane, a.q_out + wofs);
    if (!more) break;
    item = next;
    row = nrow;
    mt = nmt;
    wofs = nwofs;
    cur = nxt;
    for (int k = 0; k < NKC; ++k) bop[k] = nbop[k];
  }
}

// workgroups resident at once on the current device for a kernel (cached per device)
template <int NKC, bool SR>
static unsigned q8_resident_grid() {
  static unsigned cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1024;
  if (cached[dev] == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_q8_fast<NKC, SR>, Q8_NW * 64, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 ||
        cus <= 0)
      return 1024;
    cached[dev] = (unsigned)(per_cu * cus);
  }
  return cached[dev];
}

static inline bool q8_fast_ok(int cd, int nkc, int64_t N) { return cd == LM_BF16 && nkc > 0 && (N % 128) == 0; }

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
