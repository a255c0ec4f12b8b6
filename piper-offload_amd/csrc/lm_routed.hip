// lm_routed.hip -- routed-LoRA residual: out = y + sum_i s_i ((x A_i^T) B_i^T + bias_i)
// (P/lora.py:801-829, _routed_residual), the inference path of the reference's
// routed mode, which adds the LoRA contribution after a Linear instead of
// merging it into the weight.
//
// The reference's operation order and roundings, all in the output dtype
// (bf16 or fp16) with fp32 matmul accumulation:
//   p_i    = dt(x A_i^T)                       [T, r_i]
//   ps_i   = dt(p_i s_i)
//   part_i = dt(ps_i B_i^T)                    [T, N]
//   part_i = dt(part_i + dt(bias_i s_i))       (when a bias is present)
//   total  = part_0, then dt(total + part_i)
//   out    = dt(y + total)
//
// At most 16 tokens (decode): one kernel, k_routed_small, and no workspace.
// Otherwise three:
// * k_routed_down: MFMA x A^T over a K split per workgroup; the partial sums
//   of all factors' rank chunks go to an fp32 workspace [S][T][C * 16]
//   (C = sum of ceil(r_i / 16));
// * k_routed_finalize: sums the S partials in split order and writes
//   ps = dt(dt(p) s) once per token, in the dtype, [T][C * 16];
// * k_routed_up: a wave keeps the B operands of one 64-column tile in
//   registers and walks 16-token tiles: one MFMA chain per factor, the rest
//   of the rounding chain and one read and one write of y / out: the only
//   traffic that scales with T N.
// Lane layout (the merge kernels' convention): a wave owns 16 tokens; lane l
// holds token l & 15 and columns 16 (l >> 4) .. + 15 of a 64-column tile.
#include "lm_impl.h"

namespace {

constexpr int RT_NW = 4;
constexpr int RT_MAX_FACTORS = 8;
constexpr int RT_MAX_CHUNKS = 16;  // sum of ceil(rank / 16) over the factors

struct RoutedArgs {
  const uint16_t* x;    // [T, K]
  const uint16_t* y;    // [T, N] (the Linear output)
  uint16_t* out;        // [T, N] (may alias y)
  float* part;          // [S][T][C * 16]
  uint16_t* ps;         // [T][C * 16]: dt(dt(p) s) of each factor's ranks (zero past the rank)
  int64_t T, K, N;
  int64_t kspan;        // K columns per split (multiple of 16)
  int S, nf, nchunks;
  int tiles_per_wg;     // token tiles per up workgroup
  const uint16_t* a[RT_MAX_FACTORS];
  const uint16_t* b[RT_MAX_FACTORS];
  const uint16_t* bias[RT_MAX_FACTORS];
  float s[RT_MAX_FACTORS];
  int rank[RT_MAX_FACTORS];
  int chunk0[RT_MAX_FACTORS];  // first rank chunk of factor i
  int cfac[RT_MAX_CHUNKS];     // factor of rank chunk c
};

// 4 consecutive 16-bit values from row `row` of a [rows, cols] matrix at
// column c (zero outside the matrix); 8-byte loads when cols % 4 == 0
__device__ __forceinline__ v4i16 load4(const uint16_t* p, int64_t rows, int64_t cols, int64_t row, int64_t c) {
  v4i16 v = {0, 0, 0, 0};
  if (row >= rows) return v;
  const uint16_t* q = p + row * cols + c;
  if ((cols & 3) == 0) {
    if (c + 3 < cols) v = __builtin_bit_cast(v4i16, *(const uint2*)q);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (c + i < cols) v[i] = (short)q[i];
  }
  return v;
}

typedef short rt_v8i16 __attribute__((ext_vector_type(8)));
typedef __bf16 rt_v8bf16 __attribute__((ext_vector_type(8)));
typedef _Float16 rt_v8f16 __attribute__((ext_vector_type(8)));

// 8 consecutive 16-bit values (zero outside the matrix); 16-byte loads when cols % 8 == 0
__device__ __forceinline__ rt_v8i16 load8(const uint16_t* p, int64_t rows, int64_t cols, int64_t row, int64_t c) {
  rt_v8i16 v = {0, 0, 0, 0, 0, 0, 0, 0};
  if (row >= rows) return v;
  const uint16_t* q = p + row * cols + c;
  if ((cols & 7) == 0) {
    if (c + 7 < cols) v = __builtin_bit_cast(rt_v8i16, *(const uint4*)q);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (c + i < cols) v[i] = (short)q[i];
  }
  return v;
}

// D = A B + C over K = 32: lane l supplies row l & 15, k = 8 (l >> 4) .. + 7
template <bool HALF>
__device__ __forceinline__ v4f32 mfma32(const rt_v8i16& a, const rt_v8i16& b, const v4f32& acc) {
  if constexpr (HALF)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(rt_v8f16, a), __builtin_bit_cast(rt_v8f16, b),
                                                  acc, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(rt_v8bf16, a), __builtin_bit_cast(rt_v8bf16, b),
                                                   acc, 0, 0, 0);
}

template <bool HALF>
__device__ __forceinline__ v4f32 mfma1(const v4i16& a, const v4i16& b, const v4f32& acc) {
  if constexpr (HALF)
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4f16, a), __builtin_bit_cast(v4f16, b), acc, 0,
                                                 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc, 0, 0, 0);
}

// grid (token tiles, S); RT_NW waves split the workgroup's K range.  For rank
// chunk c the MFMA computes D[r][t] = sum_k A_i[r][k] x[t][k]: lane l holds
// ranks 16 c' + 4 (l >> 4) + 0..3 of token l & 15.  The waves' sums meet in
// LDS, one chunk at a time, and wave 0 writes the split's partial.
template <bool HALF>
__global__ __launch_bounds__(RT_NW * 64) void k_routed_down(RoutedArgs a) {
  __shared__ float sh[RT_NW][64][4];
  const int lane = threadIdx.x & 63, wave = wave_index(), rl = lane & 15, g = lane >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * 16;
  const int split = blockIdx.y;
  const int64_t kb = (int64_t)split * a.kspan, ke = kb + a.kspan < a.K ? kb + a.kspan : a.K;
  for (int i = 0; i < a.nf; ++i) {
    const int nck = (a.rank[i] + 15) / 16;
    for (int cc = 0; cc < nck; ++cc) {
      // RT_DU K steps of 32 per round: their 16-byte loads are all issued
      // before the MFMAs (loads past K, the split or the rows read zeros)
      constexpr int RT_DU = 8;
      v4f32 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int64_t k0 = kb + 32 * wave; k0 < ke; k0 += 32 * RT_NW * RT_DU) {
        rt_v8i16 av[RT_DU], xv[RT_DU];
#pragma unroll
        for (int u = 0; u < RT_DU; ++u) {
          const int64_t k = k0 + (int64_t)u * 32 * RT_NW + 8 * g;
          const bool in = k < ke;
          av[u] = in ? load8(a.a[i], a.rank[i], a.K, 16 * cc + rl, k) : (rt_v8i16){0, 0, 0, 0, 0, 0, 0, 0};
          xv[u] = in ? load8(a.x, a.T, a.K, t0 + rl, k) : (rt_v8i16){0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < RT_DU; ++u) acc = mfma32<HALF>(av[u], xv[u], acc);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) sh[wave][lane][j] = acc[j];
      __syncthreads();
      const int64_t t = t0 + rl;
      if (wave == 0 && t < a.T) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float sum = 0.0f;
          for (int w = 0; w < RT_NW; ++w) sum += sh[w][lane][j];
          v[j] = sum;
        }
        const int c = a.chunk0[i] + cc;
        float* dst = a.part + ((int64_t)split * a.T + t) * (a.nchunks * 16) + c * 16 + 4 * g;
        *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
      }
      __syncthreads();
    }
  }
}

// one thread per (token, chunk, 4 ranks): sum the S partials in split order
// and apply p_i = dt(p), ps_i = dt(p_i s_i)
template <bool HALF>
__global__ __launch_bounds__(256) void k_routed_finalize(RoutedArgs a) {
  constexpr int DT = HALF ? F16 : BF16;
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (t, c, g)
  const int64_t per_t = (int64_t)a.nchunks * 4;
  if (q >= a.T * per_t) return;
  const int64_t t = q / per_t;
  const int rem = (int)(q - t * per_t), c = rem >> 2, g = rem & 3;
  const int64_t off = t * (a.nchunks * 16) + c * 16 + 4 * g;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int sp = 0; sp < a.S; ++sp) {
    const float4 w = *(const float4*)(a.part + (int64_t)sp * a.T * (a.nchunks * 16) + off);
    v[0] += w.x;
    v[1] += w.y;
    v[2] += w.z;
    v[3] += w.w;
  }
  const float s_ = a.s[a.cfac[c]];
  uint32_t w[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    w[h] = (uint32_t)bits_dt<DT>(round_dt<DT>(round_dt<DT>(v[2 * h]) * s_)) |
           ((uint32_t)bits_dt<DT>(round_dt<DT>(round_dt<DT>(v[2 * h + 1]) * s_)) << 16);
  *(uint2*)(a.ps + off) = make_uint2(w[0], w[1]);
}

// grid (column-tile groups, token groups).  Every wave owns one 64-column
// tile: its B operands (all rank chunks, CMAX at most) stay in registers
// while it walks the token tiles of its token group.  Per token tile it needs
// the partial sums of p (L2) and the Linear output y (HBM); both are
// requested one token tile ahead, after the current tile's own loads, so that
// waiting for the current tile never waits for the prefetch (loads complete
// in order).
template <bool HALF, int CMAX>
__global__ __launch_bounds__(RT_NW * 64) void k_routed_up(RoutedArgs a) {
  constexpr int DT = HALF ? F16 : BF16;
  const int lane = threadIdx.x & 63, wave = wave_index(), rl = lane & 15, g = lane >> 4;
  const int64_t mt = (int64_t)blockIdx.x * RT_NW + wave;  // the wave's column tile
  const int64_t ntiles = (a.N + 63) / 64;
  if (mt >= ntiles) return;
  const int64_t c0 = mt * 64 + 16 * g;  // the lane's 16 output columns
  const bool vec = (a.N & 7) == 0, full = vec && c0 + 16 <= a.N;
  // B operands: MFMA k4, chunk c: position p = lane & 15 is column
  // 16 (p >> 2) + 4 k4 + (p & 3), ranks 16 c' + 4 g + 0..3 of the chunk's factor
  v4i16 bo[CMAX][4];
  const int p = lane & 15;
#pragma unroll
  for (int c = 0; c < CMAX; ++c)
    if (c < a.nchunks) {
      const int i = a.cfac[c], cc = c - a.chunk0[i];
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4)
        bo[c][k4] = load4(a.b[i], a.N, a.rank[i], mt * 64 + 16 * (p >> 2) + 4 * k4 + (p & 3), 16 * cc + 4 * g);
    }
  // bias * s of the lane's columns, per factor (rounded once)
  const int64_t tiles = (a.T + 15) / 16;
  const int64_t tb = (int64_t)blockIdx.y * a.tiles_per_wg;
  const int64_t te = tb + a.tiles_per_wg < tiles ? tb + a.tiles_per_wg : tiles;
  const int64_t rowstride = (int64_t)a.nchunks * 16;
  // per token tile: the ps operands (token rl, 4 ranks per chunk) and y
  v4i16 pp[CMAX];
  uint4 y0 = make_uint4(0, 0, 0, 0), y1 = y0;
  auto load_tile = [&](int64_t tt, v4i16 (&pv)[CMAX], uint4& v0, uint4& v1) {
    const int64_t t = tt * 16 + rl;
    const bool ok = tt < te && t < a.T;
#pragma unroll
    for (int c = 0; c < CMAX; ++c) {
      pv[c] = (v4i16){0, 0, 0, 0};
      if (c < a.nchunks && ok) pv[c] = __builtin_bit_cast(v4i16, *(const uint2*)(a.ps + t * rowstride + c * 16 + 4 * g));
    }
    if (ok && full) {
      const uint4* yr4 = (const uint4*)(a.y + t * a.N + c0);
      v0 = yr4[0];
      v1 = yr4[1];
    }
  };
  load_tile(tb, pp, y0, y1);
  for (int64_t tt = tb; tt < te; ++tt) {
    const int64_t t = tt * 16 + rl;
    const bool tok = t < a.T;
    v4i16 ps[CMAX];
#pragma unroll
    for (int c = 0; c < CMAX; ++c) ps[c] = pp[c];
    const uint4 cy0 = y0, cy1 = y1;
    load_tile(tt + 1, pp, y0, y1);  // the next token tile, behind this one's loads
    float total[16];
    v4f32 acc[4];
#pragma unroll
    for (int c = 0; c < CMAX; ++c) {
      if (c < a.nchunks) {
        const int i = a.cfac[c], cc = c - a.chunk0[i];
        if (cc == 0) {
#pragma unroll
          for (int k4 = 0; k4 < 4; ++k4) acc[k4] = (v4f32){0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) acc[k4] = mfma1<HALF>(bo[c][k4], ps[c], acc[k4]);
        if (c + 1 == a.nchunks || a.cfac[c + 1] != i) {  // the factor's last chunk: its part is complete
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            float part = round_dt<DT>(acc[j >> 2][j & 3]);
            if (a.bias[i] && c0 + j < a.N)
              part = round_dt<DT>(part + round_dt<DT>(val_dt<DT>(a.bias[i][c0 + j]) * a.s[i]));
            total[j] = i == 0 ? part : round_dt<DT>(total[j] + part);
          }
        }
      }
    }
    if (!tok || c0 >= a.N) continue;
    uint16_t* orow = a.out + t * a.N + c0;
    if (full) {
      const uint32_t yw[8] = {cy0.x, cy0.y, cy0.z, cy0.w, cy1.x, cy1.y, cy1.z, cy1.w};
      uint32_t ow[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float lo = round_dt<DT>(val_dt<DT>(yw[k] & 0xffffu) + total[2 * k]);
        const float hi = round_dt<DT>(val_dt<DT>(yw[k] >> 16) + total[2 * k + 1]);
        ow[k] = (uint32_t)bits_dt<DT>(lo) | ((uint32_t)bits_dt<DT>(hi) << 16);
      }
      ((uint4*)orow)[0] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      ((uint4*)orow)[1] = make_uint4(ow[4], ow[5], ow[6], ow[7]);
    } else {
      const uint16_t* yr = a.y + t * a.N + c0;
      for (int j = 0; j < 16 && c0 + j < a.N; ++j) orow[j] = bits_dt<DT>(round_dt<DT>(val_dt<DT>(yr[j]) + total[j]));
    }
  }
}

// ---- one launch for at most 16 tokens (decode) ---------------------------------
// Three launches cost more than their work when T is small.  Here every
// workgroup computes the whole down projection of the one token tile (its
// RT_SNW waves split K, one round of RT_DU loads each at K = 4096; the sums
// meet in LDS), applies the first two roundings into LDS, then each wave
// finishes one 64-column tile as k_routed_up does.  The wave's y values and
// (for at most two rank chunks) B operands are requested before the down
// projection, so their latency overlaps it.  Every workgroup recomputes the
// down projection (x and A are read from L2 after the first).
constexpr int RT_SNW = 16;

template <bool HALF, int CMAX>
__global__ __launch_bounds__(RT_SNW * 64) void k_routed_small(RoutedArgs a) {
  constexpr int DT = HALF ? F16 : BF16;
  constexpr bool PRE = CMAX <= 2;  // B operands loaded up front
  __shared__ float sh[RT_SNW][64][4];
  __shared__ uint32_t spw[16][RT_MAX_CHUNKS * 8];      // ps of token t: ranks 2j, 2j + 1 in word j
  const int lane = threadIdx.x & 63, wave = wave_index(), rl = lane & 15, g = lane >> 4;
  const int64_t mt = (int64_t)blockIdx.x * RT_SNW + wave;
  const bool tile = mt < (a.N + 63) / 64;
  const int64_t c0 = mt * 64 + 16 * g, t = rl;
  const bool tok = tile && t < a.T, full = (a.N & 7) == 0 && c0 + 16 <= a.N;
  const int p = lane & 15;
  uint4 y0 = make_uint4(0, 0, 0, 0), y1 = y0;
  if (tok && full) {
    const uint4* yr4 = (const uint4*)(a.y + t * a.N + c0);
    y0 = yr4[0];
    y1 = yr4[1];
  }
  v4i16 bo[PRE ? CMAX : 1][4];
  if constexpr (PRE) {
#pragma unroll
    for (int c = 0; c < CMAX; ++c) {
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) bo[c][k4] = (v4i16){0, 0, 0, 0};
      if (tile && c < a.nchunks) {
        const int i = a.cfac[c], cc = c - a.chunk0[i];
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4)
          bo[c][k4] = load4(a.b[i], a.N, a.rank[i], mt * 64 + 16 * (p >> 2) + 4 * k4 + (p & 3), 16 * cc + 4 * g);
      }
    }
  }
  constexpr int RT_DU = 8;
  for (int c = 0; c < a.nchunks; ++c) {
    const int i = a.cfac[c], cc = c - a.chunk0[i];
    v4f32 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t k0 = 32 * wave; k0 < a.K; k0 += 32 * RT_SNW * RT_DU) {
      rt_v8i16 av[RT_DU], xv[RT_DU];
#pragma unroll
      for (int u = 0; u < RT_DU; ++u) {
        const int64_t k = k0 + (int64_t)u * 32 * RT_SNW + 8 * g;
        const bool in = k < a.K;
        av[u] = in ? load8(a.a[i], a.rank[i], a.K, 16 * cc + rl, k) : (rt_v8i16){0, 0, 0, 0, 0, 0, 0, 0};
        xv[u] = in ? load8(a.x, a.T, a.K, rl, k) : (rt_v8i16){0, 0, 0, 0, 0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < RT_DU; ++u) acc = mfma32<HALF>(av[u], xv[u], acc);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) sh[wave][lane][j] = acc[j];
    __syncthreads();
    if (wave == 0) {  // lane: token rl, ranks 16 cc + 4 g + 0..3
      uint32_t w2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float v[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          float sum = 0.0f;
          for (int w = 0; w < RT_SNW; ++w) sum += sh[w][lane][2 * h + e];
          v[e] = round_dt<DT>(round_dt<DT>(sum) * a.s[i]);
        }
        w2[h] = (uint32_t)bits_dt<DT>(v[0]) | ((uint32_t)bits_dt<DT>(v[1]) << 16);
      }
      spw[rl][c * 8 + 2 * g] = w2[0];
      spw[rl][c * 8 + 2 * g + 1] = w2[1];
    }
    __syncthreads();
  }
  if (!tile) return;
  float total[16];
  v4f32 acc[4];
#pragma unroll
  for (int c = 0; c < CMAX; ++c) {
    if (c < a.nchunks) {
      const int i = a.cfac[c], cc = c - a.chunk0[i];
      if (cc == 0) {
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) acc[k4] = (v4f32){0.0f, 0.0f, 0.0f, 0.0f};
      }
      const v4i16 psv = __builtin_bit_cast(v4i16, make_uint2(spw[rl][c * 8 + 2 * g], spw[rl][c * 8 + 2 * g + 1]));
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) {
        v4i16 bv;
        if constexpr (PRE)
          bv = bo[c][k4];
        else
          bv = load4(a.b[i], a.N, a.rank[i], mt * 64 + 16 * (p >> 2) + 4 * k4 + (p & 3), 16 * cc + 4 * g);
        acc[k4] = mfma1<HALF>(bv, psv, acc[k4]);
      }
      if (c + 1 == a.nchunks || a.cfac[c + 1] != i) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          float part = round_dt<DT>(acc[j >> 2][j & 3]);
          if (a.bias[i] && c0 + j < a.N)
            part = round_dt<DT>(part + round_dt<DT>(val_dt<DT>(a.bias[i][c0 + j]) * a.s[i]));
          total[j] = i == 0 ? part : round_dt<DT>(total[j] + part);
        }
      }
    }
  }
  if (!tok || c0 >= a.N) return;
  uint16_t* orow = a.out + t * a.N + c0;
  if (full) {
    const uint32_t yw[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
    uint32_t ow[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float lo = round_dt<DT>(val_dt<DT>(yw[k] & 0xffffu) + total[2 * k]);
      const float hi = round_dt<DT>(val_dt<DT>(yw[k] >> 16) + total[2 * k + 1]);
      ow[k] = (uint32_t)bits_dt<DT>(lo) | ((uint32_t)bits_dt<DT>(hi) << 16);
    }
    ((uint4*)orow)[0] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    ((uint4*)orow)[1] = make_uint4(ow[4], ow[5], ow[6], ow[7]);
  } else {
    const uint16_t* yr = a.y + t * a.N + c0;
    for (int j = 0; j < 16 && c0 + j < a.N; ++j) orow[j] = bits_dt<DT>(round_dt<DT>(val_dt<DT>(yr[j]) + total[j]));
  }
}

// K splits of the down projection: about 2048 workgroups in all (the kernel
// streams x, so it needs occupancy), at least 256 columns of K per split
int64_t routed_splits(int64_t T, int64_t K) {
  const int64_t tiles = (T + 15) / 16;
  int64_t S = (K + 255) / 256;
  const int64_t want = (2048 + tiles - 1) / (tiles > 0 ? tiles : 1);
  if (S > want) S = want;
  return S < 1 ? 1 : S;
}

}  // namespace

extern "C" size_t lm_routed_workspace_size(int64_t T, int64_t K, const lm_routed_factor* factors, int32_t count) {
  if (T <= 16) return 0;  // the single-launch path keeps everything in LDS
  int chunks = 0;
  for (int i = 0; i < count && factors; ++i) chunks += (factors[i].rank + 15) / 16;
  const int64_t S = routed_splits(T, K);
  const size_t tt = (size_t)(T > 0 ? T : 0) * (size_t)chunks * 16;
  return align256((size_t)S * tt * sizeof(float)) + align256(tt * sizeof(uint16_t)) + 256;
}

extern "C" int lm_routed_residual(const void* x, const void* y, void* out, int64_t T, int64_t K, int64_t N,
                                  int32_t dtype, const lm_routed_factor* factors, int32_t count, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (!x || !y || !out || !factors) return fail(LM_EINVAL, "routed residual pointers must be non-null");
  if (T < 0 || K <= 0 || N <= 0) return fail(LM_EINVAL, "routed residual needs K, N > 0 and T >= 0");
  if (dtype != LM_BF16 && dtype != LM_F16)
    return fail(LM_EUNSUPPORTED, "routed residual dtype must be bfloat16 or float16, got dtype id %d", dtype);
  if (count < 1 || count > RT_MAX_FACTORS)
    return fail(LM_EUNSUPPORTED, "routed residual takes 1..%d factors, got %d", RT_MAX_FACTORS, count);
  if ((K & 3) != 0) return fail(LM_EUNSUPPORTED, "routed residual needs in_features %% 4 == 0, got %lld", (long long)K);
  if ((((uintptr_t)x) & 7) != 0) return fail(LM_EINVAL, "routed residual input must be 8-byte aligned");
  RoutedArgs a;
  memset(&a, 0, sizeof a);
  int chunks = 0;
  for (int i = 0; i < count; ++i) {
    const lm_routed_factor& f = factors[i];
    if (!f.a || !f.b) return fail(LM_EINVAL, "routed factor %d has a null A or B", i);
    if (f.rank <= 0 || f.rank > 64) return fail(LM_EUNSUPPORTED, "routed factor %d rank %d outside 1..64", i, f.rank);
    if ((((uintptr_t)f.a) & 7) != 0 || (((uintptr_t)f.b) & 7) != 0)
      return fail(LM_EINVAL, "routed factor %d must be 8-byte aligned", i);
    a.a[i] = (const uint16_t*)f.a;
    a.b[i] = (const uint16_t*)f.b;
    a.bias[i] = (const uint16_t*)f.bias;
    a.s[i] = f.strength;
    a.rank[i] = f.rank;
    a.chunk0[i] = chunks;
    const int nck = (f.rank + 15) / 16;
    if (chunks + nck > RT_MAX_CHUNKS)
      return fail(LM_EUNSUPPORTED, "routed factors need more than %d rank chunks of 16", RT_MAX_CHUNKS);
    for (int c = chunks; c < chunks + nck; ++c) a.cfac[c] = i;
    chunks += nck;
  }
  if (T == 0) return LM_OK;
  const size_t need = lm_routed_workspace_size(T, K, factors, count);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(LM_EWORKSPACE, "routed residual workspace too small: %zu < %zu bytes", workspace_bytes, need);
  if (((uintptr_t)workspace & 255) != 0) return fail(LM_EINVAL, "workspace must be 256-byte aligned");
  const int64_t tiles = (T + 15) / 16;
  const int64_t S = routed_splits(T, K);
  a.x = (const uint16_t*)x;
  a.y = (const uint16_t*)y;
  a.out = (uint16_t*)out;
  a.part = (float*)workspace;
  a.ps = (uint16_t*)((uint8_t*)workspace + align256((size_t)S * (size_t)T * (size_t)chunks * 16 * sizeof(float)));
  a.T = T;
  a.K = K;
  a.N = N;
  a.S = (int)S;
  a.kspan = ((K + S - 1) / S + 15) / 16 * 16;
  a.nf = count;
  a.nchunks = chunks;
  // up kernel: one 64-column tile per wave, token tiles split into groups so
  // that there are about 4096 waves in all
  const int64_t ntiles = (N + 63) / 64;
  const int64_t colgroups = (ntiles + RT_NW - 1) / RT_NW;
  int64_t tgroups = (4096 + ntiles - 1) / ntiles;
  if (tgroups > tiles) tgroups = tiles;
  if (tgroups < 1) tgroups = 1;
  a.tiles_per_wg = (int)((tiles + tgroups - 1) / tgroups);
  tgroups = (tiles + a.tiles_per_wg - 1) / a.tiles_per_wg;
  if (tiles > 0x7fffffff || S > 65535 || tgroups > 65535 || colgroups > 0x7fffffff)
    return fail(LM_EUNSUPPORTED, "routed residual grid too large");
  hipStream_t st = (hipStream_t)stream;
  TimedLaunch timed("routed", st);
  const dim3 block(RT_NW * 64);
  if (T <= 16) {  // one token tile: a single launch
    const dim3 sgrid((unsigned)((ntiles + RT_SNW - 1) / RT_SNW)), sblock(RT_SNW * 64);
#define RT_SM(H_)                                                                                 \
  if (chunks <= 1) hipLaunchKernelGGL((k_routed_small<H_, 1>), sgrid, sblock, 0, st, a);      \
  else if (chunks <= 2) hipLaunchKernelGGL((k_routed_small<H_, 2>), sgrid, sblock, 0, st, a); \
  else if (chunks <= 4) hipLaunchKernelGGL((k_routed_small<H_, 4>), sgrid, sblock, 0, st, a); \
  else hipLaunchKernelGGL((k_routed_small<H_, RT_MAX_CHUNKS>), sgrid, sblock, 0, st, a);
    if (dtype == LM_F16) { RT_SM(true) } else { RT_SM(false) }
#undef RT_SM
    LAUNCH_CHECK();
    return LM_OK;
  }
  const dim3 ugrid((unsigned)colgroups, (unsigned)tgroups);
#define RT_UP(H_)                                                                                    \
  if (chunks <= 1) hipLaunchKernelGGL((k_routed_up<H_, 1>), ugrid, block, 0, st, a);                \
  else if (chunks <= 2) hipLaunchKernelGGL((k_routed_up<H_, 2>), ugrid, block, 0, st, a);           \
  else if (chunks <= 4) hipLaunchKernelGGL((k_routed_up<H_, 4>), ugrid, block, 0, st, a);           \
  else hipLaunchKernelGGL((k_routed_up<H_, RT_MAX_CHUNKS>), ugrid, block, 0, st, a);
  const dim3 fgrid((unsigned)((T * chunks * 4 + 255) / 256));
  if (dtype == LM_F16) {
    hipLaunchKernelGGL(k_routed_down<true>, dim3((unsigned)tiles, (unsigned)S), block, 0, st, a);
    hipLaunchKernelGGL(k_routed_finalize<true>, fgrid, dim3(256), 0, st, a);
    RT_UP(true)
  } else {
    hipLaunchKernelGGL(k_routed_down<false>, dim3((unsigned)tiles, (unsigned)S), block, 0, st, a);
    hipLaunchKernelGGL(k_routed_finalize<false>, fgrid, dim3(256), 0, st, a);
    RT_UP(false)
  }
#undef RT_UP
  LAUNCH_CHECK();
  return LM_OK;
}
