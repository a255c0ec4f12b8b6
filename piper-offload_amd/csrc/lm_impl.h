#pragma once
// lm_impl.h -- MI355X (gfx950) kernels and C ABI for piper-offload's
// LoRA-merge hot path.  See include/lora_merge.h for the entry points and
// the reference functions each one replaces (P/ = src/piper_offload/).
//
// Kernel families
//   k_prep      : stages B and A into the MFMA-ready layouts Bp / At and
//                 clears the reduction slots (one launch per call or stack).
//   k_rows      : per-row qparam formats (INT8 per-row, scaled FP8 per-row).
//                 One workgroup owns 16 full rows; its waves split the
//                 columns, keep merged bf16 values of up to CACHE macro tiles
//                 in registers, reduce the row amax/min through LDS, then
//                 quantize (recomputing tiles that did not fit the cache).
//   k_rows_split: per-row INT8 / FP8 rows too long for a workgroup's
//                 registers at rank above 32: an amax pass into per-row
//                 workspace slots, then a pass that merges again and
//                 quantizes, each over freely tiled 64-column tiles.
//   k_blocks    : block-local formats (NVFP4 block 16, MX block 32, GGUF
//                 Q8_0 block 32), dense bf16 weights, dequantize-to-dense,
//                 and the two passes of per-tensor / two-level formats.
// Every element's delta comes from the same MFMA chain (tile_delta), so a
// fused merge and the dense merge of the same inputs see identical values.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "../../include/lora_merge.h"
#include "lm_device.h"

using namespace lm;

// ---------------------------------------------------------------------------
// error plumbing (thread-local message, defined in lm_common.hip)
// ---------------------------------------------------------------------------
int lm_fail_v(int code, const char* fmt, va_list ap);
static inline int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
static inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  int rc = lm_fail_v(code, fmt, ap);
  va_end(ap);
  return rc;
}
#define HIP_TRY(expr)                                                                        \
  do {                                                                                       \
    hipError_t e_ = (expr);                                                                  \
    if (e_ != hipSuccess) return fail(LM_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)
#define LAUNCH_CHECK() HIP_TRY(hipGetLastError())

// ---------------------------------------------------------------------------
// workspace layout (per tensor): At | Bp | reduction slots
// ---------------------------------------------------------------------------
static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
static inline int rpad_of(int rank) { return rank <= 0 ? 0 : (rank <= 16 ? 16 : (rank <= 32 ? 32 : 64)); }
static inline int64_t npad_of(int64_t N) { return (N + 127) / 128 * 128; }
static inline int64_t mpad_of(int64_t M) { return (M + 15) / 16 * 16; }

// reduction slots: 64 words for the block formats' per-tensor passes, then
// (for the two-pass long-row kernels) Mpad words of row amax bits and Mpad
// copies of the input row scales
// then, for the pruned per-tensor amax of two-level NVFP4: the Euclidean norms
// of B's rows and A's columns (Mpad + Npad floats) and one upper bound of
// max |merged| per 16-row x 128-column tile
struct WsLayout {
  size_t at_off, bp_off, red_off, nrm_off, ub_off, total;
};
static inline int64_t red_words(int64_t M) { return 64 + 2 * mpad_of(M); }
static inline int64_t ub_words(int64_t M, int64_t N) { return mpad_of(M) / 16 * (npad_of(N) / 128); }
static WsLayout ws_layout(int64_t M, int64_t N, int rank) {
  WsLayout w;
  int rp = rpad_of(rank);
  w.at_off = 0;
  w.bp_off = align256((size_t)npad_of(N) * rp * 2);
  w.red_off = w.bp_off + align256((size_t)mpad_of(M) * rp * 2);
  w.nrm_off = w.red_off + align256((size_t)red_words(M) * 4);
  w.ub_off = w.nrm_off + align256((size_t)(mpad_of(M) + npad_of(N)) * 4);
  w.total = w.ub_off + align256((size_t)ub_words(M, N) * 4);
  return w;
}

// ---------------------------------------------------------------------------
// prep: factors -> MFMA-ready layouts, clear reduction slots
// ---------------------------------------------------------------------------
struct PrepItem {
  const uint16_t* b;
  const uint16_t* a;
  int64_t ldb, lda;
  int64_t M, N;
  int rank, rpad;
  uint16_t* at;
  uint16_t* bp;
  uint32_t* red;
  int64_t nred;        // leading words of red to clear: 64, or 64 + Mpad for the two-pass rows
  int64_t work_begin;  // prefix of per-item work units (k_prep1: 0)
  int64_t block_begin; // prefix of per-item k_prep_many workgroups
  int vec_b;           // B rows load 4 ranks at once (ldb, rank % 4 == 0, 8-byte aligned)
  int at_order;        // At order: AT_PLAIN, AT_ROWS16 (row kernels, rank 16), AT_NV16 (NVFP4 kernels, rank 16)
  float* nrm;          // with norms: ||B_i|| for rows [0, Mpad), then ||A_j|| for columns [0, Npad)
  int norms;           // bf16 factors: compute nrm (the pruned NVFP4 amax bounds the delta by them)
  float* ub;           // the item's tile-bound region (not written by prep)
};

// At for the per-row kernels at rank <= 16 (RPAD 16): per 64-column tile,
// 1024 elements ordered [h][lane][kk][i], so that lane l's A^T fragments of
// the tile's 4 MFMAs (k = 2h + kk) arrive in two 16-byte loads, each load
// of the wave covering 1 KiB contiguously.  Lane l = p + 16 g takes column
// 16 (p >> 2) + 4 k + (p & 3) of the tile at ranks 4 g + i (the same
// columns and ranks as the plain At[col][g][kc][i] order).
__host__ __device__ inline int64_t at_rows16_offset(int64_t col, int g) {
  const int c = (int)(col & 63), k = (c >> 2) & 3, lane = ((c >> 4) << 2) + (c & 3) + 16 * g;
  return (col >> 6) * 1024 + (((k >> 1) * 64 + lane) * 2 + (k & 1)) * 4;
}
// At for the NVFP4 kernels at rank <= 16 (RPAD 16): per 128-column macro
// tile, 2048 elements ordered [kp][lane][kk][i], so that lane l's A^T
// fragments of the tile's 8 MFMAs (k = 2 kp + kk) arrive in four 16-byte
// loads, each load of the wave covering 1 KiB contiguously.  Lane
// l = p + 16 g takes column 32 (p >> 2) + 4 k + (p & 3) of the tile at ranks
// 4 g + i (the columns and ranks of the plain order).
__host__ __device__ inline int64_t at_nv16_offset(int64_t col, int g) {
  const int c = (int)(col & 127), r = c & 31, k = r >> 2, lane = ((c >> 5) << 2) + (r & 3) + 16 * g;
  return (col >> 7) * 2048 + ((k >> 1) * 64 + lane) * 8 + (k & 1) * 4;
}
enum : int { AT_PLAIN = 0, AT_ROWS16 = 1, AT_NV16 = 2 };

__device__ __forceinline__ void prep_unit(const PrepItem& it, int64_t u) {
  // units: [0, Npad*rpad/4) for At, then [.., + Mpad*rpad/4) for Bp, then 1
  // for red.  rpad is 16, 32 or 64: a unit is (column or row, g, kc) with
  // rpad/4 units per column or row and rpad/16 chunks kc.
  const int64_t npad = (it.N + 127) / 128 * 128, mpad = (it.M + 15) / 16 * 16;
  const int lq = it.rpad == 16 ? 2 : (it.rpad == 32 ? 3 : 4), lk = lq - 2;  // log2(rpad/4), log2(nkc)
  const int64_t n_at = npad * it.rpad / 4, n_bp = mpad * it.rpad / 4;          // 0 without factors
  const int nkc = it.rpad >> 4;
  if (u < n_at) {
    // At[col][g][kc][i]
    const int64_t col = u >> lq;
    const int rem = (int)(u & ((1 << lq) - 1));
    const int g = rem >> lk, kc = rem & (nkc - 1);
    uint16_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = kc * 16 + 4 * g + i;
      v[i] = (k < it.rank && col < it.N) ? ((const LM_GLOBAL uint16_t*)it.a)[(int64_t)k * it.lda + col] : (uint16_t)0;
    }
    const lm_u32x2 w = {(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16)};
    const int64_t off = it.at_order == AT_ROWS16 ? at_rows16_offset(col, g)
                      : it.at_order == AT_NV16 ? at_nv16_offset(col, g) : col * it.rpad + (g * nkc + kc) * 4;
    *(LM_GLOBAL lm_u32x2*)((LM_GLOBAL uint16_t*)it.at + off) = w;
    return;
  }
  u -= n_at;
  if (u < n_bp) {
    const int64_t row = u >> lq;
    const int rem = (int)(u & ((1 << lq) - 1));
    const int g = rem >> lk, kc = rem & (nkc - 1);
    const int k0 = kc * 16 + 4 * g;
    const LM_GLOBAL uint16_t* b = (const LM_GLOBAL uint16_t*)it.b;
    lm_u32x2 w = {0u, 0u};
    if (it.vec_b) {
      if (row < it.M && k0 < it.rank) w = *(const LM_GLOBAL lm_u32x2*)(b + row * it.ldb + k0);
    } else {
      uint16_t v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = k0 + i;
        v[i] = (k < it.rank && row < it.M) ? b[row * it.ldb + k] : (uint16_t)0;
      }
      w = lm_u32x2{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16)};
    }
    *(LM_GLOBAL lm_u32x2*)((LM_GLOBAL uint16_t*)it.bp + row * it.rpad + (g * nkc + kc) * 4) = w;
    return;
  }
  u -= n_bp;
  const int64_t n_red = (it.nred + 63) / 64;
  if (u < n_red) {
    if (it.red) {  // unit u clears words [64 u, 64 u + 64) (nred is a multiple of 16)
      LM_GLOBAL lm_u32x4* r = (LM_GLOBAL lm_u32x4*)it.red + 16 * u;
      const int n4 = (int)((it.nred - 64 * u) >> 2) < 16 ? (int)((it.nred - 64 * u) >> 2) : 16;
      for (int i = 0; i < n4; ++i) r[i] = lm_u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  u -= n_red;
  // norms (bf16 factors): sqrt of the fp32 sum of squares, raised by 2^-16
  // relative so that it bounds the true norm (the sum's rounding and the
  // square root's error are far below that); padding rows and columns are 0
  const LM_GLOBAL uint16_t* src;
  int64_t stride;
  bool live;
  if (u < mpad) {
    live = u < it.M;
    src = (const LM_GLOBAL uint16_t*)it.b + (live ? u * it.ldb : 0);
    stride = 1;
  } else {
    const int64_t col = u - mpad;
    live = col < it.N;
    src = (const LM_GLOBAL uint16_t*)it.a + (live ? col : 0);
    stride = it.lda;
  }
  // (B rows 8 bytes per load, A columns unrolled by 8, so that a thread's
  // loads are in flight together: with one 2-byte load per rank step the 8B
  // NVFP4 stack's prep launch took 108 us, now 60 us)
  float ss = 0.0f;
  if (live && stride == 1 && it.vec_b) {  // a B row, 4 ranks (8 bytes) per load
    const LM_GLOBAL lm_u32x2* s2 = (const LM_GLOBAL lm_u32x2*)src;
    for (int k4 = 0; k4 < it.rank / 4; k4 += 4) {
      lm_u32x2 w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = k4 + j < it.rank / 4 ? s2[k4 + j] : lm_u32x2{0u, 0u};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v0 = bf16_lo(w[j].x), v1 = bf16_hi(w[j].x), v2 = bf16_lo(w[j].y), v3 = bf16_hi(w[j].y);
        ss = __builtin_fmaf(v0, v0, ss);
        ss = __builtin_fmaf(v1, v1, ss);
        ss = __builtin_fmaf(v2, v2, ss);
        ss = __builtin_fmaf(v3, v3, ss);
      }
    }
  } else if (live) {
    int k = 0;
    for (; k + 8 <= it.rank; k += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = u2f((uint32_t)src[(k + j) * stride] << 16);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(v[j], v[j], ss);
    }
    for (; k < it.rank; ++k) {
      const float v = u2f((uint32_t)src[k * stride] << 16);
      ss = __builtin_fmaf(v, v, ss);
    }
  }
  ((LM_GLOBAL float*)it.nrm)[u] = live ? __builtin_sqrtf(ss) * (1.0f + 0x1p-16f) : 0.0f;
}

// B rows can be read 4 ranks (8 bytes) at a time
static inline int prep_vec_b(const PrepItem& it) {
  return it.b && (it.ldb % 4) == 0 && (it.rank % 4) == 0 && ((uintptr_t)it.b & 7) == 0 ? 1 : 0;
}
__host__ __device__ static inline int64_t prep_units(const PrepItem& it) {
  const int64_t npad = (it.N + 127) / 128 * 128, mpad = (it.M + 15) / 16 * 16;
  return npad * it.rpad / 4 + mpad * it.rpad / 4 + (it.nred + 63) / 64 + (it.norms ? mpad + npad : 0);
}

static __global__ __launch_bounds__(256) void k_prep1(PrepItem it, int64_t total) {
  for (int64_t u = blockIdx.x * 256ll + threadIdx.x; u < total; u += (int64_t)gridDim.x * 256) prep_unit(it, u);
}
// One workgroup per PREP_PER_BLOCK units of one item: the item is found once
// per workgroup (block_begin), not per unit.
static constexpr int PREP_PER_BLOCK = 1024;
static __global__ __launch_bounds__(256) void k_prep_many(const PrepItem* __restrict__ items, int count) {
  int lo = 0, hi = count - 1;
  const int64_t b = blockIdx.x;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (items[mid].block_begin <= b) lo = mid;
    else hi = mid - 1;
  }
  const PrepItem& it = items[lo];
  const int64_t units = prep_units(it);
  const int64_t u0 = (b - it.block_begin) * PREP_PER_BLOCK;
#pragma unroll
  for (int j = 0; j < PREP_PER_BLOCK / 256; ++j) {
    const int64_t u = u0 + j * 256 + threadIdx.x;
    if (u < units) prep_unit(it, u);
  }
}

int launch_prep(const PrepItem& it, hipStream_t st);
// asynchronous host -> device copy through pinned staging (lm_common.hip)
int lm_stage_h2d(void* dst, const void* src, size_t bytes, hipStream_t st);

// kernel timer (lm_timer_enable / lm_timer_read): bracket a launch on `st`
bool lm_timer_on();
void lm_timer_mark(const char* family, hipStream_t st, bool begin);
struct TimedLaunch {
  const char* family;
  hipStream_t st;
  bool on;
  TimedLaunch(const char* f, hipStream_t s) : family(f), st(s), on(lm_timer_on()) {
    if (on) lm_timer_mark(family, st, true);
  }
  ~TimedLaunch() {
    if (on) lm_timer_mark(family, st, false);
  }
};

// ---------------------------------------------------------------------------
// shared argument blocks
// ---------------------------------------------------------------------------
enum RowKind : int { K_INT8 = 0, K_E4M3 = 1, K_E5M2 = 2 };

struct RowArgs {
  const void* q;         // int8 / fp8 codes [M, N]
  const void* scale;     // per-row (or per-tensor) scale, storage dtype scale_dt
  const int8_t* zp;      // int8 zero point or null
  const uint16_t* dense; // requant-only input (compute dtype)
  void* q_out;
  void* scale_out;
  int8_t* zp_out;
  const uint16_t* at;
  const uint16_t* bp;
  int64_t M, N;
  float strength;
  int qmin, qmax;
  uint64_t seed;
  uint32_t* red;         // two-pass long rows: the workspace reduction slots (null otherwise)
};

template <int KIND>
struct FmtLimit;
template <>
struct FmtLimit<K_E4M3> {
  static constexpr float v = 448.0f;
  static constexpr int fmt = E4M3;
};
template <>
struct FmtLimit<K_E5M2> {
  static constexpr float v = 57344.0f;
  static constexpr int fmt = E5M2;
};

// per-row quantization parameters
struct RowQP {
  float s, inv, rcp, zp;
};

// INT8 qparams (P/_triton_int8_lora.py:123-186) -- computed by one thread
template <int CD, int SDT, bool ASYM>
__device__ RowQP int8_qparams(float mn, float mx, int qmin, int qmax, float& stored_scale, int& zp_out) {
  mn = round_dt<CD>(mn);
  mx = round_dt<CD>(mx);
  float scale;
  if constexpr (ASYM) {
    float range = round_dt<CD>(mx - mn);
    scale = range / (float)(qmax - qmin);
  } else {
    scale = __builtin_fmaxf(-mn, mx) / ((float)(qmax - qmin) / 2.0f);
  }
  scale = round_dt<CD>(scale);
  scale = __builtin_fmaxf(scale, kEps);
  scale = round_dt<CD>(scale);
  int zp = 0;
  if constexpr (ASYM) {
    float ratio = round_dt<CD>(mn / scale);
    zp = qmin - (int)__builtin_rintf(ratio);
    zp = zp < qmin ? qmin : (zp > qmax ? qmax : zp);
  }
  stored_scale = scale;
  zp_out = zp;
  RowQP qp;
  qp.s = round_dt<SDT>(scale);  // the quantize step reads the stored qparam
  qp.inv = round_dt<SDT>(1.0f / qp.s);
  qp.rcp = 1.0f / qp.s;
  qp.zp = (float)zp;
  return qp;
}

// FP8 qparams (P/_triton_float8_lora.py:249-271)
template <int CD, int KIND>
__device__ RowQP fp8_qparams(float amax, float& stored_scale) {
  float scale = round_dt<CD>(amax / FmtLimit<KIND>::v);
  if (scale == 0.0f) scale = kEps;
  stored_scale = scale;
  RowQP qp;
  qp.s = scale;
  qp.inv = 0.0f;
  qp.rcp = 1.0f / scale;
  qp.zp = 0.0f;
  return qp;
}

// ---- row-format tile: load 16 codes (or dense values) and merge -------------
template <int KIND, int CD, int SDT, int NKC, bool FROM_DENSE, bool HAS_LORA>
__device__ __forceinline__ void row_merged_tile(const RowArgs& a, int64_t row, bool rok, int64_t c0, int lane,
                                                int64_t mt_col0, const v4i16 (&bop)[NKC], float s_in, float z_in,
                                                float (&m)[16]) {
  const int64_t N = a.N;
  const bool full = rok && (c0 + 16 <= N) && ((N & 15) == 0);
  if constexpr (FROM_DENSE) {
    if (full) {
      const uint4* p = (const uint4*)(a.dense + row * N + c0);
      uint4 w0 = p[0], w1 = p[1];
      uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int j = 0; j < 16; ++j) m[j] = val_dt<CD>((j & 1) ? (w[j >> 1] >> 16) : (w[j >> 1] & 0xffffu));
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) m[j] = (rok && c0 + j < N) ? val_dt<CD>(a.dense[row * N + c0 + j]) : 0.0f;
    }
    return;
  } else {
    uint32_t w[4];
    if (full) {
      uint4 v = *(const uint4*)((const uint8_t*)a.q + row * N + c0);
      w[0] = v.x;
      w[1] = v.y;
      w[2] = v.z;
      w[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t x = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          int64_t c = c0 + 4 * i + b;
          if (rok && c < N) x |= (uint32_t)((const uint8_t*)a.q)[row * N + c] << (8 * b);
        }
        w[i] = x;
      }
    }
    float d[16];
    if constexpr (HAS_LORA) tile_delta<16, NKC, CD == F16>(a.at, mt_col0, lane, bop, d);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float base;
      if constexpr (KIND == K_INT8) {
        int qv = (int)(int8_t)(w[j >> 2] >> (8 * (j & 3)));
        base = round_dt<CD>(((float)qv - z_in) * s_in);
      } else {
        base = round_dt<CD>(fp8_decode<FmtLimit<KIND>::fmt>(w[j >> 2], j & 3) * s_in);
      }
      float v = base;
      if constexpr (HAS_LORA) v = round_dt<CD>(__builtin_fmaf(d[j], a.strength, base));
      const bool valid = rok && (c0 + j < N);
      m[j] = valid ? v : 0.0f;
    }
  }
}

template <int KIND, int SDT, bool SR>
__device__ __forceinline__ void row_quant_store(const RowArgs& a, int64_t row, bool rok, int64_t c0, const RowQP& qp,
                                                const float (&m)[16]) {
  const int64_t N = a.N;
  if (!rok || c0 >= N) return;
  const bool full = (c0 + 16 <= N) && ((N & 15) == 0);
  uint32_t h[16];
  if constexpr (SR) sr_bits<16>(a.seed, (uint64_t)(row * N + c0), h);
  uint32_t w[4];
  if constexpr (KIND == K_INT8) {
    int codes[16];
    if constexpr (SR) {
      // integer stochastic rounding on the 13-bit grid (sr_i8_pair)
      const float lo = 1536.0f + (float)a.qmin, hi = 1536.0f + (float)a.qmax, base = 1536.0f + qp.zp;
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        const uint32_t pr = sr_i8_pair(h[j], sr_i8_t(m[j], qp.rcp, base, lo, hi),
                                       sr_i8_t(m[j + 1], qp.rcp, base, lo, hi), (65535u - h[j]) << 16,
                                       (65535u - h[j + 1]) << 16);
        codes[j] = (int)(int8_t)(pr & 0xffu);
        codes[j + 1] = (int)(int8_t)((pr >> 16) & 0xffu);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float x = round_dt<SDT>(m[j] * qp.inv);
        int q = (int)__builtin_rintf(x) + (int)qp.zp;
        codes[j] = q < a.qmin ? a.qmin : (q > a.qmax ? a.qmax : q);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)(codes[4 * i] & 0xff) | ((uint32_t)(codes[4 * i + 1] & 0xff) << 8) |
             ((uint32_t)(codes[4 * i + 2] & 0xff) << 16) | ((uint32_t)(codes[4 * i + 3] & 0xff) << 24);
  } else {
    constexpr float L = FmtLimit<KIND>::v;
    constexpr int F = FmtLimit<KIND>::fmt;
    float x[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] = __builtin_fminf(__builtin_fmaxf(div_rn(m[j], qp.s, qp.rcp), -L), L);
    if constexpr (SR) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = sr_fp8<F>(x[4 * i], h[4 * i], L) | (sr_fp8<F>(x[4 * i + 1], h[4 * i + 1], L) << 8) |
               (sr_fp8<F>(x[4 * i + 2], h[4 * i + 2], L) << 16) | (sr_fp8<F>(x[4 * i + 3], h[4 * i + 3], L) << 24);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = fp8_pack4<F>(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
    }
  }
  uint8_t* dst = (uint8_t*)a.q_out + row * N + c0;
  if (full) {
    *(uint4*)dst = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    for (int j = 0; j < 16 && c0 + j < N; ++j) dst[j] = (uint8_t)(w[j >> 2] >> (8 * (j & 3)));
  }
}

// ---- k_rows: per-row formats ------------------------------------------------
template <int KIND, int CD, int SDT, bool ASYM, bool SR, int NKC, bool FROM_DENSE, int NW, int CACHE>
__device__ __forceinline__ void rows_body(const RowArgs& a, int64_t row0, int scale_dt) {
  __shared__ float sh_mx[NW][16];
  __shared__ float sh_mn[NW][16];
  __shared__ float sh_qp[4][16];
  const int lane = threadIdx.x & 63, wave = wave_index(), rl = lane & 15, g = lane >> 4;
  const int64_t row = row0 + rl;
  const bool rok = row < a.M;
  const int64_t N = a.N;
  const int ntiles = (int)((N + 63) >> 6);

  v4i16 bop[NKC];
  float s_in = 0.0f, z_in = 0.0f;
  if constexpr (!FROM_DENSE) {
    load_bop<NKC>(a.bp, row, lane, bop);
    if (rok) {
      s_in = load_scalar(a.scale, row, scale_dt);
      if (KIND == K_INT8 && a.zp) z_in = (float)a.zp[row];
    }
  }

  uint32_t cache[CACHE][8];
  float vmx = 0.0f, vmn = 0.0f;
  auto account = [&](const float (&m)[16]) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if constexpr (KIND == K_INT8) {
        vmx = __builtin_fmaxf(vmx, m[j]);
        vmn = __builtin_fminf(vmn, m[j]);
      } else {
        vmx = __builtin_fmaxf(vmx, __builtin_fabsf(m[j]));
      }
    }
  };
  // pass 1: merge, cache, reduce
#pragma unroll
  for (int i = 0; i < CACHE; ++i) {
    const int mt = wave + i * NW;
    if (mt < ntiles) {
      float m[16];
      row_merged_tile<KIND, CD, SDT, NKC, FROM_DENSE, !FROM_DENSE>(a, row, rok, (int64_t)mt * 64 + 16 * g, lane,
                                                                    (int64_t)mt * 64, bop, s_in, z_in, m);
      account(m);
#pragma unroll
      for (int k = 0; k < 8; ++k) cache[i][k] = (uint32_t)bits_dt<CD>(m[2 * k]) | ((uint32_t)bits_dt<CD>(m[2 * k + 1]) << 16);
    }
  }
  for (int mt = wave + CACHE * NW; mt < ntiles; mt += NW) {
    float m[16];
    row_merged_tile<KIND, CD, SDT, NKC, FROM_DENSE, !FROM_DENSE>(a, row, rok, (int64_t)mt * 64 + 16 * g, lane,
                                                                  (int64_t)mt * 64, bop, s_in, z_in, m);
    account(m);
  }
  vmx = lanes_max32(lanes_max16(vmx));
  if constexpr (KIND == K_INT8) vmn = lanes_min32(lanes_min16(vmn));
  if (g == 0) {
    sh_mx[wave][rl] = vmx;
    sh_mn[wave][rl] = vmn;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int t = threadIdx.x;
    float mx = 0.0f, mn = 0.0f;
    for (int w = 0; w < NW; ++w) {
      mx = __builtin_fmaxf(mx, sh_mx[w][t]);
      mn = __builtin_fminf(mn, sh_mn[w][t]);
    }
    const int64_t r = row0 + t;
    RowQP qp;
    float stored;
    if constexpr (KIND == K_INT8) {
      int zp;
      qp = int8_qparams<CD, SDT, ASYM>(mn, mx, a.qmin, a.qmax, stored, zp);
      if (r < a.M) {
        store_scalar(a.scale_out, r, SDT, stored);
        if (a.zp_out) a.zp_out[r] = (int8_t)zp;
      }
    } else {
      qp = fp8_qparams<CD, KIND>(mx, stored);
      if (r < a.M) ((float*)a.scale_out)[r] = stored;
    }
    sh_qp[0][t] = qp.s;
    sh_qp[1][t] = qp.inv;
    sh_qp[2][t] = qp.rcp;
    sh_qp[3][t] = qp.zp;
  }
  __syncthreads();
  RowQP qp;
  qp.s = sh_qp[0][rl];
  qp.inv = sh_qp[1][rl];
  qp.rcp = sh_qp[2][rl];
  qp.zp = sh_qp[3][rl];
  // pass 2: quantize cached tiles, recompute the rest
#pragma unroll
  for (int i = 0; i < CACHE; ++i) {
    const int mt = wave + i * NW;
    if (mt < ntiles) {
      float m[16];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        m[2 * k] = val_dt<CD>(cache[i][k] & 0xffffu);
        m[2 * k + 1] = val_dt<CD>(cache[i][k] >> 16);
      }
      row_quant_store<KIND, SDT, SR>(a, row, rok, (int64_t)mt * 64 + 16 * g, qp, m);
    }
  }
  for (int mt = wave + CACHE * NW; mt < ntiles; mt += NW) {
    float m[16];
    row_merged_tile<KIND, CD, SDT, NKC, FROM_DENSE, !FROM_DENSE>(a, row, rok, (int64_t)mt * 64 + 16 * g, lane,
                                                                  (int64_t)mt * 64, bop, s_in, z_in, m);
    row_quant_store<KIND, SDT, SR>(a, row, rok, (int64_t)mt * 64 + 16 * g, qp, m);
  }
}

template <int KIND, int CD, int SDT, bool ASYM, bool SR, int NKC, bool FROM_DENSE, int NW, int CACHE>
__global__ __launch_bounds__(NW * 64) void k_rows(RowArgs a, int scale_dt) {
  rows_body<KIND, CD, SDT, ASYM, SR, NKC, FROM_DENSE, NW, CACHE>(a, (int64_t)blockIdx.x * 16, scale_dt);
}

// stack: items[] in device memory, tile_begin[] = prefix of row tiles
struct RowStackItem {
  RowArgs a;
  int64_t tile_begin;
};
template <int KIND, int CD, int SDT, bool SR, int NKC, int NW, int CACHE>
__global__ __launch_bounds__(NW * 64) void k_rows_stack(const RowStackItem* __restrict__ items, int count,
                                                        int scale_dt) {
  int lo = 0, hi = count - 1;
  const int64_t t = blockIdx.x;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (items[mid].tile_begin <= t) lo = mid;
    else hi = mid - 1;
  }
  const RowArgs a = items[lo].a;
  rows_body<KIND, CD, SDT, false, SR, NKC, false, NW, CACHE>(a, (t - items[lo].tile_begin) * 16, scale_dt);
}


// ---- fast per-row kernels -----------------------------------------------------
// Specialization of rows_body for the production layouts: bf16 factors,
// N % 64 == 0, INT8 symmetric with fp32 scales or scaled FP8 (fp32 scales).
// Merged values stay packed bf16 (v_cvt_pk_bf16_f32) from pass 1 to pass 2;
// the row amax is a running fp32 max of |merged| before the bf16 rounding
// (rounding is monotone, so bf16(max |m|) = max |bf16(m)|), one v_max3 per
// pair; round-to-nearest uses the 1.5*2^23 magic add; INT8 stochastic
// rounding works on the integer grid (an exact reformulation of the
// reference's u < p selection) and FP8 stochastic rounding uses the hardware
// conversions (sr_fp8_nword).
// Global inputs of one 64-column macro tile for one lane: 16 codes of its row
// and the 4 A^T operands of its MFMAs.  Loading is split from the arithmetic
// so that a wave can have several tiles' loads in flight.
template <int NKC>
struct FastTileIn {
  uint4 raw;
  v4i16 aop[4][NKC];
};

// A lane's addresses, computed once per row group, as 32-bit offsets from the
// wave-uniform tensor bases (the fast kernels need M N < 2^32): tile mt adds
// 64 mt code bytes, 64 mt RPAD A^T elements and 8 mt Philox blocks, all
// wave-uniform, so a tile's loads and store are global_load/store with a
// scalar base, one offset register and an immediate.
struct FastLane {
  const LM_GLOBAL uint8_t* q;    // codes (uniform)
  LM_GLOBAL uint8_t* out;        // output codes (uniform)
  const LM_GLOBAL uint16_t* at;  // prepared A^T (uniform)
  uint32_t off;                  // (clamped row) N + 16 (lane >> 4)
  uint32_t aoff;                 // the lane's A^T operand offset in tile 0
  uint32_t ctr;                  // Philox counter of the lane's first offset in tile 0 (even)
};

template <int NKC, bool R16 = false>
__device__ __forceinline__ FastLane fast_lane(const RowArgs& a, int64_t rowc, int lane) {
  constexpr int RPAD = NKC * 16;
  static_assert(!R16 || NKC == 1, "the rows16 operand order is for rank 16");
  const int p = lane & 15, g = lane >> 4;
  FastLane L;
  L.q = (const LM_GLOBAL uint8_t*)a.q;
  L.out = (LM_GLOBAL uint8_t*)a.q_out;
  L.at = (const LM_GLOBAL uint16_t*)a.at;
  L.off = (uint32_t)rowc * (uint32_t)a.N + 16u * (uint32_t)g;
  L.aoff = R16 ? (uint32_t)lane * 8u : (uint32_t)((16 * (p >> 2) + (p & 3)) * RPAD + g * (NKC * 4));
  // N % 64 == 0: off / 8 is even, so the lane's second Philox block (offsets
  // +8 .. +15) is counter | 1; rows past M never store, so their counter is moot
  L.ctr = L.off >> 3;
  return L;
}

__device__ __forceinline__ uint4 fast_load_codes(const FastLane& L, int mt) {
  const lm_u32x4 raw = *(const LM_GLOBAL lm_u32x4*)(L.q + (uint32_t)(mt * 64) + L.off);
  return make_uint4(raw.x, raw.y, raw.z, raw.w);
}
template <int NKC, bool R16 = false>
__device__ __forceinline__ void fast_load_aop(const FastLane& L, int mt, v4i16 (&aop)[4][NKC]) {
  constexpr int RPAD = NKC * 16;
  const LM_GLOBAL uint16_t* at = L.at + (uint32_t)(mt * (64 * RPAD)) + L.aoff;
  if constexpr (R16) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const lm_u32x4 w = *(const LM_GLOBAL lm_u32x4*)(at + 512 * h);
      aop[2 * h][0] = __builtin_bit_cast(v4i16, lm_u32x2{w.x, w.y});
      aop[2 * h + 1][0] = __builtin_bit_cast(v4i16, lm_u32x2{w.z, w.w});
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) load_kchunks_g<NKC>(at + 4 * k * RPAD, aop[k]);
  }
}
template <int NKC, bool R16 = false>
__device__ __forceinline__ void fast_load_tile(const FastLane& L, int mt, FastTileIn<NKC>& t) {
  t.raw = fast_load_codes(L, mt);
  fast_load_aop<NKC, R16>(L, mt, t.aop);
}

// the 16 deltas of a lane's share of one 16 x 64 tile (4 MFMA chains)
template <int NKC>
__device__ __forceinline__ void fast_tile_delta(const v4i16 (&aop)[4][NKC], const v4i16 (&bop)[NKC], float (&d)[16]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const v4f32 acc = mfma_chain<NKC, false>(aop[k], bop);
    d[4 * k + 0] = acc[0];
    d[4 * k + 1] = acc[1];
    d[4 * k + 2] = acc[2];
    d[4 * k + 3] = acc[3];
  }
}
// merged values of one tile before their bf16 rounding into m[16], given the
// codes and deltas; with AMAX, amax = max(amax, |m|) (the maximum of the
// bf16-rounded values is bf16r of it)
// LUT: INT8 only, lut = the lane's row of bf16(RN(q s)) for the 256 code
// bytes (rows_fast_body), read instead of converting and scaling each code
template <int KIND, bool AMAX = true, bool LUT = false>
__device__ __forceinline__ void fast_merge_vals(const RowArgs& a, const uint4& raw, const float (&d)[16], float s_in,
                                                float (&m)[16], float& amax, const float* lut = nullptr) {
  static_assert(!LUT || KIND == K_INT8, "the dequant table is for INT8 codes");
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t word = w[k >> 1];
    float x0, x1;
    if constexpr (LUT) {
      const int b0 = (2 * k) & 3, b1 = (2 * k + 1) & 3;
      const float base0 = lut[(word >> (8 * b0)) & 0xffu], base1 = lut[(word >> (8 * b1)) & 0xffu];
      m[2 * k] = __builtin_fmaf(d[2 * k], a.strength, base0);
      m[2 * k + 1] = __builtin_fmaf(d[2 * k + 1], a.strength, base1);
      if constexpr (AMAX) amax = max3_abs(amax, m[2 * k], m[2 * k + 1]);
      continue;
    } else if constexpr (KIND == K_INT8) {
      // signed byte -> fp32 is one sign-extending SDWA convert; RN(q * s)
      const int b0 = (2 * k) & 3, b1 = (2 * k + 1) & 3;
      x0 = (float)(int8_t)(word >> (8 * b0)) * s_in;
      x1 = (float)(int8_t)(word >> (8 * b1)) * s_in;
    } else {
      const v2f32 c = (k & 1) ? fp8_decode_pair<FmtLimit<KIND>::fmt, true>(word)
                              : fp8_decode_pair<FmtLimit<KIND>::fmt, false>(word);
      x0 = c.x * s_in;
      x1 = c.y * s_in;
    }
    m[2 * k] = __builtin_fmaf(d[2 * k], a.strength, bf16r(x0));
    m[2 * k + 1] = __builtin_fmaf(d[2 * k + 1], a.strength, bf16r(x1));
    if constexpr (AMAX) amax = max3_abs(amax, m[2 * k], m[2 * k + 1]);
  }
}
template <int KIND, int NKC, bool AMAX = true, bool LUT = false>
__device__ __forceinline__ void fast_merged_f32(const RowArgs& a, const uint4& raw, const v4i16 (&aop)[4][NKC],
                                                const v4i16 (&bop)[NKC], float s_in, float (&m)[16], float& amax,
                                                const float* lut = nullptr) {
  float d[16];
  fast_tile_delta<NKC>(aop, bop, d);
  fast_merge_vals<KIND, AMAX, LUT>(a, raw, d, s_in, m, amax, lut);
}
// merged bf16 pairs of one tile into out[8]; amax = max(amax, |merged|) in fp32
template <int KIND, int NKC, bool LUT = false>
__device__ __forceinline__ void fast_merged_tile(const RowArgs& a, const uint4& raw, const v4i16 (&aop)[4][NKC],
                                                 const v4i16 (&bop)[NKC], float s_in,
                                                 uint32_t (&out)[8], float& amax, const float* lut = nullptr) {
  float m[16];
  fast_merged_f32<KIND, NKC, true, LUT>(a, raw, aop, bop, s_in, m, amax, lut);
#pragma unroll
  for (int k = 0; k < 8; ++k) out[k] = pack_bf16x2(m[2 * k], m[2 * k + 1]);
}

// quantize and store one tile given its bf16-valued merged values m[16];
// old[i] is any register the INT8 stochastic path may overwrite for pair i
// SBF: INT8 qparams stored in bf16 (the reference rounds the quantize step's
// v * RN(1 / s) to the qparam dtype, P/_triton_int8_lora.py:190-236)
template <int KIND, bool SR, bool SBF = false>
__device__ __forceinline__ void fast_quant_store_vals(const RowArgs& a, const FastLane& L, bool rok, int mt,
                                                      const RowQP& qp, const float (&m)[16], const uint32_t (&old)[8]) {
  if (!rok) return;
  uint32_t nw[8];  // complemented Philox words: 65535 - h in each half
  if constexpr (SR) sr_nwords16_even(a.seed, L.ctr + 8u * (uint32_t)mt, nw);
  uint32_t out[4];
  if constexpr (KIND == K_INT8) {
    uint32_t y[16];
    if constexpr (SR) {
      // integer stochastic rounding on the 13-bit grid (sr_i8_pair): the word
      // nw[i] holds 65535 - h of elements 2i (high half) and 2i + 1 (low
      // half), which are the random operands' top bits
      const float lo = 1536.0f + (float)a.qmin, hi = 1536.0f + (float)a.qmax;
      uint32_t pr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float t0 = sr_i8_t(m[2 * i], qp.rcp, 1536.0f, lo, hi);
        const float t1 = sr_i8_t(m[2 * i + 1], qp.rcp, 1536.0f, lo, hi);
        pr[i] = sr_i8_pair(old[i], t0, t1, nw[i], nw[i] << 16);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = pack_sr_i8(pr[2 * i], pr[2 * i + 1]);
    } else {
      const float qmin = (float)a.qmin, qmax = (float)a.qmax;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float x = __builtin_amdgcn_fmed3f(SBF ? bf16r(m[j] * qp.inv) : m[j] * qp.inv, qmin, qmax);
        y[j] = f2u(x + 12582912.0f);  // low byte = rint(x) (two's complement)
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = pack_low_bytes(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
    }
  } else {
    constexpr float L8 = FmtLimit<KIND>::v;
    constexpr int F = FmtLimit<KIND>::fmt;
    float x[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] = __builtin_amdgcn_fmed3f(div_rn(m[j], qp.s, qp.rcp), -L8, L8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (SR) out[i] = sr_fp8_nword<F>(x + 4 * i, nw + 2 * i);
      else out[i] = fp8_pack4<F>(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
    }
  }
  store_b128_guarded((LM_GLOBAL lm_u32x4*)(L.out + (uint32_t)(mt * 64) + L.off), lm_u32x4{out[0], out[1], out[2], out[3]});
}
// the same from the packed bf16 pairs w[8] of a cached tile
template <int KIND, bool SR, bool SBF = false>
__device__ __forceinline__ void fast_quant_store(const RowArgs& a, const FastLane& L, bool rok, int mt,
                                                 const RowQP& qp, const uint32_t (&w)[8]) {
  float m[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m[2 * i] = bf16_lo(w[i]);
    m[2 * i + 1] = bf16_hi(w[i]);
  }
  fast_quant_store_vals<KIND, SR, SBF>(a, L, rok, mt, qp, m, w);
}

// Tiles of A^T operands a wave keeps in flight ahead of the arithmetic (the
// codes of the cached tiles are all requested up front).  One tile's operands
// hold 8, 16 or 32 VGPRs for NKC 1, 2, 4.
// (Rank 16: 6 tiles ahead measured 1% faster than 4 on the 8B INT8 stack,
// SR 3.99 -> 3.95 ms per step on one box, RTN unchanged, at 123 VGPRs; 8
// ahead spills.)
template <int NKC, bool SR>
constexpr int fast_prefetch() { return NKC == 1 ? 6 : 2; }

// LCACHE: merged tiles per wave kept in LDS after the register cache (2 KiB
// each: [half][lane][4 words], so the two 16-byte writes of a lane are
// consecutive across lanes); tiles beyond CACHE + LCACHE are merged twice.
template <int KIND, bool SR, int NKC, int NW, int CACHE, int PF_ = fast_prefetch<NKC, SR>(), int LCACHE = 0,
          bool R16 = false, bool SBF = false>
__device__ __forceinline__ void rows_fast_body(const RowArgs& a, int64_t row0) {
  static_assert(!SBF || KIND == K_INT8, "bf16 qparams are an INT8 layout");
  __shared__ float sh_mx[16][NW];
  __shared__ lm_u32x4 lcache[LCACHE > 0 ? LCACHE : 1][NW][2][64];
  constexpr int PF = PF_ < CACHE ? PF_ : CACHE;
  const int lane = threadIdx.x & 63, wave = wave_index(), rl = lane & 15;
  const int64_t row = row0 + rl;
  const bool rok = row < a.M;
  // rows past M load row M-1 (valid memory); their results are never stored
  const int64_t rowc = rok ? row : a.M - 1;
  const int ntiles = (int)(a.N >> 6);
  const FastLane L = fast_lane<NKC, R16>(a, rowc, lane);
  v4i16 bop[NKC];
  load_bop_g<NKC>(a.bp, row, lane, bop);
  const float s_in = !rok ? 0.0f
                     : SBF ? bf16_val(((const LM_GLOBAL uint16_t*)a.scale)[row]) : ((const LM_GLOBAL float*)a.scale)[row];
  uint32_t cache[CACHE][8];
  float amax = 0.0f;
  // INT8 in 8-wave workgroups: the dequantized base bf16(RN(q s)) comes
  // from a per-row table of the 256 code bytes in LDS (16 KiB), two address
  // instructions per element instead of the sign-extending convert, the
  // product and the bf16 rounding; the values are the same.  8B stack
  // (bench.py, bit-identical): RTN 3.79 -> 3.43 ms per step, SR 4.14 ->
  // 4.06 ms.  (The 16-wave long-row kernel, one workgroup per CU with 4 LDS
  // tiles per wave, measured slower with it and keeps the arithmetic.)
  constexpr bool LUT = KIND == K_INT8 && NW == 8 && LCACHE <= 2;
  // rows 260 floats apart: lanes of different rows reading the same code byte
  // fall in different banks
  constexpr int LSTRIDE = 260;
  __shared__ __attribute__((aligned(16))) float lut[LUT ? 16 * LSTRIDE : 1];
  const float* lrow = lut + (LUT ? rl * LSTRIDE : 0);
  const bool bfree = wave + (CACHE - 1) * NW < ntiles;  // wave-uniform
  uint4 raw[CACHE];
  if (bfree) {
    // every cache slot holds a tile: the codes of all CACHE tiles (4 VGPRs
    // each) are requested at once, before the table is built, so a wave
    // keeps CACHE KiB of HBM reads in flight
#pragma unroll
    for (int i = 0; i < CACHE; ++i) raw[i] = fast_load_codes(L, wave + i * NW);
  }
  if constexpr (LUT) {
    // thread t of the 512 fills row t / 32 for the codes q = 4 (t % 32) .. + 3 and -q
    // (RN and the bf16 rounding are odd functions, so the entry of -q is the
    // negated entry of q); the row's first thread also fills -128
    const int r = (int)(threadIdx.x >> 5), q0 = 4 * (int)(threadIdx.x & 31);
    const float s = row0 + r >= a.M ? 0.0f  // (rows past M: s_in is 0 as well)
                    : SBF ? bf16_val(((const LM_GLOBAL uint16_t*)a.scale)[row0 + r])
                          : ((const LM_GLOBAL float*)a.scale)[row0 + r];
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = bf16r((float)(q0 + j) * s);
    float* lr = lut + r * LSTRIDE;
    *(float4*)(lr + q0) = make_float4(v[0], v[1], v[2], v[3]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (q0 + j > 0) lr[256 - q0 - j] = -v[j];
    if (q0 == 0) lr[128] = bf16r(-128.0f * s);
    __syncthreads();
  }
  if (bfree) {
    // branch-free; the A^T operands (L2-resident, 4 NKC VGPRs per MFMA) run
    // PF tiles ahead
    v4i16 aop[PF][4][NKC];
#pragma unroll
    for (int i = 0; i < PF; ++i) fast_load_aop<NKC, R16>(L, wave + i * NW, aop[i]);
#pragma unroll
    for (int i = 0; i < CACHE; ++i) {
      fast_merged_tile<KIND, NKC, LUT>(a, raw[i], aop[i % PF], bop, s_in, cache[i], amax, lrow);
      if (i + PF < CACHE) fast_load_aop<NKC, R16>(L, wave + (i + PF) * NW, aop[i % PF]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < CACHE; ++i) {
      const int mt = wave + i * NW;
      if (mt < ntiles) {
        FastTileIn<NKC> in;
        fast_load_tile<NKC, R16>(L, mt, in);
        fast_merged_tile<KIND, NKC, LUT>(a, in.raw, in.aop, bop, s_in, cache[i], amax, lrow);
      }
    }
  }
  // tiles beyond the register cache: one tile of loads ahead (the last
  // prefetch re-reads the final tile instead of branching); the first LCACHE
  // of them are kept in LDS
  if (wave + CACHE * NW < ntiles) {
    FastTileIn<NKC> cur;
    fast_load_tile<NKC, R16>(L, wave + CACHE * NW, cur);
    int l = 0;
    for (int mt = wave + CACHE * NW; mt < ntiles; mt += NW, ++l) {
      FastTileIn<NKC> nxt;
      fast_load_tile<NKC, R16>(L, mt + NW < ntiles ? mt + NW : mt, nxt);
      uint32_t t[8];
      fast_merged_tile<KIND, NKC, LUT>(a, cur.raw, cur.aop, bop, s_in, t, amax, lrow);
      if (LCACHE > 0 && l < LCACHE) {
        lcache[l][wave][0][lane] = lm_u32x4{t[0], t[1], t[2], t[3]};
        lcache[l][wave][1][lane] = lm_u32x4{t[4], t[5], t[6], t[7]};
      }
      cur = nxt;
    }
  }
  float vmx = bf16r(amax);  // = max |bf16(merged)| of the lane
  vmx = lanes_max32(lanes_max16(vmx));
  if ((lane >> 4) == 0) sh_mx[rl][wave] = vmx;
  __syncthreads();
  // Every lane derives its row's qparams from the NW wave maxima itself (the
  // lanes of a row agree), so no second barrier and no single-wave section.
  float mx = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; ++w) mx = __builtin_fmaxf(mx, sh_mx[rl][w]);
  const bool writer = wave == 0 && (lane >> 4) == 0 && rok;  // one scale store per row
  float stored;
  RowQP qp;
  if constexpr (KIND == K_INT8) {
    int zp;
    qp = int8_qparams<BF16, SBF ? BF16 : F32, false>(-mx, mx, a.qmin, a.qmax, stored, zp);
    if (writer && SBF) ((LM_GLOBAL uint16_t*)a.scale_out)[row] = bf16_bits(stored);
    if (writer && !SBF) ((LM_GLOBAL float*)a.scale_out)[row] = stored;
    if (writer && a.zp_out) ((LM_GLOBAL int8_t*)a.zp_out)[row] = 0;
  } else {
    qp = fp8_qparams<BF16, KIND>(mx, stored);
    if (writer) ((LM_GLOBAL float*)a.scale_out)[row] = stored;
  }
#pragma unroll
  for (int i = 0; i < CACHE; ++i) {
    const int mt = wave + i * NW;
    if (mt < ntiles) fast_quant_store<KIND, SR, SBF>(a, L, rok, mt, qp, cache[i]);
  }
#pragma unroll
  for (int l = 0; l < LCACHE; ++l) {
    const int mt = wave + (CACHE + l) * NW;
    if (mt < ntiles) {
      const lm_u32x4 lo = lcache[l][wave][0][lane], hi = lcache[l][wave][1][lane];
      const uint32_t t[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      fast_quant_store<KIND, SR, SBF>(a, L, rok, mt, qp, t);
    }
  }
  if (wave + (CACHE + LCACHE) * NW < ntiles) {
    FastTileIn<NKC> cur;
    fast_load_tile<NKC, R16>(L, wave + (CACHE + LCACHE) * NW, cur);
    for (int mt = wave + (CACHE + LCACHE) * NW; mt < ntiles; mt += NW) {
      FastTileIn<NKC> nxt;
      fast_load_tile<NKC, R16>(L, mt + NW < ntiles ? mt + NW : mt, nxt);
      uint32_t t[8];
      float unused = 0.0f;
      fast_merged_tile<KIND, NKC, LUT>(a, cur.raw, cur.aop, bop, s_in, t, unused, lrow);
      fast_quant_store<KIND, SR, SBF>(a, L, rok, mt, qp, t);
      cur = nxt;
    }
  }
}

// Rank 16 with the 8-tile cache fits 128 VGPRs: two 512-thread workgroups per
// CU (4 waves per SIMD), which the bound below holds the compiler to (and the
// 16-wave kernel's 10-tile cache, and rank 32's 6 register tiles, to 128
// VGPRs as well).
template <int NKC, int CACHE>
constexpr int fast_min_waves() { return (NKC == 1 && CACHE <= 10) || (NKC == 2 && CACHE <= 6) ? 4 : 1; }

template <int KIND, bool SR, int NKC, int NW, int CACHE, int PF_ = fast_prefetch<NKC, SR>(), int LCACHE = 0,
          bool SBF = false>
__global__ __launch_bounds__(NW * 64, (fast_min_waves<NKC, CACHE>())) void k_rows_fast(RowArgs a) {
  rows_fast_body<KIND, SR, NKC, NW, CACHE, PF_, LCACHE, false, SBF>(a, (int64_t)blockIdx.x * 16);
}
// The item that owns 16-row group t: the last of the `count` ascending first
// groups begins[] that is <= t.  Every lane compares four entries per pass
// of 256 (one 16-byte load from a table that stays in L2) and the wave counts
// them with ballots, instead of a chain of dependent scalar loads.
__device__ __forceinline__ int stack_item_of(const int32_t* __restrict__ begins, int count, int32_t t) {
  const int lane = threadIdx.x & 63;
  int n = 0;
  for (int base = 0; base < count; base += 256) {
    const int i0 = base + 4 * lane;
    int32_t v[4] = {INT32_MAX, INT32_MAX, INT32_MAX, INT32_MAX};
    if (i0 + 3 < count) {
      const lm_u32x4 w = *(const LM_GLOBAL lm_u32x4*)((const LM_GLOBAL int32_t*)begins + i0);
      v[0] = (int32_t)w.x; v[1] = (int32_t)w.y; v[2] = (int32_t)w.z; v[3] = (int32_t)w.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i0 + j < count) v[j] = begins[i0 + j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) n += __builtin_popcountll(__ballot(v[j] <= t));
  }
  return n - 1;
}

template <int KIND, bool SR, int NKC, int NW, int CACHE, int PF_ = fast_prefetch<NKC, SR>(), int LCACHE = 0,
          bool R16 = false, bool SBF = false>
__global__ __launch_bounds__(NW * 64, (fast_min_waves<NKC, CACHE>())) void k_rows_fast_stack(const RowStackItem* __restrict__ items,
                                                                                             const int32_t* __restrict__ begins,
                                                                                             int count) {
  const int32_t t = (int32_t)xcd_unit(blockIdx.x, gridDim.x);
  const int it = __builtin_amdgcn_readfirstlane(stack_item_of(begins, count, t));
  const RowArgs a = items[it].a;
  rows_fast_body<KIND, SR, NKC, NW, CACHE, PF_, LCACHE, R16, SBF>(a, (int64_t)(t - begins[it]) * 16);
}

// ---- long rows in two passes ------------------------------------------------
// A workgroup that owns whole rows has to hold their merged values between
// the row reduction and the requant; for rows of more than 8192 merged
// values per 16-row group and rank above 32 that cache fills the register
// file (one workgroup per CU) and the kernel waits on memory with its phases
// serialized.  k_rows_split instead tiles the weight freely and runs twice:
//   pass 1 (QUANT = false): merge, reduce max |bf16(merged)| per row, fold it
//           into the row's slot of red with an atomic max (non-negative floats
//           order like their bits; prep cleared the slots), and copy the input
//           row scales into the workspace;
//   pass 2 (QUANT = true):  recompute the same merged values from the codes,
//           derive the row's qparams from the slot, quantize and store.
// Pass 2 reads the input scales from the workspace copy, so outputs may alias
// inputs (a workgroup of one column range may overwrite the row scale while
// another still needs it).  Both passes address codes, A^T operands and
// Philox counters exactly as k_rows_fast does, so results are bit-identical.
// A wave covers RB 16-row blocks (they share each tile's A^T operands) and
// TPW 64-column tiles; the SPLIT_NW waves of a workgroup share the same rows
// and a range of SPLIT_NW x TPW tiles (interleaved with IL, else consecutive
// per wave).
static constexpr int SPLIT_NW = 4;
template <int KIND, bool SR, int NKC, int RB, int TPW, bool QUANT, int IL = 0>
__global__ __launch_bounds__(SPLIT_NW * 64) void k_rows_split(RowArgs a, int wg_per_group) {
  // (the per-lane wave index: wave_index() left the VALU count unchanged)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, rl = lane & 15;
  const int ntiles = (int)(a.N >> 6);
  const int64_t grp = blockIdx.x / wg_per_group;
  // IL: the workgroup's waves take interleaved tiles (wave w: w, w + 4, ...)
  // of its 4 TPW, so that at any time they read neighbouring 64-byte halves
  // of the same 128-byte lines
  const int wgi = (int)(blockIdx.x - grp * wg_per_group);
  const int t0 = IL ? wgi * SPLIT_NW * TPW + wave : (wgi * SPLIT_NW + wave) * TPW;
  constexpr int TS = IL ? SPLIT_NW : 1;  // tile stride of a wave
  if (t0 >= ntiles) return;  // wave-uniform; the kernel has no barrier
  const int64_t mpad = (a.M + 15) / 16 * 16;
  LM_GLOBAL uint32_t* rmax = (LM_GLOBAL uint32_t*)a.red + 64;
  LM_GLOBAL float* s_copy = (LM_GLOBAL float*)(rmax + mpad);
  FastLane L[RB];
  v4i16 bop[RB][NKC];
  float s_in[RB], amax[RB];
  bool rok[RB];
  int64_t row[RB];
  RowQP qp[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    row[rb] = grp * (16 * RB) + 16 * rb + rl;
    rok[rb] = row[rb] < a.M;
    // rows past M work on row M-1 (valid memory) and never store
    const int64_t rowc = rok[rb] ? row[rb] : a.M - 1;
    L[rb] = fast_lane<NKC>(a, rowc, lane);
    load_bop<NKC>(a.bp, rowc, lane, bop[rb]);
    amax[rb] = 0.0f;
    if constexpr (QUANT) {
      s_in[rb] = s_copy[rowc];
      const float mx = u2f(rmax[rowc]);
      const bool writer = t0 == 0 && (lane >> 4) == 0 && rok[rb];  // one scale store per row
      float stored;
      if constexpr (KIND == K_INT8) {
        int zp;
        qp[rb] = int8_qparams<BF16, F32, false>(-mx, mx, a.qmin, a.qmax, stored, zp);
        if (writer && a.zp_out) a.zp_out[row[rb]] = 0;
      } else {
        qp[rb] = fp8_qparams<BF16, KIND>(mx, stored);
      }
      if (writer) ((float*)a.scale_out)[row[rb]] = stored;
    } else {
      s_in[rb] = ((const LM_GLOBAL float*)a.scale)[rowc];
    }
  }
  // merge (and requant) of one row block of one tile
  auto block = [&](int rb, int mt, const uint4& codes, const float (&d)[16]) {
    float m[16];
    fast_merge_vals<KIND, !QUANT>(a, codes, d, s_in[rb], m, amax[rb]);
    if constexpr (QUANT) {
      uint32_t old[8];
#pragma unroll
      for (int j = 0; j < 16; ++j) m[j] = bf16r(m[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) old[i] = f2u(m[2 * i]);
      fast_quant_store_vals<KIND, SR>(a, L[rb], rok[rb], mt, qp[rb], m, old);
    }
  };
  // one tile: the deltas of every row block first (the MFMAs consume the A^T
  // operands), then the next tile's operands and codes are requested, then
  // the merge / requant arithmetic of this tile hides their latency
  v4i16 aop[4][NKC];
  uint4 raw[RB];
  auto load = [&](int mt) {
    fast_load_aop<NKC>(L[0], mt, aop);  // A^T offsets depend on the lane only
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) raw[rb] = fast_load_codes(L[rb], mt);
  };
  auto tile = [&](int mt, int next) {
    float d[RB][16];
    uint4 cur[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      fast_tile_delta<NKC>(aop, bop[rb], d[rb]);
      cur[rb] = raw[rb];
    }
    if (next >= 0) load(next);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) block(rb, mt, cur[rb], d[rb]);
  };
  // The amax pass holds two row blocks' deltas instead of RB: row block rb
  // is merged while rb + 1's MFMAs run, each row block's next codes are
  // requested as soon as its current ones are merged, and the next A^T
  // operands once the last MFMA has read them.
  auto tile_amax = [&](int mt, int next) {
    float d[2][16];
    fast_tile_delta<NKC>(aop, bop[0], d[0]);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (rb + 1 < RB) fast_tile_delta<NKC>(aop, bop[rb + 1], d[(rb + 1) & 1]);
      else if (next >= 0) fast_load_aop<NKC>(L[0], next, aop);
      float m[16];
      fast_merge_vals<KIND, true>(a, raw[rb], d[rb & 1], s_in[rb], m, amax[rb]);
      if (next >= 0) raw[rb] = fast_load_codes(L[rb], next);
    }
  };
  load(t0);
  if (t0 + TS * (TPW - 1) < ntiles) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      if constexpr (QUANT) tile(t0 + TS * i, i + 1 < TPW ? t0 + TS * (i + 1) : -1);
      else tile_amax(t0 + TS * i, i + 1 < TPW ? t0 + TS * (i + 1) : -1);
    }
  } else {
    for (int mt = t0; mt < ntiles; mt += TS) {
      if constexpr (QUANT) tile(mt, mt + TS < ntiles ? mt + TS : -1);
      else tile_amax(mt, mt + TS < ntiles ? mt + TS : -1);
    }
  }
  if constexpr (!QUANT) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float vmx = bf16r(amax[rb]);  // = max |bf16(merged)| of the lane
      vmx = lanes_max32(lanes_max16(vmx));
      if ((lane >> 4) == 0 && rok[rb]) {
        atomicMax((uint32_t*)(rmax + row[rb]), f2u(vmx));
        if (t0 == 0) s_copy[row[rb]] = s_in[rb];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// k_blocks: block-local formats, dense weights, dequant, per-tensor passes
// ---------------------------------------------------------------------------
enum BlkFmt : int {
  B_NVFP4 = 0,
  B_MXFP4 = 1,
  B_MXE4M3 = 2,
  B_MXE5M2 = 3,
  B_Q8_0 = 4,
  B_DENSE = 5,   // plain bf16/fp16 weight (addmm_)
  B_INT8 = 6,    // per-tensor / per-row INT8 (dequant, per-tensor passes)
  B_E4M3 = 7,    // per-tensor / per-row FP8
  B_E5M2 = 8,
};
enum BlkPass : int {
  P_FULL = 0,     // merge + requant in one pass (block-local formats)
  P_AMAX = 1,     // reduce max|merged| (and max(-min)) into red[]
  P_QUANT = 2,    // quantize with the global qparams derived from red[]
  P_TODENSE = 3,  // write merged (or dequantized) values to a dense output
};

struct BlkArgs {
  const void* q;
  const void* scale;
  const void* aux;        // nvfp4: per-tensor scale in (float*); int8: zero point (int8*)
  const uint16_t* dense;  // requant-only input
  void* q_out;
  void* scale_out;
  void* aux_out;          // nvfp4: per-tensor scale out; int8: zero point out
  void* out;              // P_TODENSE output
  const uint16_t* at;
  const uint16_t* bp;
  uint32_t* red;
  int64_t M, N, ld;       // ld: row stride of dense weights (B_DENSE)
  float strength;
  uint64_t seed;
  int swizzled;
  int mx_mode;
  int out_dt;
  int scale_dt;
  int qmin, qmax;
  int asym;
  int64_t group;          // INT8/FP8 qparam group (N or M*N)
  int tpw;                // macro tiles per wave
};

template <int F>
struct BlkTraits {
  static constexpr int SPAN = (F == B_MXFP4 || F == B_MXE4M3 || F == B_MXE5M2 || F == B_Q8_0) ? 32 : 16;
};


typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// load the lane's SPAN base (dequantized) values; returns false if row invalid
template <int F, int CD>
__device__ __forceinline__ void blk_load_base(const BlkArgs& a, int64_t row, bool rok, int64_t c0, float gscale,
                                              float (&base)[BlkTraits<F>::SPAN], float& aux_val) {
  constexpr int SPAN = BlkTraits<F>::SPAN;
  const int64_t N = a.N;
  if (!rok || c0 >= N) {
#pragma unroll
    for (int j = 0; j < SPAN; ++j) base[j] = 0.0f;
    return;
  }
  if constexpr (F == B_NVFP4) {
    uint2 w = *(const uint2*)((const uint8_t*)a.q + row * (N / 2) + c0 / 2);
    uint32_t sc = ((const uint8_t*)a.scale)[blocked_offset(row, c0 / 16, N / 16, a.swizzled)];
    float bs = round_dt<CD>(fp8_value<E4M3>(sc));
    if (a.aux) bs = round_dt<CD>(bs * gscale);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      uint32_t word = j < 8 ? w.x : w.y;
      uint32_t code = (word >> (4 * (j & 7))) & 15u;
      base[j] = round_dt<CD>(e2m1_value(code) * bs);
    }
  } else if constexpr (F == B_MXFP4 || F == B_MXE4M3 || F == B_MXE5M2) {
    uint32_t sc = ((const uint8_t*)a.scale)[blocked_offset(row, c0 / 32, N / 32, a.swizzled)];
    float s = e8m0_value(sc);
    float sr = round_dt<CD>(s);
    if constexpr (F == B_MXFP4) {
      uint4 w = *(const uint4*)((const uint8_t*)a.q + row * (N / 2) + c0 / 2);
      uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        uint32_t code = (ws[j >> 3] >> (4 * (j & 7))) & 15u;
        base[j] = round_dt<CD>(e2m1_value(code) * sr);
      }
    } else {
      const uint4* p = (const uint4*)((const uint8_t*)a.q + row * N + c0);
      uint4 w0 = p[0], w1 = p[1];
      uint32_t ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        float lp = fp8_decode<F == B_MXE4M3 ? E4M3 : E5M2>(ws[j >> 2], j & 3);
        base[j] = round_dt<CD>(lp * sr);
      }
    }
  } else if constexpr (F == B_Q8_0) {
    const int64_t ofs = row * (N / 32 * 34) + (c0 / 32) * 34;
    const uint8_t* p8 = (const uint8_t*)a.q + (ofs & ~(int64_t)3);
    const int sh = (int)(ofs & 3);
    u32x4_a4 v0 = *(const u32x4_a4*)p8, v1 = *(const u32x4_a4*)(p8 + 16);
    // sh == 0 needs only bytes 32..33 of the window: never read past the block
    uint32_t v8 = sh ? *(const uint32_t*)(p8 + 32) : (uint32_t)*(const uint16_t*)(p8 + 32);
    uint32_t win[9] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3], v8};
    uint32_t blk[9];
#pragma unroll
    for (int k = 0; k < 8; ++k) blk[k] = __builtin_amdgcn_alignbyte(win[k + 1], win[k], sh);
    blk[8] = win[8] >> (8 * sh);
    // blk bytes: [d lo][d hi][q0..q31]
    float d = round_dt<CD>(f16_val(blk[0] & 0xffffu));
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      int bi = j + 2;
      int qv = (int)(int8_t)(blk[bi >> 2] >> (8 * (bi & 3)));
      base[j] = round_dt<CD>(d * (float)qv);
    }
  } else if constexpr (F == B_DENSE) {
    const uint16_t* p = (const uint16_t*)a.q + row * a.ld + c0;
    if (c0 + 16 <= N && (a.ld & 7) == 0) {
      uint4 w0 = ((const uint4*)p)[0], w1 = ((const uint4*)p)[1];
      uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int j = 0; j < 16; ++j) base[j] = val_dt<CD>((j & 1) ? (w[j >> 1] >> 16) : (w[j >> 1] & 0xffffu));
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) base[j] = (c0 + j < N) ? val_dt<CD>(p[j]) : 0.0f;
    }
  } else {  // B_INT8 / B_E4M3 / B_E5M2: per-row, per-tensor or per-group scale (16 | group)
    const int64_t qi = a.group == N ? row : (a.group == a.M * N ? 0 : (row * N + c0) / a.group);
    const float s = load_scalar(a.scale, qi, a.scale_dt);
    float z = 0.0f;
    if constexpr (F == B_INT8) z = a.aux ? (float)((const int8_t*)a.aux)[qi] : 0.0f;
    const uint8_t* p = (const uint8_t*)a.q + row * N + c0;
    const bool full = (c0 + 16 <= N) && ((N & 15) == 0);
    uint32_t w[4];
    if (full) {
      uint4 v = *(const uint4*)p;
      w[0] = v.x;
      w[1] = v.y;
      w[2] = v.z;
      w[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t x = 0;
        for (int b = 0; b < 4; ++b)
          if (c0 + 4 * i + b < N) x |= (uint32_t)p[4 * i + b] << (8 * b);
        w[i] = x;
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float v;
      if constexpr (F == B_INT8) v = round_dt<CD>(((float)(int)(int8_t)(w[j >> 2] >> (8 * (j & 3))) - z) * s);
      else v = round_dt<CD>(fp8_decode<F == B_E4M3 ? E4M3 : E5M2>(w[j >> 2], j & 3) * s);
      base[j] = (c0 + j < N) ? v : 0.0f;
    }
  }
  (void)aux_val;
}

// quantize + store one lane's block (block-local formats, or INT8/FP8 with
// global qparams in P_QUANT)
template <int F, int CD, bool SR>
__device__ __forceinline__ void blk_store(const BlkArgs& a, int64_t row, int64_t c0, const float (&m)[BlkTraits<F>::SPAN],
                                          float gscale, const RowQP& gqp) {
  constexpr int SPAN = BlkTraits<F>::SPAN;
  const int64_t N = a.N;
  uint32_t h[SPAN];
  if constexpr (SR) sr_bits<SPAN>(a.seed, (uint64_t)(row * N + c0), h);
  if constexpr (F == B_NVFP4) {
    float bmax = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) bmax = __builtin_fmaxf(bmax, __builtin_fabsf(m[j]));
    const bool two = a.aux != nullptr;
    float bscale = bmax / 6.0f;
    float fs = two ? bscale / gscale : bscale;
    fs = __builtin_fminf(__builtin_fmaxf(fs, 0.015625f), 448.0f);
    uint32_t sc8 = fp8_encode1<E4M3>(fs);
    fs = fp8_value<E4M3>(sc8);
    ((uint8_t*)a.scale_out)[blocked_offset(row, c0 / 16, N / 16, a.swizzled)] = (uint8_t)sc8;
    float recip = two ? (1.0f / gscale) / fs : 0.0f;
    float rfs = 1.0f / fs;
    float x[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float nrm = two ? m[j] * recip : div_rn(m[j], fs, rfs);
      x[j] = __builtin_fminf(__builtin_fmaxf(nrm, -6.0f), 6.0f);
    }
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      uint32_t byte = e2m1_pack2(x[2 * t], x[2 * t + 1]);
      if constexpr (SR) {
        uint32_t c0c = sr_e2m1(x[2 * t], byte & 15u, h[2 * t]);
        uint32_t c1c = sr_e2m1(x[2 * t + 1], byte >> 4, h[2 * t + 1]);
        byte = c0c | (c1c << 4);
      }
      packed[t >> 2] |= byte << (8 * (t & 3));
    }
    *(uint2*)((uint8_t*)a.q_out + row * (N / 2) + c0 / 2) = make_uint2(packed[0], packed[1]);
  } else if constexpr (F == B_MXFP4 || F == B_MXE4M3 || F == B_MXE5M2) {
    constexpr int emax = F == B_MXFP4 ? 2 : (F == B_MXE4M3 ? 8 : 15);
    constexpr float maxpos = F == B_MXFP4 ? 6.0f : (F == B_MXE4M3 ? 448.0f : 57344.0f);
    constexpr int mbits = F == B_MXFP4 ? 1 : (F == B_MXE4M3 ? 3 : 2);
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(m[j]));
    float inv;
    uint32_t enc = mx_scale(amax, a.mx_mode, emax, maxpos, mbits, inv);
    ((uint8_t*)a.scale_out)[blocked_offset(row, c0 / 32, N / 32, a.swizzled)] = (uint8_t)enc;
    float x[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) x[j] = __builtin_fminf(__builtin_fmaxf(m[j] * inv, -maxpos), maxpos);
    if constexpr (F == B_MXFP4) {
      uint32_t packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        uint32_t byte = e2m1_pack2(x[2 * t], x[2 * t + 1]);
        if constexpr (SR) {
          uint32_t c0c = sr_e2m1(x[2 * t], byte & 15u, h[2 * t]);
          uint32_t c1c = sr_e2m1(x[2 * t + 1], byte >> 4, h[2 * t + 1]);
          byte = c0c | (c1c << 4);
        }
        packed[t >> 2] |= byte << (8 * (t & 3));
      }
      *(uint4*)((uint8_t*)a.q_out + row * (N / 2) + c0 / 2) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    } else {
      constexpr int FF = F == B_MXE4M3 ? E4M3 : E5M2;
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (SR)
          w[i] = sr_fp8<FF>(x[4 * i], h[4 * i], maxpos) | (sr_fp8<FF>(x[4 * i + 1], h[4 * i + 1], maxpos) << 8) |
                 (sr_fp8<FF>(x[4 * i + 2], h[4 * i + 2], maxpos) << 16) |
                 (sr_fp8<FF>(x[4 * i + 3], h[4 * i + 3], maxpos) << 24);
        else
          w[i] = fp8_pack4<FF>(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
      }
      uint4* dst = (uint4*)((uint8_t*)a.q_out + row * N + c0);
      dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
      dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
  } else if constexpr (F == B_Q8_0) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(m[j]));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t blk[9];
    blk[0] = (uint32_t)f16_bits(d);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      int q = (int)__builtin_roundf(m[j] * id);
      if constexpr (SR) {  // integer stochastic rounding on the 13-bit grid (sr_i8_pair)
        const uint32_t pr = sr_i8_pair(h[j], sr_i8_t(m[j], id, 1536.0f, 1409.0f, 1663.0f), 1536.0f,
                                       (65535u - h[j]) << 16, 0u);
        q = (int)(int8_t)(pr & 0xffu);
      }
      int bi = j + 2;
      if ((bi & 3) == 0) blk[bi >> 2] = 0u;
      blk[bi >> 2] |= ((uint32_t)q & 0xffu) << (8 * (bi & 3));
    }
    const int64_t ofs = row * (N / 32 * 34) + (c0 / 32) * 34;
    uint8_t* base = (uint8_t*)a.q_out + ofs;
    if ((ofs & 3) == 0) {
      u32x4_a4 v0 = {blk[0], blk[1], blk[2], blk[3]}, v1 = {blk[4], blk[5], blk[6], blk[7]};
      *(u32x4_a4*)base = v0;
      *(u32x4_a4*)(base + 16) = v1;
      *(uint16_t*)(base + 32) = (uint16_t)blk[8];
    } else {  // ofs % 4 == 2: a short first, then 8 aligned dwords
      *(uint16_t*)base = (uint16_t)blk[0];
      uint32_t sh[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) sh[k] = __builtin_amdgcn_alignbyte(blk[k + 1], blk[k], 2);
      u32x4_a4 v0 = {sh[0], sh[1], sh[2], sh[3]}, v1 = {sh[4], sh[5], sh[6], sh[7]};
      *(u32x4_a4*)(base + 2) = v0;
      *(u32x4_a4*)(base + 18) = v1;
    }
  } else if constexpr (F == B_DENSE) {
    uint16_t* p = (uint16_t*)a.q_out + row * a.ld + c0;
    if (c0 + 16 <= N && (a.ld & 7) == 0) {
      uint32_t w[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k] = (uint32_t)bits_dt<CD>(m[2 * k]) | ((uint32_t)bits_dt<CD>(m[2 * k + 1]) << 16);
      ((uint4*)p)[0] = make_uint4(w[0], w[1], w[2], w[3]);
      ((uint4*)p)[1] = make_uint4(w[4], w[5], w[6], w[7]);
    } else {
      for (int j = 0; j < 16 && c0 + j < N; ++j) p[j] = bits_dt<CD>(m[j]);
    }
  } else {  // per-tensor INT8 / FP8 quantize with global qparams
    RowArgs ra;
    ra.q_out = a.q_out;
    ra.N = N;
    ra.qmin = a.qmin;
    ra.qmax = a.qmax;
    ra.seed = a.seed;
    constexpr int KIND = F == B_INT8 ? K_INT8 : (F == B_E4M3 ? K_E4M3 : K_E5M2);
    float mm[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) mm[j] = m[j];
    if (a.scale_dt == BF16) row_quant_store<KIND, BF16, SR>(ra, row, true, c0, gqp, mm);
    else row_quant_store<KIND, F32, SR>(ra, row, true, c0, gqp, mm);
  }
}

// global qparams for per-tensor INT8/FP8 from red[0] = max, red[1] = max(-min)
template <int F, int CD>
__device__ RowQP tensor_qparams(const BlkArgs& a, float& stored, int& zp) {
  const float mx = u2f(a.red[0]), mn = -u2f(a.red[1]);
  if constexpr (F == B_INT8) {
    if (a.scale_dt == BF16) {
      return a.asym ? int8_qparams<CD, BF16, true>(mn, mx, a.qmin, a.qmax, stored, zp)
                    : int8_qparams<CD, BF16, false>(mn, mx, a.qmin, a.qmax, stored, zp);
    }
    return a.asym ? int8_qparams<CD, F32, true>(mn, mx, a.qmin, a.qmax, stored, zp)
                  : int8_qparams<CD, F32, false>(mn, mx, a.qmin, a.qmax, stored, zp);
  } else {
    zp = 0;
    return fp8_qparams<CD, F == B_E4M3 ? K_E4M3 : K_E5M2>(mx, stored);
  }
}

template <int F, int CD, int NKC, bool SR, bool FROM_DENSE, int PASS, bool HAS_LORA>
__global__ __launch_bounds__(256) void k_blocks(BlkArgs a) {
  constexpr int SPAN = BlkTraits<F>::SPAN;
  constexpr int MTW = 4 * SPAN;
  __shared__ float sh_red[2][4];
  const int lane = threadIdx.x & 63, wave = wave_index(), rl = lane & 15, g = lane >> 4;
  const int64_t M = a.M, N = a.N;
  const int ntiles = (int)((N + MTW - 1) / MTW);
  const int tpw = a.tpw;
  const int groups_per_rt = (ntiles + tpw - 1) / tpw;
  const int64_t unit = (int64_t)blockIdx.x * 4 + wave;
  const int64_t rt = unit / groups_per_rt;
  const int grp = (int)(unit % groups_per_rt);
  const int64_t row = rt * 16 + rl;
  const bool active = rt * 16 < M;  // whole wave uniform
  const bool rok = active && row < M;

  float gscale = 1.0f;
  if constexpr (F == B_NVFP4) {
    if (a.aux) {
      if constexpr (PASS == P_QUANT) {
        gscale = __builtin_fmaxf(u2f(a.red[0]) / 2688.0f, kEps);
      } else {
        gscale = *(const float*)a.aux;
      }
    }
  }
  RowQP gqp = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (PASS == P_QUANT && (F == B_INT8 || F == B_E4M3 || F == B_E5M2)) {
    float stored;
    int zp;
    gqp = tensor_qparams<F, CD>(a, stored, zp);
  }
  // the per-tensor global scale used by dequant stays the INPUT per-tensor scale
  float gin = 1.0f;
  if constexpr (F == B_NVFP4) gin = a.aux ? *(const float*)a.aux : 1.0f;

  v4i16 bop[NKC];
  if constexpr (HAS_LORA && !FROM_DENSE) load_bop<NKC>(a.bp, active ? row : 0, lane, bop);

  float vmx = 0.0f, vmn = 0.0f;
  if (active) {
    for (int k = 0; k < tpw; ++k) {
      const int mt = grp * tpw + k;
      if (mt >= ntiles) break;
      const int64_t mt_col0 = (int64_t)mt * MTW;
      const int64_t c0 = mt_col0 + SPAN * g;
      float m[SPAN];
      if constexpr (FROM_DENSE) {
#pragma unroll
        for (int j = 0; j < SPAN; ++j) m[j] = (rok && c0 + j < N) ? val_dt<CD>(a.dense[row * N + c0 + j]) : 0.0f;
      } else {
        float base[SPAN];
        float auxv = 0.0f;
        blk_load_base<F, CD>(a, row, rok, c0, gin, base, auxv);
        if constexpr (HAS_LORA) {
          float d[SPAN];
          tile_delta<SPAN, NKC, CD == F16>(a.at, mt_col0, lane, bop, d);
#pragma unroll
          for (int j = 0; j < SPAN; ++j) {
            float v;
            if constexpr (F == B_NVFP4) {
              float upd = d[j] * a.strength;
              v = (upd == 0.0f) ? base[j] : round_dt<CD>(__builtin_fmaf(d[j], a.strength, base[j]));
            } else {
              v = round_dt<CD>(__builtin_fmaf(d[j], a.strength, base[j]));
            }
            m[j] = (rok && c0 + j < N) ? v : 0.0f;
          }
        } else {
#pragma unroll
          for (int j = 0; j < SPAN; ++j) m[j] = base[j];
        }
      }
      if constexpr (PASS == P_AMAX) {
#pragma unroll
        for (int j = 0; j < SPAN; ++j) {
          if constexpr (F == B_INT8) {
            vmx = __builtin_fmaxf(vmx, m[j]);
            vmn = __builtin_fminf(vmn, m[j]);
          } else {
            vmx = __builtin_fmaxf(vmx, __builtin_fabsf(m[j]));
          }
        }
      } else if constexpr (PASS == P_TODENSE) {
        if (rok) {
          for (int j = 0; j < SPAN && c0 + j < N; ++j) store_scalar(a.out, row * N + c0 + j, a.out_dt, m[j]);
        }
      } else {
        if (rok && c0 < N) blk_store<F, CD, SR>(a, row, c0, m, gscale, gqp);
      }
    }
  }
  if constexpr (PASS == P_AMAX) {
    vmx = wave_max(vmx);
    float nmn = wave_max(-vmn);
    if (lane == 0) {
      sh_red[0][wave] = vmx;
      sh_red[1][wave] = nmn;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float x = __builtin_fmaxf(__builtin_fmaxf(sh_red[0][0], sh_red[0][1]), __builtin_fmaxf(sh_red[0][2], sh_red[0][3]));
      float y = __builtin_fmaxf(__builtin_fmaxf(sh_red[1][0], sh_red[1][1]), __builtin_fmaxf(sh_red[1][2], sh_red[1][3]));
      atomicMax(&a.red[0], f2u(x));  // non-negative floats order like their bits
      atomicMax(&a.red[1], f2u(y + 0.0f));
    }
  }
}

// zero the padding entries of a swizzled 128x4 scale layout
static __global__ __launch_bounds__(256) void k_zero_swizzle_pad(uint8_t* scale, int64_t M, int64_t scols, int64_t total) {
  const int64_t ncb = (scols + 3) / 4;
  for (int64_t o = blockIdx.x * 256ll + threadIdx.x; o < total; o += (int64_t)gridDim.x * 256) {
    int64_t tile = o / 512, w = o % 512;
    int64_t row_lane = w / 16, rem = w % 16, rgrp = rem / 4, cib = rem % 4;
    int64_t rb = tile / ncb, cb = tile % ncb;
    int64_t row = rb * 128 + rgrp * 32 + row_lane, scol = cb * 4 + cib;
    if (row >= M || scol >= scols) scale[o] = 0;
  }
}

// writes the per-tensor outputs once every workgroup of the quantize pass has
// consumed the inputs (the outputs may alias them)
template <int F, int CD>
__global__ void k_finalize(BlkArgs a) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  if constexpr (F == B_NVFP4) {
    if (a.aux_out) *(float*)a.aux_out = __builtin_fmaxf(u2f(a.red[0]) / 2688.0f, kEps);
  } else {
    float stored;
    int zp;
    (void)tensor_qparams<F, CD>(a, stored, zp);
    store_scalar(a.scale_out, 0, F == B_INT8 ? a.scale_dt : F32, stored);
    if (F == B_INT8 && a.aux_out) *(int8_t*)a.aux_out = (int8_t)zp;
  }
}
template <int F>
static int run_finalize(const BlkArgs& a, int cd, hipStream_t st) {
  if (cd == LM_F16) hipLaunchKernelGGL((k_finalize<F, F16>), dim3(1), dim3(64), 0, st, a);
  else hipLaunchKernelGGL((k_finalize<F, BF16>), dim3(1), dim3(64), 0, st, a);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
struct Ctx {
  hipStream_t st;
  uint16_t* at = nullptr;
  uint16_t* bp = nullptr;
  uint32_t* red = nullptr;
  float* nrm = nullptr;  // ws_layout's norms region
  float* ub = nullptr;   // ws_layout's tile-bound region
  int nkc = 0;
};

static inline int check_lora(const lm_lora* l, int64_t M, int64_t N) {
  if (!l) return LM_OK;
  if (!l->b || !l->a) return fail(LM_EINVAL, "LoRA factor pointers must be non-null");
  if (l->rank <= 0) return fail(LM_EINVAL, "LoRA rank must be positive, got %d", l->rank);
  if (l->rank > 64) return fail(LM_EUNSUPPORTED, "LoRA rank %d exceeds the supported maximum 64", l->rank);
  if (l->dtype != LM_BF16 && l->dtype != LM_F16)
    return fail(LM_EUNSUPPORTED, "LoRA factors must be bfloat16 or float16, got dtype id %d", l->dtype);
  if (l->ldb < l->rank || l->lda < N) return fail(LM_EINVAL, "LoRA factor leading dimensions are too small");
  (void)M;
  return LM_OK;
}

// rows_split: the call runs the two-pass long-row kernels, whose row amax
// slots the prep launch clears
static inline int setup(Ctx& c, int64_t M, int64_t N, const lm_lora* l, void* ws, size_t wsb, void* stream,
                        bool rows_split = false, bool norms = false, int at_order = AT_PLAIN) {
  c.st = (hipStream_t)stream;
  const int rank = l ? l->rank : 0;
  WsLayout w = ws_layout(M, N, rank);
  if (!ws) return fail(LM_EWORKSPACE, "workspace pointer is null (need %zu bytes)", w.total);
  if (wsb < w.total) return fail(LM_EWORKSPACE, "workspace too small: %zu < %zu bytes", wsb, w.total);
  if (((uintptr_t)ws & 255) != 0) return fail(LM_EINVAL, "workspace must be 256-byte aligned");
  uint8_t* base = (uint8_t*)ws;
  c.at = (uint16_t*)(base + w.at_off);
  c.bp = (uint16_t*)(base + w.bp_off);
  c.red = (uint32_t*)(base + w.red_off);
  c.nkc = rpad_of(rank) / 16;
  PrepItem it{};
  it.b = l ? (const uint16_t*)l->b : nullptr;
  it.a = l ? (const uint16_t*)l->a : nullptr;
  it.ldb = l ? l->ldb : 0;
  it.lda = l ? l->lda : 0;
  it.M = M;
  it.N = N;
  it.rank = rank;
  it.rpad = rpad_of(rank);
  it.at = c.at;
  it.bp = c.bp;
  it.red = c.red;
  it.nred = rows_split ? 64 + mpad_of(M) : 64;
  it.work_begin = 0;
  it.block_begin = 0;
  it.vec_b = prep_vec_b(it);
  it.at_order = at_order;
  c.nrm = (float*)(base + w.nrm_off);
  c.ub = (float*)(base + w.ub_off);
  it.nrm = c.nrm;
  it.norms = norms && l != nullptr && l->dtype == LM_BF16 ? 1 : 0;
  return launch_prep(it, c.st);
}

static inline int check_rounding(const lm_rounding* r) {
  if (!r) return LM_OK;
  if (r->mode != LM_ROUND_NEAREST && r->mode != LM_ROUND_STOCHASTIC)
    return fail(LM_EINVAL, "unknown rounding mode %d", r->mode);
  return LM_OK;
}
static inline bool is_sr(const lm_rounding* r) { return r && r->mode == LM_ROUND_STOCHASTIC; }
static inline uint64_t seed_of(const lm_rounding* r) { return r ? r->seed : 0; }

// dispatch helpers: NKC in {1,2,4}
#define NKC_SWITCH(nkc, ...)                                             \
  switch (nkc) {                                                         \
    case 1: { constexpr int NKC_ = 1; __VA_ARGS__; } break;              \
    case 2: { constexpr int NKC_ = 2; __VA_ARGS__; } break;              \
    case 4: { constexpr int NKC_ = 4; __VA_ARGS__; } break;              \
    default: return fail(LM_EUNSUPPORTED, "unsupported rank padding");   \
  }

// ranks are padded to 16, 32 or 64 (rpad_of), so nkc is 1, 2 or 4
static inline int nkc_bucket(int nkc) { return nkc; }

static inline unsigned blocks_for(int64_t M, int64_t N, int mtw, int tpw) {
  int64_t ntiles = (N + mtw - 1) / mtw;
  int64_t groups = (ntiles + tpw - 1) / tpw;
  int64_t units = (M + 15) / 16 * groups;
  return (unsigned)((units + 3) / 4);
}

template <int F, int NKC, bool SR, bool FROM_DENSE, int PASS, bool HAS_LORA>
static int run_blocks_cd(const BlkArgs& a, int cd, hipStream_t st) {
  constexpr int SPAN = BlkTraits<F>::SPAN;
  unsigned nb = blocks_for(a.M, a.N, 4 * SPAN, a.tpw);
  if (nb == 0) return LM_OK;
  TimedLaunch timed(PASS == P_FULL ? "blocks_full" : PASS == P_AMAX ? "blocks_amax" : PASS == P_QUANT ? "blocks_quant"
                                                                                                    : "todense",
                    st);
  if (cd == LM_F16)
    hipLaunchKernelGGL((k_blocks<F, F16, NKC, SR, FROM_DENSE, PASS, HAS_LORA>), dim3(nb), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((k_blocks<F, BF16, NKC, SR, FROM_DENSE, PASS, HAS_LORA>), dim3(nb), dim3(256), 0, st, a);
  LAUNCH_CHECK();
  return LM_OK;
}

// run a block kernel for the given pass with optional LoRA / SR
template <int F, int PASS>
static int run_blocks(const BlkArgs& a, int cd, int nkc, bool sr, bool from_dense, hipStream_t st) {
  if (from_dense) {
    if (sr) return run_blocks_cd<F, 1, true, true, PASS, false>(a, cd, st);
    return run_blocks_cd<F, 1, false, true, PASS, false>(a, cd, st);
  }
  if (nkc == 0) {
    if (sr) return run_blocks_cd<F, 1, true, false, PASS, false>(a, cd, st);
    return run_blocks_cd<F, 1, false, false, PASS, false>(a, cd, st);
  }
  if (sr) {
    NKC_SWITCH(nkc_bucket(nkc), return (run_blocks_cd<F, NKC_, true, false, PASS, true>(a, cd, st)));
  } else {
    NKC_SWITCH(nkc_bucket(nkc), return (run_blocks_cd<F, NKC_, false, false, PASS, true>(a, cd, st)));
  }
  return LM_OK;
}

static BlkArgs blk_args_base(const Ctx& c, int64_t M, int64_t N, const lm_lora* l, const lm_rounding* r) {
  BlkArgs a;
  memset(&a, 0, sizeof a);
  a.at = c.at;
  a.bp = c.bp;
  a.red = c.red;
  a.M = M;
  a.N = N;
  a.ld = N;
  a.strength = l ? l->strength : 0.0f;
  a.seed = seed_of(r);
  a.tpw = 4;
  a.group = N;
  return a;
}

// ---------------------------------------------------------------------------
// per-row kernels dispatch
// ---------------------------------------------------------------------------
// NW waves per workgroup, CACHE macro tiles of 64 columns cached per wave.
static constexpr int ROW_NW = 8;
static constexpr int ROW_CACHE = 8;

template <int KIND, int CD, int SDT, bool ASYM, bool SR, bool FROM_DENSE>
static int run_rows_nkc(const RowArgs& a, int nkc, int scale_dt, hipStream_t st) {
  dim3 grid((unsigned)((a.M + 15) / 16)), block(ROW_NW * 64);
  TimedLaunch timed("rows", st);
  if (FROM_DENSE || nkc == 0) {
    hipLaunchKernelGGL((k_rows<KIND, CD, SDT, ASYM, SR, 1, FROM_DENSE, ROW_NW, ROW_CACHE>), grid, block, 0, st, a,
                       scale_dt);
  } else {
    NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_rows<KIND, CD, SDT, ASYM, SR, NKC_, FROM_DENSE, ROW_NW, ROW_CACHE>),
                                                   grid, block, 0, st, a, scale_dt));
  }
  LAUNCH_CHECK();
  return LM_OK;
}

// fast path eligibility: bf16 factors, N % 64 == 0, INT8 symmetric fp32 scales or FP8
// The fast kernels address codes, A^T operands and Philox counters with 32-bit
// offsets: M N < 2^32 (4 GiB of codes per tensor) and N RPAD < 2^32.
static inline bool rows_fast_ok(int kind, int cd, int sdt, bool asym, int nkc, int64_t M, int64_t N) {
  return cd == LM_BF16 && nkc > 0 && (N % 64) == 0 && (kind != K_INT8 || (!asym && (sdt == LM_F32 || sdt == LM_BF16))) &&
         M * N < (INT64_C(1) << 32) && N * 64 < (INT64_C(1) << 32);
}

// Rows with more macro tiles per wave than the register cache holds are
// merged twice (the surplus tiles are recomputed in pass 2).  Two remedies,
// measured on MI355X:
// * rank 16 (128 VGPRs): 16-wave workgroups halve the tiles per wave at the
//   same occupancy (4 waves per SIMD); 8B down_proj rows [4096, 14336]:
//   RTN 1.44 -> 1.21 ms, SR 1.51 -> 1.46 ms for the 32 layers;
// * a 16-tile cache: pays for rank 64 (FP8 [8192, 8192] r64: RTN 0.124 ->
//   0.083 ms, SR 0.137 -> 0.115 ms) and for round-to-nearest at rank 32, while
//   stochastic rounding at rank 32 is VALU-bound and loses the occupancy it
//   costs (those rows recompute).
// Rows of up to 8 tiles per wave: rank 16 caches them all in registers; rank
// 32 keeps 4 in registers and 4 in LDS (64 KiB per workgroup), which brings
// it to 106 VGPRs and two workgroups per CU instead of one.  INT8 at rank 32
// keeps 6 in registers and 2 in LDS (116 VGPRs, 32 KiB), which leaves room
// for the dequantization table: config 2 ([14336, 4096] r32) SR 0.0499 ->
// 0.0481 ms, RTN 0.0424 -> 0.0420 ms, bit-identical.
template <int KIND, int NKC>
constexpr int row_reg_cache() { return NKC == 2 ? (KIND == K_INT8 ? 6 : 4) : 8; }
template <int KIND, int NKC>
constexpr int row_lds_cache() { return NKC == 2 ? (KIND == K_INT8 ? 2 : 4) : 0; }
static constexpr int ROW_DEEP_CACHE = 16;
static constexpr int ROW_NW_WIDE = 16;
// 16-wave rows keep 10 tiles per wave in registers and 4 more in LDS (128 KiB
// per workgroup, one workgroup per CU), so a 14336-column row (224 tiles) is
// merged once; the A^T operands run 2 tiles ahead instead of 4 to make room
// (128 VGPRs, a few spilled).  The 32 down_proj of the 8B stack, against 8
// register tiles and 4 ahead (2 of 14 tiles merged twice): SR 1.298 -> 1.268
// ms, RTN 1.140 -> 1.074 ms.
static constexpr int ROW_WIDE_CACHE = 10;
static constexpr int ROW_WIDE_PF = 2;
static constexpr int ROW_WIDE_LDS = 4;
enum RowsMode : int { ROWS_REGULAR = 0, ROWS_WIDE = 1, ROWS_DEEP = 2 };
static inline int rows_long_mode(int nkc, bool sr, int64_t N) {
  const int64_t tpw = (N / 64 + ROW_NW - 1) / ROW_NW;
  if (tpw <= ROW_CACHE) return ROWS_REGULAR;
  if (nkc == 1) return ROWS_WIDE;
  return (nkc == 4 || !sr) ? ROWS_DEEP : ROWS_REGULAR;
}

template <int KIND, bool SR, int NKC, bool SBF = false>
static int launch_rows_fast(const RowArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.M + 15) / 16));
  TimedLaunch timed("rows", st);
  const int mode = rows_long_mode(NKC, SR, a.N);
  if (mode == ROWS_WIDE) {
    if constexpr (NKC == 1)
      hipLaunchKernelGGL((k_rows_fast<KIND, SR, NKC, ROW_NW_WIDE, ROW_WIDE_CACHE, ROW_WIDE_PF, ROW_WIDE_LDS, SBF>),
                         grid, dim3(ROW_NW_WIDE * 64), 0, st, a);
  } else if (mode == ROWS_DEEP) {
    if constexpr (NKC == 4 || !SR)
      hipLaunchKernelGGL((k_rows_fast<KIND, SR, NKC, ROW_NW, ROW_DEEP_CACHE, NKC == 4 ? 1 : 2, 0, SBF>), grid,
                         dim3(ROW_NW * 64), 0, st, a);
  } else {
    hipLaunchKernelGGL((k_rows_fast<KIND, SR, NKC, ROW_NW, row_reg_cache<KIND, NKC>(), fast_prefetch<NKC, SR>(),
                                    row_lds_cache<KIND, NKC>(), SBF>),
                       grid, dim3(ROW_NW * 64), 0, st, a);
  }
  LAUNCH_CHECK();
  return LM_OK;
}

// Two-pass long rows (k_rows_split): wave tiles of 16 RB rows x 64 TPW
// columns.  The amax pass has little arithmetic per A^T operand and shares
// each tile's operands among 8 row blocks (128 rows); the quant pass, which
// holds the Philox state and the quantized words as well, among 4.  Measured
// on MI355X, FP8 [8192, 8192] rank 64, stochastic: amax pass 28.6 us at
// RB 8 (30.4 at RB 4, 42 at RB 2); quant pass 53.9 us at RB 4, TPW 8 (56.3 at
// RB 2, 58.3 without the one-tile operand prefetch).
static constexpr int SPLIT_RB1 = 8, SPLIT_TPW1 = 8, SPLIT_RB2 = 4, SPLIT_TPW2 = 8;
// the workgroup's 4 waves take interleaved tiles (amax pass 25.9 -> 24.0 us,
// quant pass 50.7 -> 49.8 us on FP8 config 3, stochastic)
static constexpr int SPLIT_IL = 1;
// whether a per-row merge runs the two-pass kernels: rows too long for the
// register cache at rank above 32, where the cached kernel runs one
// workgroup per CU
static inline bool rows_split_wanted(int kind, int cd, int sdt, bool asym, bool sr, int nkc, int64_t M, int64_t N) {
  return rows_fast_ok(kind, cd, sdt, asym, nkc, M, N) && sdt == LM_F32 && nkc == 4 &&
         rows_long_mode(nkc, sr, N) == ROWS_DEEP;
}
template <int KIND, bool SR, int NKC, int RB, int TPW, bool QUANT, int IL = 0>
static int launch_rows_split_pass(const RowArgs& a, hipStream_t st) {
  const int64_t waves = (a.N / 64 + TPW - 1) / TPW;
  const int64_t wg_per_group = (waves + SPLIT_NW - 1) / SPLIT_NW;
  const int64_t groups = (a.M + 16 * RB - 1) / (16 * RB);
  if (groups * wg_per_group > 0x7fffffff) return fail(LM_EUNSUPPORTED, "weight too large for one row launch");
  {
    TimedLaunch timed("rows", st);
    hipLaunchKernelGGL((k_rows_split<KIND, SR, NKC, RB, TPW, QUANT, IL>), dim3((unsigned)(groups * wg_per_group)),
                       dim3(SPLIT_NW * 64), 0, st, a, (int)wg_per_group);
  }
  LAUNCH_CHECK();
  return LM_OK;
}
template <int KIND, bool SR, int NKC>
static int launch_rows_split(const RowArgs& a, hipStream_t st) {
  const int rc = launch_rows_split_pass<KIND, SR, NKC, SPLIT_RB1, SPLIT_TPW1, false, SPLIT_IL>(a, st);
  return rc ? rc : launch_rows_split_pass<KIND, SR, NKC, SPLIT_RB2, SPLIT_TPW2, true, SPLIT_IL>(a, st);
}

template <int KIND, bool FROM_DENSE>
static int run_rows(const RowArgs& a, int cd, int sdt, bool asym, bool sr, int nkc, hipStream_t st) {
  if (!FROM_DENSE && rows_fast_ok(KIND, cd, sdt, asym, nkc, a.M, a.N)) {
    if (a.red) {  // the caller chose the two-pass kernels (rows_split_wanted: rank bucket 64) and had prep clear the slots
      if (nkc_bucket(nkc) != 4) return fail(LM_EINVAL, "two-pass rows need the rank-64 bucket");
      return sr ? launch_rows_split<KIND, true, 4>(a, st) : launch_rows_split<KIND, false, 4>(a, st);
    }
    if constexpr (KIND == K_INT8) {
      if (sdt == LM_BF16) {
        if (sr) {
          NKC_SWITCH(nkc_bucket(nkc), return (launch_rows_fast<KIND, true, NKC_, true>(a, st)));
        } else {
          NKC_SWITCH(nkc_bucket(nkc), return (launch_rows_fast<KIND, false, NKC_, true>(a, st)));
        }
      }
    }
    if (sr) {
      NKC_SWITCH(nkc_bucket(nkc), return (launch_rows_fast<KIND, true, NKC_>(a, st)));
    } else {
      NKC_SWITCH(nkc_bucket(nkc), return (launch_rows_fast<KIND, false, NKC_>(a, st)));
    }
  }
#define RR(CD_, SDT_, AS_, SR_) return run_rows_nkc<KIND, CD_, SDT_, AS_, SR_, FROM_DENSE>(a, nkc, sdt, st)
  if (KIND != K_INT8) {
    asym = false;
    sdt = LM_F32;
  }
  if (cd == LM_F16) {
    if (sdt == LM_BF16) {
      if (asym) { if (sr) RR(F16, BF16, true, true); else RR(F16, BF16, true, false); }
      else { if (sr) RR(F16, BF16, false, true); else RR(F16, BF16, false, false); }
    } else {
      if (asym) { if (sr) RR(F16, F32, true, true); else RR(F16, F32, true, false); }
      else { if (sr) RR(F16, F32, false, true); else RR(F16, F32, false, false); }
    }
  } else {
    if (sdt == LM_BF16) {
      if (asym) { if (sr) RR(BF16, BF16, true, true); else RR(BF16, BF16, true, false); }
      else { if (sr) RR(BF16, BF16, false, true); else RR(BF16, BF16, false, false); }
    } else {
      if (asym) { if (sr) RR(BF16, F32, true, true); else RR(BF16, F32, true, false); }
      else { if (sr) RR(BF16, F32, false, true); else RR(BF16, F32, false, false); }
    }
  }
#undef RR
}

static inline int check_nvfp4(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return fail(LM_EINVAL, "NVFP4 merge requires a non-empty weight");
  if (N % 16 != 0) return fail(LM_EINVAL, "NVFP4 requires columns divisible by 16, got %lld", (long long)N);
  return LM_OK;
}
static inline int zero_swizzle_pad(uint8_t* scale, int64_t M, int64_t scols, hipStream_t st) {
  int64_t total = (M + 127) / 128 * 512 * ((scols + 3) / 4);
  if ((M % 128) == 0 && (scols % 4) == 0) return LM_OK;
  int64_t nb = (total + 255) / 256;
  if (nb > 4096) nb = 4096;
  hipLaunchKernelGGL(k_zero_swizzle_pad, dim3((unsigned)nb), dim3(256), 0, st, scale, M, scols, total);
  LAUNCH_CHECK();
  return LM_OK;
}

