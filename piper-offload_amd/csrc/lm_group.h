// lm_group.h -- per-group INT8 / scaled-FP8 layouts: TorchAO block_size
// (1, g) with g < N, one scale (and INT8 zero point) per g consecutive
// elements of a row, stored [M, N / g] (P/int8_adapter.py:144-188,
// P/float8_adapter.py:63-98).  The quantization recipe is the per-row one
// applied to each group (P/_triton_int8_lora.py:98-237, _block_numel).
//
// Supported group sizes: 16, 32 and multiples of 64, dividing N.  A lane
// holds 16 consecutive columns of a 64-column tile (row lane & 15, columns
// 16 (lane >> 4) ..), so a group of 16 is one lane, a group of 32 two lanes
// (xor 16) and a group of 64 or more the four lanes of its row (xor 16, 32)
// over g / 64 tiles.  One wave works on one unit: a 64-column tile (g <= 64)
// or one group (g >= 64) of 16 rows.  Groups are independent, so there is no
// workgroup-level exchange; groups of more than one tile are merged twice
// (max, then quantize), which keeps the register footprint of any g small.
#pragma once
#include "lm_impl.h"

static constexpr int GROUP_NW = 4;

static inline bool group_size_ok(int64_t N, int64_t g) {
  return g > 0 && g < N && N % g == 0 && (g == 16 || g == 32 || g % 64 == 0);
}

template <int KIND, int CD, int SDT, bool ASYM, bool SR, int NKC, bool FROM_DENSE>
__global__ __launch_bounds__(GROUP_NW * 64) void k_groups(RowArgs a, int scale_dt, int64_t g) {
  const int lane = threadIdx.x & 63, rl = lane & 15, gi = lane >> 4;
  const int64_t N = a.N;
  const int64_t T = g >= 64 ? g / 64 : 1;                    // tiles per unit
  const int64_t units = g >= 64 ? N / g : (N + 63) / 64;     // units per 16-row group
  const int64_t item = (int64_t)blockIdx.x * GROUP_NW + (threadIdx.x >> 6);
  if (item >= ((a.M + 15) / 16) * units) return;
  const int64_t rgrp = item / units, u = item - rgrp * units;
  const int64_t row = rgrp * 16 + rl;
  const bool rok = row < a.M;
  const int64_t col0 = u * 64 * T;
  const int64_t c_lane = col0 + 16 * gi;  // the lane's first column in the unit's first tile
  const bool live = rok && c_lane < N;    // the lane holds columns of the weight
  const int64_t qi = live ? (row * N + c_lane) / g : 0;  // the lane's group (all its columns share it)

  v4i16 bop[NKC];
  float s_in = 0.0f, z_in = 0.0f;
  if constexpr (!FROM_DENSE) {
    load_bop<NKC>(a.bp, row, lane, bop);  // Bp holds ceil(M / 16) * 16 rows
    if (live) {
      s_in = load_scalar(a.scale, qi, scale_dt);
      if (KIND == K_INT8 && a.zp) z_in = (float)a.zp[qi];
    }
  }
  // group statistics; min / max include 0, as the per-row recipe does
  float vmx = 0.0f, vmn = 0.0f;
  float m[16];
  for (int64_t t = 0; t < T; ++t) {
    row_merged_tile<KIND, CD, SDT, NKC, FROM_DENSE, !FROM_DENSE>(a, row, rok, c_lane + 64 * t, lane, col0 + 64 * t,
                                                                  bop, s_in, z_in, m);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if constexpr (KIND == K_INT8) {
        vmx = __builtin_fmaxf(vmx, m[j]);
        vmn = __builtin_fminf(vmn, m[j]);
      } else {
        vmx = __builtin_fmaxf(vmx, __builtin_fabsf(m[j]));
      }
    }
  }
  if (g >= 32) {
    vmx = lanes_max16(vmx);
    if constexpr (KIND == K_INT8) vmn = lanes_min16(vmn);
  }
  if (g >= 64) {
    vmx = lanes_max32(vmx);
    if constexpr (KIND == K_INT8) vmn = lanes_min32(vmn);
  }
  // one store per group: its first lane
  const bool writer = live && (g >= 64 ? gi == 0 : (g == 32 ? (gi & 1) == 0 : true));
  RowQP qp;
  float stored;
  if constexpr (KIND == K_INT8) {
    int zp;
    qp = int8_qparams<CD, SDT, ASYM>(vmn, vmx, a.qmin, a.qmax, stored, zp);
    if (writer) {
      store_scalar(a.scale_out, qi, SDT, stored);
      if (a.zp_out) a.zp_out[qi] = (int8_t)zp;
    }
  } else {
    qp = fp8_qparams<CD, KIND>(vmx, stored);
    if (writer) ((float*)a.scale_out)[qi] = stored;
  }
  if (T == 1) {
    row_quant_store<KIND, SDT, SR>(a, row, rok, c_lane, qp, m);
  } else {
    for (int64_t t = 0; t < T; ++t) {
      row_merged_tile<KIND, CD, SDT, NKC, FROM_DENSE, !FROM_DENSE>(a, row, rok, c_lane + 64 * t, lane,
                                                                    col0 + 64 * t, bop, s_in, z_in, m);
      row_quant_store<KIND, SDT, SR>(a, row, rok, c_lane + 64 * t, qp, m);
    }
  }
}

template <int KIND, int CD, int SDT, bool ASYM, bool SR, bool FROM_DENSE>
static int run_groups_nkc(const RowArgs& a, int64_t g, int nkc, int scale_dt, hipStream_t st) {
  const int64_t units = g >= 64 ? a.N / g : (a.N + 63) / 64;
  const int64_t items = ((a.M + 15) / 16) * units;
  const dim3 grid((unsigned)((items + GROUP_NW - 1) / GROUP_NW)), block(GROUP_NW * 64);
  TimedLaunch timed("groups", st);
  if (FROM_DENSE || nkc == 0) {
    hipLaunchKernelGGL((k_groups<KIND, CD, SDT, ASYM, SR, 1, FROM_DENSE>), grid, block, 0, st, a, scale_dt, g);
  } else {
    NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_groups<KIND, CD, SDT, ASYM, SR, NKC_, FROM_DENSE>), grid, block,
                                                   0, st, a, scale_dt, g));
  }
  LAUNCH_CHECK();
  return LM_OK;
}

// the group kernel for a compute dtype, scale dtype, mapping and rounding
template <int KIND, bool FROM_DENSE>
static int run_groups(const RowArgs& a, int64_t g, int cd, int sdt, bool asym, bool sr, int nkc, hipStream_t st) {
  if ((a.M + 15) / 16 * ((a.N + 63) / 64) >= (INT64_C(1) << 33))
    return fail(LM_EUNSUPPORTED, "per-group weight too large for one launch");
#define RG(CD_, SDT_, AS_, SR_) return run_groups_nkc<KIND, CD_, SDT_, AS_, SR_, FROM_DENSE>(a, g, nkc, sdt, st)
  if constexpr (KIND != K_INT8) {
    (void)asym;
    if (cd == LM_F16) { if (sr) RG(F16, F32, false, true); else RG(F16, F32, false, false); }
    else { if (sr) RG(BF16, F32, false, true); else RG(BF16, F32, false, false); }
  } else if (cd == LM_F16) {
    if (sdt == LM_BF16) {
      if (asym) { if (sr) RG(F16, BF16, true, true); else RG(F16, BF16, true, false); }
      else { if (sr) RG(F16, BF16, false, true); else RG(F16, BF16, false, false); }
    } else {
      if (asym) { if (sr) RG(F16, F32, true, true); else RG(F16, F32, true, false); }
      else { if (sr) RG(F16, F32, false, true); else RG(F16, F32, false, false); }
    }
  } else {
    if (sdt == LM_BF16) {
      if (asym) { if (sr) RG(BF16, BF16, true, true); else RG(BF16, BF16, true, false); }
      else { if (sr) RG(BF16, BF16, false, true); else RG(BF16, BF16, false, false); }
    } else {
      if (asym) { if (sr) RG(BF16, F32, true, true); else RG(BF16, F32, true, false); }
      else { if (sr) RG(BF16, F32, false, true); else RG(BF16, F32, false, false); }
    }
  }
#undef RG
}
