// lm_rows_stack.h -- the INT8 stack's grouped launches of the fast row
// kernels, shared by lm_stack.hip (fp32 qparams) and lm_stack_sbf.hip (bf16
// qparams, compiled as its own translation unit so the two sets of kernels
// build in parallel).
#pragma once
#include "lm_impl.h"

// 16-row groups [0, tiles[0]) over the n_regular items at d0 run in the
// 8-wave kernel; groups [0, tiles[1]) of the count - n_regular items after
// them (rows longer than the register cache) in the 16-wave kernel at rank
// 16 or the deep-cache kernel above.  begins[] holds each item's first group
// within its launch.  SBF: bf16 qparams.  Launch errors are read by the
// caller (hipGetLastError).
template <bool SBF>
static int int8_stack_fast_launch(const RowStackItem* d0, const int32_t* begins, int n_regular, int count,
                                   const int64_t (&tiles)[2], int nkc_max, bool sr, hipStream_t st) {
  const dim3 block(ROW_NW * 64);
  if (tiles[0] > 0) {
    const dim3 grid((unsigned)tiles[0]);
#define RF(SR_)                                                                                                     \
  NKC_SWITCH(nkc_bucket(nkc_max),                                                                                   \
             hipLaunchKernelGGL((k_rows_fast_stack<K_INT8, SR_, NKC_, ROW_NW, row_reg_cache<K_INT8, NKC_>(),         \
                                                   fast_prefetch<NKC_, SR_>(), row_lds_cache<K_INT8, NKC_>(), NKC_ == 1,  \
                                                   SBF>),                                                             \
                                grid, block, 0, st, d0, begins, n_regular))
    if (sr) { RF(true); } else { RF(false); }
#undef RF
  }
  if (tiles[1] > 0) {
    const dim3 grid((unsigned)tiles[1]);
    const RowStackItem* d1 = d0 + n_regular;
    const int n_deep = count - n_regular;
    if (nkc_bucket(nkc_max) == 1) {  // ROWS_WIDE: 16-wave workgroups
      const dim3 wblock(ROW_NW_WIDE * 64);
      if (sr)
        hipLaunchKernelGGL((k_rows_fast_stack<K_INT8, true, 1, ROW_NW_WIDE, ROW_WIDE_CACHE, ROW_WIDE_PF,
                                              ROW_WIDE_LDS, true, SBF>),
                           grid, wblock, 0, st, d1, begins + n_regular, n_deep);
      else
        hipLaunchKernelGGL((k_rows_fast_stack<K_INT8, false, 1, ROW_NW_WIDE, ROW_WIDE_CACHE, ROW_WIDE_PF,
                                              ROW_WIDE_LDS, true, SBF>),
                           grid, wblock, 0, st, d1, begins + n_regular, n_deep);
    } else {  // ROWS_DEEP
#define RD(SR_, PF_)                                                                                               \
  NKC_SWITCH(nkc_bucket(nkc_max),                                                                                  \
             if constexpr (NKC_ != 1 && (NKC_ == 4 || !SR_))                                                       \
                 hipLaunchKernelGGL((k_rows_fast_stack<K_INT8, SR_, NKC_, ROW_NW, ROW_DEEP_CACHE, PF_, 0, false, SBF>), \
                                    grid, block, 0, st, d1, begins + n_regular, n_deep))
      if (sr) { RD(true, 1); } else if (nkc_max == 4) { RD(false, 1); } else { RD(false, 2); }
#undef RD
    }
  }
  return LM_OK;
}

// the bf16-qparam instantiation (lm_stack_sbf.hip)
__attribute__((visibility("hidden"))) int int8_stack_fast_launch_sbf(const RowStackItem* d0, const int32_t* begins,
                                                                      int n_regular, int count,
                                                                      const int64_t (&tiles)[2], int nkc_max, bool sr,
                                                                      hipStream_t st);
