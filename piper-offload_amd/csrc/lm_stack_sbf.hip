// lm_stack_sbf.hip -- INT8 stack launches with bf16 qparams (see lm_rows_stack.h).
#include "lm_rows_stack.h"

int int8_stack_fast_launch_sbf(const RowStackItem* d0, const int32_t* begins, int n_regular, int count,
                                const int64_t (&tiles)[2], int nkc_max, bool sr, hipStream_t st) {
  return int8_stack_fast_launch<true>(d0, begins, n_regular, count, tiles, nkc_max, sr, st);
}
