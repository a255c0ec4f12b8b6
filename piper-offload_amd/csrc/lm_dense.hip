// lm_dense.hip -- plain bf16/fp16 weight merge (addmm_) entry point.
#include "lm_impl.h"

// ---------------------------------------------------------------------------
// dense bf16 / fp16 weight: w += strength * B@A
// ---------------------------------------------------------------------------
extern "C" int lm_dense_merge(void* w, int64_t M, int64_t N, int64_t ldw, const lm_lora* lora, void* workspace,
                              size_t workspace_bytes, void* stream) {
  int rc;
  if (!w || !lora) return fail(LM_EINVAL, "dense merge pointers must be non-null");
  if (M <= 0 || N <= 0 || ldw < N) return fail(LM_EINVAL, "dense merge shape is invalid");
  if ((rc = check_lora(lora, M, N))) return rc;
  Ctx c;
  if ((rc = setup(c, M, N, lora, workspace, workspace_bytes, stream))) return rc;
  BlkArgs a = blk_args_base(c, M, N, lora, nullptr);
  a.q = w;
  a.q_out = w;
  a.ld = ldw;
  return run_blocks<B_DENSE, P_FULL>(a, lora->dtype, c.nkc, false, false, c.st);
}

