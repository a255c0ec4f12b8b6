// lm_q8.hip -- GGUF Q8_0 merge / requant and GGUF dequant entry points.
#include "lm_q8_fast.h"

// ---------------------------------------------------------------------------
// GGUF Q8_0
// ---------------------------------------------------------------------------
static int check_q8(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return fail(LM_EINVAL, "Q8_0 merge requires a non-empty weight");
  if (N % 32 != 0) return fail(LM_EINVAL, "Q8_0 requires logical columns divisible by 32, got %lld", (long long)N);
  return LM_OK;
}
extern "C" int lm_q8_0_merge(const uint8_t* packed, uint8_t* packed_out, int64_t M, int64_t N, const lm_lora* lora,
                             const lm_rounding* rounding, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if (!packed || !packed_out) return fail(LM_EINVAL, "Q8_0 pointers must be non-null");
  if (!lora) return fail(LM_EINVAL, "lm_q8_0_merge requires LoRA factors");
  if ((rc = check_q8(M, N))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  if ((rc = check_rounding(rounding))) return rc;
  Ctx c;
  if ((rc = setup(c, M, N, lora, workspace, workspace_bytes, stream))) return rc;
  if (q8_fast_ok(lora->dtype, c.nkc, M, N)) {
    Q8Args qa;
    qa.q = packed;
    qa.q_out = packed_out;
    qa.at = c.at;
    qa.bp = c.bp;
    qa.M = M;
    qa.N = N;
    qa.strength = lora->strength;
    qa.seed = rounding ? rounding->seed : 0;
    return q8_fast_run(qa, c.nkc, is_sr(rounding), c.st);
  }
  BlkArgs a = blk_args_base(c, M, N, lora, rounding);
  a.q = packed;
  a.q_out = packed_out;
  return run_blocks<B_Q8_0, P_FULL>(a, lora->dtype, c.nkc, is_sr(rounding), false, c.st);
}
extern "C" int lm_q8_0_requant(const void* dense, int32_t dense_dtype, uint8_t* packed_out, int64_t M, int64_t N,
                               const lm_rounding* rounding, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if (!dense || !packed_out) return fail(LM_EINVAL, "Q8_0 requant pointers must be non-null");
  if ((rc = check_q8(M, N))) return rc;
  if ((rc = check_rounding(rounding))) return rc;
  Ctx c;
  if ((rc = setup(c, M, N, nullptr, workspace, workspace_bytes, stream))) return rc;
  BlkArgs a = blk_args_base(c, M, N, nullptr, rounding);
  a.dense = (const uint16_t*)dense;
  a.q_out = packed_out;
  return run_blocks<B_Q8_0, P_FULL>(a, dense_dtype, 0, is_sr(rounding), true, c.st);
}
bool gguf_block_sizes(int type, int* bs, int* ts);                                       // lm_gguf.hip
int gguf_dequant_run(const uint8_t* src, int type, int64_t nelem, void* out, int dt, hipStream_t st);  // lm_gguf.hip

extern "C" int lm_gguf_dequant(const uint8_t* packed, int32_t quant_type, int64_t rows, int64_t cols, const lm_lora* lora,
                               void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  int rc, bs, ts;
  if (!gguf_block_sizes(quant_type, &bs, &ts))
    return fail(LM_EUNSUPPORTED, "Unsupported GGUF quant type: %d", quant_type);
  if (out_dtype != LM_BF16 && out_dtype != LM_F16 && out_dtype != LM_F32)
    return fail(LM_EINVAL, "GGUF dequant output dtype must be bf16, f16 or f32");
  if (rows < 0 || cols < 0) return fail(LM_EINVAL, "GGUF dequant shape must be non-negative");
  if (cols % bs != 0)
    return fail(LM_EINVAL, "GGUF type %d needs logical columns divisible by %d, got %lld", quant_type, bs, (long long)cols);
  if (rows == 0 || cols == 0) return LM_OK;
  if (!packed || !out) return fail(LM_EINVAL, "GGUF dequant pointers must be non-null");
  if (!lora) {
    if (((uintptr_t)out & 15) != 0) return fail(LM_EINVAL, "GGUF dequant output must be 16-byte aligned");
    return gguf_dequant_run(packed, quant_type, rows * cols, out, out_dtype, (hipStream_t)stream);
  }
  // dequantize with a LoRA delta added: Q8_0 only (the merge extension's format)
  if (quant_type != LM_GGUF_Q8_0) return fail(LM_EUNSUPPORTED, "GGUF dequant with LoRA factors supports Q8_0 only");
  if ((rc = check_q8(rows, cols))) return rc;
  if ((rc = check_lora(lora, rows, cols))) return rc;
  Ctx c;
  if ((rc = setup(c, rows, cols, lora, workspace, workspace_bytes, stream))) return rc;
  BlkArgs a = blk_args_base(c, rows, cols, lora, nullptr);
  a.q = packed;
  a.out = out;
  a.out_dt = out_dtype;
  return run_blocks<B_Q8_0, P_TODENSE>(a, lora->dtype, c.nkc, false, false, c.st);
}
