// lm_nvfp4.hip -- NVFP4 (TorchAO NVFP4Tensor) entry points.
#include "lm_nvfp4_fast.h"

// ---------------------------------------------------------------------------
// NVFP4
// ---------------------------------------------------------------------------
static int nvfp4_common(const uint8_t* q, const uint8_t* scale, const float* pts, const void* dense, int dense_dt,
                        bool two_level, uint8_t* q_out, uint8_t* scale_out, float* pts_out, int64_t M, int64_t N,
                        int32_t swz, const lm_lora* lora, const lm_rounding* rnd, void* ws, size_t wsb, void* stream) {
  int rc;
  if ((rc = check_nvfp4(M, N))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  if ((rc = check_rounding(rnd))) return rc;
  if (!q_out || !scale_out) return fail(LM_EINVAL, "NVFP4 outputs must be non-null");
  if (two_level && !pts_out) return fail(LM_EINVAL, "two-level NVFP4 needs a per-tensor scale output");
  Ctx c;
  const int cd = lora ? lora->dtype : dense_dt;
  // the pruned amax of a two-level fast merge bounds the delta by the factors' norms (prep)
  const bool fast = lora && !dense && nv_fast_ok(cd, rpad_of(lora->rank) / 16, M, N);
  if ((rc = setup(c, M, N, lora, ws, wsb, stream, false, fast && two_level,
                  fast && nkc_bucket(rpad_of(lora->rank) / 16) == 1 ? AT_NV16 : AT_PLAIN)))
    return rc;
  const bool sr = is_sr(rnd);
  BlkArgs a = blk_args_base(c, M, N, lora, rnd);
  a.q = q;
  a.scale = scale;
  a.aux = two_level ? (const void*)(pts ? pts : (const float*)c.red) : nullptr;
  a.dense = (const uint16_t*)dense;
  a.q_out = q_out;
  a.scale_out = scale_out;
  a.aux_out = pts_out;
  a.swizzled = swz;
  if (swz && (rc = zero_swizzle_pad(scale_out, M, N / 16, c.st))) return rc;
  if (fast) {
    NvArgs na;
    na.q = q;
    na.scale = scale;
    na.gin = two_level ? pts : nullptr;
    na.q_out = q_out;
    na.scale_out = scale_out;
    na.gout = pts_out;
    na.at = c.at;
    na.bp = c.bp;
    na.red = c.red;
    na.nrm = c.nrm;
    na.ub = c.ub;
    na.M = M;
    na.N = N;
    na.strength = lora->strength;
    na.swizzled = swz;
    na.seed = rnd ? rnd->seed : 0;
    return nv_fast_run(na, c.nkc, sr, c.st);
  }
  if (two_level) {
    if ((rc = run_blocks<B_NVFP4, P_AMAX>(a, cd, c.nkc, false, dense != nullptr, c.st))) return rc;
    if ((rc = run_blocks<B_NVFP4, P_QUANT>(a, cd, c.nkc, sr, dense != nullptr, c.st))) return rc;
    return run_finalize<B_NVFP4>(a, cd, c.st) ? fail(LM_EHIP, "finalize launch failed") : LM_OK;
  }
  return run_blocks<B_NVFP4, P_FULL>(a, cd, c.nkc, sr, dense != nullptr, c.st);
}

extern "C" int lm_nvfp4_merge(const uint8_t* q, const uint8_t* scale, const float* per_tensor_scale, uint8_t* q_out,
                              uint8_t* scale_out, float* per_tensor_scale_out, int64_t M, int64_t N, int32_t swizzled,
                              const lm_lora* lora, const lm_rounding* rounding, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (!q || !scale) return fail(LM_EINVAL, "NVFP4 inputs must be non-null");
  if (!lora) return fail(LM_EINVAL, "lm_nvfp4_merge requires LoRA factors");
  return nvfp4_common(q, scale, per_tensor_scale, nullptr, 0, per_tensor_scale != nullptr, q_out, scale_out,
                      per_tensor_scale_out, M, N, swizzled, lora, rounding, workspace, workspace_bytes, stream);
}
extern "C" int lm_nvfp4_requant(const void* dense, int32_t dense_dtype, uint8_t* q_out, uint8_t* scale_out,
                                float* per_tensor_scale_out, int64_t M, int64_t N, int32_t swizzled,
                                const lm_rounding* rounding, void* workspace, size_t workspace_bytes, void* stream) {
  if (!dense) return fail(LM_EINVAL, "dense input must be non-null");
  if (dense_dtype != LM_BF16 && dense_dtype != LM_F16) return fail(LM_EUNSUPPORTED, "requant input must be bf16/fp16");
  return nvfp4_common(nullptr, nullptr, nullptr, dense, dense_dtype, per_tensor_scale_out != nullptr, q_out, scale_out,
                      per_tensor_scale_out, M, N, swizzled, nullptr, rounding, workspace, workspace_bytes, stream);
}
extern "C" int lm_nvfp4_dequant(const uint8_t* q, const uint8_t* scale, const float* per_tensor_scale, int64_t M, int64_t N,
                                int32_t swizzled, const lm_lora* lora, void* out, int32_t out_dtype, void* workspace,
                                size_t workspace_bytes, void* stream) {
  int rc;
  if (!q || !scale || !out) return fail(LM_EINVAL, "NVFP4 dequant pointers must be non-null");
  if ((rc = check_nvfp4(M, N))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  Ctx c;
  if ((rc = setup(c, M, N, lora, workspace, workspace_bytes, stream))) return rc;
  BlkArgs a = blk_args_base(c, M, N, lora, nullptr);
  a.q = q;
  a.scale = scale;
  a.aux = per_tensor_scale;
  a.swizzled = swizzled;
  a.out = out;
  a.out_dt = out_dtype;
  const int cd = lora ? lora->dtype : (out_dtype == LM_F16 ? LM_F16 : LM_BF16);
  return run_blocks<B_NVFP4, P_TODENSE>(a, cd, c.nkc, false, false, c.st);
}

