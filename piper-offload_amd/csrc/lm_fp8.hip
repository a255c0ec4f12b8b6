// lm_fp8.hip -- scaled FP8 (TorchAO Float8Tensor) entry points.
#include "lm_group.h"

// ---------------------------------------------------------------------------
// FP8
// ---------------------------------------------------------------------------
static int check_fp8_layout(int64_t M, int64_t N, int64_t group, int32_t fmt) {
  if (M <= 0 || N <= 0) return fail(LM_EINVAL, "FP8 merge requires a non-empty weight");
  if (fmt != LM_E4M3 && fmt != LM_E5M2) return fail(LM_EUNSUPPORTED, "FP8 storage must be e4m3fn or e5m2");
  if (group != N && group != M * N && !group_size_ok(N, group))
    return fail(LM_EUNSUPPORTED,
                "FP8 supports per-row, per-tensor and per-group layouts (group 16, 32 or a multiple of 64 dividing "
                "N), got group %lld for N=%lld",
                (long long)group, (long long)N);
  return LM_OK;
}

static int fp8_common(const uint8_t* q, const float* scale, const void* dense, int dense_dt, uint8_t* q_out,
                      float* scale_out, int64_t M, int64_t N, int64_t group, int32_t fmt, const lm_lora* lora,
                      const lm_rounding* rnd, void* ws, size_t wsb, void* stream) {
  int rc;
  if ((rc = check_fp8_layout(M, N, group, fmt))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  if ((rc = check_rounding(rnd))) return rc;
  if (!q_out || !scale_out) return fail(LM_EINVAL, "FP8 outputs must be non-null");
  const int cd = lora ? lora->dtype : dense_dt;
  const bool sr = is_sr(rnd);
  const bool split = !dense && group == N && lora &&
                     rows_split_wanted(fmt == LM_E4M3 ? K_E4M3 : K_E5M2, cd, LM_F32, false, sr,
                                       rpad_of(lora->rank) / 16, M, N);
  Ctx c;
  if ((rc = setup(c, M, N, lora, ws, wsb, stream, split))) return rc;
  if (group == N || group != M * N) {  // per-row, or per-group
    RowArgs a;
    memset(&a, 0, sizeof a);
    a.q = q;
    a.scale = scale;
    a.dense = (const uint16_t*)dense;
    a.q_out = q_out;
    a.scale_out = scale_out;
    a.at = c.at;
    a.bp = c.bp;
    a.M = M;
    a.N = N;
    a.strength = lora ? lora->strength : 0.0f;
    a.seed = seed_of(rnd);
    a.red = split ? c.red : nullptr;
    if (group != N) {
      if (fmt == LM_E4M3) {
        if (dense) return run_groups<K_E4M3, true>(a, group, cd, LM_F32, false, sr, 0, c.st);
        return run_groups<K_E4M3, false>(a, group, cd, LM_F32, false, sr, c.nkc, c.st);
      }
      if (dense) return run_groups<K_E5M2, true>(a, group, cd, LM_F32, false, sr, 0, c.st);
      return run_groups<K_E5M2, false>(a, group, cd, LM_F32, false, sr, c.nkc, c.st);
    }
    if (fmt == LM_E4M3) {
      if (dense) return run_rows<K_E4M3, true>(a, cd, LM_F32, false, sr, 0, c.st);
      return run_rows<K_E4M3, false>(a, cd, LM_F32, false, sr, c.nkc, c.st);
    }
    if (dense) return run_rows<K_E5M2, true>(a, cd, LM_F32, false, sr, 0, c.st);
    return run_rows<K_E5M2, false>(a, cd, LM_F32, false, sr, c.nkc, c.st);
  }
  BlkArgs a = blk_args_base(c, M, N, lora, rnd);
  a.q = q;
  a.scale = scale;
  a.dense = (const uint16_t*)dense;
  a.q_out = q_out;
  a.scale_out = scale_out;
  a.scale_dt = LM_F32;
  a.group = group;
  if (fmt == LM_E4M3) {
    if ((rc = run_blocks<B_E4M3, P_AMAX>(a, cd, c.nkc, false, dense != nullptr, c.st))) return rc;
    if ((rc = run_blocks<B_E4M3, P_QUANT>(a, cd, c.nkc, sr, dense != nullptr, c.st))) return rc;
    return run_finalize<B_E4M3>(a, cd, c.st) ? fail(LM_EHIP, "finalize launch failed") : LM_OK;
  }
  if ((rc = run_blocks<B_E5M2, P_AMAX>(a, cd, c.nkc, false, dense != nullptr, c.st))) return rc;
  if ((rc = run_blocks<B_E5M2, P_QUANT>(a, cd, c.nkc, sr, dense != nullptr, c.st))) return rc;
  return run_finalize<B_E5M2>(a, cd, c.st) ? fail(LM_EHIP, "finalize launch failed") : LM_OK;
}

extern "C" int lm_fp8_merge(const uint8_t* q, const float* scale, uint8_t* q_out, float* scale_out, int64_t M, int64_t N,
                            int64_t group, int32_t fp8_dtype, const lm_lora* lora, const lm_rounding* rounding,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !scale) return fail(LM_EINVAL, "FP8 inputs must be non-null");
  if (!lora) return fail(LM_EINVAL, "lm_fp8_merge requires LoRA factors");
  return fp8_common(q, scale, nullptr, 0, q_out, scale_out, M, N, group, fp8_dtype, lora, rounding, workspace,
                    workspace_bytes, stream);
}
extern "C" int lm_fp8_requant(const void* dense, int32_t dense_dtype, uint8_t* q_out, float* scale_out, int64_t M,
                              int64_t N, int64_t group, int32_t fp8_dtype, const lm_rounding* rounding, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (!dense) return fail(LM_EINVAL, "dense input must be non-null");
  if (dense_dtype != LM_BF16 && dense_dtype != LM_F16) return fail(LM_EUNSUPPORTED, "requant input must be bf16/fp16");
  return fp8_common(nullptr, nullptr, dense, dense_dtype, q_out, scale_out, M, N, group, fp8_dtype, nullptr, rounding,
                    workspace, workspace_bytes, stream);
}
extern "C" int lm_fp8_dequant(const uint8_t* q, const float* scale, int64_t M, int64_t N, int64_t group, int32_t fp8_dtype,
                              const lm_lora* lora, void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes,
                              void* stream) {
  int rc;
  if (!q || !scale || !out) return fail(LM_EINVAL, "FP8 dequant pointers must be non-null");
  if ((rc = check_fp8_layout(M, N, group, fp8_dtype))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  Ctx c;
  if ((rc = setup(c, M, N, lora, workspace, workspace_bytes, stream))) return rc;
  BlkArgs a = blk_args_base(c, M, N, lora, nullptr);
  a.q = q;
  a.scale = scale;
  a.scale_dt = LM_F32;
  a.group = group;
  a.out = out;
  a.out_dt = out_dtype;
  const int cd = lora ? lora->dtype : (out_dtype == LM_F16 ? LM_F16 : LM_BF16);
  if (fp8_dtype == LM_E4M3) return run_blocks<B_E4M3, P_TODENSE>(a, cd, c.nkc, false, false, c.st);
  return run_blocks<B_E5M2, P_TODENSE>(a, cd, c.nkc, false, false, c.st);
}

