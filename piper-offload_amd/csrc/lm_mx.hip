// lm_mx.hip -- MX (TorchAO MXTensor: MXFP4 / MXFP8) entry points.
#include "lm_mx_fast.h"

// ---------------------------------------------------------------------------
// MX
// ---------------------------------------------------------------------------
static int check_mx(int64_t M, int64_t N, int32_t elem, int32_t scaling) {
  if (M <= 0 || N <= 0) return fail(LM_EINVAL, "MX merge requires a non-empty weight");
  if (N % 32 != 0) return fail(LM_EINVAL, "MX requires columns divisible by 32, got %lld", (long long)N);
  if (elem != LM_E2M1 && elem != LM_E4M3 && elem != LM_E5M2) return fail(LM_EUNSUPPORTED, "unsupported MX element dtype");
  if (scaling < 0 || scaling > 3) return fail(LM_EINVAL, "unknown MX scaling mode %d", scaling);
  return LM_OK;
}
template <int PASS>
static int run_mx(const BlkArgs& a, int elem, int cd, int nkc, bool sr, bool from_dense, hipStream_t st) {
  if (elem == LM_E2M1) return run_blocks<B_MXFP4, PASS>(a, cd, nkc, sr, from_dense, st);
  if (elem == LM_E4M3) return run_blocks<B_MXE4M3, PASS>(a, cd, nkc, sr, from_dense, st);
  return run_blocks<B_MXE5M2, PASS>(a, cd, nkc, sr, from_dense, st);
}
extern "C" int lm_mx_merge(uint8_t* q, uint8_t* scale, int64_t M, int64_t N, int32_t elem_dtype, int32_t scaling,
                           int32_t swizzled, const lm_lora* lora, const lm_rounding* rounding, void* workspace,
                           size_t workspace_bytes, void* stream) {
  int rc;
  if (!q || !scale) return fail(LM_EINVAL, "MX pointers must be non-null");
  if (!lora) return fail(LM_EINVAL, "lm_mx_merge requires LoRA factors");
  if ((rc = check_mx(M, N, elem_dtype, scaling))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  if ((rc = check_rounding(rounding))) return rc;
  Ctx c;
  const int nkc = rpad_of(lora->rank) / 16;
  const bool fast = mx_fast_ok(lora->dtype, nkc, M, N);
  // rank 16 on the fast kernel: A^T in its macro-tile order
  if ((rc = setup(c, M, N, lora, workspace, workspace_bytes, stream, false, false,
                  fast && nkc_bucket(nkc) == 1 ? AT_NV16 : AT_PLAIN)))
    return rc;
  if (fast) {
    MxArgs ma;
    ma.q = q;
    ma.scale = scale;
    ma.at = c.at;
    ma.bp = c.bp;
    ma.M = M;
    ma.N = N;
    ma.strength = lora->strength;
    ma.swizzled = swizzled;
    ma.mode = scaling;
    ma.seed = rounding ? rounding->seed : 0;
    return mx_fast_run(ma, elem_dtype, c.nkc, is_sr(rounding), c.st);
  }
  BlkArgs a = blk_args_base(c, M, N, lora, rounding);
  a.q = q;
  a.scale = scale;
  a.q_out = q;
  a.scale_out = scale;
  a.swizzled = swizzled;
  a.mx_mode = scaling;
  return run_mx<P_FULL>(a, elem_dtype, lora->dtype, c.nkc, is_sr(rounding), false, c.st);
}
extern "C" int lm_mx_requant(const void* dense, int32_t dense_dtype, uint8_t* q_out, uint8_t* scale_out, int64_t M,
                             int64_t N, int32_t elem_dtype, int32_t scaling, int32_t swizzled, const lm_rounding* rounding,
                             void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if (!dense || !q_out || !scale_out) return fail(LM_EINVAL, "MX requant pointers must be non-null");
  if ((rc = check_mx(M, N, elem_dtype, scaling))) return rc;
  if ((rc = check_rounding(rounding))) return rc;
  Ctx c;
  if ((rc = setup(c, M, N, nullptr, workspace, workspace_bytes, stream))) return rc;
  BlkArgs a = blk_args_base(c, M, N, nullptr, rounding);
  a.dense = (const uint16_t*)dense;
  a.q_out = q_out;
  a.scale_out = scale_out;
  a.swizzled = swizzled;
  a.mx_mode = scaling;
  if (swizzled && (rc = zero_swizzle_pad(scale_out, M, N / 32, c.st))) return rc;
  return run_mx<P_FULL>(a, elem_dtype, dense_dtype, 0, is_sr(rounding), true, c.st);
}
extern "C" int lm_mx_dequant(const uint8_t* q, const uint8_t* scale, int64_t M, int64_t N, int32_t elem_dtype,
                             int32_t swizzled, const lm_lora* lora, void* out, int32_t out_dtype, void* workspace,
                             size_t workspace_bytes, void* stream) {
  int rc;
  if (!q || !scale || !out) return fail(LM_EINVAL, "MX dequant pointers must be non-null");
  if ((rc = check_mx(M, N, elem_dtype, 0))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  Ctx c;
  if ((rc = setup(c, M, N, lora, workspace, workspace_bytes, stream))) return rc;
  BlkArgs a = blk_args_base(c, M, N, lora, nullptr);
  a.q = q;
  a.scale = scale;
  a.swizzled = swizzled;
  a.out = out;
  a.out_dt = out_dtype;
  const int cd = lora ? lora->dtype : (out_dtype == LM_F16 ? LM_F16 : LM_BF16);
  return run_mx<P_TODENSE>(a, elem_dtype, cd, c.nkc, false, false, c.st);
}

