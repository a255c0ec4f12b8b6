// lm_int8.hip -- INT8 (TorchAO Int8Tensor) merge / requant / dequant entry points.
#include "lm_group.h"

// ---------------------------------------------------------------------------
// INT8
// ---------------------------------------------------------------------------
static int check_int8_layout(int64_t M, int64_t N, int64_t group, int32_t scale_dtype) {
  if (M <= 0 || N <= 0) return fail(LM_EINVAL, "INT8 merge requires a non-empty weight, got [%lld, %lld]", (long long)M, (long long)N);
  if (scale_dtype != LM_F32 && scale_dtype != LM_BF16)
    return fail(LM_EUNSUPPORTED, "INT8 scales must be float32 or bfloat16, got dtype id %d", scale_dtype);
  if (group != N && group != M * N && !group_size_ok(N, group))
    return fail(LM_EUNSUPPORTED,
                "INT8 supports per-row (group=N), per-tensor (group=M*N) and per-group layouts (group 16, 32 or a "
                "multiple of 64 dividing N), got group %lld for N=%lld",
                (long long)group, (long long)N);
  return LM_OK;
}

static int int8_common(const int8_t* q, const void* scale, const int8_t* zp, const void* dense, int dense_dt, int8_t* q_out,
                       void* scale_out, int8_t* zp_out, int64_t M, int64_t N, int64_t group, int32_t sdt, int32_t asym,
                       int32_t reduce_range, const lm_lora* lora, const lm_rounding* rnd, void* ws, size_t wsb,
                       void* stream) {
  int rc;
  if ((rc = check_int8_layout(M, N, group, sdt))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  if ((rc = check_rounding(rnd))) return rc;
  if (!q_out || !scale_out) return fail(LM_EINVAL, "INT8 outputs must be non-null");
  const int cd = lora ? lora->dtype : dense_dt;
  const bool sr = is_sr(rnd);
  const bool split = !dense && group == N && lora &&
                     rows_split_wanted(K_INT8, cd, sdt, asym != 0, sr, rpad_of(lora->rank) / 16, M, N);
  Ctx c;
  if ((rc = setup(c, M, N, lora, ws, wsb, stream, split))) return rc;
  const int qmin = reduce_range ? -64 : -128, qmax = reduce_range ? 63 : 127;
  if (group == N || group != M * N) {  // per-row, or per-group
    RowArgs a;
    memset(&a, 0, sizeof a);
    a.q = q;
    a.scale = scale;
    a.zp = zp;
    a.dense = (const uint16_t*)dense;
    a.q_out = q_out;
    a.scale_out = scale_out;
    a.zp_out = zp_out;
    a.at = c.at;
    a.bp = c.bp;
    a.M = M;
    a.N = N;
    a.strength = lora ? lora->strength : 0.0f;
    a.qmin = qmin;
    a.qmax = qmax;
    a.seed = seed_of(rnd);
    a.red = split ? c.red : nullptr;
    if (group != N) {
      if (dense) return run_groups<K_INT8, true>(a, group, cd, sdt, asym != 0, sr, 0, c.st);
      return run_groups<K_INT8, false>(a, group, cd, sdt, asym != 0, sr, c.nkc, c.st);
    }
    if (dense) return run_rows<K_INT8, true>(a, cd, sdt, asym != 0, sr, 0, c.st);
    return run_rows<K_INT8, false>(a, cd, sdt, asym != 0, sr, c.nkc, c.st);
  }
  // per-tensor: two passes
  BlkArgs a = blk_args_base(c, M, N, lora, rnd);
  a.q = q;
  a.scale = scale;
  a.aux = zp;
  a.dense = (const uint16_t*)dense;
  a.q_out = q_out;
  a.scale_out = scale_out;
  a.aux_out = zp_out;
  a.scale_dt = sdt;
  a.qmin = qmin;
  a.qmax = qmax;
  a.asym = asym;
  a.group = group;
  if ((rc = run_blocks<B_INT8, P_AMAX>(a, cd, c.nkc, false, dense != nullptr, c.st))) return rc;
  if ((rc = run_blocks<B_INT8, P_QUANT>(a, cd, c.nkc, sr, dense != nullptr, c.st))) return rc;
  return run_finalize<B_INT8>(a, cd, c.st) ? fail(LM_EHIP, "finalize launch failed") : LM_OK;
}

extern "C" int lm_int8_merge(const int8_t* q, const void* scale, const int8_t* zero_point, int8_t* q_out, void* scale_out,
                             int8_t* zero_point_out, int64_t M, int64_t N, int64_t group, int32_t scale_dtype,
                             int32_t asymmetric, int32_t reduce_range, const lm_lora* lora, const lm_rounding* rounding,
                             void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !scale) return fail(LM_EINVAL, "INT8 inputs must be non-null");
  if (!lora) return fail(LM_EINVAL, "lm_int8_merge requires LoRA factors");
  if (asymmetric && (!zero_point_out)) return fail(LM_EINVAL, "asymmetric INT8 merge requires a zero-point output");
  return int8_common(q, scale, zero_point, nullptr, 0, q_out, scale_out, zero_point_out, M, N, group, scale_dtype,
                     asymmetric, reduce_range, lora, rounding, workspace, workspace_bytes, stream);
}

extern "C" int lm_int8_requant(const void* dense, int32_t dense_dtype, int8_t* q_out, void* scale_out,
                               int8_t* zero_point_out, int64_t M, int64_t N, int64_t group, int32_t scale_dtype,
                               int32_t asymmetric, int32_t reduce_range, const lm_rounding* rounding, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (!dense) return fail(LM_EINVAL, "dense input must be non-null");
  if (dense_dtype != LM_BF16 && dense_dtype != LM_F16)
    return fail(LM_EUNSUPPORTED, "requant input must be bfloat16 or float16");
  if ((N & 7) != 0 && group == N) {
    // the dense fast path needs 16-byte rows; the masked path handles the rest
  }
  return int8_common(nullptr, nullptr, nullptr, dense, dense_dtype, q_out, scale_out, zero_point_out, M, N, group,
                     scale_dtype, asymmetric, reduce_range, nullptr, rounding, workspace, workspace_bytes, stream);
}

extern "C" int lm_int8_dequant(const int8_t* q, const void* scale, const int8_t* zero_point, int64_t M, int64_t N,
                               int64_t group, int32_t scale_dtype, const lm_lora* lora, void* out, int32_t out_dtype,
                               void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if (!q || !scale || !out) return fail(LM_EINVAL, "INT8 dequant pointers must be non-null");
  if ((rc = check_int8_layout(M, N, group, scale_dtype))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  Ctx c;
  if ((rc = setup(c, M, N, lora, workspace, workspace_bytes, stream))) return rc;
  BlkArgs a = blk_args_base(c, M, N, lora, nullptr);
  a.q = q;
  a.scale = scale;
  a.aux = zero_point;
  a.scale_dt = scale_dtype;
  a.group = group;
  a.out = out;
  a.out_dt = out_dtype;
  const int cd = lora ? lora->dtype : (out_dtype == LM_F16 ? LM_F16 : LM_BF16);
  return run_blocks<B_INT8, P_TODENSE>(a, cd, c.nkc, false, false, c.st);
}


// ---------------------------------------------------------------------------
// lm_int8_merge_noalloc: lm_int8_merge with its workspace in a static device
// array, for callers that cannot allocate (code under HIP graph capture, tight
// serving loops).  Each GPU holds its own copy of `scratch` from module load to
// process exit.  Host code never passes the array's name to a kernel or a copy
// (it is a host-side stand-in, not a device address): the address comes from
// hipGetSymbolAddress, taken once per device with that device current on the
// first call there, and kept per device.  Every call on a GPU shares that
// GPU's array; the factor-relayout kernel rewrites the whole region a call
// reads (the transposed A, the packed B and the cleared reduction slots), so
// nothing of an earlier call survives into a later one.  Calls that overlap
// on one GPU (several streams or threads) race on the array.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[LM_NOALLOC_SCRATCH_BYTES];

#include <mutex>
namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};
}  // namespace

static int scratch_of_current_device(void** out) {
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kScratchDevices)
    return fail(LM_EUNSUPPORTED, "lm_int8_merge_noalloc supports device ordinals below %d, got %d", kScratchDevices, dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(LM_EHIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LM_OK;
}

extern "C" int lm_int8_merge_noalloc(const int8_t* q, const void* scale, const int8_t* zero_point, int8_t* q_out,
                                     void* scale_out, int8_t* zero_point_out, int64_t M, int64_t N, int64_t group,
                                     int32_t scale_dtype, int32_t asymmetric, int32_t reduce_range, const lm_lora* lora,
                                     const lm_rounding* rounding, void* stream) {
  int rc;
  if (!lora) return fail(LM_EINVAL, "lm_int8_merge_noalloc requires LoRA factors");
  if ((rc = check_int8_layout(M, N, group, scale_dtype))) return rc;
  if ((rc = check_lora(lora, M, N))) return rc;
  const size_t need = lm_workspace_size(M, N, lora->rank);
  if (need > (size_t)LM_NOALLOC_SCRATCH_BYTES)
    return fail(LM_EWORKSPACE,
                "lm_int8_merge_noalloc: a [%lld, %lld] rank-%d merge needs %zu bytes of scratch, above the %zu-byte "
                "static array; use lm_int8_merge with a caller workspace",
                (long long)M, (long long)N, (int)lora->rank, need, (size_t)LM_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = scratch_of_current_device(&ws))) return rc;
  return lm_int8_merge(q, scale, zero_point, q_out, scale_out, zero_point_out, M, N, group, scale_dtype, asymmetric,
                       reduce_range, lora, rounding, ws, (size_t)LM_NOALLOC_SCRATCH_BYTES, stream);
}
