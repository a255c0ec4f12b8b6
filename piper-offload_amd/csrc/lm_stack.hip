// lm_stack.hip -- grouped multi-target (stack) entry points.
#include "lm_nvfp4_fast.h"
#include "lm_rows_stack.h"

// ---------------------------------------------------------------------------
// stacks
// ---------------------------------------------------------------------------
// Stack workspace: the descriptor tables, 256 bytes of slack, then the
// per-item regions.
extern "C" size_t lm_stack_workspace_extra(int32_t count) {
  return align256((size_t)count * sizeof(PrepItem)) + align256((size_t)count * sizeof(RowStackItem)) +
         align256((size_t)count * sizeof(BlkArgs)) + 256;
}

static int stack_layout(const lm_stack_item* items, int32_t count, void* ws, size_t wsb, PrepItem* preps,
                        size_t& cursor) {
  uint8_t* base = (uint8_t*)ws;
  for (int i = 0; i < count; ++i) {
    const lm_stack_item& s = items[i];
    int rc;
    if ((rc = check_lora(&s.lora, s.M, s.N))) return rc;
    WsLayout w = ws_layout(s.M, s.N, s.lora.rank);
    if (cursor + w.total > wsb) return fail(LM_EWORKSPACE, "stack workspace too small at item %d", i);
    PrepItem& p = preps[i];
    p.b = (const uint16_t*)s.lora.b;
    p.a = (const uint16_t*)s.lora.a;
    p.ldb = s.lora.ldb;
    p.lda = s.lora.lda;
    p.M = s.M;
    p.N = s.N;
    p.rank = s.lora.rank;
    p.rpad = rpad_of(s.lora.rank);
    p.at = (uint16_t*)(base + cursor + w.at_off);
    p.bp = (uint16_t*)(base + cursor + w.bp_off);
    p.red = (uint32_t*)(base + cursor + w.red_off);
    p.nrm = (float*)(base + cursor + w.nrm_off);
    p.ub = (float*)(base + cursor + w.ub_off);
    p.nred = 64;
    p.vec_b = prep_vec_b(p);
    cursor += w.total;
  }
  return LM_OK;
}

static int stack_prep(PrepItem* preps, int32_t count, uint8_t* dev_items, hipStream_t st) {
  int64_t blocks = 0;
  for (int i = 0; i < count; ++i) {
    preps[i].work_begin = 0;
    preps[i].block_begin = blocks;
    blocks += (prep_units(preps[i]) + PREP_PER_BLOCK - 1) / PREP_PER_BLOCK;
  }
  if (blocks > 0x7fffffff) return fail(LM_EUNSUPPORTED, "stack factors too large for one prep launch");
  int rc = lm_stage_h2d(dev_items, preps, sizeof(PrepItem) * count, st);
  if (rc != LM_OK) return rc;
  TimedLaunch timed("prep", st);
  hipLaunchKernelGGL(k_prep_many, dim3((unsigned)blocks), dim3(256), 0, st, (const PrepItem*)dev_items, count);
  LAUNCH_CHECK();
  return LM_OK;
}

extern "C" int lm_int8_merge_stack(const lm_stack_item* items, int32_t count, int32_t scale_dtype, int32_t rounding_mode,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  if (count <= 0) return LM_OK;
  if (!items || !workspace) return fail(LM_EINVAL, "stack items and workspace must be non-null");
  if (scale_dtype != LM_F32 && scale_dtype != LM_BF16) return fail(LM_EUNSUPPORTED, "INT8 scales must be f32/bf16");
  if (((uintptr_t)workspace & 255) != 0) return fail(LM_EINVAL, "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const size_t extra = lm_stack_workspace_extra(count);
  if (workspace_bytes < extra) return fail(LM_EWORKSPACE, "stack workspace too small");
  uint8_t* base = (uint8_t*)workspace;
  uint8_t* dev_prep = base;
  uint8_t* dev_rows = base + align256((size_t)count * sizeof(PrepItem));
  size_t cursor = extra;
  // host tables; lm_stage_h2d copies them into pinned staging before returning
  // the rows table and, right after its region, the items' first groups
  // (begins, int32, in launch order): one upload into the RowStackItem and
  // BlkArgs regions of the workspace (the INT8 stack does not use the latter)
  const size_t rows_bytes = align256((size_t)count * sizeof(RowStackItem));
  static_assert(sizeof(BlkArgs) >= sizeof(int32_t), "begins fit the BlkArgs region");
  PrepItem* preps = (PrepItem*)calloc(count, sizeof(PrepItem));
  RowStackItem* rows = (RowStackItem*)calloc(1, rows_bytes + (size_t)count * sizeof(int32_t));
  if (!preps || !rows) {
    free(preps);
    free(rows);
    return fail(LM_EINVAL, "host allocation failed");
  }
  int32_t* begins = (int32_t*)((uint8_t*)rows + rows_bytes);
  int rc = stack_layout(items, count, workspace, workspace_bytes, preps, cursor);
  int nkc_max = 0, cd = items[0].lora.dtype;
  for (int i = 0; i < count; ++i) {
    const int nkc = rpad_of(items[i].lora.rank) / 16;
    nkc_max = nkc > nkc_max ? nkc : nkc_max;
  }
  const bool sr = rounding_mode == LM_ROUND_STOCHASTIC;
  bool fast = true;
  for (int i = 0; i < count; ++i) fast = fast && rows_fast_ok(K_INT8, cd, scale_dtype, false, nkc_max, items[i].M, items[i].N);
  // fast kernels: items whose rows want the deep register cache go to a
  // second launch; each launch numbers its 16-row groups from 0
  int n_regular = 0;
  for (int i = 0; i < count; ++i) n_regular += (fast && rows_long_mode(nkc_max, sr, items[i].N) != ROWS_REGULAR) ? 0 : 1;
  int64_t tiles[2] = {0, 0};
  int slot[2] = {0, n_regular};
  // rank 16 on the fast kernels: A^T in the row kernels' tile order
  const bool r16 = fast && nkc_bucket(nkc_max) == 1;
  for (int i = 0; i < count; ++i) preps[i].at_order = r16 ? AT_ROWS16 : AT_PLAIN;
  for (int i = 0; rc == LM_OK && i < count; ++i) {
    const lm_stack_item& s = items[i];
    if (s.lora.dtype != cd) rc = fail(LM_EUNSUPPORTED, "all stack items must share one factor dtype");
    if (s.M <= 0 || s.N <= 0 || !s.q || !s.scale || !s.q_out || !s.scale_out)
      rc = fail(LM_EINVAL, "stack item %d has an invalid shape or null pointer", i);
    const int grp = (fast && rows_long_mode(nkc_max, sr, s.N) != ROWS_REGULAR) ? 1 : 0;
    RowStackItem& r = rows[slot[grp]++];
    RowArgs& a = r.a;
    a.q = s.q;
    a.scale = s.scale;
    a.zp = nullptr;
    a.q_out = s.q_out;
    a.scale_out = s.scale_out;
    a.at = preps[i].at;
    a.bp = preps[i].bp;
    a.M = s.M;
    a.N = s.N;
    a.strength = s.lora.strength;
    a.qmin = -128;
    a.qmax = 127;
    a.seed = s.seed;
    a.red = nullptr;
    r.tile_begin = tiles[grp];
    begins[slot[grp] - 1] = (int32_t)tiles[grp];
    tiles[grp] += (s.M + 15) / 16;
  }
  if (rc == LM_OK && (tiles[0] > 0x7fffffff || tiles[1] > 0x7fffffff))
    rc = fail(LM_EUNSUPPORTED, "stack too large for one launch");
  if (rc == LM_OK) rc = stack_prep(preps, count, dev_prep, st);
  if (rc == LM_OK) {
    // every item uses the largest rank bucket: the prepared layouts are per item,
    // so items with a smaller rank must have the same padding.  Re-check.
    for (int i = 0; i < count; ++i)
      if (nkc_bucket(rpad_of(items[i].lora.rank) / 16) != nkc_bucket(nkc_max))
        rc = fail(LM_EUNSUPPORTED, "stack items must share one rank bucket (16/32/64)");
  }
  if (rc == LM_OK) rc = lm_stage_h2d(dev_rows, rows, rows_bytes + sizeof(int32_t) * count, st);
  const int32_t* dev_begins = (const int32_t*)(dev_rows + rows_bytes);
  if (rc == LM_OK) {
    const dim3 block(ROW_NW * 64);
    TimedLaunch timed("rows_stack", st);
    const RowStackItem* d0 = (const RowStackItem*)dev_rows;
    if (fast) {
      rc = scale_dtype == LM_BF16 ? int8_stack_fast_launch_sbf(d0, dev_begins, n_regular, count, tiles, nkc_max, sr, st)
                                  : int8_stack_fast_launch<false>(d0, dev_begins, n_regular, count, tiles, nkc_max, sr, st);
    } else {
      const dim3 grid((unsigned)tiles[0]);
#define RS(CD_, SDT_, SR_) NKC_SWITCH(nkc_bucket(nkc_max), hipLaunchKernelGGL((k_rows_stack<K_INT8, CD_, SDT_, SR_, NKC_, ROW_NW, ROW_CACHE>), grid, block, 0, st, d0, count, scale_dtype))
    if (cd == LM_F16) {
      if (scale_dtype == LM_BF16) { if (sr) { RS(F16, BF16, true); } else { RS(F16, BF16, false); } }
      else { if (sr) { RS(F16, F32, true); } else { RS(F16, F32, false); } }
    } else {
      if (scale_dtype == LM_BF16) { if (sr) { RS(BF16, BF16, true); } else { RS(BF16, BF16, false); } }
      else { if (sr) { RS(BF16, F32, true); } else { RS(BF16, F32, false); } }
    }
#undef RS
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) rc = fail(LM_EHIP, "stack launch: %s", hipGetErrorString(e));
  }
  free(preps);
  free(rows);
  return rc;
}

// Grouped NVFP4 merge.  Two-level items: the pruned amax (bound-and-seed and
// refine launches over all of them), then one quant launch; single-level
// items: one quant launch.  `dev_items` is workspace for the descriptor table
// (the BlkArgs region of lm_stack_workspace_extra).
static int nv_stack_fast(const lm_stack_item* items, int32_t count, int32_t swizzled, bool sr, const PrepItem* preps,
                         uint8_t* dev_items, hipStream_t st) {
  static_assert(sizeof(NvStackItem) <= sizeof(BlkArgs), "NVFP4 stack descriptors must fit the workspace slot");
  NvStackItem* h = (NvStackItem*)calloc(count, sizeof(NvStackItem));
  if (!h) return fail(LM_EINVAL, "host allocation failed");
  // two-level items first, then single-level ones; each group numbers its
  // 16-row units from 0 and gets its own quant launch
  int n_two = 0;
  for (int i = 0; i < count; ++i) n_two += items[i].aux != nullptr ? 1 : 0;
  int64_t tiles[2] = {0, 0};
  int64_t bounds = 0, refines = 0;  // the pruned amax: 128-row bound chunks, 512-tile refine chunks
  int slot[2] = {0, n_two};
  int rc = LM_OK;
  for (int i = 0; i < count && rc == LM_OK; ++i) {
    const lm_stack_item& s = items[i];
    if (!s.q || !s.scale || !s.q_out || !s.scale_out) rc = fail(LM_EINVAL, "stack item %d has a null pointer", i);
    if (s.aux && !s.aux_out) rc = fail(LM_EINVAL, "stack item %d: two-level NVFP4 needs a per-tensor scale output", i);
    if (s.aux && !preps[i].norms) rc = fail(LM_EINVAL, "stack item %d: two-level NVFP4 without its norm workspace", i);
    const int grp = s.aux != nullptr ? 0 : 1;
    NvStackItem& it = h[slot[grp]++];
    NvArgs& a = it.a;
    a.q = (const uint8_t*)s.q;
    a.scale = (const uint8_t*)s.scale;
    a.gin = (const float*)s.aux;
    a.q_out = (uint8_t*)s.q_out;
    a.scale_out = (uint8_t*)s.scale_out;
    a.gout = (float*)s.aux_out;
    a.at = preps[i].at;
    a.bp = preps[i].bp;
    a.red = preps[i].red;
    a.nrm = preps[i].norms ? preps[i].nrm : nullptr;
    a.ub = preps[i].ub;
    a.M = s.M;
    a.N = s.N;
    a.strength = s.lora.strength;
    a.swizzled = swizzled;
    a.seed = s.seed;
    it.tile_begin = tiles[grp];
    tiles[grp] += nv_units(s.M, s.N);
    it.bound_begin = bounds;
    it.refine_begin = refines;
    if (grp == 0) {
      bounds += nv_bound_units(s.M);
      refines += nv_refine_units(s.M, s.N);
    }
    if (rc == LM_OK && swizzled) rc = zero_swizzle_pad((uint8_t*)s.scale_out, s.M, s.N / 16, st);
  }
  if (rc == LM_OK) rc = lm_stage_h2d(dev_items, h, sizeof(NvStackItem) * count, st);
  if (rc == LM_OK && (bounds > 0x7fffffff || refines > 0x7fffffff))
    rc = fail(LM_EUNSUPPORTED, "nvfp4 stack too large for one launch");
  const int nkc = preps[0].rpad / 16;
  const dim3 block(NV_NW * 64);
  const NvStackItem* d = (const NvStackItem*)dev_items;
  // block scales staged in LDS: plain layout, rows of at most NV_LSC_TILES macro tiles
  bool lsc = !swizzled;
  for (int i = 0; i < count; ++i) lsc = lsc && (items[i].N >> 7) <= NV_LSC_TILES;
  if (rc == LM_OK && n_two > 0) {
    TimedLaunch timed("nvfp4", st);
    NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_nv_bound_stack<NKC_>), dim3((unsigned)bounds), block, 0, st, d,
                                                   n_two));
    NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_nv_refine_stack<NKC_>), dim3((unsigned)refines), block, 0, st, d,
                                                   n_two));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) rc = fail(LM_EHIP, "nvfp4 pruned amax launches: %s", hipGetErrorString(e));
  }
  if (rc == LM_OK && n_two > 0) {
    TimedLaunch timed("nvfp4", st);
#define NQ2(SR_, LSC_)                                                                                     \
  NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_nv_quant_stack<NKC_, SR_, true, LSC_>), dim3((unsigned)tiles[0]), \
                                                 block, 0, st, d, n_two))
    if (lsc) { if (sr) { NQ2(true, true); } else { NQ2(false, true); } }
    else { if (sr) { NQ2(true, false); } else { NQ2(false, false); } }
#undef NQ2
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) rc = fail(LM_EHIP, "nvfp4 quant launch: %s", hipGetErrorString(e));
  }
  if (rc == LM_OK && tiles[1] > 0) {
    TimedLaunch timed("nvfp4", st);
#define NQ(SR_, LSC_)                                                                                       \
  NKC_SWITCH(nkc_bucket(nkc), hipLaunchKernelGGL((k_nv_quant_stack<NKC_, SR_, false, LSC_>), dim3((unsigned)tiles[1]), \
                                                 block, 0, st, d + n_two, count - n_two))
    if (lsc) { if (sr) { NQ(true, true); } else { NQ(false, true); } }
    else { if (sr) { NQ(true, false); } else { NQ(false, false); } }
#undef NQ
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) rc = fail(LM_EHIP, "nvfp4 quant launch: %s", hipGetErrorString(e));
  }
  free(h);
  return rc;
}

// NVFP4 stack: the grouped fast kernels when every item qualifies; otherwise
// every item is processed by its own block-kernel launches after one grouped
// prep (two-level items need their own amax pass).
extern "C" int lm_nvfp4_merge_stack(const lm_stack_item* items, int32_t count, int32_t swizzled, int32_t rounding_mode,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  if (count <= 0) return LM_OK;
  if (!items || !workspace) return fail(LM_EINVAL, "stack items and workspace must be non-null");
  if (((uintptr_t)workspace & 255) != 0) return fail(LM_EINVAL, "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const size_t extra = lm_stack_workspace_extra(count);
  if (workspace_bytes < extra) return fail(LM_EWORKSPACE, "stack workspace too small");
  uint8_t* base = (uint8_t*)workspace;
  size_t cursor = extra;
  PrepItem* preps = (PrepItem*)calloc(count, sizeof(PrepItem));
  if (!preps) return fail(LM_EINVAL, "host allocation failed");
  int rc = stack_layout(items, count, workspace, workspace_bytes, preps, cursor);
  bool fast = rc == LM_OK;
  for (int i = 0; fast && i < count; ++i)
    fast = nv_fast_ok(items[i].lora.dtype, preps[i].rpad / 16, items[i].M, items[i].N) &&
           nkc_bucket(preps[i].rpad / 16) == nkc_bucket(preps[0].rpad / 16) && check_nvfp4(items[i].M, items[i].N) == 0;
  // two-level items with bf16 factors: the factors' norms for the pruned
  // amax; rank 16 on the fast kernels: A^T in their macro-tile order
  for (int i = 0; rc == LM_OK && i < count; ++i) {
    preps[i].norms = items[i].aux && items[i].lora.dtype == LM_BF16 ? 1 : 0;
    preps[i].at_order = fast && nkc_bucket(preps[0].rpad / 16) == 1 ? AT_NV16 : AT_PLAIN;
  }
  if (rc == LM_OK) rc = stack_prep(preps, count, base, st);
  if (fast && rc == LM_OK) {
    uint8_t* dev_blk = base + align256((size_t)count * sizeof(PrepItem)) + align256((size_t)count * sizeof(RowStackItem));
    rc = nv_stack_fast(items, count, swizzled, rounding_mode == LM_ROUND_STOCHASTIC, preps, dev_blk, st);
    free(preps);
    return rc;
  }
  lm_rounding rnd;
  rnd.mode = rounding_mode;
  rnd.reserved = 0;
  for (int i = 0; rc == LM_OK && i < count; ++i) {
    const lm_stack_item& s = items[i];
    if ((rc = check_nvfp4(s.M, s.N))) break;
    rnd.seed = s.seed;
    Ctx c;
    c.st = st;
    c.at = preps[i].at;
    c.bp = preps[i].bp;
    c.red = preps[i].red;
    c.nkc = preps[i].rpad / 16;
    const bool two = s.aux != nullptr;
    BlkArgs a = blk_args_base(c, s.M, s.N, &s.lora, &rnd);
    a.q = s.q;
    a.scale = s.scale;
    a.aux = s.aux;
    a.q_out = s.q_out;
    a.scale_out = s.scale_out;
    a.aux_out = s.aux_out;
    a.swizzled = swizzled;
    const bool sr = rounding_mode == LM_ROUND_STOCHASTIC;
    if (swizzled && (rc = zero_swizzle_pad((uint8_t*)s.scale_out, s.M, s.N / 16, st))) break;
    if (two) {
      if ((rc = run_blocks<B_NVFP4, P_AMAX>(a, s.lora.dtype, c.nkc, false, false, st))) break;
      if ((rc = run_blocks<B_NVFP4, P_QUANT>(a, s.lora.dtype, c.nkc, sr, false, st))) break;
      if (run_finalize<B_NVFP4>(a, s.lora.dtype, st)) rc = fail(LM_EHIP, "finalize launch failed");
    } else {
      rc = run_blocks<B_NVFP4, P_FULL>(a, s.lora.dtype, c.nkc, sr, false, st);
    }
  }
  free(preps);
  return rc;
}
