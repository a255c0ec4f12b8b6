/*
 * lora_merge.h -- C ABI of the MI355X (gfx950) LoRA-merge library
 * (libpiper_lora_merge.so, built from piper-offload_amd/csrc).
 *
 * Each entry point replaces one function of piper-offload's fused merge
 * path.  Citations use P/ = src/piper_offload/ of the reference:
 *
 *   lm_int8_merge   <- merge_int8_lora     P/_triton_int8_lora.py:267-407
 *   lm_fp8_merge    <- merge_float8_lora   P/_triton_float8_lora.py:486-588
 *   lm_nvfp4_merge  <- merge_nvfp4_lora    P/_triton_nvfp4_lora.py:515-595
 *   lm_mx_merge     <- merge_mx_lora_      P/_triton_mx_lora.py:333-425
 *   lm_dense_merge  <- RegularAdapter.merge_lora_ (addmm_)
 *                                          P/tensor_adapters.py:686-696
 *   lm_q8_0_merge   <- (no reference counterpart: the reference routes GGUF
 *                      only, P/gguf_adapter.py:160-284; requant follows the
 *                      ggml Q8_0 recipe)
 *   lm_gguf_dequant <- dequantize          P/gguf_dequant.py:303-331
 *   lm_*_requant, lm_*_dequant           <- the portable dequantize_* /
 *                      requantize_* shims (P/_torchao_int8.py:113-173,
 *                      P/_torchao_float8.py:93-161, P/_torchao_nvfp4.py:106-197,
 *                      P/_torchao_mx.py:143-207) as single fused kernels
 *   lm_*_merge_stack <- the per-target loop of merge_lora()
 *                      (P/merge.py:121-125) as one grouped launch
 *
 * Conventions
 *  - All pointers are device pointers unless noted; tensors are row-major
 *    and contiguous unless a leading dimension is given.  M = out rows,
 *    N = logical in columns, rank = r.
 *  - `stream` is a hipStream_t passed as void*.  No entry point allocates
 *    device memory (scratch comes from the caller's `workspace`, sized by
 *    lm_workspace_size()) and none synchronizes: every call is asynchronous
 *    on `stream`.  The *_stack entry points copy their descriptor tables
 *    into the workspace through pinned host staging owned by the library,
 *    so the caller's item array may be reused as soon as the call returns;
 *    the workspace must stay allocated until the stream has run the call
 *    (stream-ordered allocators such as torch's satisfy this).
 *  - Return value: LM_OK or an lm_status; lm_last_error() returns a
 *    thread-local message for the last failure on the calling thread.
 *  - The deterministic path rounds to nearest even.  Stochastic rounding
 *    draws u = k * 2^-16, k a 16-bit half of word (idx & 7) >> 1 of
 *    Philox4x32-7(counter = idx >> 3, key = seed) (high half for even idx,
 *    words 1 and 3 complemented), idx = row * N + col.
 *  - merged = round_compute(fma(delta, strength, base)), delta the fp32
 *    accumulation of B@A on bf16/fp16 MFMA.
 */
#ifndef PIPER_LORA_MERGE_H
#define PIPER_LORA_MERGE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LM_ABI_VERSION 1

/* element / storage dtypes */
enum lm_dtype {
  LM_F32 = 0,
  LM_BF16 = 1,
  LM_F16 = 2,
  LM_E4M3 = 3, /* float8_e4m3fn */
  LM_E5M2 = 4, /* float8_e5m2 */
  LM_E2M1 = 5, /* packed fp4, even column in the low nibble */
  LM_E8M0 = 6
};

/* rounding of terminal codes */
enum lm_rounding_mode {
  LM_ROUND_NEAREST = 0,
  LM_ROUND_STOCHASTIC = 1
};

/* MX E8M0 scale calculation (P/_triton_mx_lora.py:23-26) */
enum lm_mx_scaling { LM_MX_FLOOR = 0, LM_MX_RCEIL = 1, LM_MX_CEIL = 2, LM_MX_EVEN = 3 };

/* GGUF quant types (ggml numbering) */
/* GGML quantization type ids (the values of gguf.GGMLQuantizationType) of the
 * types P/gguf_dequant.py:278-294 dispatches */
enum lm_gguf_type {
  LM_GGUF_F32 = 0,
  LM_GGUF_F16 = 1,
  LM_GGUF_Q4_0 = 2,
  LM_GGUF_Q4_1 = 3,
  LM_GGUF_Q5_0 = 6,
  LM_GGUF_Q5_1 = 7,
  LM_GGUF_Q8_0 = 8,
  LM_GGUF_Q2_K = 10,
  LM_GGUF_Q3_K = 11,
  LM_GGUF_Q4_K = 12,
  LM_GGUF_Q5_K = 13,
  LM_GGUF_Q6_K = 14,
  LM_GGUF_IQ4_NL = 20,
  LM_GGUF_IQ4_XS = 23,
  LM_GGUF_BF16 = 30
};

enum lm_status {
  LM_OK = 0,
  LM_EINVAL = 1,       /* bad shape / dtype / pointer: maps to ValueError */
  LM_EUNSUPPORTED = 2, /* valid but not implemented layout: ValueError */
  LM_EWORKSPACE = 3,   /* workspace too small */
  LM_EHIP = 4          /* HIP runtime failure: RuntimeError */
};

/* One LoRA update B@A scaled by `strength` (P/lora.py:595-626 stages B and A
 * on the target device in the compute dtype). */
typedef struct lm_lora {
  const void* b; /* [M, rank], row stride ldb elements */
  const void* a; /* [rank, N], row stride lda elements */
  int64_t ldb;
  int64_t lda;
  int32_t rank;
  int32_t dtype; /* LM_BF16 or LM_F16 (the compute dtype) */
  float strength;
  int32_t reserved;
} lm_lora;

/* Rounding request; `seed` is the uint64 from derive_seed()
 * (P/seeding.py:10-36, P/lora.py:356-359). */
typedef struct lm_rounding {
  int32_t mode; /* lm_rounding_mode */
  int32_t reserved;
  uint64_t seed;
} lm_rounding;

int lm_version(void);
const char* lm_last_error(void);

/* Bytes of workspace any entry point below needs for one tensor of this
 * shape and rank (stack entries: sum over items + lm_stack_workspace_extra). */
size_t lm_workspace_size(int64_t M, int64_t N, int32_t rank);
size_t lm_stack_workspace_extra(int32_t count);

/* ---------------- INT8 (TorchAO Int8Tensor) ---------------------------
 * q: int8 [M, N]; scale: [M*N/group] in scale_dtype (LM_F32/LM_BF16);
 * zero_point: int8 [M*N/group] or NULL (symmetric).  group = N (per-row),
 * M*N (per-tensor) or g < N per-group (TorchAO block_size (1, g): 16, 32 or a
 * multiple of 64 dividing N; qparams [M, N/g] row-major), as the Triton
 * path's _block_numel (P/_triton_int8_lora.py:251-264).  Outputs may alias
 * inputs (in-place merge). */
int lm_int8_merge(const int8_t* q, const void* scale, const int8_t* zero_point, int8_t* q_out, void* scale_out,
                  int8_t* zero_point_out, int64_t M, int64_t N, int64_t group, int32_t scale_dtype, int32_t asymmetric,
                  int32_t reduce_range, const lm_lora* lora, const lm_rounding* rounding, void* workspace,
                  size_t workspace_bytes, void* stream);
/* lm_int8_merge without a workspace argument: NO counterpart in the reference.
 * It is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The call
 * allocates nothing: its scratch is a static device array of
 * LM_NOALLOC_SCRATCH_BYTES that each GPU holds until the process ends.  A
 * shape whose lm_workspace_size(M, N, rank) exceeds that fails with
 * LM_EWORKSPACE before any device work.  All calls on one GPU share its
 * array: calls that overlap on one GPU (several streams or threads) race.
 * Results equal lm_int8_merge's bit for bit. */
#define LM_NOALLOC_SCRATCH_BYTES (8u << 20)
int lm_int8_merge_noalloc(const int8_t* q, const void* scale, const int8_t* zero_point, int8_t* q_out,
                          void* scale_out, int8_t* zero_point_out, int64_t M, int64_t N, int64_t group,
                          int32_t scale_dtype, int32_t asymmetric, int32_t reduce_range, const lm_lora* lora,
                          const lm_rounding* rounding, void* stream);
int lm_int8_requant(const void* dense, int32_t dense_dtype, int8_t* q_out, void* scale_out, int8_t* zero_point_out,
                    int64_t M, int64_t N, int64_t group, int32_t scale_dtype, int32_t asymmetric, int32_t reduce_range,
                    const lm_rounding* rounding, void* workspace, size_t workspace_bytes, void* stream);
/* dequantize (lora == NULL) or dequantize + merge without requant. */
int lm_int8_dequant(const int8_t* q, const void* scale, const int8_t* zero_point, int64_t M, int64_t N, int64_t group,
                    int32_t scale_dtype, const lm_lora* lora, void* out, int32_t out_dtype, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---------------- scaled FP8 (TorchAO Float8Tensor) -------------------
 * q: fp8 [M, N] (fp8_dtype LM_E4M3/LM_E5M2); scale: fp32 [M*N/group];
 * group = N (per-row), M*N (per-tensor) or g < N per-group (16, 32 or a
 * multiple of 64 dividing N; P/float8_adapter.py:63-98). */
int lm_fp8_merge(const uint8_t* q, const float* scale, uint8_t* q_out, float* scale_out, int64_t M, int64_t N,
                 int64_t group, int32_t fp8_dtype, const lm_lora* lora, const lm_rounding* rounding, void* workspace,
                 size_t workspace_bytes, void* stream);
int lm_fp8_requant(const void* dense, int32_t dense_dtype, uint8_t* q_out, float* scale_out, int64_t M, int64_t N,
                   int64_t group, int32_t fp8_dtype, const lm_rounding* rounding, void* workspace,
                   size_t workspace_bytes, void* stream);
int lm_fp8_dequant(const uint8_t* q, const float* scale, int64_t M, int64_t N, int64_t group, int32_t fp8_dtype,
                   const lm_lora* lora, void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes,
                   void* stream);

/* ---------------- NVFP4 (TorchAO NVFP4Tensor) -------------------------
 * q: uint8 [M, N/2]; scale: e4m3 [M, N/16] or swizzled
 * [ceil(M/128)*32, ceil(N/64)*16]; per_tensor_scale: fp32[1] or NULL
 * (single-level).  scale_out is fully written (swizzle padding zeroed). */
int lm_nvfp4_merge(const uint8_t* q, const uint8_t* scale, const float* per_tensor_scale, uint8_t* q_out,
                   uint8_t* scale_out, float* per_tensor_scale_out, int64_t M, int64_t N, int32_t swizzled,
                   const lm_lora* lora, const lm_rounding* rounding, void* workspace, size_t workspace_bytes,
                   void* stream);
int lm_nvfp4_requant(const void* dense, int32_t dense_dtype, uint8_t* q_out, uint8_t* scale_out,
                     float* per_tensor_scale_out, int64_t M, int64_t N, int32_t swizzled, const lm_rounding* rounding,
                     void* workspace, size_t workspace_bytes, void* stream);
int lm_nvfp4_dequant(const uint8_t* q, const uint8_t* scale, const float* per_tensor_scale, int64_t M, int64_t N,
                     int32_t swizzled, const lm_lora* lora, void* out, int32_t out_dtype, void* workspace,
                     size_t workspace_bytes, void* stream);

/* ---------------- MX (TorchAO MXTensor: MXFP4 / MXFP8) ----------------
 * In place.  elem_dtype LM_E2M1 (q: uint8 [M, N/2]) or LM_E4M3/LM_E5M2
 * (q: [M, N]); scale: e8m0 [M, N/32] or swizzled [ceil(M/128)*32,
 * ceil(N/128)*16]; scaling = lm_mx_scaling. */
int lm_mx_merge(uint8_t* q, uint8_t* scale, int64_t M, int64_t N, int32_t elem_dtype, int32_t scaling, int32_t swizzled,
                const lm_lora* lora, const lm_rounding* rounding, void* workspace, size_t workspace_bytes,
                void* stream);
int lm_mx_requant(const void* dense, int32_t dense_dtype, uint8_t* q_out, uint8_t* scale_out, int64_t M, int64_t N,
                  int32_t elem_dtype, int32_t scaling, int32_t swizzled, const lm_rounding* rounding, void* workspace,
                  size_t workspace_bytes, void* stream);
int lm_mx_dequant(const uint8_t* q, const uint8_t* scale, int64_t M, int64_t N, int32_t elem_dtype, int32_t swizzled,
                  const lm_lora* lora, void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes,
                  void* stream);

/* ---------------- GGUF Q8_0 ------------------------------------------
 * packed: uint8 [M, N/32*34], blocks [fp16 d][32 x int8]. */
int lm_q8_0_merge(const uint8_t* packed, uint8_t* packed_out, int64_t M, int64_t N, const lm_lora* lora,
                  const lm_rounding* rounding, void* workspace, size_t workspace_bytes, void* stream);
int lm_q8_0_requant(const void* dense, int32_t dense_dtype, uint8_t* packed_out, int64_t M, int64_t N,
                    const lm_rounding* rounding, void* workspace, size_t workspace_bytes, void* stream);
/* GGUF dequantize of `rows` rows of `cols` logical elements of any
 * lm_gguf_type (replaces P/gguf_dequant.py:303-331 `dequantize`; out dtype
 * LM_BF16/LM_F16/LM_F32, the reference's `dtype`, which is also the precision
 * every step rounds to).  `packed` holds rows*cols/block whole blocks back to
 * back (any alignment); `out` is 16-byte aligned.  With `lora` NULL no
 * workspace is used.  A non-NULL `lora` adds strength*B@A to the dequantized
 * values (Q8_0 only; workspace as lm_workspace_size).  An unknown type returns
 * LM_EUNSUPPORTED (the reference raises NotImplementedError). */
int lm_gguf_dequant(const uint8_t* packed, int32_t quant_type, int64_t rows, int64_t cols, const lm_lora* lora,
                    void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------- plain bf16/fp16 weight (addmm_) ---------------------
 * w: [M, N] row stride ldw, dtype = lora->dtype; w += strength * B@A. */
int lm_dense_merge(void* w, int64_t M, int64_t N, int64_t ldw, const lm_lora* lora, void* workspace,
                   size_t workspace_bytes, void* stream);

/* ---------------- routed LoRA residual --------------------------------
 * Replaces _routed_residual (P/lora.py:801-829), the POST-hook contribution
 * of routed mode (P/lora.py:869-930):
 *   out = dt(y + sum_i dt(dt(dt(dt(x A_i^T) s_i) B_i^T) + dt(bias_i s_i)))
 * with every matmul accumulated in fp32 and every step rounded to the
 * output dtype `dtype` (LM_BF16 / LM_F16), in the reference's order (the sum
 * over factors left to right).  x: [T, K]; y, out: [T, N] (out may alias y);
 * a: [rank, K]; b: [N, rank]; bias: [N] or NULL; all row-major in `dtype`,
 * 8-byte aligned, K % 4 == 0, rank 1..64, at most 8 factors and 16 rank
 * chunks of 16 in all.  Workspace: lm_routed_workspace_size bytes, 256-byte
 * aligned; that size is 0 (and `workspace` may be NULL) for T <= 16, which
 * runs as a single launch. */
typedef struct lm_routed_factor {
  const void* a;
  const void* b;
  const void* bias;
  float strength;
  int32_t rank;
} lm_routed_factor;
size_t lm_routed_workspace_size(int64_t T, int64_t K, const lm_routed_factor* factors, int32_t count);
int lm_routed_residual(const void* x, const void* y, void* out, int64_t T, int64_t K, int64_t N, int32_t dtype,
                       const lm_routed_factor* factors, int32_t count, void* workspace, size_t workspace_bytes,
                       void* stream);

/* ---------------- stacks: many targets, one grouped launch ------------
 * `items` is a HOST array of `count` descriptors.  Each target gets its own
 * seed (derive_seed(param_path, merge_index)).  An item's outputs may alias
 * its own inputs (in place); items must not share buffers with each other
 * (the NVFP4 round-to-nearest stack runs one item's quantization while
 * other items are still being read). */
typedef struct lm_stack_item {
  const void* q;        /* packed codes in */
  const void* scale;    /* scales in */
  const void* aux;      /* int8: zero point or NULL; nvfp4: per_tensor_scale or NULL */
  void* q_out;
  void* scale_out;
  void* aux_out;
  int64_t M;
  int64_t N;
  lm_lora lora;
  uint64_t seed;
} lm_stack_item;

/* INT8 per-row symmetric stack (scale_dtype LM_F32/LM_BF16). */
int lm_int8_merge_stack(const lm_stack_item* items, int32_t count, int32_t scale_dtype, int32_t rounding_mode,
                        void* workspace, size_t workspace_bytes, void* stream);
/* NVFP4 stack (two-level when aux != NULL). */
int lm_nvfp4_merge_stack(const lm_stack_item* items, int32_t count, int32_t swizzled, int32_t rounding_mode,
                         void* workspace, size_t workspace_bytes, void* stream);

/* ---------------- instrumentation -------------------------------------
 * No reference counterpart.  When enabled, every entry point brackets its
 * main kernel launches with hipEvents on the caller's stream, keyed by kernel
 * family ("rows", "rows_stack", "blocks_full", "blocks_amax",
 * "blocks_quant", "todense", "prep", "nvfp4", "mx", "q8", "gguf").  lm_timer_read synchronizes the
 * recorded events and returns the summed milliseconds and launch count of one
 * family.  Enabling (or re-enabling) clears the record. */
int lm_timer_enable(int32_t enable);
int lm_timer_read(const char* family, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif
#endif /* PIPER_LORA_MERGE_H */
