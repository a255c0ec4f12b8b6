// lm_gguf.hip -- GGUF dequantize for every type the reference dispatches
// (P/gguf_dequant.py:278-294; P/ = the reference's src/piper_offload/).
//
// Layout.  A GGUF tensor is a flat run of fixed-size blocks (the ggml block
// structs; BS logical elements in TS bytes).  A 256-thread workgroup owns
// 2048 consecutive logical elements: NB = 2048 / BS whole blocks, NB * TS
// bytes, which is a multiple of 16 for every type.  It stages those bytes
// into LDS with 16-byte loads (byte loads when the base is not 16-byte
// aligned), then each lane decodes 8 consecutive elements of one block and
// writes them with one 16-byte store (two for fp32).  The work is HBM-bound:
// TS/BS bytes read and 2 (or 4) bytes written per element.
//
// Arithmetic.  The reference evaluates each type as a few torch ops in the
// output dtype: each op computes in fp32 and rounds to that dtype, and fp16
// block scales are first converted to it.  rnd<DT> is that rounding, applied
// after every op in the reference's order; contraction into FMA is off in
// this file so the fp32 output keeps the separate roundings too.
#include "lm_impl.h"

#pragma clang fp contract(off)

namespace {

enum GgType : int {
  GT_F32 = 0, GT_F16 = 1, GT_Q4_0 = 2, GT_Q4_1 = 3, GT_Q5_0 = 6, GT_Q5_1 = 7, GT_Q8_0 = 8, GT_Q2_K = 10,
  GT_Q3_K = 11, GT_Q4_K = 12, GT_Q5_K = 13, GT_Q6_K = 14, GT_IQ4_NL = 20, GT_IQ4_XS = 23, GT_BF16 = 30
};

// (block elements, block bytes, alignment of a block start within a
// 16-byte-aligned chunk) -- the ggml block structs
template <int T> struct Gg;
template <> struct Gg<GT_Q4_0> { static constexpr int BS = 32, TS = 18, AL = 2; };
template <> struct Gg<GT_IQ4_NL> { static constexpr int BS = 32, TS = 18, AL = 2; };
template <> struct Gg<GT_Q4_1> { static constexpr int BS = 32, TS = 20, AL = 4; };
template <> struct Gg<GT_Q5_0> { static constexpr int BS = 32, TS = 22, AL = 2; };
template <> struct Gg<GT_Q5_1> { static constexpr int BS = 32, TS = 24, AL = 8; };
template <> struct Gg<GT_Q8_0> { static constexpr int BS = 32, TS = 34, AL = 2; };
template <> struct Gg<GT_Q2_K> { static constexpr int BS = 256, TS = 84, AL = 4; };
template <> struct Gg<GT_Q3_K> { static constexpr int BS = 256, TS = 110, AL = 2; };
template <> struct Gg<GT_Q4_K> { static constexpr int BS = 256, TS = 144, AL = 16; };
template <> struct Gg<GT_Q5_K> { static constexpr int BS = 256, TS = 176, AL = 16; };
template <> struct Gg<GT_Q6_K> { static constexpr int BS = 256, TS = 210, AL = 2; };
template <> struct Gg<GT_IQ4_XS> { static constexpr int BS = 256, TS = 136, AL = 8; };

constexpr int GG_THREADS = 256;
constexpr int GG_CHUNK = GG_THREADS * 8;  // logical elements per workgroup

// IQ4_NL / IQ4_XS non-linear code book (ggml kvalues_iq4nl)
__constant__ int8_t kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// fp32 -> fp16 RNE -> fp32.  Written as the conversion instruction itself:
// left to the optimizer, fp16(d * q) becomes v_fma_mixlo_f16(d, q, +0), and
// the +0 addend turns a -0 product into +0 where torch's fp16 multiply keeps -0.
DEV float f16r(float x) {
  uint32_t h = __builtin_bit_cast(uint32_t, x);
  asm("v_cvt_f16_f32 %0, %0" : "+v"(h));  // output tied to the input
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int DT>
DEV float rnd(float x) {
  if constexpr (DT == LM_BF16) return bf16r(x);
  else if constexpr (DT == LM_F16) return f16r(x);
  else return x;
}

// LDS reads at a statically known alignment A (bytes)
DEV uint32_t ld16(const uint8_t* p) { return *(const uint16_t*)p; }
DEV float ldf16(const uint8_t* p) { return (float)__builtin_bit_cast(_Float16, (uint16_t)ld16(p)); }
template <int A>
DEV uint32_t ld4(const uint8_t* p) {
  if constexpr (A >= 4) return *(const uint32_t*)p;
  else return ld16(p) | (ld16(p + 2) << 16);
}
// 8 bytes as two words: byte k of the run is (w[k >> 2] >> 8 (k & 3)) & 255
template <int A>
DEV void ld8(const uint8_t* p, uint32_t (&w)[2]) {
  if constexpr (A >= 8) {
    const uint2 v = *(const uint2*)p;
    w[0] = v.x;
    w[1] = v.y;
  } else {
    w[0] = ld4<A>(p);
    w[1] = ld4<A>(p + 4);
  }
}
DEV uint32_t byte_of(const uint32_t (&w)[2], int k) { return (w[k >> 2] >> (8 * (k & 3))) & 255u; }
// 4-bit field of byte k at bit offset sh (0 or 4)
DEV uint32_t nib_of(const uint32_t (&w)[2], int k, uint32_t sh) {
  return __builtin_amdgcn_ubfe(w[k >> 2], 8 * (k & 3) + sh, 4);
}
DEV uint32_t bits_of(const uint32_t (&w)[2], int k, uint32_t sh, uint32_t n) {
  return __builtin_amdgcn_ubfe(w[k >> 2], 8 * (k & 3) + sh, n);
}

// Decode the 8 elements e0 .. e0+7 (e0 % 8 == 0) of the block at b (LDS).
template <int T, int DT>
DEV void decode8(const uint8_t* b, int e0, const int8_t* iq4, float (&v)[8]) {
  constexpr int A = Gg<T>::AL;
  if constexpr (T == GT_Q8_0) {  // P/gguf_dequant.py:57-61
    const float d = rnd<DT>(ldf16(b));
    uint32_t w[2];
    ld8<A>(b + 2 + e0, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = rnd<DT>(d * (float)(int8_t)byte_of(w, i));
  } else if constexpr (T == GT_Q4_0 || T == GT_IQ4_NL || T == GT_Q4_1) {
    // :107-115 / :226-242 / :95-104: element e is nibble (e >= 16) of qs[e & 15]
    constexpr int QS = T == GT_Q4_1 ? 4 : 2;
    const float d = rnd<DT>(ldf16(b));
    uint32_t w[2];
    ld8<A>(b + QS + (e0 & 15), w);
    const uint32_t sh = e0 >= 16 ? 4u : 0u;
    if constexpr (T == GT_Q4_1) {
      const float m = rnd<DT>(ldf16(b + 2));
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = rnd<DT>(rnd<DT>(d * (float)nib_of(w, i, sh)) + m);
    } else if constexpr (T == GT_Q4_0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = rnd<DT>(d * (float)((int)nib_of(w, i, sh) - 8));
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = rnd<DT>(d * (float)iq4[nib_of(w, i, sh)]);
    }
  } else if constexpr (T == GT_Q5_0 || T == GT_Q5_1) {
    // :80-92 / :64-77: bit e of the little-endian qh word is bit 4 of element e
    constexpr bool ONE = T == GT_Q5_1;
    const float d = rnd<DT>(ldf16(b));
    const uint32_t qh = ld4<ONE ? 4 : 2>(b + (ONE ? 4 : 2)) >> e0;
    uint32_t w[2];
    ld8<ONE ? 8 : 2>(b + (ONE ? 8 : 6) + (e0 & 15), w);
    const uint32_t sh = e0 >= 16 ? 4u : 0u;
    if constexpr (ONE) {
      const float m = rnd<DT>(ldf16(b + 2));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t q = nib_of(w, i, sh) | (((qh >> i) & 1u) << 4);
        v[i] = rnd<DT>(rnd<DT>(d * (float)q) + m);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int q = (int)(nib_of(w, i, sh) | (((qh >> i) & 1u) << 4)) - 16;
        v[i] = rnd<DT>(d * (float)q);
      }
    }
  } else if constexpr (T == GT_Q2_K) {
    // :200-211: scales[16] | qs[64] | d | dmin; 2-bit field 2 ((e & 127) >> 5) of qs[32 (e >> 7) + (e & 31)]
    const float d = rnd<DT>(ldf16(b + 80)), dmin = rnd<DT>(ldf16(b + 82));
    const uint32_t sc = b[e0 >> 4];
    const float dl = rnd<DT>(d * (float)(sc & 15u)), ml = rnd<DT>(dmin * (float)(sc >> 4));
    uint32_t w[2];
    ld8<A>(b + 16 + 32 * (e0 >> 7) + (e0 & 31), w);
    const uint32_t sh = 2u * (uint32_t)((e0 & 127) >> 5);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = rnd<DT>(rnd<DT>(dl * (float)bits_of(w, i, sh, 2)) - ml);
  } else if constexpr (T == GT_Q3_K) {
    // :172-197: hmask[32] | qs[64] | scales[12] | d
    const float d = rnd<DT>(ldf16(b + 108));
    const int is = e0 >> 4;
    const uint32_t lo = is < 8 ? (b[96 + is] & 15u) : (uint32_t)(b[96 + is - 8] >> 4);
    const uint32_t hi = (b[96 + 8 + (is & 3)] >> (2 * (is >> 2))) & 3u;
    const float dl = rnd<DT>(d * (float)((int)(lo | (hi << 4)) - 32));
    uint32_t hm[2], qs[2];
    ld8<A>(b + (e0 & 31), hm);
    ld8<A>(b + 32 + 32 * (e0 >> 7) + (e0 & 31), qs);
    const uint32_t sh = 2u * (uint32_t)((e0 & 127) >> 5), hb = (uint32_t)(e0 >> 5);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q = (int)bits_of(qs, i, sh, 2) - (bits_of(hm, i, hb, 1) ? 0 : 4);
      v[i] = rnd<DT>(dl * (float)q);
    }
  } else if constexpr (T == GT_Q4_K || T == GT_Q5_K) {
    // :157-169 / :137-154: d | dmin | scales[12] | (qh[32] |) qs[128]; sub-block j = e >> 5
    constexpr bool FIVE = T == GT_Q5_K;
    const float d = rnd<DT>(ldf16(b)), dmin = rnd<DT>(ldf16(b + 2));
    const int j = e0 >> 5;
    const uint8_t* s = b + 4;
    uint32_t sc, mn;  // :44-49
    if (j < 4) {
      sc = s[j] & 63u;
      mn = s[4 + j] & 63u;
    } else {
      sc = (s[j + 4] & 15u) | ((uint32_t)(s[j - 4] >> 6) << 4);
      mn = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
    const float ds = rnd<DT>(d * (float)sc), dm = rnd<DT>(dmin * (float)mn);
    uint32_t w[2];
    ld8<8>(b + (FIVE ? 48 : 16) + 32 * (j >> 1) + (e0 & 31), w);
    const uint32_t sh = 4u * (uint32_t)(j & 1);
    uint32_t h[2] = {0u, 0u};
    if constexpr (FIVE) ld8<8>(b + 16 + (e0 & 31), h);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t q = nib_of(w, i, sh);
      if constexpr (FIVE) q |= bits_of(h, i, (uint32_t)j, 1) << 4;
      v[i] = rnd<DT>(rnd<DT>(ds * (float)q) - dm);
    }
  } else if constexpr (T == GT_Q6_K) {
    // :118-134: ql[128] | qh[64] | scales[16] (int8) | d
    const float d = rnd<DT>(ldf16(b + 208));
    const int h = e0 >> 7, r = e0 & 127;
    const float ds = rnd<DT>(d * (float)(int8_t)b[192 + (e0 >> 4)]);
    uint32_t ql[2], qh[2];
    ld8<A>(b + 64 * h + (r & 63), ql);
    ld8<A>(b + 128 + 32 * h + (r & 31), qh);
    const uint32_t sl = 4u * (uint32_t)(r >> 6), shh = 2u * (uint32_t)(r >> 5);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q = (int)(nib_of(ql, i, sl) | (bits_of(qh, i, shh, 2) << 4)) - 32;
      v[i] = rnd<DT>(ds * (float)q);
    }
  } else if constexpr (T == GT_IQ4_XS) {
    // :245-274: d | scales_h (u16) | scales_l[4] | qs[128]; sub-block j = e >> 5
    const float d = rnd<DT>(ldf16(b));
    const int j = e0 >> 5, p = e0 & 31;
    const uint32_t lo = (b[4 + (j >> 1)] >> (4 * (j & 1))) & 15u, hi = (ld16(b + 2) >> (2 * j)) & 3u;
    const float dl = rnd<DT>(d * (float)((int)(lo | (hi << 4)) - 32));
    uint32_t w[2];
    ld8<A>(b + 8 + 16 * j + (p & 15), w);
    const uint32_t sh = p >= 16 ? 4u : 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = rnd<DT>(dl * (float)iq4[nib_of(w, i, sh)]);
  }
}

template <int DT>
DEV void store8(void* out, int64_t i0, const float (&v)[8]) {
  if constexpr (DT == LM_F32) {
    float4* o = (float4*)((float*)out + i0);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else if constexpr (DT == LM_BF16) {
    *(uint4*)((uint16_t*)out + i0) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                 pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  } else {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)v[2 * k]);
      const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)v[2 * k + 1]);
      w[k] = lo | (hi << 16);
    }
    *(uint4*)((uint16_t*)out + i0) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// block-quantized types: one workgroup per 2048-element chunk
template <int T, int DT>
__global__ __launch_bounds__(GG_THREADS) void k_gguf_blocks(const uint8_t* __restrict__ src, int64_t nblocks,
                                                           void* __restrict__ out, int aligned) {
  constexpr int BS = Gg<T>::BS, TS = Gg<T>::TS, NB = GG_CHUNK / BS, BYTES = NB * TS;
  static_assert(BYTES % 16 == 0, "chunk must be whole 16-byte words");
  __shared__ __align__(16) uint8_t lds[BYTES];
  __shared__ int8_t iq4[16];
  const int tid = threadIdx.x;
  if constexpr (T == GT_IQ4_NL || T == GT_IQ4_XS) {
    if (tid < 16) iq4[tid] = kIq4Values[tid];
  }
  const int64_t b0 = (int64_t)blockIdx.x * NB;
  const int nb = (int)(nblocks - b0 < NB ? nblocks - b0 : NB);
  const int len = nb * TS;
  const uint8_t* g = src + b0 * TS;
  if (aligned) {
    for (int i = tid * 16; i < len; i += GG_THREADS * 16) {
      if (i + 16 <= len) {
        *(uint4*)(lds + i) = *(const uint4*)(g + i);
      } else {
        for (int k = i; k < len; ++k) lds[k] = g[k];
      }
    }
  } else {
    for (int i = tid; i < len; i += GG_THREADS) lds[i] = g[i];
  }
  __syncthreads();
  const int e = tid * 8, blk = e / BS;
  if (blk >= nb) return;
  float v[8];
  decode8<T, DT>(lds + blk * TS, e % BS, iq4, v);
  store8<DT>(out, b0 * BS + e, v);
}

// F32 / F16 / BF16 (:214-223, then .to(dtype) at :328-330): elementwise
template <int T, int DT>
__global__ __launch_bounds__(GG_THREADS) void k_gguf_plain(const uint8_t* __restrict__ src, int64_t n,
                                                          void* __restrict__ out, int aligned) {
  constexpr int ES = T == GT_F32 ? 4 : 2;
  const int64_t i0 = ((int64_t)blockIdx.x * GG_THREADS + threadIdx.x) * 8;
  if (i0 >= n) return;
  float v[8];
  if (aligned && i0 + 8 <= n) {
    uint32_t w[8];
    const uint4* p = (const uint4*)(src + i0 * ES);
    const uint4 a = p[0];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    if constexpr (ES == 4) {
      const uint4 c = p[1];
      w[4] = c.x; w[5] = c.y; w[6] = c.z; w[7] = c.w;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (T == GT_F32) v[i] = rnd<DT>(u2f(w[i]));
      else {
        const uint32_t h = (w[i >> 1] >> (16 * (i & 1))) & 0xffffu;
        v[i] = rnd<DT>(T == GT_F16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)h) : u2f(h << 16));
      }
    }
    store8<DT>(out, i0, v);
    return;
  }
  // unaligned source or the ragged tail: element at a time from bytes
  for (int i = 0; i < 8 && i0 + i < n; ++i) {
    const uint8_t* p = src + (i0 + i) * ES;
    float x;
    if constexpr (T == GT_F32) x = u2f((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
    else {
      const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
      x = T == GT_F16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)h) : u2f(h << 16);
    }
    x = rnd<DT>(x);
    if constexpr (DT == LM_F32) ((float*)out)[i0 + i] = x;
    else if constexpr (DT == LM_BF16) ((uint16_t*)out)[i0 + i] = (uint16_t)(pack_bf16x2(0.0f, x) >> 16);
    else ((uint16_t*)out)[i0 + i] = __builtin_bit_cast(uint16_t, (_Float16)x);
  }
}

template <int T>
int launch_blocks(const uint8_t* src, int64_t nblocks, void* out, int dt, int aligned, hipStream_t st) {
  const dim3 grid((unsigned)((nblocks + GG_CHUNK / Gg<T>::BS - 1) / (GG_CHUNK / Gg<T>::BS))), block(GG_THREADS);
  if (dt == LM_BF16) hipLaunchKernelGGL((k_gguf_blocks<T, LM_BF16>), grid, block, 0, st, src, nblocks, out, aligned);
  else if (dt == LM_F16) hipLaunchKernelGGL((k_gguf_blocks<T, LM_F16>), grid, block, 0, st, src, nblocks, out, aligned);
  else hipLaunchKernelGGL((k_gguf_blocks<T, LM_F32>), grid, block, 0, st, src, nblocks, out, aligned);
  LAUNCH_CHECK();
  return LM_OK;
}
template <int T>
int launch_plain(const uint8_t* src, int64_t n, void* out, int dt, int aligned, hipStream_t st) {
  const dim3 grid((unsigned)((n + GG_CHUNK - 1) / GG_CHUNK)), block(GG_THREADS);
  if (dt == LM_BF16) hipLaunchKernelGGL((k_gguf_plain<T, LM_BF16>), grid, block, 0, st, src, n, out, aligned);
  else if (dt == LM_F16) hipLaunchKernelGGL((k_gguf_plain<T, LM_F16>), grid, block, 0, st, src, n, out, aligned);
  else hipLaunchKernelGGL((k_gguf_plain<T, LM_F32>), grid, block, 0, st, src, n, out, aligned);
  LAUNCH_CHECK();
  return LM_OK;
}

}  // namespace

// (block elements, block bytes) of a type the reference dispatches; false otherwise
bool gguf_block_sizes(int type, int* bs, int* ts) {
  int b = 0, t = 0;
  switch (type) {
    case GT_F32: b = 1; t = 4; break;
    case GT_F16: case GT_BF16: b = 1; t = 2; break;
#define GGS(T_) case T_: b = Gg<T_>::BS; t = Gg<T_>::TS; break;
    GGS(GT_Q4_0) GGS(GT_Q4_1) GGS(GT_Q5_0) GGS(GT_Q5_1) GGS(GT_Q8_0) GGS(GT_Q2_K) GGS(GT_Q3_K) GGS(GT_Q4_K)
    GGS(GT_Q5_K) GGS(GT_Q6_K) GGS(GT_IQ4_NL) GGS(GT_IQ4_XS)
#undef GGS
    default: return false;
  }
  *bs = b;
  *ts = t;
  return true;
}

// Dequantize `nelem` logical elements (whole blocks) of `type` into `out`
// (16-byte aligned, dtype dt).  Called by lm_gguf_dequant after validation.
int gguf_dequant_run(const uint8_t* src, int type, int64_t nelem, void* out, int dt, hipStream_t st) {
  int bs, ts;
  if (!gguf_block_sizes(type, &bs, &ts)) return fail(LM_EUNSUPPORTED, "unsupported GGUF quant type %d", type);
  const int aligned = ((uintptr_t)src & 15) == 0;
  TimedLaunch timed("gguf", st);
  switch (type) {
    case GT_F32: return launch_plain<GT_F32>(src, nelem, out, dt, aligned, st);
    case GT_F16: return launch_plain<GT_F16>(src, nelem, out, dt, aligned, st);
    case GT_BF16: return launch_plain<GT_BF16>(src, nelem, out, dt, aligned, st);
#define GGL(T_) case T_: return launch_blocks<T_>(src, nelem / bs, out, dt, aligned, st);
    GGL(GT_Q4_0) GGL(GT_Q4_1) GGL(GT_Q5_0) GGL(GT_Q5_1) GGL(GT_Q8_0) GGL(GT_Q2_K) GGL(GT_Q3_K) GGL(GT_Q4_K)
    GGL(GT_Q5_K) GGL(GT_Q6_K) GGL(GT_IQ4_NL) GGL(GT_IQ4_XS)
#undef GGL
  }
  return fail(LM_EUNSUPPORTED, "unsupported GGUF quant type %d", type);
}
