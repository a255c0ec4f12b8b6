"""The reference's portable merge paths in torch CPU ops: the CPU baseline.

TEST AND BENCHMARK INFRASTRUCTURE.  Only ``tests/`` and ``bench.py``'s
``cpu_baseline`` leg use this module; the product path never does.

The reference merges a TorchAO INT8 weight without its Triton kernel as
(P/int8_adapter.py:349-411 with the fused path unavailable):

* dequantize to the compute dtype (``Int8Tensor.dequantize``,
  P/_torchao_int8.py:113-116): bf16(q * s);
* ``addmm_(b, a, alpha=strength)`` on the dense weight
  (RegularAdapter.merge_lora_, P/tensor_adapters.py:686-696);
* requantize with fresh per-row scales (``Int8Tensor.from_hp``,
  P/_torchao_int8.py:119-173), whose arithmetic the Triton kernel restates
  (P/_triton_int8_lora.py:123-236): s = bf16(max(bf16(amax / 127.5), 2^-23)),
  q = clamp(rint(v * (1 / s)), -128, 127);
* with a rounding seed, replace only the codes by stochastic rounding of
  v / s with a ``torch.rand`` stream from a CPU generator seeded by it
  (P/_torchao_int8.py:176-213, P/_stochastic_quantization.py:6-60).

TorchAO is not importable here, so its ``from_hp`` is restated from that
recipe.  The stochastic codes use torch's CPU generator (the reference's
portable stream), not the Philox stream of the HIP kernels: only the
deterministic codes are comparable bit for bit with the oracle.

The other formats follow the same three steps, each adapter's
``_torch_merge_*_lora_`` (dequantize, ``addmm_``, requantize, copy back):

* scaled FP8 per row, P/float8_adapter.py:101-120: dequant bf16(fp32(q) * s)
  (P/_triton_float8_lora.py:80-85); requant s = bf16(amax / 448) with a zero
  row floored to 2^-23 (P/_torchao_float8.py:192-223), codes
  e4m3(clamp(v / s, +-448));
* NVFP4, P/nvfp4_adapter.py:119-135: dequant bf16(code * bf16(bf16(e4m3) g));
  requant g = max(amax / 2688, 2^-23), block scale e4m3(clamp(bmax / 6 / g,
  2^-6, 448)), codes e2m1(clamp(v ((1 / g) / s), +-6)) with ties to even
  (P/_triton_nvfp4_lora.py:251-367, P/_torchao_nvfp4.py:106-231);
* MXFP4 (FLOOR scales), P/mx_adapter.py:139-159: dequant
  bf16(bf16(code) * bf16(2^e)); requant e = clamp(exponent(amax) - 2, -127,
  128), codes e2m1(clamp(v * 2^-e, +-6)) (P/_triton_mx_lora.py:115-295,
  P/_torchao_mx.py:149-266);
* GGUF Q8_0: dequant bf16(bf16(d) * q) (P/gguf_dequant.py:57-61), requant by
  ggml's quantize_row_q8_0 (d = amax / 127, q = round half away(x / d); the
  reference has no GGUF requant).

Stochastic codes choose between the two neighbouring representable values
with P(up) = (x - lo) / (hi - lo) and a ``torch.rand`` uniform, as the
reference's portable codebook rounding does (P/_stochastic_quantization.py).
"""

from __future__ import annotations

import torch

EPS = torch.finfo(torch.float32).eps


def int8_dequant(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16(q * s) for per-row fp32 scales [M, 1]."""
    return (q.to(torch.float32) * scale).to(torch.bfloat16)


def int8_requant(dense: torch.Tensor, *, rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric INT8 codes and fp32 scales [M, 1] of a bf16 weight."""
    v = dense.to(torch.float32)
    amax = v.abs().amax(dim=1, keepdim=True)
    scale = (amax / torch.full_like(amax, 127.5)).to(torch.bfloat16).to(torch.float32)
    scale = scale.clamp_min(EPS).to(torch.bfloat16).to(torch.float32)
    q = torch.round(v * (1.0 / scale)).clamp_(-128, 127)
    if rounding_seed is not None:
        y = (v / scale).clamp(-128, 127)
        lower = torch.floor(y)
        p = y - lower
        g = torch.Generator(device="cpu").manual_seed(int(rounding_seed) % (1 << 63))
        u = torch.rand(y.shape, generator=g, dtype=torch.float32)
        interior = (y > -128) & (y < 127) & (p > 0)
        q = torch.where(interior, lower + (u < p).to(torch.float32), q)
    return q.to(torch.int8), scale


def int8_merge(q: torch.Tensor, scale: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
               rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One portable merge: dequantize, addmm_, requantize (codes and scales)."""
    dense = int8_dequant(q, scale)
    dense.addmm_(b, a, alpha=strength)
    return int8_requant(dense, rounding_seed=rounding_seed)


# ---- shared stochastic selection over a sorted magnitude grid -----------------
def _sr_grid(x: torch.Tensor, grid: torch.Tensor, det_mag: torch.Tensor, rounding_seed: int) -> torch.Tensor:
    """Magnitudes of stochastic codes: |x| rounded to one of its two neighbours on ``grid`` (sorted,
    non-negative), P(up) = (|x| - lo) / (hi - lo); values on the grid and beyond its end keep det_mag."""
    mag = x.abs()
    hi_i = torch.searchsorted(grid, mag.contiguous(), right=False).clamp_(1, grid.numel() - 1)
    lo, hi = grid[hi_i - 1], grid[hi_i]
    p = ((mag - lo) / (hi - lo)).clamp_(0, 1)
    g = torch.Generator(device="cpu").manual_seed(int(rounding_seed) % (1 << 63))
    u = torch.rand(x.shape, generator=g, dtype=torch.float32)
    inside = (mag > 0) & (mag < grid[-1]) & (p > 0)
    return torch.where(inside, torch.where(u < p, hi, lo), det_mag)


# ---- scaled FP8 e4m3fn, per row -----------------------------------------------
_FP8_GRID = torch.arange(0, 127, dtype=torch.uint8).view(torch.float8_e4m3fn).float()  # 0 .. 448


def fp8_dequant(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16(fp32(q) * s): ``q`` e4m3fn codes as uint8 [M, N], per-row fp32 scales [M, 1]."""
    return (q.view(torch.float8_e4m3fn).to(torch.float32) * scale).to(torch.bfloat16)


def fp8_requant(dense: torch.Tensor, *, rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    v = dense.to(torch.float32)
    amax = v.abs().amax(dim=1, keepdim=True)
    scale = (amax / torch.full_like(amax, 448.0)).to(torch.bfloat16).to(torch.float32)
    scale = torch.where(scale == 0, torch.full_like(scale, EPS), scale)
    x = (v / scale).clamp_(-448.0, 448.0)
    q = x.to(torch.float8_e4m3fn)
    if rounding_seed is not None:
        mag = _sr_grid(x, _FP8_GRID, q.to(torch.float32).abs(), rounding_seed)
        q = torch.where(x < 0, -mag, mag).to(torch.float8_e4m3fn)
        q = torch.where((x == 0) & torch.signbit(x), torch.full_like(q, -0.0), q)
    return q.view(torch.uint8), scale


def fp8_merge(q: torch.Tensor, scale: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
              rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    dense = fp8_dequant(q, scale)
    dense.addmm_(b, a, alpha=strength)
    return fp8_requant(dense, rounding_seed=rounding_seed)


# ---- E2M1 (NVFP4 and MXFP4 codes) ----------------------------------------------
_E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
# RNE thresholds of P/_triton_nvfp4_lora.py:55-85: a magnitude at or below an even-code midpoint stays
# below it, one at an odd-code midpoint rounds up (ties to even)
_E2M1_MID = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
_E2M1_TIE_UP = torch.tensor([False, True, False, True, False, True, False])


def _e2m1_codes(x: torch.Tensor) -> torch.Tensor:
    """RNE e2m1 codes (sign in bit 3, -0 kept) of values already clamped to +-6."""
    mag = x.abs()
    c = torch.zeros(x.shape, dtype=torch.int64)
    for k in range(7):
        up = mag >= _E2M1_MID[k] if _E2M1_TIE_UP[k] else mag > _E2M1_MID[k]
        c += up.to(torch.int64)
    return c | (torch.signbit(x).to(torch.int64) << 3)


def _e2m1_values(codes: torch.Tensor) -> torch.Tensor:
    v = _E2M1[codes & 7]
    return torch.where((codes & 8) != 0, -v, v)


def _unpack_fp4(q: torch.Tensor) -> torch.Tensor:
    """[M, N/2] packed bytes -> [M, N] codes, the even column in the low nibble."""
    q = q.to(torch.int64)
    return torch.stack([q & 15, q >> 4], dim=-1).reshape(q.shape[0], -1)


def _pack_fp4(codes: torch.Tensor) -> torch.Tensor:
    c = codes.reshape(codes.shape[0], -1, 2)
    return (c[..., 0] | (c[..., 1] << 4)).to(torch.uint8)


def _fp4_codes(nrm: torch.Tensor, rounding_seed: int | None) -> torch.Tensor:
    codes = _e2m1_codes(nrm)
    if rounding_seed is not None:
        mag = _sr_grid(nrm, _E2M1, _E2M1[codes & 7], rounding_seed)
        codes = torch.bucketize(mag, _E2M1) | (codes & 8)
    return codes


# ---- NVFP4 (two-level, plain scales) ------------------------------------------
def nvfp4_dequant(q: torch.Tensor, scale: torch.Tensor, per_tensor_scale: torch.Tensor | None) -> torch.Tensor:
    """bf16(code * bf16(bf16(e4m3) * g)): packed codes [M, N/2], e4m3 block scales as uint8 [M, N/16]."""
    bs = scale.view(torch.float8_e4m3fn).to(torch.float32).to(torch.bfloat16).to(torch.float32)
    if per_tensor_scale is not None:
        bs = (bs * per_tensor_scale.to(torch.float32)).to(torch.bfloat16).to(torch.float32)
    v = _e2m1_values(_unpack_fp4(q))
    return (v * bs.repeat_interleave(16, dim=1)).to(torch.bfloat16)


def nvfp4_requant(dense: torch.Tensor, *, two_level: bool = True,
                  rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    v = dense.to(torch.float32)
    M, N = v.shape
    g = None
    if two_level:
        amax = v.abs().amax().reshape(1)
        g = torch.clamp_min(amax / torch.full_like(amax, 2688.0), EPS)
    blocks = v.reshape(M, N // 16, 16)
    bscale = blocks.abs().amax(dim=-1) / torch.full((M, N // 16), 6.0)
    fs = bscale / g if g is not None else bscale
    sc8 = fs.clamp(2.0 ** -6, 448.0).to(torch.float8_e4m3fn)
    fs = sc8.to(torch.float32)
    if g is not None:
        recip = (1.0 / g) / fs
        nrm = blocks * recip[..., None]
    else:
        nrm = blocks / fs[..., None]
    codes = _fp4_codes(nrm.clamp(-6.0, 6.0).reshape(M, N), rounding_seed)
    return _pack_fp4(codes), sc8.view(torch.uint8), g


def nvfp4_merge(q, scale, per_tensor_scale, b, a, strength, *, rounding_seed=None):  # noqa: ANN001, ANN201
    dense = nvfp4_dequant(q, scale, per_tensor_scale)
    dense.addmm_(b, a, alpha=strength)
    return nvfp4_requant(dense, two_level=per_tensor_scale is not None, rounding_seed=rounding_seed)


# ---- MXFP4, FLOOR scales (the MX default scaling mode) ---------------------------
def mxfp4_dequant(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16(bf16(code) * bf16(2^e)): packed codes [M, N/2], e8m0 scale codes [M, N/32] (0 -> 2^-127)."""
    e = scale.to(torch.int32)
    s = torch.where(e == 0, torch.full(e.shape, 2.0 ** -127), torch.ldexp(torch.ones(e.shape), e - 127))
    s = torch.where(e == 255, torch.full(e.shape, float("nan")), s).to(torch.bfloat16).to(torch.float32)
    v = _e2m1_values(_unpack_fp4(q)).to(torch.bfloat16).to(torch.float32)
    return (v * s.repeat_interleave(32, dim=1)).to(torch.bfloat16)


def mxfp4_requant(dense: torch.Tensor, *, rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    v = dense.to(torch.float32)
    M, N = v.shape
    blocks = v.reshape(M, N // 32, 32)
    amax = blocks.abs().amax(dim=-1)
    ex = ((amax.view(torch.int32) >> 23) & 255) - 127
    unb = (ex - 2).clamp(-127, 128)
    enc = (unb + 127).to(torch.uint8)
    scale = torch.clamp_min(((unb + 127).to(torch.int32) << 23).view(torch.float32), 2.0 ** -126)
    nrm = (blocks * (1.0 / scale)[..., None]).clamp(-6.0, 6.0)
    codes = _fp4_codes(nrm.reshape(M, N), rounding_seed)
    return _pack_fp4(codes), enc


def mxfp4_merge(q, scale, b, a, strength, *, rounding_seed=None):  # noqa: ANN001, ANN201
    dense = mxfp4_dequant(q, scale)
    dense.addmm_(b, a, alpha=strength)
    return mxfp4_requant(dense, rounding_seed=rounding_seed)


# ---- GGUF Q8_0 -------------------------------------------------------------------
def q8_0_dequant(packed: torch.Tensor, N: int) -> torch.Tensor:
    """bf16(bf16(d) * q) of 34-byte blocks [fp16 d][32 x int8]."""
    M = packed.shape[0]
    blk = packed.reshape(M, N // 32, 34)
    d = blk[..., :2].contiguous().view(torch.float16).to(torch.bfloat16).to(torch.float32)
    q = blk[..., 2:].contiguous().view(torch.int8).to(torch.float32)
    return (q * d).to(torch.bfloat16).reshape(M, N)


def q8_0_requant(dense: torch.Tensor, *, rounding_seed: int | None = None) -> torch.Tensor:
    v = dense.to(torch.float32)
    M, N = v.shape
    blocks = v.reshape(M, N // 32, 32)
    d = blocks.abs().amax(dim=-1, keepdim=True) / torch.full((M, N // 32, 1), 127.0)
    inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
    x = blocks * inv
    # round half away from zero, exactly: 0.5 - 2^-25 keeps x + 0.5 from rounding up below a half
    q = torch.trunc(x + torch.copysign(torch.full_like(x, 0.5 - 2.0 ** -25), x))
    if rounding_seed is not None:
        lower = torch.floor(x)
        p = x - lower
        g = torch.Generator(device="cpu").manual_seed(int(rounding_seed) % (1 << 63))
        u = torch.rand(x.shape, generator=g, dtype=torch.float32)
        inside = (x > -127) & (x < 127) & (p > 0)
        q = torch.where(inside, lower + (u < p).to(torch.float32), q)
    out = torch.empty((M, N // 32, 34), dtype=torch.uint8)
    out[..., :2] = d.to(torch.float16).view(torch.uint8).reshape(M, N // 32, 2)
    out[..., 2:] = q.clamp(-127, 127).to(torch.int8).view(torch.uint8)
    return out.reshape(M, N // 32 * 34)


def q8_0_merge(packed, N, b, a, strength, *, rounding_seed=None):  # noqa: ANN001, ANN201
    dense = q8_0_dequant(packed, N)
    dense.addmm_(b, a, alpha=strength)
    return q8_0_requant(dense, rounding_seed=rounding_seed)
