"""CPU oracle for the LoRA-merge hot path -- TEST INFRASTRUCTURE ONLY.

This package is the checker for the HIP kernels.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product package never does.

It wraps ``liblm_oracle.so`` (built from ``lm_oracle.c`` by ``Makefile``),
a C restatement of the reference's fused-merge arithmetic, and adds
``derive_seed`` (P/seeding.py:10-36) in Python.  Arrays are numpy:
bf16/fp16 values travel as their uint16 bit patterns, 8-bit formats as
uint8 codes.

Citation shorthand: P/ = /root/reference/src/piper_offload/.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from hashlib import blake2s

import numpy as np

__all__ = [
    "DT_F32", "DT_BF16", "DT_F16", "DT_E4M3", "DT_E5M2", "DT_E2M1", "DT_E8M0",
    "SR_OFF", "SR_PHILOX8", "SR_TRITON",
    "MX_FLOOR", "MX_RCEIL", "MX_CEIL", "MX_EVEN",
    "derive_seed", "lib", "load",
]

DT_F32, DT_BF16, DT_F16, DT_E4M3, DT_E5M2, DT_E2M1, DT_E8M0 = 0, 1, 2, 3, 4, 5, 6
SR_OFF, SR_PHILOX8, SR_TRITON = 0, 1, 2
MX_FLOOR, MX_RCEIL, MX_CEIL, MX_EVEN = 0, 1, 2, 3

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblm_oracle.so")
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_U64 = ctypes.c_uint64
_F = ctypes.c_float

_SIGS = {
    "lmo_philox4x32": (None, [_P, ctypes.c_uint32, ctypes.c_uint32, _I, _P]),
    "lmo_sr_rounds": (_I, []),
    "lmo_uniforms": (None, [_I, _U64, _U64, _I64, _P]),
    "lmo_merge_dense": (None, [_P, _P, _I, _I64, _I64, _P, _I64, _P, _I64, _I, _I, _F, _I]),
    "lmo_routed_residual": (None, [_P, _P, _P, _I64, _I64, _I64, _I, _I, _P, _P, _P, _P, _P]),
    "lmo_int8_dequant": (None, [_P, _P, _I, _P, _I64, _I64, _I64, _I, _P]),
    "lmo_int8_requant": (None, [_P, _I, _I64, _I64, _I64, _I, _I, _I, _I, _U64, _P, _P, _P]),
    "lmo_fp8_dequant": (None, [_P, _I, _P, _I64, _I64, _I64, _I, _P]),
    "lmo_fp8_requant": (None, [_P, _I, _I64, _I64, _I64, _I, _I, _U64, _P, _P]),
    "lmo_blocked_scale_offset": (_I64, [_I64, _I64, _I64, _I]),
    "lmo_nvfp4_dequant": (None, [_P, _P, _P, _I64, _I64, _I, _I, _P]),
    "lmo_nvfp4_requant": (None, [_P, _I, _I64, _I64, _I, _I, _I, _U64, _P, _P, _P]),
    "lmo_mx_dequant": (None, [_P, _P, _I, _I64, _I64, _I, _I, _P]),
    "lmo_mx_requant": (None, [_P, _I, _I64, _I64, _I, _I, _I, _I, _U64, _P, _P]),
    "lmo_q8_0_dequant": (None, [_P, _I64, _I64, _I, _P]),
    "lmo_q8_0_requant": (None, [_P, _I, _I64, _I64, _I, _U64, _P]),
    "lmo_gguf_sizes": (_I, [_I, _P, _P]),
    "lmo_gguf_dequant": (_I, [_P, _I, _I64, _I, _P]),
    "lmo_f32_to_bf16": (None, [_P, _P, _I64]),
    "lmo_f32_to_f16": (None, [_P, _P, _I64]),
    "lmo_f16_to_f32": (None, [_P, _P, _I64]),
    "lmo_f32_to_fp8": (None, [_I, _P, _P, _I64]),
    "lmo_fp8_to_f32": (None, [_I, _P, _P, _I64]),
    "lmo_f32_to_e2m1": (None, [_P, _P, _I64]),
    "lmo_e8m0_to_f32": (None, [_P, _P, _I64]),
    "lmo_mx_scale": (None, [_P, _I64, _I, _I, _P, _P]),
    "lmo_sr_int": (None, [_P, _P, _P, _I64, _I, _I, _P]),
    "lmo_sr_int13": (None, [_P, _P, _P, _P, _I64, _I, _I, _P]),
    "lmo_sr_h16": (None, [ctypes.c_uint64, ctypes.c_uint64, _I64, _P]),
    "lmo_sr_e2m1": (None, [_P, _P, _P, _I64, _P]),
    "lmo_sr_fp8": (None, [_I, _P, _P, _I64, _F, _P]),
    "lmo_version": (_I, []),
}


def build() -> str:
    """Compile the oracle with ``make`` (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib_ = ctypes.CDLL(_LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib_, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib_
    return _lib


def lib() -> ctypes.CDLL:
    return load()


def _p(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ---------------------------------------------------------------------------
# derive_seed (P/seeding.py:10-36): blake2s-64 over a versioned typed encoding
# ---------------------------------------------------------------------------
def derive_seed(*parts: str | int) -> int:
    h = blake2s(digest_size=8)
    h.update(b"piper-offload-seed-v1\0")
    for part in parts:
        if isinstance(part, str):
            enc = part.encode("utf-8")
            h.update(b"s")
            h.update(len(enc).to_bytes(8, "little"))
            h.update(enc)
        elif isinstance(part, int) and not isinstance(part, bool):
            if not 0 <= part < (1 << 64):
                raise ValueError("derive_seed() integer parts must be unsigned 64-bit values")
            h.update(b"i")
            h.update(part.to_bytes(8, "little"))
        else:
            raise TypeError("derive_seed() parts must be strings or unsigned 64-bit integers")
    return int.from_bytes(h.digest(), "little")


# ---------------------------------------------------------------------------
# codecs
# ---------------------------------------------------------------------------
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    load().lmo_f32_to_bf16(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    load().lmo_f32_to_f16(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    load().lmo_f16_to_f32(_p(h), _p(out), h.size)
    return out


def f32_to_fp8(x: np.ndarray, fmt: int = DT_E4M3) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    load().lmo_f32_to_fp8(fmt, _p(x), _p(out), x.size)
    return out


def fp8_to_f32(c: np.ndarray, fmt: int = DT_E4M3) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.uint8)
    out = np.empty(c.shape, np.float32)
    load().lmo_fp8_to_f32(fmt, _p(c), _p(out), c.size)
    return out


def f32_to_e2m1(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    load().lmo_f32_to_e2m1(_p(x), _p(out), x.size)
    return out


E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                       dtype=np.float32)


def e8m0_to_f32(c: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.uint8)
    out = np.empty(c.shape, np.float32)
    load().lmo_e8m0_to_f32(_p(c), _p(out), c.size)
    return out


def mx_scale(amax: np.ndarray, fmt: int, mode: int) -> tuple[np.ndarray, np.ndarray]:
    amax = np.ascontiguousarray(amax, dtype=np.float32)
    codes = np.empty(amax.shape, np.uint8)
    inv = np.empty(amax.shape, np.float32)
    load().lmo_mx_scale(_p(amax), amax.size, fmt, mode, _p(codes), _p(inv))
    return codes, inv


def philox4x32(ctr: tuple[int, int, int, int], key: tuple[int, int], rounds: int = 10) -> tuple[int, ...]:
    c = np.array(ctr, dtype=np.uint32)
    out = np.empty(4, np.uint32)
    load().lmo_philox4x32(_p(c), key[0], key[1], rounds, _p(out))
    return tuple(int(v) for v in out)


def sr_rounds() -> int:
    """Philox rounds of the SR_PHILOX8 stream (the HIP kernels' SR_ROUNDS)."""
    return int(load().lmo_sr_rounds())


def uniforms(seed: int, start: int, n: int, mode: int = SR_PHILOX8) -> np.ndarray:
    out = np.empty(n, np.float32)
    load().lmo_uniforms(mode, seed, start, n, _p(out))
    return out


def sr_int(x, det, u, qmin, qmax):
    x = np.ascontiguousarray(x, np.float32)
    det = np.ascontiguousarray(det, np.int32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty(x.shape, np.int32)
    load().lmo_sr_int(_p(x), _p(det), _p(u), x.size, qmin, qmax, _p(out))
    return out


def sr_int13(v, rcp, zp, h, qmin, qmax):
    """Integer stochastic rounding of v / s + zp on the 13-bit grid (rcp = RN(1 / s), h = 16-bit draws)."""
    v = np.ascontiguousarray(v, np.float32)
    rcp = np.ascontiguousarray(np.broadcast_to(np.asarray(rcp, np.float32), v.shape))
    zp = np.ascontiguousarray(np.broadcast_to(np.asarray(zp, np.float32), v.shape))
    h = np.ascontiguousarray(np.broadcast_to(np.asarray(h, np.uint32), v.shape))
    out = np.empty(v.shape, np.int32)
    load().lmo_sr_int13(_p(v), _p(rcp), _p(zp), _p(h), v.size, qmin, qmax, _p(out))
    return out


def sr_h16(seed: int, start: int, n: int) -> np.ndarray:
    """The 16-bit Philox draws of offsets start .. start + n - 1 (uniform = h * 2^-16)."""
    out = np.empty(n, np.uint32)
    load().lmo_sr_h16(seed, start, n, _p(out))
    return out


def sr_e2m1(x, det, u):
    x = np.ascontiguousarray(x, np.float32)
    det = np.ascontiguousarray(det, np.uint8)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty(x.shape, np.uint8)
    load().lmo_sr_e2m1(_p(x), _p(det), _p(u), x.size, _p(out))
    return out


def sr_fp8(x, u, fmt=DT_E4M3, limit=448.0):
    x = np.ascontiguousarray(x, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty(x.shape, np.uint8)
    load().lmo_sr_fp8(fmt, _p(x), _p(u), x.size, limit, _p(out))
    return out


# ---------------------------------------------------------------------------
# merge building blocks (dense arrays are uint16 bf16 bits unless cd=DT_F32)
# ---------------------------------------------------------------------------
def _dense_empty(shape, cd):
    return np.empty(shape, np.float32 if cd == DT_F32 else np.uint16)


def merge_dense(base: np.ndarray, b: np.ndarray, a: np.ndarray, strength: float, *, cd: int = DT_BF16,
                fdt: int = DT_BF16, keep_zero_update: bool = False) -> np.ndarray:
    """merged = round_cd(fmaf(B@A (k ascending), strength, base))."""
    base = np.ascontiguousarray(base)
    b = np.ascontiguousarray(b)
    a = np.ascontiguousarray(a)
    M, N = base.shape
    r = a.shape[0] if a is not None else 0
    out = _dense_empty((M, N), cd)
    load().lmo_merge_dense(_p(base), _p(out), cd, M, N, _p(b), b.shape[1] if b.ndim == 2 else 0, _p(a), N, fdt, r,
                           float(strength), int(keep_zero_update))
    return out


def routed_residual(x, y, factors, *, dt=DT_BF16):
    """out = dt(y + sum_i part_i), factors = [(a [r, K], b [N, r], bias [N] or None, strength)], all arrays of dt
    bit patterns (uint16); the reference's _routed_residual (P/lora.py:801-829) with fp32 matmul sums."""
    x = np.ascontiguousarray(x)
    y = np.ascontiguousarray(y)
    T, K = x.shape
    N = y.shape[1]
    nf = len(factors)
    keep = [(np.ascontiguousarray(a), np.ascontiguousarray(b), None if bias is None else np.ascontiguousarray(bias))
            for a, b, bias, _s in factors]
    ptr = ctypes.c_void_p * nf
    a_p = ptr(*[_p(a) for a, _b, _c in keep])
    b_p = ptr(*[_p(b) for _a, b, _c in keep])
    c_p = ptr(*[_p(c) for _a, _b, c in keep])
    s_arr = (ctypes.c_float * nf)(*[float(f[3]) for f in factors])
    r_arr = (ctypes.c_int32 * nf)(*[int(a.shape[0]) for a, _b, _c in keep])
    out = np.empty_like(y)
    load().lmo_routed_residual(_p(x), _p(y), _p(out), T, K, N, dt, nf, a_p, b_p, c_p, s_arr, r_arr)
    return out


def int8_dequant(q, scale, zp, group, *, scale_dt=DT_F32, cd=DT_BF16):
    q = np.ascontiguousarray(q, np.int8)
    M, N = q.shape
    scale = np.ascontiguousarray(scale)
    zp = None if zp is None else np.ascontiguousarray(zp, np.int8)
    out = _dense_empty((M, N), cd)
    load().lmo_int8_dequant(_p(q), _p(scale), scale_dt, _p(zp), M, N, group, cd, _p(out))
    return out


def int8_requant(dense, group, *, cd=DT_BF16, scale_dt=DT_F32, asymmetric=False, reduce_range=False,
                 sr_mode=SR_OFF, seed=0):
    dense = np.ascontiguousarray(dense)
    M, N = dense.shape
    nq = M * N // group
    q = np.empty((M, N), np.int8)
    scale = np.empty(nq, np.float32 if scale_dt == DT_F32 else np.uint16)
    zp = np.empty(nq, np.int8)
    load().lmo_int8_requant(_p(dense), cd, M, N, group, scale_dt, int(asymmetric), int(reduce_range), sr_mode,
                            seed, _p(q), _p(scale), _p(zp))
    return q, scale, zp


def fp8_dequant(q, scale, group, *, fmt=DT_E4M3, cd=DT_BF16):
    q = np.ascontiguousarray(q, np.uint8)
    M, N = q.shape
    scale = np.ascontiguousarray(scale, np.float32)
    out = _dense_empty((M, N), cd)
    load().lmo_fp8_dequant(_p(q), fmt, _p(scale), M, N, group, cd, _p(out))
    return out


def fp8_requant(dense, group, *, fmt=DT_E4M3, cd=DT_BF16, sr_mode=SR_OFF, seed=0):
    dense = np.ascontiguousarray(dense)
    M, N = dense.shape
    q = np.empty((M, N), np.uint8)
    scale = np.empty(M * N // group, np.float32)
    load().lmo_fp8_requant(_p(dense), cd, M, N, group, fmt, sr_mode, seed, _p(q), _p(scale))
    return q, scale


def blocked_scale_shape(M: int, N: int, block: int, swizzled: bool) -> tuple[int, int]:
    if not swizzled:
        return M, N // block
    return (M + 127) // 128 * 32, (N // block + 3) // 4 * 16


def blocked_scale_offset(row, scale_col, scale_cols, swizzled) -> int:
    return int(load().lmo_blocked_scale_offset(row, scale_col, scale_cols, int(swizzled)))


def nvfp4_dequant(q, scale, pts, *, swizzled=False, cd=DT_BF16):
    q = np.ascontiguousarray(q, np.uint8)
    M, half = q.shape
    N = half * 2
    scale = np.ascontiguousarray(scale, np.uint8)
    pts_arr = None if pts is None else np.ascontiguousarray(np.asarray(pts, np.float32).reshape(1))
    out = _dense_empty((M, N), cd)
    load().lmo_nvfp4_dequant(_p(q), _p(scale), _p(pts_arr), M, N, int(swizzled), cd, _p(out))
    return out


def nvfp4_requant(dense, *, swizzled=False, two_level=True, cd=DT_BF16, sr_mode=SR_OFF, seed=0):
    dense = np.ascontiguousarray(dense)
    M, N = dense.shape
    q = np.empty((M, N // 2), np.uint8)
    scale = np.zeros(blocked_scale_shape(M, N, 16, swizzled), np.uint8)
    pts = np.zeros(1, np.float32)
    load().lmo_nvfp4_requant(_p(dense), cd, M, N, int(swizzled), int(two_level), sr_mode, seed, _p(q), _p(scale),
                             _p(pts))
    return q, scale, (pts if two_level else None)


def mx_dequant(q, scale, fmt, N, *, swizzled=False, cd=DT_BF16):
    q = np.ascontiguousarray(q, np.uint8)
    M = q.shape[0]
    scale = np.ascontiguousarray(scale, np.uint8)
    out = _dense_empty((M, N), cd)
    load().lmo_mx_dequant(_p(q), _p(scale), fmt, M, N, int(swizzled), cd, _p(out))
    return out


def mx_requant(dense, fmt, mode=MX_FLOOR, *, swizzled=False, cd=DT_BF16, sr_mode=SR_OFF, seed=0):
    dense = np.ascontiguousarray(dense)
    M, N = dense.shape
    q = np.empty((M, N // 2) if fmt == DT_E2M1 else (M, N), np.uint8)
    scale = np.zeros(blocked_scale_shape(M, N, 32, swizzled), np.uint8)
    load().lmo_mx_requant(_p(dense), cd, M, N, fmt, mode, int(swizzled), sr_mode, seed, _p(q), _p(scale))
    return q, scale


def q8_0_dequant(packed, N, *, cd=DT_BF16):
    packed = np.ascontiguousarray(packed, np.uint8)
    M = packed.shape[0]
    out = _dense_empty((M, N), cd)
    load().lmo_q8_0_dequant(_p(packed), M, N, cd, _p(out))
    return out


def q8_0_requant(dense, *, cd=DT_BF16, sr_mode=SR_OFF, seed=0):
    dense = np.ascontiguousarray(dense)
    M, N = dense.shape
    packed = np.empty((M, N // 32 * 34), np.uint8)
    load().lmo_q8_0_requant(_p(dense), cd, M, N, sr_mode, seed, _p(packed))
    return packed


def gguf_sizes(quant_type: int) -> tuple[int, int] | None:
    """(block size, bytes per block) of a GGUF type the reference dequantizes."""
    b, t = ctypes.c_int(0), ctypes.c_int(0)
    if not load().lmo_gguf_sizes(int(quant_type), ctypes.byref(b), ctypes.byref(t)):
        return None
    return b.value, t.value


def gguf_dequant(packed, quant_type: int, *, cd=DT_BF16):
    """P/gguf_dequant.py:303-331 over a flat run of whole blocks (uint8 bytes);
    returns the logical values as a 1-D array (bf16/fp16 bit patterns or fp32)."""
    packed = np.ascontiguousarray(packed, np.uint8).reshape(-1)
    sizes = gguf_sizes(quant_type)
    if sizes is None:
        raise NotImplementedError(f"GGUF quant type {quant_type} is not dispatched by the reference")
    bs, ts = sizes
    if packed.size % ts:
        raise ValueError("packed bytes are not a whole number of blocks")
    nblocks = packed.size // ts
    out = _dense_empty((nblocks * bs,), cd)
    load().lmo_gguf_dequant(_p(packed), int(quant_type), nblocks, cd, _p(out))
    return out
