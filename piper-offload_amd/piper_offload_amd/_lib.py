"""ctypes binding of ``libpiper_lora_merge.so`` (the C ABI in include/lora_merge.h).

There is no fallback: when the HIP library is missing or no GPU is present,
:func:`lib` raises, so the product path never silently runs on the CPU.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

__all__ = [
    "LM_F32", "LM_BF16", "LM_F16", "LM_E4M3", "LM_E5M2", "LM_E2M1", "LM_E8M0",
    "LM_ROUND_NEAREST", "LM_ROUND_STOCHASTIC",
    "LoraStruct", "RoundingStruct", "RoutedFactor", "StackItem",
    "check", "lib", "library_path", "torch_dtype_id", "workspace",
]

LM_F32, LM_BF16, LM_F16, LM_E4M3, LM_E5M2, LM_E2M1, LM_E8M0 = 0, 1, 2, 3, 4, 5, 6
LM_ROUND_NEAREST, LM_ROUND_STOCHASTIC = 0, 1
LM_OK, LM_EINVAL, LM_EUNSUPPORTED, LM_EWORKSPACE, LM_EHIP = 0, 1, 2, 3, 4

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_lib", "libpiper_lora_merge.so")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_SZ = ctypes.c_size_t


class LoraStruct(ctypes.Structure):
    """Mirror of ``lm_lora``."""

    _fields_ = [
        ("b", _P), ("a", _P), ("ldb", _I64), ("lda", _I64),
        ("rank", _I32), ("dtype", _I32), ("strength", ctypes.c_float), ("reserved", _I32),
    ]


class RoundingStruct(ctypes.Structure):
    """Mirror of ``lm_rounding``."""

    _fields_ = [("mode", _I32), ("reserved", _I32), ("seed", ctypes.c_uint64)]


class StackItem(ctypes.Structure):
    """Mirror of ``lm_stack_item``."""

    _fields_ = [
        ("q", _P), ("scale", _P), ("aux", _P), ("q_out", _P), ("scale_out", _P), ("aux_out", _P),
        ("M", _I64), ("N", _I64), ("lora", LoraStruct), ("seed", ctypes.c_uint64),
    ]


class RoutedFactor(ctypes.Structure):
    """Mirror of ``lm_routed_factor``."""

    _fields_ = [("a", _P), ("b", _P), ("bias", _P), ("strength", ctypes.c_float), ("rank", _I32)]


_L = ctypes.POINTER(LoraStruct)
_R = ctypes.POINTER(RoundingStruct)

_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "lm_version": (_I32, []),
    "lm_last_error": (ctypes.c_char_p, []),
    "lm_workspace_size": (_SZ, [_I64, _I64, _I32]),
    "lm_stack_workspace_extra": (_SZ, [_I32]),
    "lm_int8_merge": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _L, _R, _P, _SZ, _P]),
    "lm_int8_merge_noalloc": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _L, _R, _P]),
    "lm_int8_requant": (_I32, [_P, _I32, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _R, _P, _SZ, _P]),
    "lm_int8_dequant": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I32, _L, _P, _I32, _P, _SZ, _P]),
    "lm_fp8_merge": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I32, _L, _R, _P, _SZ, _P]),
    "lm_fp8_requant": (_I32, [_P, _I32, _P, _P, _I64, _I64, _I64, _I32, _R, _P, _SZ, _P]),
    "lm_fp8_dequant": (_I32, [_P, _P, _I64, _I64, _I64, _I32, _L, _P, _I32, _P, _SZ, _P]),
    "lm_nvfp4_merge": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _L, _R, _P, _SZ, _P]),
    "lm_nvfp4_requant": (_I32, [_P, _I32, _P, _P, _P, _I64, _I64, _I32, _R, _P, _SZ, _P]),
    "lm_nvfp4_dequant": (_I32, [_P, _P, _P, _I64, _I64, _I32, _L, _P, _I32, _P, _SZ, _P]),
    "lm_mx_merge": (_I32, [_P, _P, _I64, _I64, _I32, _I32, _I32, _L, _R, _P, _SZ, _P]),
    "lm_mx_requant": (_I32, [_P, _I32, _P, _P, _I64, _I64, _I32, _I32, _I32, _R, _P, _SZ, _P]),
    "lm_mx_dequant": (_I32, [_P, _P, _I64, _I64, _I32, _I32, _L, _P, _I32, _P, _SZ, _P]),
    "lm_q8_0_merge": (_I32, [_P, _P, _I64, _I64, _L, _R, _P, _SZ, _P]),
    "lm_q8_0_requant": (_I32, [_P, _I32, _P, _I64, _I64, _R, _P, _SZ, _P]),
    "lm_gguf_dequant": (_I32, [_P, _I32, _I64, _I64, _L, _P, _I32, _P, _SZ, _P]),
    "lm_dense_merge": (_I32, [_P, _I64, _I64, _I64, _L, _P, _SZ, _P]),
    "lm_int8_merge_stack": (_I32, [ctypes.POINTER(StackItem), _I32, _I32, _I32, _P, _SZ, _P]),
    "lm_nvfp4_merge_stack": (_I32, [ctypes.POINTER(StackItem), _I32, _I32, _I32, _P, _SZ, _P]),
    "lm_routed_workspace_size": (_SZ, [_I64, _I64, ctypes.POINTER(RoutedFactor), _I32]),
    "lm_routed_residual": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I32, ctypes.POINTER(RoutedFactor), _I32, _P, _SZ,
                                  _P]),
    "lm_timer_enable": (_I32, [_I32]),
    "lm_timer_read": (_I32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> str:
    return _LIB_PATH


def load_library() -> ctypes.CDLL:
    """Load the shared library and bind every exported signature (no GPU needed)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"piper_offload_amd: HIP library not built ({_LIB_PATH} is missing); "
                    "run __graft_entry__.build() or `make -C piper-offload_amd/csrc`."
                )
            handle = ctypes.CDLL(_LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def lib() -> ctypes.CDLL:
    """Return the bound library for a GPU call; raises without a HIP device."""
    handle = load_library()
    if not torch.cuda.is_available():
        raise RuntimeError("piper_offload_amd: the LoRA-merge kernels need a ROCm GPU (torch.cuda is unavailable)")
    return handle


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def timer_enable(enable: bool = True) -> None:
    """Start (and clear) or stop the library's per-kernel-family HIP event timer."""
    check(load_library().lm_timer_enable(int(enable)))


def timer_read(family: str) -> tuple[float, int]:
    """(summed milliseconds, launches) recorded for one kernel family; synchronizes its events."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int64(0)
    check(load_library().lm_timer_read(family.encode(), ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


def check(rc: int) -> None:
    """Map an lm_status to the reference's exception types."""
    if rc == LM_OK:
        return
    msg = (load_library().lm_last_error() or b"").decode("utf-8", "replace")
    if rc in (LM_EINVAL, LM_EUNSUPPORTED, LM_EWORKSPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)


def torch_dtype_id(dtype: torch.dtype) -> int:
    if dtype is torch.bfloat16:
        return LM_BF16
    if dtype is torch.float16:
        return LM_F16
    if dtype is torch.float32:
        return LM_F32
    if dtype is torch.float8_e4m3fn:
        return LM_E4M3
    if dtype is torch.float8_e5m2:
        return LM_E5M2
    raise ValueError(f"unsupported dtype {dtype}")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """A 256-byte aligned scratch tensor from torch's caching allocator."""
    return torch.empty(max(int(nbytes), 256) + 256, dtype=torch.uint8, device=device)


def aligned_ptr(ws: torch.Tensor) -> int:
    p = ws.data_ptr()
    return (p + 255) & ~255


def lora_struct(b: torch.Tensor, a: torch.Tensor, strength: float) -> LoraStruct:
    return LoraStruct(
        b.data_ptr(), a.data_ptr(), b.stride(0), a.stride(0), a.shape[0], torch_dtype_id(b.dtype), float(strength), 0
    )


def rounding_struct(rounding_seed: int | None) -> RoundingStruct:
    if rounding_seed is None:
        return RoundingStruct(LM_ROUND_NEAREST, 0, 0)
    if not 0 <= int(rounding_seed) < (1 << 64):
        raise ValueError("rounding_seed must be an unsigned 64-bit integer")
    return RoundingStruct(LM_ROUND_STOCHASTIC, 0, int(rounding_seed))


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
