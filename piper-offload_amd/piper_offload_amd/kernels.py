"""Drop-in replacements for piper-offload's fused merge functions.

Each public function keeps the exact signature, argument meaning, return
value and ``ValueError`` behaviour of the reference function it replaces
(P/ = the reference's src/piper_offload/), and calls the HIP kernels through
the C ABI:

* :func:`merge_int8_lora`   <- P/_triton_int8_lora.py:267-407
* :func:`merge_float8_lora` <- P/_triton_float8_lora.py:486-588
* :func:`merge_nvfp4_lora`  <- P/_triton_nvfp4_lora.py:515-595
* :func:`merge_mx_lora_`    <- P/_triton_mx_lora.py:333-425
* :func:`merge_q8_0_lora`   -- GGUF Q8_0 merge (no reference counterpart)
* :func:`merge_dense_lora_` <- RegularAdapter.merge_lora_ (P/tensor_adapters.py:686-696)
* :func:`dequantize_gguf`   <- P/gguf_dequant.py:303-331 (all 15 dispatched types)

The ``*_into`` variants write into caller-provided (possibly aliasing)
outputs; the adapters use them to merge in place without a copy.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib as L

__all__ = [
    "dequantize_float8",
    "GGUF_DEQUANT_TYPES",
    "dequantize_gguf",
    "dequantize_int8",
    "dequantize_mx",
    "dequantize_nvfp4",
    "merge_dense_lora_",
    "merge_float8_lora",
    "merge_float8_lora_into",
    "merge_int8_lora",
    "merge_int8_lora_into",
    "merge_mx_lora_",
    "merge_nvfp4_lora",
    "merge_nvfp4_lora_into",
    "merge_q8_0_lora",
    "requantize_float8",
    "requantize_int8",
    "requantize_mx",
    "requantize_nvfp4",
    "requantize_q8_0",
]

GGML_Q8_0 = 8
_Q8_0_BLOCK, _Q8_0_BYTES = 32, 34
_FACTOR_DTYPES = (torch.bfloat16, torch.float16)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _run(name: str, device: torch.device, ws_bytes: int, *args: object) -> None:
    """Call one C entry point with a fresh workspace on the current stream.

    The workspace comes from torch's caching allocator on the same stream, so
    releasing it after the (asynchronous) launch is stream-ordered.
    """
    handle = L.lib()
    with torch.cuda.device(device):
        ws = L.workspace(ws_bytes, device)
        rc = getattr(handle, name)(*args, L.aligned_ptr(ws), ws_bytes, L.stream_ptr(device))
    L.check(rc)


def _factors(b: torch.Tensor, a: torch.Tensor, rows: int, cols: int, label: str) -> tuple[torch.Tensor, torch.Tensor]:
    if b.ndim != 2 or a.ndim != 2:
        raise ValueError(f"{label} merge expects rank-two tensors.")
    if b.dtype is not a.dtype:
        raise ValueError(f"{label} merge requires matching LoRA factor dtypes.")
    if b.dtype not in _FACTOR_DTYPES:
        raise ValueError(f"{label} HIP merge supports bfloat16 and float16 LoRA factors, got {b.dtype}.")
    rank = a.shape[0]
    if rows == 0 or cols == 0 or rank == 0:
        raise ValueError(f"{label} merge requires non-empty weight and factors.")
    if tuple(b.shape) != (rows, rank) or a.shape[1] != cols:
        raise ValueError(f"LoRA factors do not match the {label} weight shape.")
    if rank > 64:
        raise ValueError(f"{label} HIP merge supports LoRA rank up to 64, got {rank}.")
    return b.contiguous(), a.contiguous()


def _same_device(label: str, *tensors: torch.Tensor | None) -> torch.device:
    first = tensors[0]
    assert first is not None
    if first.device.type != "cuda":
        raise ValueError(f"{label} HIP merge requires GPU tensors.")
    for t in tensors[1:]:
        if t is not None and t.device != first.device:
            raise ValueError(f"{label} HIP merge requires all tensors on one GPU device.")
    return first.device


# ---------------------------------------------------------------------------
# INT8
# ---------------------------------------------------------------------------
def _group_ok(cols: int, group: int) -> bool:
    """Per-group sizes the group kernels take: 16, 32 or a multiple of 64, dividing the columns."""
    return 0 < group < cols and cols % group == 0 and (group in (16, 32) or group % 64 == 0)


def _int8_group(shape: tuple[int, int], block_size: tuple[int, ...]) -> int:
    """Elements per qparam: per-tensor, per-row or per-group (1, g) layouts (P/_triton_int8_lora.py:251-264)."""
    rows, cols = shape
    block_size = tuple(block_size)
    if block_size == (rows, cols):
        return rows * cols
    if block_size == (1, cols):
        return cols
    if len(block_size) == 2 and block_size[0] == 1 and _group_ok(cols, block_size[1]):
        return block_size[1]
    raise ValueError(
        "HIP INT8 merge supports two-dimensional per-tensor, per-row and per-group layouts (group 16, 32 or a "
        f"multiple of 64 dividing the columns), got shape {shape} with block size {block_size}."
    )


def _qparam_shape(shape: tuple[int, int], group: int) -> tuple[int, int]:
    rows, cols = shape
    if group == rows * cols and group != cols:
        return (1, 1)
    return (rows, cols // group)


def merge_int8_lora_into(
    qdata: torch.Tensor, scale: torch.Tensor, zero_point: torch.Tensor | None, block_size: tuple[int, ...],
    b: torch.Tensor, a: torch.Tensor, strength: float, *, asymmetric: bool, reduce_range: bool,
    rounding_seed: int | None, out_qdata: torch.Tensor, out_scale: torch.Tensor, out_zero_point: torch.Tensor | None,
) -> None:
    device = _same_device("INT8", qdata, scale, b, a, zero_point)
    if qdata.dtype is not torch.int8:
        raise ValueError(f"HIP INT8 merge requires int8 weight storage, got {qdata.dtype}.")
    if qdata.ndim != 2:
        raise ValueError("HIP INT8 merge expects rank-two tensors.")
    if scale.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"HIP INT8 merge supports float32 and bfloat16 scales, got {scale.dtype}.")
    rows, cols = qdata.shape
    b, a = _factors(b, a, rows, cols, "INT8")
    group = _int8_group((rows, cols), block_size)
    nq = rows * cols // group
    if scale.numel() != nq:
        raise ValueError("INT8 scale shape does not match the quantization block layout.")
    if zero_point is not None and (zero_point.dtype is not torch.int8 or zero_point.numel() != nq):
        raise ValueError("INT8 zero-point storage does not match the quantization blocks.")
    for t in (qdata, scale, zero_point, out_qdata, out_scale, out_zero_point):
        if t is not None and not t.is_contiguous():
            raise ValueError("HIP INT8 merge requires contiguous storage.")
    lora = L.lora_struct(b, a, strength)
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, a.shape[0])
    _run("lm_int8_merge", device, ws_bytes,
         _ptr(qdata), _ptr(scale), _ptr(zero_point), _ptr(out_qdata), _ptr(out_scale), _ptr(out_zero_point),
         rows, cols, group, L.torch_dtype_id(scale.dtype), int(asymmetric), int(reduce_range),
         ctypes.byref(lora), ctypes.byref(rnd))


def merge_int8_lora(
    qdata: torch.Tensor, scale: torch.Tensor, zero_point: torch.Tensor | None, block_size: tuple[int, int],
    b: torch.Tensor, a: torch.Tensor, strength: float, *, asymmetric: bool, reduce_range: bool,
    rounding_seed: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Return raw affine-INT8 buffers after one LoRA merge (P/_triton_int8_lora.py:267-279)."""
    qdata = qdata.contiguous()
    scale = scale.contiguous()
    zero_point = None if zero_point is None else zero_point.contiguous()
    out_q = torch.empty_like(qdata)
    out_s = torch.empty_like(scale)
    out_z = torch.empty(scale.shape, device=scale.device, dtype=torch.int8)
    merge_int8_lora_into(qdata, scale, zero_point, block_size, b, a, strength, asymmetric=asymmetric,
                         reduce_range=reduce_range, rounding_seed=rounding_seed, out_qdata=out_q, out_scale=out_s,
                         out_zero_point=out_z)
    return out_q, out_s, out_z


def requantize_int8(dense: torch.Tensor, block_size: tuple[int, int], *, scale_dtype: torch.dtype = torch.float32,
                    asymmetric: bool = False, reduce_range: bool = False, rounding_seed: int | None = None
                    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Encode a dense bf16/fp16 tensor with the fused INT8 requant kernel."""
    device = _same_device("INT8", dense)
    dense = dense.contiguous()
    rows, cols = dense.shape
    group = _int8_group((rows, cols), block_size)
    nq = rows * cols // group
    qshape = _qparam_shape((rows, cols), group)
    out_q = torch.empty((rows, cols), device=device, dtype=torch.int8)
    out_s = torch.empty(qshape, device=device, dtype=scale_dtype)
    out_z = torch.empty(qshape, device=device, dtype=torch.int8)
    assert out_s.numel() == nq
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, 0)
    _run("lm_int8_requant", device, ws_bytes, _ptr(dense), L.torch_dtype_id(dense.dtype), _ptr(out_q), _ptr(out_s),
         _ptr(out_z), rows, cols, group, L.torch_dtype_id(scale_dtype), int(asymmetric), int(reduce_range),
         ctypes.byref(rnd))
    return out_q, out_s, out_z


def dequantize_int8(qdata: torch.Tensor, scale: torch.Tensor, zero_point: torch.Tensor | None,
                    block_size: tuple[int, int], *, dtype: torch.dtype = torch.bfloat16,
                    lora: tuple[torch.Tensor, torch.Tensor, float] | None = None) -> torch.Tensor:
    """Dense INT8 dequantize, or dequantize + LoRA merge without requant when ``lora`` is given."""
    device = _same_device("INT8", qdata, scale)
    qdata = qdata.contiguous()
    rows, cols = qdata.shape
    group = _int8_group((rows, cols), block_size)
    out = torch.empty((rows, cols), device=device, dtype=dtype)
    lora_s, rank = None, 0
    if lora is not None:
        b, a = _factors(lora[0], lora[1], rows, cols, "INT8")
        lora_s, rank = L.lora_struct(b, a, lora[2]), a.shape[0]
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, rank)
    _run("lm_int8_dequant", device, ws_bytes, _ptr(qdata), _ptr(scale.contiguous()),
         _ptr(None if zero_point is None else zero_point.contiguous()), rows, cols, group,
         L.torch_dtype_id(scale.dtype), None if lora_s is None else ctypes.byref(lora_s), _ptr(out),
         L.torch_dtype_id(dtype))
    return out


# ---------------------------------------------------------------------------
# scaled FP8
# ---------------------------------------------------------------------------
def _fp8_group(shape: tuple[int, int], block_size: tuple[int, ...], scale: torch.Tensor) -> int:
    """Elements per scale: per-row, per-tensor or per-group (1, g) layouts (P/float8_adapter.py:63-98)."""
    rows, cols = shape
    block_size = tuple(block_size)
    if block_size == (1, cols):
        if tuple(scale.shape) != (rows, 1):
            raise ValueError(f"HIP per-row scaled-FP8 merge expects scale shape {(rows, 1)}, got {tuple(scale.shape)}.")
        return cols
    if block_size == (rows, cols):
        if scale.numel() != 1:
            raise ValueError("HIP per-tensor scaled-FP8 merge expects one scale.")
        return rows * cols
    if len(block_size) == 2 and block_size[0] == 1 and _group_ok(cols, block_size[1]):
        g = block_size[1]
        if tuple(scale.shape) != (rows, cols // g):
            raise ValueError(f"HIP per-group scaled-FP8 merge expects scale shape {(rows, cols // g)}, "
                             f"got {tuple(scale.shape)}.")
        return g
    raise ValueError(
        "HIP scaled-FP8 merge supports per-row, per-tensor and per-group layouts (group 16, 32 or a multiple of 64 "
        f"dividing the columns), got block_size={block_size!r}."
    )


def merge_float8_lora_into(qdata: torch.Tensor, scale: torch.Tensor, block_size: tuple[int, ...], b: torch.Tensor,
                           a: torch.Tensor, strength: float, *, rounding_seed: int | None, out_qdata: torch.Tensor,
                           out_scale: torch.Tensor) -> None:
    device = _same_device("scaled-FP8", qdata, scale, b, a)
    if qdata.dtype not in (torch.float8_e4m3fn, torch.float8_e5m2):
        raise ValueError(f"HIP scaled-FP8 merge supports E4M3FN and E5M2 storage, got {qdata.dtype}.")
    if qdata.ndim != 2:
        raise ValueError("HIP scaled-FP8 merge expects rank-two tensors.")
    if scale.dtype is not torch.float32:
        raise ValueError("HIP scaled-FP8 merge expects float32 scales.")
    rows, cols = qdata.shape
    b, a = _factors(b, a, rows, cols, "scaled-FP8")
    group = _fp8_group((rows, cols), block_size, scale)
    lora = L.lora_struct(b, a, strength)
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, a.shape[0])
    _run("lm_fp8_merge", device, ws_bytes, _ptr(qdata), _ptr(scale), _ptr(out_qdata), _ptr(out_scale), rows, cols,
         group, L.torch_dtype_id(qdata.dtype), ctypes.byref(lora), ctypes.byref(rnd))


def merge_float8_lora(qdata: torch.Tensor, scale: torch.Tensor, block_size: tuple[int, ...], b: torch.Tensor,
                      a: torch.Tensor, strength: float, *, rounding_seed: int | None = None
                      ) -> tuple[torch.Tensor, torch.Tensor]:
    """Return raw scaled-FP8 buffers after one merge (P/_triton_float8_lora.py:486-495)."""
    qdata = qdata.contiguous()
    scale = scale.contiguous()
    out_q = torch.empty_like(qdata)
    out_s = torch.empty_like(scale)
    merge_float8_lora_into(qdata, scale, block_size, b, a, strength, rounding_seed=rounding_seed, out_qdata=out_q,
                           out_scale=out_s)
    return out_q, out_s


def requantize_float8(dense: torch.Tensor, block_size: tuple[int, int], *, fp8_dtype: torch.dtype = torch.float8_e4m3fn,
                      rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    device = _same_device("scaled-FP8", dense)
    dense = dense.contiguous()
    rows, cols = dense.shape
    block_size = tuple(block_size)
    if block_size == (1, cols):
        sshape = (rows, 1)
    elif block_size == (rows, cols):
        sshape = (1, 1)
    elif len(block_size) == 2 and block_size[0] == 1 and block_size[1] > 0 and cols % block_size[1] == 0:
        sshape = (rows, cols // block_size[1])
    else:
        sshape = (1, 1)  # rejected by _fp8_group below
    out_q = torch.empty((rows, cols), device=device, dtype=fp8_dtype)
    out_s = torch.empty(sshape, device=device, dtype=torch.float32)
    group = _fp8_group((rows, cols), block_size, out_s)
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, 0)
    _run("lm_fp8_requant", device, ws_bytes, _ptr(dense), L.torch_dtype_id(dense.dtype), _ptr(out_q), _ptr(out_s),
         rows, cols, group, L.torch_dtype_id(fp8_dtype), ctypes.byref(rnd))
    return out_q, out_s


def dequantize_float8(qdata: torch.Tensor, scale: torch.Tensor, block_size: tuple[int, int], *,
                      dtype: torch.dtype = torch.bfloat16,
                      lora: tuple[torch.Tensor, torch.Tensor, float] | None = None) -> torch.Tensor:
    device = _same_device("scaled-FP8", qdata, scale)
    qdata = qdata.contiguous()
    rows, cols = qdata.shape
    group = _fp8_group((rows, cols), block_size, scale)
    out = torch.empty((rows, cols), device=device, dtype=dtype)
    lora_s, rank = None, 0
    if lora is not None:
        b, a = _factors(lora[0], lora[1], rows, cols, "scaled-FP8")
        lora_s, rank = L.lora_struct(b, a, lora[2]), a.shape[0]
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, rank)
    _run("lm_fp8_dequant", device, ws_bytes, _ptr(qdata), _ptr(scale.contiguous()), rows, cols, group,
         L.torch_dtype_id(qdata.dtype), None if lora_s is None else ctypes.byref(lora_s), _ptr(out),
         L.torch_dtype_id(dtype))
    return out


# ---------------------------------------------------------------------------
# NVFP4
# ---------------------------------------------------------------------------
def _nvfp4_scale_shape(rows: int, cols: int, swizzled: bool) -> tuple[int, int]:
    if swizzled:
        return (rows + 127) // 128 * 32, (cols + 63) // 64 * 16
    return rows, cols // 16


def merge_nvfp4_lora_into(qdata: torch.Tensor, scale: torch.Tensor, per_tensor_scale: torch.Tensor | None,
                          block_size: int, is_swizzled_scales: bool, b: torch.Tensor, a: torch.Tensor, strength: float,
                          *, rounding_seed: int | None, out_qdata: torch.Tensor, out_scale: torch.Tensor,
                          out_per_tensor_scale: torch.Tensor | None) -> None:
    device = _same_device("NVFP4", qdata, scale, b, a, per_tensor_scale)
    if qdata.dtype is not torch.uint8:
        raise ValueError(f"HIP NVFP4 merge expects packed uint8 data, got {qdata.dtype}.")
    if scale.dtype is not torch.float8_e4m3fn:
        raise ValueError("HIP NVFP4 merge expects E4M3FN block scales.")
    if qdata.ndim != 2 or scale.ndim != 2:
        raise ValueError("HIP NVFP4 merge expects rank-two tensors.")
    if not qdata.is_contiguous() or not scale.is_contiguous():
        raise ValueError("HIP NVFP4 merge requires contiguous packed data and scales.")
    if block_size != 16:
        raise ValueError("HIP NVFP4 merge requires block_size=16.")
    rows, packed_cols = qdata.shape
    cols = packed_cols * 2
    if packed_cols % 8 != 0:
        raise ValueError("HIP NVFP4 merge requires columns divisible by 16.")
    b, a = _factors(b, a, rows, cols, "NVFP4")
    if tuple(scale.shape) != _nvfp4_scale_shape(rows, cols, is_swizzled_scales):
        raise ValueError("NVFP4 scale shape does not match its swizzle metadata.")
    if per_tensor_scale is not None and (per_tensor_scale.dtype is not torch.float32 or per_tensor_scale.numel() != 1):
        raise ValueError("HIP NVFP4 merge expects one float32 per-tensor scale.")
    lora = L.lora_struct(b, a, strength)
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, a.shape[0])
    _run("lm_nvfp4_merge", device, ws_bytes, _ptr(qdata), _ptr(scale.view(torch.uint8)), _ptr(per_tensor_scale),
         _ptr(out_qdata), _ptr(out_scale.view(torch.uint8)), _ptr(out_per_tensor_scale), rows, cols,
         int(is_swizzled_scales), ctypes.byref(lora), ctypes.byref(rnd))


def merge_nvfp4_lora(qdata: torch.Tensor, scale: torch.Tensor, per_tensor_scale: torch.Tensor | None, block_size: int,
                     is_swizzled_scales: bool, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                     rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Return packed NVFP4 buffers after one merge (P/_triton_nvfp4_lora.py:515-526)."""
    out_q = torch.empty_like(qdata)
    out_s = torch.zeros_like(scale)
    out_pts = None if per_tensor_scale is None else torch.empty_like(per_tensor_scale)
    merge_nvfp4_lora_into(qdata, scale, per_tensor_scale, block_size, is_swizzled_scales, b, a, strength,
                          rounding_seed=rounding_seed, out_qdata=out_q, out_scale=out_s,
                          out_per_tensor_scale=out_pts)
    return out_q, out_s, out_pts


def requantize_nvfp4(dense: torch.Tensor, *, two_level: bool = True, swizzled: bool = False,
                     rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    device = _same_device("NVFP4", dense)
    dense = dense.contiguous()
    rows, cols = dense.shape
    out_q = torch.empty((rows, cols // 2), device=device, dtype=torch.uint8)
    out_s = torch.zeros(_nvfp4_scale_shape(rows, cols, swizzled), device=device, dtype=torch.float8_e4m3fn)
    out_pts = torch.empty((), device=device, dtype=torch.float32) if two_level else None
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, 0)
    _run("lm_nvfp4_requant", device, ws_bytes, _ptr(dense), L.torch_dtype_id(dense.dtype), _ptr(out_q),
         _ptr(out_s.view(torch.uint8)), _ptr(out_pts), rows, cols, int(swizzled), ctypes.byref(rnd))
    return out_q, out_s, out_pts


def dequantize_nvfp4(qdata: torch.Tensor, scale: torch.Tensor, per_tensor_scale: torch.Tensor | None, *,
                     swizzled: bool = False, dtype: torch.dtype = torch.bfloat16,
                     lora: tuple[torch.Tensor, torch.Tensor, float] | None = None) -> torch.Tensor:
    device = _same_device("NVFP4", qdata, scale)
    rows, cols = qdata.shape[0], qdata.shape[1] * 2
    out = torch.empty((rows, cols), device=device, dtype=dtype)
    lora_s, rank = None, 0
    if lora is not None:
        b, a = _factors(lora[0], lora[1], rows, cols, "NVFP4")
        lora_s, rank = L.lora_struct(b, a, lora[2]), a.shape[0]
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, rank)
    _run("lm_nvfp4_dequant", device, ws_bytes, _ptr(qdata.contiguous()), _ptr(scale.contiguous().view(torch.uint8)),
         _ptr(per_tensor_scale), rows, cols, int(swizzled), None if lora_s is None else ctypes.byref(lora_s),
         _ptr(out), L.torch_dtype_id(dtype))
    return out


# ---------------------------------------------------------------------------
# MX
# ---------------------------------------------------------------------------
_FP4_DTYPE = getattr(torch, "float4_e2m1fn_x2", None)
_E8M0_DTYPE = getattr(torch, "float8_e8m0fnu", None)


def _mx_format(elem_dtype: object) -> int:
    if elem_dtype is torch.float8_e4m3fn:
        return L.LM_E4M3
    if elem_dtype is torch.float8_e5m2:
        return L.LM_E5M2
    if elem_dtype is _FP4_DTYPE and _FP4_DTYPE is not None:
        return L.LM_E2M1
    raise ValueError(f"HIP MX merge does not support element dtype {elem_dtype}.")


def _mx_scale_shape(rows: int, cols: int, swizzled: bool) -> tuple[int, int]:
    if not swizzled:
        return rows, cols // 32
    return (rows + 127) // 128 * 32, (cols + 127) // 128 * 16


def merge_mx_lora_(qdata: torch.Tensor, scale: torch.Tensor, elem_dtype: torch.dtype, block_size: int,
                   orig_dtype: torch.dtype, b: torch.Tensor, a: torch.Tensor, strength: float, *, scaling_mode: int,
                   swizzled: bool, rounding_seed: int | None = None) -> None:
    """Merge one staged update directly into raw MX storage (P/_triton_mx_lora.py:333-346)."""
    device = _same_device("MX", qdata, scale, b, a)
    if qdata.ndim != 2 or scale.ndim != 2 or b.ndim != 2 or a.ndim != 2:
        raise ValueError("HIP MX merge expects rank-two tensors.")
    if block_size != 32:
        raise ValueError("HIP MX merge supports block size 32.")
    if b.dtype is not a.dtype or b.dtype is not orig_dtype:
        raise ValueError("HIP MX merge requires factors in the weight's original dtype.")
    if orig_dtype is not torch.bfloat16:
        raise ValueError(f"HIP MX merge supports bfloat16 weights and factors, got {orig_dtype}.")
    if not qdata.is_contiguous() or not scale.is_contiguous():
        raise ValueError("HIP MX merge requires contiguous MX storage.")
    if scaling_mode not in (0, 1, 2, 3):
        raise ValueError(f"Unsupported MX scaling mode id {scaling_mode}.")
    rows, rank = b.shape
    if a.shape[0] != rank:
        raise ValueError("LoRA factor inner dimensions do not match.")
    cols = a.shape[1]
    if cols % 32 != 0:
        raise ValueError("HIP MX merge requires columns divisible by 32.")
    fmt = _mx_format(elem_dtype)
    expected_q = (rows, cols // 2) if fmt == L.LM_E2M1 else (rows, cols)
    if tuple(qdata.shape) != expected_q:
        raise ValueError("MX qdata shape does not match its element format and LoRA factors.")
    if tuple(scale.shape) != _mx_scale_shape(rows, cols, swizzled):
        raise ValueError("MX scale shape does not match its block layout.")
    if _E8M0_DTYPE is not None and scale.dtype is not _E8M0_DTYPE and scale.dtype is not torch.uint8:
        raise ValueError(f"HIP MX merge expects E8M0 scales, got {scale.dtype}.")
    b, a = _factors(b, a, rows, cols, "MX")
    lora = L.lora_struct(b, a, strength)
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, rank)
    _run("lm_mx_merge", device, ws_bytes, _ptr(qdata), _ptr(scale), rows, cols, fmt, int(scaling_mode),
         int(swizzled), ctypes.byref(lora), ctypes.byref(rnd))


def requantize_mx(dense: torch.Tensor, elem_dtype: torch.dtype, *, scaling_mode: int = 0, swizzled: bool = False,
                  rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    device = _same_device("MX", dense)
    dense = dense.contiguous()
    rows, cols = dense.shape
    fmt = _mx_format(elem_dtype)
    out_q = torch.empty((rows, cols // 2) if fmt == L.LM_E2M1 else (rows, cols), device=device,
                        dtype=torch.uint8 if fmt == L.LM_E2M1 else elem_dtype)
    out_s = torch.zeros(_mx_scale_shape(rows, cols, swizzled), device=device, dtype=torch.uint8)
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, 0)
    _run("lm_mx_requant", device, ws_bytes, _ptr(dense), L.torch_dtype_id(dense.dtype), _ptr(out_q), _ptr(out_s),
         rows, cols, fmt, int(scaling_mode), int(swizzled), ctypes.byref(rnd))
    return out_q, out_s


def dequantize_mx(qdata: torch.Tensor, scale: torch.Tensor, elem_dtype: torch.dtype, cols: int, *,
                  swizzled: bool = False, dtype: torch.dtype = torch.bfloat16,
                  lora: tuple[torch.Tensor, torch.Tensor, float] | None = None) -> torch.Tensor:
    device = _same_device("MX", qdata, scale)
    rows = qdata.shape[0]
    fmt = _mx_format(elem_dtype)
    out = torch.empty((rows, cols), device=device, dtype=dtype)
    lora_s, rank = None, 0
    if lora is not None:
        b, a = _factors(lora[0], lora[1], rows, cols, "MX")
        lora_s, rank = L.lora_struct(b, a, lora[2]), a.shape[0]
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, rank)
    _run("lm_mx_dequant", device, ws_bytes, _ptr(qdata.contiguous()), _ptr(scale.contiguous()), rows, cols, fmt,
         int(swizzled), None if lora_s is None else ctypes.byref(lora_s), _ptr(out), L.torch_dtype_id(dtype))
    return out


# ---------------------------------------------------------------------------
# GGUF Q8_0
# ---------------------------------------------------------------------------
def q8_0_logical_shape(packed_shape: tuple[int, ...]) -> tuple[int, ...]:
    """P/gguf_dequant.py:297-300 for Q8_0: 34 bytes hold 32 elements."""
    return (*packed_shape[:-1], packed_shape[-1] // _Q8_0_BYTES * _Q8_0_BLOCK)


def merge_q8_0_lora(packed: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                    rounding_seed: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Merge into GGUF Q8_0 bytes: dequantize (bf16), add strength*B@A, re-block per ggml."""
    device = _same_device("Q8_0", packed, b, a)
    if packed.dtype is not torch.uint8 or packed.ndim != 2:
        raise ValueError("HIP Q8_0 merge expects rank-two uint8 GGUF bytes.")
    if packed.shape[1] % _Q8_0_BYTES != 0:
        raise ValueError("Q8_0 rows must hold whole 34-byte blocks.")
    packed = packed.contiguous()
    rows, cols = q8_0_logical_shape(tuple(packed.shape))
    b, a = _factors(b, a, rows, cols, "Q8_0")
    out = torch.empty_like(packed) if out is None else out
    lora = L.lora_struct(b, a, strength)
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, a.shape[0])
    _run("lm_q8_0_merge", device, ws_bytes, _ptr(packed), _ptr(out), rows, cols, ctypes.byref(lora),
         ctypes.byref(rnd))
    return out


def requantize_q8_0(dense: torch.Tensor, *, rounding_seed: int | None = None) -> torch.Tensor:
    device = _same_device("Q8_0", dense)
    dense = dense.contiguous()
    rows, cols = dense.shape
    if cols % _Q8_0_BLOCK != 0:
        raise ValueError("Q8_0 requires columns divisible by 32.")
    out = torch.empty((rows, cols // _Q8_0_BLOCK * _Q8_0_BYTES), device=device, dtype=torch.uint8)
    rnd = L.rounding_struct(rounding_seed)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, 0)
    _run("lm_q8_0_requant", device, ws_bytes, _ptr(dense), L.torch_dtype_id(dense.dtype), _ptr(out), rows, cols,
         ctypes.byref(rnd))
    return out


# block elements and bytes of every type P/gguf_dequant.py:278-294 dispatches
# (ggml block structs; keys are gguf.GGMLQuantizationType values)
GGUF_DEQUANT_TYPES: dict[int, tuple[int, int]] = {
    0: (1, 4), 1: (1, 2), 30: (1, 2),                      # F32, F16, BF16
    2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),    # Q4_0, Q4_1, Q5_0, Q5_1
    8: (32, 34), 20: (32, 18),                             # Q8_0, IQ4_NL
    10: (256, 84), 11: (256, 110), 12: (256, 144),         # Q2_K, Q3_K, Q4_K
    13: (256, 176), 14: (256, 210), 23: (256, 136),        # Q5_K, Q6_K, IQ4_XS
}
_GGUF_OUT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def dequantize_gguf(data: torch.Tensor, quant_type: int, *, dtype: torch.dtype = torch.bfloat16,
                    lora: tuple[torch.Tensor, torch.Tensor, float] | None = None) -> torch.Tensor:
    """GGUF dequantize on the GPU (P/gguf_dequant.py:303-331) for every type
    the reference dispatches; ``lora`` (Q8_0 only) adds strength*B@A."""
    sizes = GGUF_DEQUANT_TYPES.get(int(quant_type))
    if sizes is None:
        raise NotImplementedError(f"Unsupported GGUF quant type: {quant_type!r}")
    if dtype not in _GGUF_OUT_DTYPES:
        raise ValueError(f"HIP GGUF dequant computes in bf16, fp16 or fp32, not {dtype}.")
    block, nbytes = sizes
    device = _same_device("GGUF", data)
    if data.ndim == 0:
        raise ValueError("GGUF data must have at least one dimension.")
    shape = (*data.shape[:-1], data.shape[-1] // nbytes * block)  # P/gguf_dequant.py:297-300 on data.shape
    raw = data.view(torch.uint8)
    if raw.shape[-1] % nbytes != 0:
        raise ValueError(f"GGUF rows must hold whole {nbytes}-byte blocks of type {quant_type}.")
    raw = raw.contiguous()
    elements = raw.numel() // nbytes * block
    if math.prod(shape) != elements:
        raise ValueError(f"GGUF bytes of shape {tuple(data.shape)} do not give a tensor of shape {shape}.")
    out = torch.empty(shape, device=device, dtype=dtype)
    if elements == 0:
        return out
    cols = shape[-1]
    rows = elements // cols
    lora_s, rank = None, 0
    if lora is not None:
        if int(quant_type) != GGML_Q8_0:
            raise ValueError("GGUF dequant with LoRA factors supports Q8_0 only.")
        b, a = _factors(lora[0], lora[1], rows, cols, "GGUF")
        lora_s, rank = L.lora_struct(b, a, lora[2]), a.shape[0]
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, rank) if lora is not None else 0
    _run("lm_gguf_dequant", device, ws_bytes, _ptr(raw), int(quant_type), rows, cols,
         None if lora_s is None else ctypes.byref(lora_s), _ptr(out), L.torch_dtype_id(dtype))
    return out


# ---------------------------------------------------------------------------
# plain dense weight
# ---------------------------------------------------------------------------
def merge_dense_lora_(weight: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float) -> None:
    """``weight.addmm_(b, a, alpha=strength)`` for bf16/fp16 weights on the GPU."""
    device = _same_device("dense", weight, b, a)
    if weight.ndim != 2 or weight.stride(1) != 1:
        raise ValueError("HIP dense merge expects a row-major rank-two weight.")
    if weight.dtype is not b.dtype:
        raise ValueError("HIP dense merge requires factors in the weight dtype.")
    rows, cols = weight.shape
    b, a = _factors(b, a, rows, cols, "dense")
    lora = L.lora_struct(b, a, strength)
    ws_bytes = L.load_library().lm_workspace_size(rows, cols, a.shape[0])
    _run("lm_dense_merge", device, ws_bytes, _ptr(weight), rows, cols, weight.stride(0), ctypes.byref(lora))
