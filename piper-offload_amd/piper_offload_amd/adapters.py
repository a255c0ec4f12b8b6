"""Tensor adapters: the reference's LoRA-merge capability on the HIP kernels.

Each adapter mirrors the reference adapter of the same name (P/ = the
reference's src/piper_offload/) for the merge capability only:

* ``logical_shape`` / ``compute_dtype``           (P/tensor_adapters.py:140-220)
* ``merge_lora_(target, b, a, strength, *, rounding_seed=None)``
                                                  (P/tensor_adapters.py:233-255)
* ``validate_lora_merge``                         (P/tensor_adapters.py:258-278)
* ``dequantize`` / ``requantize(t, like=...)``    (P/tensor_adapters.py:281-318)
* ``copy_into(src, target=...)``                  (P/tensor_adapters.py:345-360)

``merge_lora_`` updates the target's existing storage in place (storage and
wrapper identity are preserved, P/torchao_structured_adapter.py:95-116).  A
layout the HIP kernels do not cover raises ``ValueError`` from
``validate_lora_merge`` -- there is no CPU fallback for GPU weights.
"""

from __future__ import annotations

from typing import Any

import torch

from . import kernels as K
from .formats import Float8Weight, GGUFWeight, Int8Weight, MXWeight, NVFP4Weight

__all__ = [
    "Float8Adapter",
    "GgufAdapter",
    "Int8Adapter",
    "MxAdapter",
    "Nvfp4Adapter",
    "RegularAdapter",
]

_FP4 = getattr(torch, "float4_e2m1fn_x2", None)
_MX_MODES = {"floor": 0, "rceil": 1, "ceil": 2, "even": 3}


def _require(t: Any, attrs: tuple[str, ...], label: str) -> Any:  # noqa: ANN401
    missing = [a for a in attrs if not hasattr(t, a)]
    if missing:
        raise TypeError(f"expected a {label} tensor, got {type(t).__name__} missing {missing}")
    return t


# ---------------------------------------------------------------------------
# plain tensors (P/tensor_adapters.py:578-708)
# ---------------------------------------------------------------------------
class RegularAdapter:
    """Plain ``torch.Tensor`` weights: ``target.addmm_(b, a, alpha=strength)``.

    GPU bf16/fp16 weights use the fused HIP merge (one pass over the weight);
    CPU tensors and other dtypes keep the exact ``addmm_`` of the reference.
    """

    @staticmethod
    def matches(t: torch.Tensor) -> bool:
        return type(t) is torch.Tensor or type(t) is torch.nn.Parameter

    @staticmethod
    def tensor_id(t: torch.Tensor) -> tuple:
        return ("regular", t.device, t.data_ptr(), t.dtype, tuple(t.shape), t.stride(), t.storage_offset())

    @staticmethod
    def compute_dtype(t: torch.Tensor) -> torch.dtype:
        return t.dtype

    @staticmethod
    def logical_shape(t: torch.Tensor) -> tuple[int, ...]:
        return tuple(t.shape)

    @staticmethod
    def merge_lora_(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                    rounding_seed: int | None = None) -> None:
        del rounding_seed
        if (target.device.type == "cuda" and target.dtype in (torch.bfloat16, torch.float16) and target.ndim == 2
                and target.stride(1) == 1 and b.dtype is target.dtype and a.shape[0] <= 64):
            K.merge_dense_lora_(target, b, a, strength)
            return
        target.addmm_(b, a, alpha=strength)


# ---------------------------------------------------------------------------
# INT8 (P/int8_adapter.py)
# ---------------------------------------------------------------------------
class Int8Adapter:
    """TorchAO ``Int8Tensor`` layout (per-row / per-tensor, symmetric or affine)."""

    ATTRS = ("qdata", "scale", "zero_point", "block_size", "reduce_range")

    @staticmethod
    def matches(t: torch.Tensor) -> bool:
        return isinstance(t, Int8Weight)

    @staticmethod
    def tensor_id(t: torch.Tensor) -> tuple:
        return ("int8", t.qdata.device, t.qdata.data_ptr(), t.scale.data_ptr(), tuple(t.qdata.shape))

    @staticmethod
    def compute_dtype(t: torch.Tensor) -> torch.dtype:
        return t.dtype

    @staticmethod
    def logical_shape(t: torch.Tensor) -> tuple[int, ...]:
        return tuple(t.qdata.shape)

    @staticmethod
    def _pre_scale(qt: Any) -> torch.Tensor | None:  # noqa: ANN401
        """``act_pre_scale`` as [1, 1] or [1, in_features], or None (P/int8_adapter.py:59-100).

        TorchAO multiplies the activation by it before the matmul, so a merge
        divides A by it along the input dimension; only layouts whose meaning
        does not depend on the activation's rank are accepted."""
        pre = getattr(qt, "act_pre_scale", None)
        if pre is None:
            return None
        if not pre.dtype.is_floating_point:
            raise ValueError(f"TorchAO INT8 act_pre_scale must be floating-point for LoRA merge, got {pre.dtype}.")
        if pre.device != qt.qdata.device:
            raise ValueError("TorchAO INT8 act_pre_scale must be on the weight device for LoRA merge, got "
                             f"{pre.device} and {qt.qdata.device}.")
        cols = qt.qdata.shape[-1]
        if pre.numel() == 1:
            norm = pre.reshape(1, 1)
        elif pre.ndim >= 1 and pre.shape[-1] == cols and all(s == 1 for s in pre.shape[:-1]):
            norm = pre.reshape(1, cols)
        else:
            raise ValueError("TorchAO INT8 act_pre_scale must be a scalar or one value per input feature with only "
                             f"singleton leading dimensions for LoRA merge; got shape {tuple(pre.shape)} for {cols} "
                             "input features.")
        if not bool(torch.isfinite(norm).all()):
            raise ValueError("TorchAO INT8 act_pre_scale must contain only finite values for LoRA merge.")
        if bool((norm == 0).any()):
            raise ValueError("TorchAO INT8 act_pre_scale must contain only non-zero values for LoRA merge.")
        return norm

    @staticmethod
    def _stored_coordinates(qt: Any, a: torch.Tensor, strength: float) -> tuple[torch.Tensor, float]:  # noqa: ANN401
        """A in stored-weight coordinates: (strength * A) / act_pre_scale, unit strength (P/int8_adapter.py:103-141)."""
        norm = Int8Adapter._pre_scale(qt)
        if norm is None:
            return a, strength
        # strength is folded in before the division, in float64, so that a tiny
        # strength keeps A / p finite when p alone would overflow it
        stored = a.to(torch.float64).mul(strength).div(norm.to(device=a.device, dtype=torch.float64)).to(a.dtype)
        if not bool(torch.isfinite(stored).all()):
            raise ValueError("TorchAO INT8 act_pre_scale produces non-finite stored-coordinate LoRA factors.")
        return stored.contiguous(), 1.0

    @staticmethod
    def validate_lora_merge(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                            rounding_seed: int | None = None) -> None:
        del rounding_seed
        qt = _require(target, Int8Adapter.ATTRS, "INT8")
        Int8Adapter._stored_coordinates(qt, a, strength)
        rows, cols = qt.qdata.shape
        K._int8_group((rows, cols), tuple(qt.block_size))
        if qt.scale.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"HIP INT8 merge supports float32 and bfloat16 scales, got {qt.scale.dtype}.")

    @staticmethod
    def merge_lora_(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                    rounding_seed: int | None = None) -> None:
        qt = _require(target, Int8Adapter.ATTRS, "INT8")
        a, strength = Int8Adapter._stored_coordinates(qt, a, strength)
        zp = qt.zero_point
        # mapping type inferred from the zero point (P/_torchao_int8.py:153-155; host sync as there)
        asymmetric = zp is not None and bool(zp.any())
        K.merge_int8_lora_into(qt.qdata, qt.scale, zp, tuple(qt.block_size), b, a, strength,
                               asymmetric=asymmetric, reduce_range=bool(qt.reduce_range),
                               rounding_seed=rounding_seed, out_qdata=qt.qdata, out_scale=qt.scale,
                               out_zero_point=zp)

    @staticmethod
    def stack_key(target: torch.Tensor) -> tuple | None:
        """Key of the grouped launch (``lm_int8_merge_stack``) that merges ``target`` exactly as
        :meth:`merge_lora_` does, or None: per-row symmetric codes with full range, no
        ``act_pre_scale``, contiguous storage, float32/bfloat16 scales.  Targets with equal keys
        share one launch."""
        qt = _require(target, Int8Adapter.ATTRS, "INT8")
        q, s, zp = qt.qdata, qt.scale, qt.zero_point
        if q.device.type != "cuda" or q.dtype is not torch.int8 or q.ndim != 2 or bool(qt.reduce_range) \
                or getattr(qt, "act_pre_scale", None) is not None or tuple(qt.block_size) != (1, q.shape[1]) \
                or s.dtype not in (torch.float32, torch.bfloat16) or s.numel() != q.shape[0] \
                or not q.is_contiguous() or not s.is_contiguous() or s.device != q.device:
            return None
        if zp is not None and bool(zp.any()):  # mapping type from the zero point, as merge_lora_ infers it
            return None
        return ("int8", q.device, s.dtype)

    @staticmethod
    def stage_lora_factors(target: torch.Tensor, factors: tuple[tuple[float, torch.Tensor, torch.Tensor], ...], *,
                           logical_shape: tuple[int, ...], compute_dtype: torch.dtype
                           ) -> tuple[torch.Tensor, torch.Tensor, float] | None:
        """Transform each logical A before packing when ``act_pre_scale`` is set (P/int8_adapter.py:302-347)."""
        qt = _require(target, Int8Adapter.ATTRS, "INT8")
        norm = Int8Adapter._pre_scale(qt)
        if norm is None:
            return None
        total = sum(a.shape[0] for _s, a, _b in factors)
        dev = qt.qdata.device
        a_packed = torch.empty((total, logical_shape[1]), device=dev, dtype=compute_dtype)
        b_packed = torch.empty((logical_shape[0], total), device=dev, dtype=compute_dtype)
        pre = norm.to(device=dev, dtype=torch.float64)
        off = 0
        for strength, a, b in factors:
            nxt = off + a.shape[0]
            a_packed[off:nxt].copy_(a.to(device=dev, dtype=torch.float64).mul(strength).div(pre))
            b_packed[:, off:nxt].copy_(b, non_blocking=True)
            off = nxt
        return b_packed, a_packed, 1.0

    @staticmethod
    def validate_prepared_lora_merge(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                                     rounding_seed: int | None = None) -> None:
        del b, rounding_seed
        _require(target, Int8Adapter.ATTRS, "INT8")
        if strength != 1.0:
            raise ValueError(f"TorchAO INT8 prepared LoRA merge requires unit strength, got {strength}.")
        if not bool(torch.isfinite(a).all()):
            raise ValueError("TorchAO INT8 prepared stored-coordinate LoRA factors must be finite.")

    @staticmethod
    def merge_prepared_lora_(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                             rounding_seed: int | None = None) -> None:
        qt = _require(target, Int8Adapter.ATTRS, "INT8")
        zp = qt.zero_point
        asymmetric = zp is not None and bool(zp.any())
        K.merge_int8_lora_into(qt.qdata, qt.scale, zp, tuple(qt.block_size), b, a, strength,
                               asymmetric=asymmetric, reduce_range=bool(qt.reduce_range),
                               rounding_seed=rounding_seed, out_qdata=qt.qdata, out_scale=qt.scale,
                               out_zero_point=zp)

    @staticmethod
    def dequantize(t: torch.Tensor) -> torch.Tensor:
        qt = _require(t, Int8Adapter.ATTRS, "INT8")
        return K.dequantize_int8(qt.qdata, qt.scale, qt.zero_point, tuple(qt.block_size), dtype=t.dtype)

    @staticmethod
    def requantize(t: torch.Tensor, *, like: torch.Tensor, rounding_seed: int | None = None) -> Int8Weight:
        qt = _require(like, Int8Adapter.ATTRS, "INT8")
        asym = qt.zero_point is not None and bool(qt.zero_point.any())
        q, s, z = K.requantize_int8(t.to(like.dtype), tuple(qt.block_size), scale_dtype=qt.scale.dtype,
                                    asymmetric=asym, reduce_range=bool(qt.reduce_range), rounding_seed=rounding_seed)
        return Int8Weight(q, s.reshape(qt.scale.shape), tuple(qt.block_size), like.dtype,
                          zero_point=None if qt.zero_point is None else z.reshape(qt.zero_point.shape),
                          act_pre_scale=getattr(qt, "act_pre_scale", None), reduce_range=bool(qt.reduce_range))

    @staticmethod
    def copy_into(src: torch.Tensor, *, target: torch.Tensor) -> None:
        for name in ("qdata", "scale", "zero_point"):
            dst = getattr(target, name)
            if dst is not None:
                dst.copy_(getattr(src, name))


# ---------------------------------------------------------------------------
# scaled FP8 (P/float8_adapter.py)
# ---------------------------------------------------------------------------
class Float8Adapter:
    ATTRS = ("qdata", "scale", "block_size")

    @staticmethod
    def matches(t: torch.Tensor) -> bool:
        return isinstance(t, Float8Weight)

    @staticmethod
    def tensor_id(t: torch.Tensor) -> tuple:
        return ("float8", t.qdata.device, t.qdata.data_ptr(), t.scale.data_ptr(), tuple(t.qdata.shape))

    @staticmethod
    def compute_dtype(t: torch.Tensor) -> torch.dtype:
        return t.dtype

    @staticmethod
    def logical_shape(t: torch.Tensor) -> tuple[int, ...]:
        return tuple(t.qdata.shape)

    @staticmethod
    def validate_lora_merge(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                            rounding_seed: int | None = None) -> None:
        del b, a, strength, rounding_seed
        f8 = _require(target, Float8Adapter.ATTRS, "Float8")
        K._fp8_group(tuple(f8.qdata.shape), tuple(f8.block_size), f8.scale)

    @staticmethod
    def merge_lora_(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                    rounding_seed: int | None = None) -> None:
        f8 = _require(target, Float8Adapter.ATTRS, "Float8")
        K.merge_float8_lora_into(f8.qdata, f8.scale, tuple(f8.block_size), b, a, strength,
                                 rounding_seed=rounding_seed, out_qdata=f8.qdata, out_scale=f8.scale)

    @staticmethod
    def dequantize(t: torch.Tensor) -> torch.Tensor:
        f8 = _require(t, Float8Adapter.ATTRS, "Float8")
        return K.dequantize_float8(f8.qdata, f8.scale, tuple(f8.block_size), dtype=t.dtype)

    @staticmethod
    def requantize(t: torch.Tensor, *, like: torch.Tensor, rounding_seed: int | None = None) -> Float8Weight:
        f8 = _require(like, Float8Adapter.ATTRS, "Float8")
        q, s = K.requantize_float8(t.to(like.dtype), tuple(f8.block_size), fp8_dtype=f8.qdata.dtype,
                                   rounding_seed=rounding_seed)
        return Float8Weight(q, s.reshape(f8.scale.shape), tuple(f8.block_size), like.dtype)

    @staticmethod
    def copy_into(src: torch.Tensor, *, target: torch.Tensor) -> None:
        target.qdata.copy_(src.qdata)
        target.scale.copy_(src.scale)


# ---------------------------------------------------------------------------
# NVFP4 (P/nvfp4_adapter.py)
# ---------------------------------------------------------------------------
class Nvfp4Adapter:
    ATTRS = ("qdata", "scale", "per_tensor_scale", "block_size", "orig_dtype", "is_swizzled_scales")

    @staticmethod
    def matches(t: torch.Tensor) -> bool:
        return isinstance(t, NVFP4Weight)

    @staticmethod
    def tensor_id(t: torch.Tensor) -> tuple:
        return ("nvfp4", t.qdata.device, t.qdata.data_ptr(), t.scale.data_ptr(), tuple(t.qdata.shape))

    @staticmethod
    def compute_dtype(t: torch.Tensor) -> torch.dtype:
        return t.orig_dtype

    @staticmethod
    def logical_shape(t: torch.Tensor) -> tuple[int, ...]:
        return (t.qdata.shape[0], t.qdata.shape[1] * 2)

    @staticmethod
    def validate_lora_merge(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                            rounding_seed: int | None = None) -> None:
        """P/nvfp4_adapter.py:227-252."""
        del b, a, strength, rounding_seed
        nv = _require(target, Nvfp4Adapter.ATTRS, "NVFP4")
        if not nv.qdata.is_contiguous():
            raise ValueError("Cannot merge LoRA into a non-contiguous (e.g. transposed) NVFP4 weight: "
                             "requantization produces the standard packed layout. Use routed LoRA for this weight.")
        if nv.per_tensor_scale is not None and nv.per_tensor_scale.numel() != 1:
            raise ValueError("Cannot merge LoRA into an NVFP4 weight with a non-scalar per_tensor_scale; "
                             "the merge recomputes a single global scale. Use routed LoRA for this weight.")
        if nv.block_size != 16:
            raise ValueError("HIP NVFP4 merge requires block_size=16.")

    @staticmethod
    def stack_key(target: torch.Tensor) -> tuple | None:
        """Key of the grouped launches (``lm_nvfp4_merge_stack``) that merge ``target`` exactly as
        :meth:`merge_lora_` does, or None; targets with equal keys (one scale layout) share them."""
        nv = _require(target, Nvfp4Adapter.ATTRS, "NVFP4")
        q, s, pts = nv.qdata, nv.scale, nv.per_tensor_scale
        if q.device.type != "cuda" or q.dtype is not torch.uint8 or q.ndim != 2 or s.ndim != 2 \
                or s.dtype is not torch.float8_e4m3fn or nv.block_size != 16 or q.shape[1] % 8 != 0 \
                or not q.is_contiguous() or not s.is_contiguous() or s.device != q.device:
            return None
        if tuple(s.shape) != K._nvfp4_scale_shape(q.shape[0], 2 * q.shape[1], bool(nv.is_swizzled_scales)):
            return None
        if pts is not None and (pts.dtype is not torch.float32 or pts.numel() != 1 or pts.device != q.device):
            return None
        return ("nvfp4", q.device, bool(nv.is_swizzled_scales))

    @staticmethod
    def merge_lora_(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                    rounding_seed: int | None = None) -> None:
        nv = _require(target, Nvfp4Adapter.ATTRS, "NVFP4")
        pts = nv.per_tensor_scale
        K.merge_nvfp4_lora_into(nv.qdata, nv.scale, pts, nv.block_size, nv.is_swizzled_scales, b, a, strength,
                                rounding_seed=rounding_seed, out_qdata=nv.qdata, out_scale=nv.scale,
                                out_per_tensor_scale=pts)

    @staticmethod
    def dequantize(t: torch.Tensor) -> torch.Tensor:
        nv = _require(t, Nvfp4Adapter.ATTRS, "NVFP4")
        return K.dequantize_nvfp4(nv.qdata, nv.scale, nv.per_tensor_scale, swizzled=nv.is_swizzled_scales,
                                  dtype=nv.orig_dtype)

    @staticmethod
    def requantize(t: torch.Tensor, *, like: torch.Tensor, rounding_seed: int | None = None) -> NVFP4Weight:
        nv = _require(like, Nvfp4Adapter.ATTRS, "NVFP4")
        q, s, pts = K.requantize_nvfp4(t.to(nv.orig_dtype), two_level=nv.per_tensor_scale is not None,
                                       swizzled=nv.is_swizzled_scales, rounding_seed=rounding_seed)
        if pts is not None:
            pts = pts.reshape(nv.per_tensor_scale.shape)
        return NVFP4Weight(q, s, pts, nv.block_size, nv.orig_dtype, nv.is_swizzled_scales)

    @staticmethod
    def copy_into(src: torch.Tensor, *, target: torch.Tensor) -> None:
        target.qdata.copy_(src.qdata)
        target.scale.copy_(src.scale)
        if target.per_tensor_scale is not None:
            target.per_tensor_scale.copy_(src.per_tensor_scale)


# ---------------------------------------------------------------------------
# MX (P/mx_adapter.py)
# ---------------------------------------------------------------------------
class MxAdapter:
    ATTRS = ("qdata", "scale", "elem_dtype", "block_size", "orig_dtype", "is_swizzled_scales")

    @staticmethod
    def matches(t: torch.Tensor) -> bool:
        return isinstance(t, MXWeight)

    @staticmethod
    def tensor_id(t: torch.Tensor) -> tuple:
        return ("mx", t.qdata.device, t.qdata.data_ptr(), t.scale.data_ptr(), tuple(t.qdata.shape))

    @staticmethod
    def compute_dtype(t: torch.Tensor) -> torch.dtype:
        return t.orig_dtype

    @staticmethod
    def logical_shape(t: torch.Tensor) -> tuple[int, ...]:
        cols = t.qdata.shape[1] * 2 if t.elem_dtype is _FP4 else t.qdata.shape[1]
        return (t.qdata.shape[0], cols)

    @staticmethod
    def _mode(mx: Any) -> int:  # noqa: ANN401
        mode = getattr(mx, "scaling_mode", None)
        mode = getattr(mode, "value", mode)
        if mode is None:
            return 0
        if isinstance(mode, int):
            return mode
        if mode not in _MX_MODES:
            raise ValueError(f"Unsupported MX scaling mode {mode!r}.")
        return _MX_MODES[mode]

    @staticmethod
    def validate_lora_merge(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                            rounding_seed: int | None = None) -> None:
        del b, a, strength, rounding_seed
        mx = _require(target, MxAdapter.ATTRS, "MX")
        if not mx.qdata.is_contiguous():
            raise ValueError("Cannot merge LoRA into a non-contiguous (e.g. transposed) MX weight: requantization "
                             "produces the standard packed layout. Use routed LoRA for this weight.")
        MxAdapter._mode(mx)

    @staticmethod
    def merge_lora_(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                    rounding_seed: int | None = None) -> None:
        mx = _require(target, MxAdapter.ATTRS, "MX")
        K.merge_mx_lora_(mx.qdata, mx.scale.view(torch.uint8), mx.elem_dtype, mx.block_size, mx.orig_dtype, b, a,
                         strength, scaling_mode=MxAdapter._mode(mx), swizzled=mx.is_swizzled_scales,
                         rounding_seed=rounding_seed)

    @staticmethod
    def dequantize(t: torch.Tensor) -> torch.Tensor:
        mx = _require(t, MxAdapter.ATTRS, "MX")
        return K.dequantize_mx(mx.qdata.view(torch.uint8), mx.scale.view(torch.uint8), mx.elem_dtype,
                               MxAdapter.logical_shape(mx)[1], swizzled=mx.is_swizzled_scales, dtype=mx.orig_dtype)

    @staticmethod
    def requantize(t: torch.Tensor, *, like: torch.Tensor, rounding_seed: int | None = None) -> MXWeight:
        mx = _require(like, MxAdapter.ATTRS, "MX")
        q, s = K.requantize_mx(t.to(mx.orig_dtype), mx.elem_dtype, scaling_mode=MxAdapter._mode(mx),
                               swizzled=mx.is_swizzled_scales, rounding_seed=rounding_seed)
        return MXWeight(q, s.view(mx.scale.dtype), mx.elem_dtype, mx.block_size, mx.orig_dtype,
                        mx.is_swizzled_scales, getattr(mx, "scaling_mode", "floor"))

    @staticmethod
    def copy_into(src: torch.Tensor, *, target: torch.Tensor) -> None:
        target.qdata.view(torch.uint8).copy_(src.qdata.view(torch.uint8))
        target.scale.view(torch.uint8).copy_(src.scale.view(torch.uint8))


# ---------------------------------------------------------------------------
# GGUF (P/gguf_adapter.py) -- Q8_0 gains a merge here
# ---------------------------------------------------------------------------
class GgufAdapter:
    @staticmethod
    def matches(t: torch.Tensor) -> bool:
        return isinstance(t, GGUFWeight) and t.dtype == torch.uint8

    @staticmethod
    def tensor_id(t: torch.Tensor) -> tuple:
        raw = t.as_subclass(torch.Tensor)
        return ("gguf", raw.device, raw.untyped_storage().data_ptr(), raw.storage_offset(), tuple(raw.shape),
                raw.stride(), t.quant_type)

    @staticmethod
    def compute_dtype(t: torch.Tensor) -> torch.dtype:  # noqa: ARG004
        return torch.bfloat16

    @staticmethod
    def logical_shape(t: torch.Tensor) -> tuple[int, ...]:
        if t.quant_type != K.GGML_Q8_0:
            raise ValueError(f"GGUF quant type {t.quant_type} has no LoRA merge; use routed LoRA.")
        return K.q8_0_logical_shape(tuple(t.shape))

    @staticmethod
    def validate_lora_merge(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                            rounding_seed: int | None = None) -> None:
        del b, a, strength, rounding_seed
        GgufAdapter.logical_shape(target)
        if target.ndim != 2 or not target.is_contiguous():
            raise ValueError("GGUF Q8_0 merge expects contiguous rank-two packed bytes.")

    @staticmethod
    def merge_lora_(target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                    rounding_seed: int | None = None) -> None:
        GgufAdapter.logical_shape(target)
        raw = target.as_subclass(torch.Tensor)
        K.merge_q8_0_lora(raw, b, a, strength, rounding_seed=rounding_seed, out=raw)

    @staticmethod
    def dequantize(t: torch.Tensor) -> torch.Tensor:
        return K.dequantize_gguf(t.as_subclass(torch.Tensor), t.quant_type, dtype=torch.bfloat16)

    @staticmethod
    def requantize(t: torch.Tensor, *, like: torch.Tensor, rounding_seed: int | None = None) -> GGUFWeight:
        if like.quant_type != K.GGML_Q8_0:
            raise ValueError(f"GGUF quant type {like.quant_type} has no requantizer.")
        return GGUFWeight(K.requantize_q8_0(t.to(torch.bfloat16), rounding_seed=rounding_seed),
                          quant_type=like.quant_type)

    @staticmethod
    def copy_into(src: torch.Tensor, *, target: torch.Tensor) -> None:
        target.as_subclass(torch.Tensor).copy_(src.as_subclass(torch.Tensor))
