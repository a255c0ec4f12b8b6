"""Packed-weight containers with the raw buffers of TorchAO / GGUF tensors.

TorchAO and gguf are not dependencies of this package.  These wrapper tensor
subclasses carry byte-identical storage under the attribute names the
reference's adapters read (P/_torchao_int8.py:30-41, P/_torchao_float8.py:22-29,
P/_torchao_nvfp4.py:18-28, P/_torchao_mx.py:28-37, P/gguf_adapter.py:61-105),
so a model built from them, or a TorchAO tensor exposing the same attributes,
goes through the same adapters and kernels.  They can be wrapped in
``nn.Parameter(..., requires_grad=False)``; arithmetic on them is not
supported (use the adapter's ``dequantize``).

Logical shape is the dense ``[out, in]`` weight; ``dtype`` is the logical
(compute) dtype.
"""

from __future__ import annotations

from typing import Any

import torch

__all__ = ["Float8Weight", "GGUFWeight", "Int8Weight", "MXWeight", "NVFP4Weight", "PackedWeight"]

_ALIAS_OPS = (torch.ops.aten.detach.default, torch.ops.aten.alias.default)


class PackedWeight(torch.Tensor):
    """Base wrapper: holds named inner tensors plus metadata."""

    TENSOR_ATTRS: tuple[str, ...] = ()
    META_ATTRS: tuple[str, ...] = ()

    @staticmethod
    def __new__(cls, *args: Any, **kwargs: Any) -> PackedWeight:  # noqa: ARG004
        shape, dtype, device = cls._logical(*args, **kwargs)
        return torch.Tensor._make_wrapper_subclass(cls, shape, dtype=dtype, device=device, requires_grad=False)

    @classmethod
    def _logical(cls, *args: Any, **kwargs: Any) -> tuple[tuple[int, ...], torch.dtype, torch.device]:
        raise NotImplementedError

    __torch_function__ = torch._C._disabled_torch_function_impl

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):  # noqa: ANN001, ANN206
        if func in _ALIAS_OPS:
            return args[0]._shallow_copy()
        raise NotImplementedError(
            f"{cls.__name__} does not support {func}; use its tensor adapter (dequantize / merge_lora_)."
        )

    def _fields(self) -> dict[str, Any]:
        return {name: getattr(self, name) for name in self.TENSOR_ATTRS + self.META_ATTRS}

    def _shallow_copy(self) -> PackedWeight:
        return type(self)(**self._fields())

    def inner_tensors(self) -> list[torch.Tensor]:
        return [t for t in (getattr(self, n) for n in self.TENSOR_ATTRS) if t is not None]

    def __repr__(self, *, tensor_contents: object | None = None) -> str:  # noqa: ARG002
        return f"{type(self).__name__}(shape={list(self.shape)}, dtype={self.dtype}, device={self.device})"


class Int8Weight(PackedWeight):
    """TorchAO ``Int8Tensor`` layout: int8 ``qdata``, ``scale`` per block, optional ``zero_point``."""

    TENSOR_ATTRS = ("qdata", "scale", "zero_point", "act_pre_scale")
    META_ATTRS = ("block_size", "dtype_", "reduce_range")

    def __init__(self, qdata: torch.Tensor, scale: torch.Tensor, block_size: tuple[int, ...],
                 dtype_: torch.dtype = torch.bfloat16, zero_point: torch.Tensor | None = None,
                 act_pre_scale: torch.Tensor | None = None, reduce_range: bool = False) -> None:
        self.qdata = qdata
        self.scale = scale
        self.zero_point = zero_point
        self.act_pre_scale = act_pre_scale
        self.block_size = tuple(block_size)
        self.dtype_ = dtype_
        self.reduce_range = bool(reduce_range)

    @classmethod
    def _logical(cls, qdata, scale, block_size, dtype_=torch.bfloat16, *_a, **_kw):  # noqa: ANN001, ANN206, ARG003
        return tuple(qdata.shape), dtype_, qdata.device


class Float8Weight(PackedWeight):
    """TorchAO ``Float8Tensor`` layout: fp8 ``qdata`` + fp32 ``scale``."""

    TENSOR_ATTRS = ("qdata", "scale")
    META_ATTRS = ("block_size", "dtype_")

    def __init__(self, qdata: torch.Tensor, scale: torch.Tensor, block_size: tuple[int, ...],
                 dtype_: torch.dtype = torch.bfloat16) -> None:
        self.qdata = qdata
        self.scale = scale
        self.block_size = tuple(block_size)
        self.dtype_ = dtype_

    @classmethod
    def _logical(cls, qdata, scale, block_size, dtype_=torch.bfloat16, *_a, **_kw):  # noqa: ANN001, ANN206, ARG003
        return tuple(qdata.shape), dtype_, qdata.device


class NVFP4Weight(PackedWeight):
    """TorchAO ``NVFP4Tensor`` layout: packed e2m1 ``qdata`` [M, N/2], e4m3 ``scale``
    per 16 elements (regular or 128x4 swizzled), optional fp32 ``per_tensor_scale``."""

    TENSOR_ATTRS = ("qdata", "scale", "per_tensor_scale")
    META_ATTRS = ("block_size", "orig_dtype", "is_swizzled_scales")

    def __init__(self, qdata: torch.Tensor, scale: torch.Tensor, per_tensor_scale: torch.Tensor | None = None,
                 block_size: int = 16, orig_dtype: torch.dtype = torch.bfloat16,
                 is_swizzled_scales: bool = False) -> None:
        self.qdata = qdata
        self.scale = scale
        self.per_tensor_scale = per_tensor_scale
        self.block_size = int(block_size)
        self.orig_dtype = orig_dtype
        self.is_swizzled_scales = bool(is_swizzled_scales)

    @classmethod
    def _logical(cls, qdata, scale, per_tensor_scale=None, block_size=16, orig_dtype=torch.bfloat16, *_a, **_kw):  # noqa: ANN001, ANN206, ARG003
        return (qdata.shape[0], qdata.shape[1] * 2), orig_dtype, qdata.device


class MXWeight(PackedWeight):
    """TorchAO ``MXTensor`` layout: MXFP4 (packed uint8 [M, N/2]) or MXFP8 ([M, N]) elements
    with e8m0 ``scale`` per 32 elements; ``scaling_mode`` is floor/rceil/ceil/even."""

    TENSOR_ATTRS = ("qdata", "scale")
    META_ATTRS = ("elem_dtype", "block_size", "orig_dtype", "is_swizzled_scales", "scaling_mode")

    def __init__(self, qdata: torch.Tensor, scale: torch.Tensor, elem_dtype: torch.dtype, block_size: int = 32,
                 orig_dtype: torch.dtype = torch.bfloat16, is_swizzled_scales: bool = False,
                 scaling_mode: str = "floor") -> None:
        self.qdata = qdata
        self.scale = scale
        self.elem_dtype = elem_dtype
        self.block_size = int(block_size)
        self.orig_dtype = orig_dtype
        self.is_swizzled_scales = bool(is_swizzled_scales)
        self.scaling_mode = scaling_mode

    @classmethod
    def _logical(cls, qdata, scale, elem_dtype, block_size=32, orig_dtype=torch.bfloat16, *_a, **_kw):  # noqa: ANN001, ANN206, ARG003
        fp4 = getattr(torch, "float4_e2m1fn_x2", None)
        cols = qdata.shape[1] * 2 if elem_dtype is fp4 else qdata.shape[1]
        return (qdata.shape[0], cols), orig_dtype, qdata.device


class GGUFWeight(torch.Tensor):
    """uint8 GGUF bytes carrying ``quant_type`` (P/gguf_adapter.py:61-105)."""

    quant_type: int

    @staticmethod
    def __new__(cls, data: torch.Tensor, *, quant_type: int) -> GGUFWeight:
        t = torch.Tensor._make_subclass(cls, data, False)
        t.quant_type = int(quant_type)
        return t

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):  # noqa: ANN001, ANN206
        result = super().__torch_function__(func, types, args, kwargs or {})
        qt = next((a.quant_type for a in args if isinstance(a, GGUFWeight)), None)
        if qt is not None:
            if isinstance(result, cls):
                result.quant_type = qt
            elif isinstance(result, (list, tuple)):
                for r in result:
                    if isinstance(r, cls):
                        r.quant_type = qt
        return result

    def __repr__(self, *, tensor_contents: object | None = None) -> str:  # noqa: ARG002
        return f"GGUFWeight(quant_type={self.quant_type}, packed_shape={list(self.shape)}, device={self.device})"
