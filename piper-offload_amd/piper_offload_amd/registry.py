"""Adapter registration and selection (P/tensor_adapter_registry.py:38-152).

Dispatch order: externally registered adapters newest-first, then the
built-ins; ``RegularAdapter`` is last and matches only plain tensors.
DTensor sharding is outside this single-GPU build, so there is no DTensor
adapter in front of the list.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Any

import torch
from torch import nn

from .adapters import Float8Adapter, GgufAdapter, Int8Adapter, MxAdapter, Nvfp4Adapter, RegularAdapter

__all__ = ["param_representation", "param_tensor_id", "register_adapter", "select_adapter", "tensor_id"]

_BUILTIN_ADAPTERS: tuple[type, ...] = (
    Nvfp4Adapter,
    MxAdapter,
    Float8Adapter,
    Int8Adapter,
    GgufAdapter,
    RegularAdapter,
)
_REGISTERED_ADAPTERS: list[type] = []


def register_adapter(adapter_cls: type) -> Callable[[], None]:
    """Register an external adapter class; returns an idempotent remover."""
    if not isinstance(adapter_cls, type):
        raise TypeError(f"register_adapter() expects an adapter class, got {type(adapter_cls).__name__}")
    if adapter_cls in _BUILTIN_ADAPTERS:
        raise ValueError(f"TensorAdapter {adapter_cls.__name__!r} is already built in")
    if adapter_cls in _REGISTERED_ADAPTERS:
        raise ValueError(f"TensorAdapter {adapter_cls.__name__!r} is already registered")
    for attr in ("matches", "tensor_id", "compute_dtype"):
        if not callable(getattr(adapter_cls, attr, None)):
            raise TypeError(f"Adapter {adapter_cls.__name__!r} does not satisfy the TensorAdapter protocol")
    _REGISTERED_ADAPTERS.insert(0, adapter_cls)
    removed = False

    def remove_adapter() -> None:
        nonlocal removed
        if not removed:
            _REGISTERED_ADAPTERS.remove(adapter_cls)
            removed = True

    return remove_adapter


def select_adapter(t: torch.Tensor) -> Any:  # noqa: ANN401
    """Return the highest-priority adapter that handles ``t``."""
    for adapter_cls in (*_REGISTERED_ADAPTERS, *_BUILTIN_ADAPTERS):
        if adapter_cls.matches(t):
            return adapter_cls()
    raise NotImplementedError(
        f"No TensorAdapter for tensor type {type(t).__name__!r}. Plain tensors are handled by RegularAdapter; "
        "tensor subclasses need a dedicated adapter registered with register_adapter()."
    )


def tensor_id(t: torch.Tensor) -> tuple[Any, ...]:
    return select_adapter(t).tensor_id(t)


def param_representation(param: torch.Tensor) -> torch.Tensor:
    """``param.data`` for plain parameters; the object itself for tensor subclasses."""
    if type(param) is nn.Parameter or type(param) is torch.Tensor:
        return param.data
    return param


def param_tensor_id(param: torch.Tensor) -> tuple[Any, ...]:
    if param.numel() == 0:
        return ("__empty__", id(param))
    return tensor_id(param_representation(param))
