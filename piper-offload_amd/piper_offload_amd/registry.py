"""Which adapter handles a tensor, and tensor identity (interface of P/tensor_adapter_registry.py:38-152).

The dispatch chain is external registrations, newest first, followed by the
built-in adapters of this build; ``RegularAdapter`` closes the chain and
matches only plain tensors.  The chain is kept as one tuple that is rebuilt
on every (rare) registration change, so a lookup is a single scan.  There is
no DTensor adapter: sharded weights are outside this single-GPU build.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Any

import torch
from torch import nn

from .adapters import Float8Adapter, GgufAdapter, Int8Adapter, MxAdapter, Nvfp4Adapter, RegularAdapter

__all__ = ["param_representation", "param_tensor_id", "register_adapter", "select_adapter", "tensor_id"]

_BUILTIN_ADAPTERS: tuple[type, ...] = (Nvfp4Adapter, MxAdapter, Float8Adapter, Int8Adapter, GgufAdapter, RegularAdapter)
_PROTOCOL = ("matches", "tensor_id", "compute_dtype")


class _Chain:
    """External adapter classes (newest first) and the dispatch tuple derived from them."""

    def __init__(self) -> None:
        self.external: list[type] = []
        self.order: tuple[type, ...] = _BUILTIN_ADAPTERS

    def rebuild(self) -> None:
        self.order = (*self.external, *_BUILTIN_ADAPTERS)


_CHAIN = _Chain()


class _Registration:
    """Handle returned by :func:`register_adapter`; calling it removes the adapter (again: no effect)."""

    __slots__ = ("adapter_cls", "active")

    def __init__(self, adapter_cls: type) -> None:
        self.adapter_cls = adapter_cls
        self.active = True

    def __call__(self) -> None:
        if self.active:
            self.active = False
            _CHAIN.external.remove(self.adapter_cls)
            _CHAIN.rebuild()


def register_adapter(adapter_cls: type) -> Callable[[], None]:
    """Put an external adapter class in front of the built-ins; returns an idempotent remover.

    The class must satisfy the adapter protocol (``matches``, ``tensor_id``,
    ``compute_dtype``) and be constructible without arguments.  Registration is
    process-global and meant for application start-up.
    """
    if not isinstance(adapter_cls, type):
        raise TypeError(f"register_adapter() expects a TensorAdapter class, got {type(adapter_cls).__name__}")
    name = adapter_cls.__name__
    if adapter_cls in _BUILTIN_ADAPTERS:
        raise ValueError(f"TensorAdapter {name!r} is already built in")
    if adapter_cls in _CHAIN.external:
        raise ValueError(f"TensorAdapter {name!r} is already registered")
    try:
        adapter_cls()
    except TypeError as exc:
        raise TypeError(f"TensorAdapter {name!r} must be constructible without arguments") from exc
    if any(not callable(getattr(adapter_cls, attr, None)) for attr in _PROTOCOL):
        raise TypeError(f"Adapter {name!r} does not satisfy the TensorAdapter protocol")
    _CHAIN.external.insert(0, adapter_cls)
    _CHAIN.rebuild()
    return _Registration(adapter_cls)


def select_adapter(t: torch.Tensor) -> Any:  # noqa: ANN401
    """An instance of the first adapter in the dispatch chain that matches ``t``."""
    found = next((cls for cls in _CHAIN.order if cls.matches(t)), None)
    if found is None:
        raise NotImplementedError(
            f"No TensorAdapter for tensor type {type(t).__name__!r}. Plain tensors are handled by RegularAdapter; "
            "tensor subclasses need a dedicated adapter registered with register_adapter()."
        )
    return found()


def tensor_id(t: torch.Tensor) -> tuple[Any, ...]:
    """The identity the matching adapter gives ``t`` (tied weights share one)."""
    return select_adapter(t).tensor_id(t)


def param_representation(param: torch.Tensor) -> torch.Tensor:
    """The object an adapter sees for a parameter.

    A plain parameter or tensor is seen through ``.data``: for a packed weight
    wrapped in a Parameter that is the packed object itself.  A parameter whose
    own class is a tensor subclass is seen as it is, since ``.data`` could
    strip its packed state.
    """
    return param.data if type(param) in (nn.Parameter, torch.Tensor) else param


def param_tensor_id(param: torch.Tensor) -> tuple[Any, ...]:
    """Tensor identity of a parameter.  Zero-element tensors all report data pointer 0,
    so they are told apart by the Python object instead."""
    return ("zero-element", id(param)) if param.numel() == 0 else tensor_id(param_representation(param))
