"""Routed LoRA: the LoRA contribution added after a Linear instead of merged into it.

The reference's routed mode (P/lora.py:792-930).  A forward hook on the
parent module stages the factors on the input's device (cached) and returns
``output + residual`` with

    residual = sum_i ((x @ A_i.T) * s_i) @ B_i.T (+ bias_i * s_i)

computed by ``lm_routed_residual``: an MFMA down projection into a small fp32
workspace, then one kernel that applies the reference's roundings (every
step in the output dtype, matmuls accumulated in fp32), multiplies by B and
adds into a new output, reading and writing the ``[T, N]`` output once.  At
most 16 tokens (decode) run as a single launch with no workspace.

Differences from the reference, on purpose:

* staged factors are kept per device and dtype while the host factors are
  unmodified (their in-place version counters), instead of copied on every
  invocation, so one post-forward hook replaces the reference's pre/post
  pair;
* the kernel is inference-only (no autograd) and takes bfloat16 / float16
  outputs; other cases raise instead of running elsewhere.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import Any

import torch
from torch import nn

from . import _lib as L
from .lora import ScaledLoRAFactor

__all__ = ["RoutedFactor", "install_routed_residual_hook", "routed_residual"]

_DTYPES = (torch.bfloat16, torch.float16)


@dataclass(slots=True, frozen=True)
class RoutedFactor:
    """Factors on the device of one invocation (P/lora.py:792-798): a [r, in], b [out, r], bias [out] or None."""

    a: torch.Tensor
    b: torch.Tensor
    strength: float
    bias: torch.Tensor | None = None


def routed_residual(x: torch.Tensor, factors: Sequence[RoutedFactor], output: torch.Tensor) -> torch.Tensor:
    """``output + sum_i s_i ((x A_i^T) B_i^T + bias_i)`` with the reference's roundings (P/lora.py:801-829).

    ``x`` [..., in], ``output`` [..., out] on one GPU; returns a new tensor
    shaped like ``output``.
    """
    if not factors:
        raise ValueError("Routed LoRA residual requires at least one factor")
    dtype = output.dtype
    if dtype not in _DTYPES:
        raise ValueError(f"HIP routed LoRA residual supports bfloat16 and float16 outputs, got {dtype}.")
    if torch.is_grad_enabled() and (x.requires_grad or output.requires_grad or any(
            f.a.requires_grad or f.b.requires_grad or (f.bias is not None and f.bias.requires_grad) for f in factors)):
        raise NotImplementedError("The HIP routed LoRA residual is inference-only; run under torch.no_grad().")
    device = output.device
    if device.type != "cuda" or x.device != device:
        raise ValueError("HIP routed LoRA residual requires the input and output on one GPU.")
    k = x.shape[-1]
    n = output.shape[-1]
    x2 = x.to(dtype=dtype).reshape(-1, k).contiguous()
    y2 = output.reshape(-1, n).contiguous()
    t = y2.shape[0]
    if x2.shape[0] != t:
        raise ValueError(f"Routed LoRA input has {x2.shape[0]} rows but the output has {t}.")
    keep = []
    arr = (L.RoutedFactor * len(factors))()
    for i, f in enumerate(factors):
        a = f.a.to(device=device, dtype=dtype).contiguous()
        b = f.b.to(device=device, dtype=dtype).contiguous()
        if a.ndim != 2 or b.ndim != 2 or a.shape[1] != k or b.shape != (n, a.shape[0]):
            raise ValueError(f"Routed LoRA factor {i} has shapes A {tuple(a.shape)}, B {tuple(b.shape)}; expected "
                             f"A [r, {k}] and B [{n}, r].")
        bias = None if f.bias is None else f.bias.to(device=device, dtype=dtype).contiguous()
        if bias is not None and bias.shape != (n,):
            raise ValueError(f"Routed LoRA factor {i} bias shape {tuple(bias.shape)} does not match ({n},).")
        keep.extend(t_ for t_ in (a, b, bias) if t_ is not None)
        arr[i].a, arr[i].b = a.data_ptr(), b.data_ptr()
        arr[i].bias = None if bias is None else bias.data_ptr()
        arr[i].strength = float(f.strength)
        arr[i].rank = a.shape[0]
    out = torch.empty_like(y2)
    if t == 0:
        return out.view(output.shape)
    handle = L.lib()
    ws_bytes = handle.lm_routed_workspace_size(t, k, arr, len(factors))
    with torch.cuda.device(device):
        # at most 16 tokens need no workspace (one launch, LDS only)
        ws = L.workspace(ws_bytes, device) if ws_bytes else None
        rc = handle.lm_routed_residual(x2.data_ptr(), y2.data_ptr(), out.data_ptr(), t, k, n, L.torch_dtype_id(dtype),
                                       arr, len(factors), None if ws is None else L.aligned_ptr(ws), ws_bytes,
                                       L.stream_ptr(device))
    L.check(rc)
    del keep
    return out.view(output.shape)


class _Stager:
    """Device copies of host factors per (device, dtype), valid while the host tensors are unmodified."""

    def __init__(self, factors: Sequence[ScaledLoRAFactor]) -> None:
        self.factors = list(factors)
        self.cache: dict[tuple[torch.device, torch.dtype], tuple[tuple[int, ...], tuple[RoutedFactor, ...]]] = {}

    def stage(self, device: torch.device, dtype: torch.dtype) -> tuple[RoutedFactor, ...]:
        versions = tuple(v for f in self.factors for t in (f.a, f.b, f.bias) if t is not None for v in (t._version,))
        key = (device, dtype)
        hit = self.cache.get(key)
        if hit is not None and hit[0] == versions:
            return hit[1]

        def dev(t: torch.Tensor | None) -> torch.Tensor | None:
            return None if t is None else t.to(device=device, non_blocking=True).to(dtype=dtype)

        staged = tuple(RoutedFactor(dev(f.a), dev(f.b), f.strength, dev(f.bias)) for f in self.factors)
        self.cache[key] = (versions, staged)
        return staged


class _RoutedHook:
    """A forward hook that returns ``output + routed residual`` for the module it is on.

    The reference stages the factors in a pre-forward hook for every
    invocation and adds the residual in a post-forward hook that must run even
    when the forward raises (to drop the staged copies).  Here the staged
    copies are cached per (device, dtype) by ``_Stager``, so one post-forward
    hook does both and there is no per-invocation state to clean up.
    """

    def __init__(self, parent: nn.Module, factors: Sequence[ScaledLoRAFactor]) -> None:
        self.stager = _Stager(factors)
        self.handle = parent.register_forward_hook(self, with_kwargs=True)

    @staticmethod
    def _input(args: tuple[Any, ...], kwargs: dict[str, Any]) -> torch.Tensor:
        """``Linear.forward``'s input, given by position or as the keyword ``input``."""
        if args:
            x = args[0]
        elif "input" in kwargs:
            x = kwargs["input"]
        else:
            raise TypeError("Routed LoRA expected the Linear input as either the first positional argument or the "
                            "'input' keyword")
        if isinstance(x, torch.Tensor):
            return x
        raise TypeError(f"Routed LoRA requires the Linear input to be a torch.Tensor; got {type(x).__name__}")

    def __call__(self, _module: nn.Module, args: tuple[Any, ...], kwargs: dict[str, Any], output: object) -> object:
        if not isinstance(output, torch.Tensor):
            return output
        x = self._input(args, kwargs)
        return routed_residual(x, self.stager.stage(x.device, output.dtype), output)

    def remove(self) -> None:
        self.handle.remove()  # a removed handle ignores further removals
        self.stager.cache.clear()


def install_routed_residual_hook(parent: nn.Module, factors: Sequence[ScaledLoRAFactor]) -> Callable[[], None]:
    """Add the routed residual of ``factors`` to every output of ``parent`` (interface of P/lora.py:869-930).

    Returns an idempotent callable that removes the hook.  One hook covers
    every LoRA targeting this parent.
    """
    if not factors:
        raise ValueError("Routed LoRA hook requires at least one factor")
    return _RoutedHook(parent, factors).remove
