"""Grouped merges: many targets in one HIP launch.

The reference applies every target of ``merge_lora()`` in a Python loop
(P/merge.py:121-125), paying staging copies, host syncs and 3-5 kernel
launches per weight.  :func:`merge_int8_stack` hands all per-row INT8
targets of a model to one grouped kernel (``lm_int8_merge_stack``);
:func:`merge_nvfp4_stack` does the NVFP4 equivalent.  Each target keeps its
own seed, so results equal per-target merges with the same seeds.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence
from dataclasses import dataclass

import torch

from . import _lib as L

__all__ = ["StackTarget", "merge_int8_stack", "merge_nvfp4_stack"]


@dataclass(slots=True)
class StackTarget:
    """One weight of a stack merge: packed storage + staged factors + seed."""

    weight: object  # Int8Weight / NVFP4Weight (or any object with the same attributes)
    b: torch.Tensor
    a: torch.Tensor
    strength: float
    seed: int = 0


def _items(targets: Sequence[StackTarget], kind: str) -> tuple[ctypes.Array, int, torch.device]:
    lib = L.lib()
    arr = (L.StackItem * len(targets))()
    total = lib.lm_stack_workspace_extra(len(targets))
    device = None
    for i, t in enumerate(targets):
        w = t.weight
        rows = w.qdata.shape[0]
        cols = w.qdata.shape[1] * (2 if kind == "nvfp4" else 1)
        if t.b.dtype not in (torch.bfloat16, torch.float16) or t.b.dtype is not t.a.dtype:
            raise ValueError("stack merge needs bf16/fp16 factors of one dtype")
        if tuple(t.b.shape) != (rows, t.a.shape[0]) or t.a.shape[1] != cols:
            raise ValueError(f"stack target {i}: LoRA factors do not match the weight shape")
        device = w.qdata.device if device is None else device
        if w.qdata.device != device:
            raise ValueError("stack merge requires all targets on one GPU")
        it = arr[i]
        it.q = w.qdata.data_ptr()
        it.scale = w.scale.data_ptr()
        it.q_out = w.qdata.data_ptr()
        it.scale_out = w.scale.data_ptr()
        if kind == "nvfp4" and w.per_tensor_scale is not None:
            it.aux = w.per_tensor_scale.data_ptr()
            it.aux_out = w.per_tensor_scale.data_ptr()
        it.M, it.N = rows, cols
        it.lora = L.lora_struct(t.b, t.a, t.strength)
        it.seed = int(t.seed)
        total += lib.lm_workspace_size(rows, cols, t.a.shape[0])
    assert device is not None
    return arr, total, device


def merge_int8_stack(targets: Sequence[StackTarget], *, stochastic: bool = True) -> None:
    """Merge many per-row symmetric INT8 weights in place with one grouped launch."""
    if not targets:
        return
    for t in targets:
        w = t.weight
        if w.qdata.dtype is not torch.int8 or tuple(w.block_size) != (1, w.qdata.shape[1]):
            raise ValueError("merge_int8_stack supports per-row INT8 weights")
        if getattr(w, "zero_point", None) is not None and bool(w.zero_point.any()):
            raise ValueError("merge_int8_stack supports symmetric INT8 weights")
    scale_dtype = targets[0].weight.scale.dtype
    if any(t.weight.scale.dtype is not scale_dtype for t in targets):
        raise ValueError("stack targets must share one scale dtype")
    arr, total, device = _items(targets, "int8")
    with torch.cuda.device(device):
        ws = L.workspace(total, device)
        rc = L.lib().lm_int8_merge_stack(arr, len(targets), L.torch_dtype_id(scale_dtype),
                                        L.LM_ROUND_STOCHASTIC if stochastic else L.LM_ROUND_NEAREST,
                                        L.aligned_ptr(ws), total, L.stream_ptr(device))
    L.check(rc)


def merge_nvfp4_stack(targets: Sequence[StackTarget], *, stochastic: bool = True) -> None:
    """Merge many NVFP4 weights in place (one grouped prep, per-target passes)."""
    if not targets:
        return
    swz = bool(targets[0].weight.is_swizzled_scales)
    if any(bool(t.weight.is_swizzled_scales) != swz for t in targets):
        raise ValueError("stack targets must share one scale layout")
    arr, total, device = _items(targets, "nvfp4")
    with torch.cuda.device(device):
        ws = L.workspace(total, device)
        rc = L.lib().lm_nvfp4_merge_stack(arr, len(targets), int(swz),
                                         L.LM_ROUND_STOCHASTIC if stochastic else L.LM_ROUND_NEAREST,
                                         L.aligned_ptr(ws), total, L.stream_ptr(device))
    L.check(rc)
