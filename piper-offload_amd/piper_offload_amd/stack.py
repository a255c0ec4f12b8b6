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

__all__ = ["StackPlan", "StackTarget", "merge_int8_stack", "merge_nvfp4_stack"]


@dataclass(slots=True)
class StackTarget:
    """One weight of a stack merge: packed storage + staged factors + seed."""

    weight: object  # Int8Weight / NVFP4Weight (or any object with the same attributes)
    b: torch.Tensor
    a: torch.Tensor
    strength: float
    seed: int = 0


def _byte_range(t: torch.Tensor) -> tuple[int, int]:
    """[first, last) bytes a tensor view can touch."""
    if t.numel() == 0:
        return t.data_ptr(), t.data_ptr()
    span = 1 + sum((n - 1) * abs(st) for n, st in zip(t.shape, t.stride()))
    return t.data_ptr(), t.data_ptr() + span * t.element_size()


def _reject_shared_buffers(targets: Sequence[StackTarget]) -> None:
    """Items of one grouped launch must not share storage: the launch merges its items in place at the same
    time, so two items over the same bytes (one weight twice, views of one fused tensor, one shared
    per-tensor scale) would read each other's outputs, with results that depend on scheduling."""
    spans = []
    for i, t in enumerate(targets):
        w = t.weight
        for name in ("qdata", "scale", "per_tensor_scale", "zero_point"):
            buf = getattr(w, name, None)
            if isinstance(buf, torch.Tensor) and buf.numel():
                lo, hi = _byte_range(buf)
                spans.append((lo, hi, i, name))
    spans.sort()
    for (lo0, hi0, i0, n0), (lo1, hi1, i1, n1) in zip(spans, spans[1:]):
        if lo1 < hi0:
            raise ValueError(f"stack targets must not share buffers: target {i0} {n0} overlaps target {i1} {n1}")


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


class StackPlan:
    """A reusable grouped merge over fixed targets.

    Building the descriptor table (pointers, shapes, factors) and sizing the
    workspace happen once; :meth:`merge` only rewrites the per-target seeds
    and issues the grouped call, asynchronously on the current stream.  The
    targets' storage and factors must stay alive and keep their addresses for
    the plan's lifetime; their contents may change between merges (that is
    the point: each merge updates the weights in place).

    Every merge reuses one workspace (the factor layouts and the descriptor
    table).  A merge therefore makes its stream wait for the previous merge's
    completion event, so merges issued on different streams run one after the
    other instead of overwriting buffers an earlier launch still reads.
    """

    def __init__(self, targets: Sequence[StackTarget], kind: str) -> None:
        if kind not in ("int8", "nvfp4"):
            raise ValueError(f"unknown stack kind {kind!r}")
        if not targets:
            raise ValueError("a stack plan needs at least one target")
        self.kind = kind
        self.targets = list(targets)
        if kind == "int8":
            for t in self.targets:
                w = t.weight
                if w.qdata.dtype is not torch.int8 or tuple(w.block_size) != (1, w.qdata.shape[1]):
                    raise ValueError("merge_int8_stack supports per-row INT8 weights")
                if getattr(w, "zero_point", None) is not None and bool(w.zero_point.any()):
                    raise ValueError("merge_int8_stack supports symmetric INT8 weights")
            self._scale_dtype = self.targets[0].weight.scale.dtype
            if any(t.weight.scale.dtype is not self._scale_dtype for t in self.targets):
                raise ValueError("stack targets must share one scale dtype")
        else:
            self._swizzled = bool(self.targets[0].weight.is_swizzled_scales)
            if any(bool(t.weight.is_swizzled_scales) != self._swizzled for t in self.targets):
                raise ValueError("stack targets must share one scale layout")
        _reject_shared_buffers(self.targets)
        self._arr, self._ws_bytes, self.device = _items(self.targets, kind)
        with torch.cuda.device(self.device):
            self._ws = L.workspace(self._ws_bytes, self.device)
        self._ws_ptr = L.aligned_ptr(self._ws)
        self._last: torch.cuda.Event | None = None  # completion of the previous merge

    def synchronize(self) -> None:
        """Wait for the last merge."""
        if self._last is not None:
            self._last.synchronize()

    def merge(self, seeds: Sequence[int] | None = None, *, stochastic: bool = True) -> None:
        """Merge every target once; ``seeds`` (one per target) replace the targets' seeds."""
        if seeds is not None:
            if len(seeds) != len(self.targets):
                raise ValueError("one seed per target is required")
            for it, seed in zip(self._arr, seeds):
                it.seed = int(seed)
        lib = L.lib()
        mode = L.LM_ROUND_STOCHASTIC if stochastic else L.LM_ROUND_NEAREST
        with torch.cuda.device(self.device):
            current = torch.cuda.current_stream(self.device)
            if self._last is not None:
                current.wait_event(self._last)
            stream = current.cuda_stream
            if self.kind == "int8":
                rc = lib.lm_int8_merge_stack(self._arr, len(self.targets), L.torch_dtype_id(self._scale_dtype), mode,
                                             self._ws_ptr, self._ws_bytes, stream)
            else:
                rc = lib.lm_nvfp4_merge_stack(self._arr, len(self.targets), int(self._swizzled), mode,
                                              self._ws_ptr, self._ws_bytes, stream)
            # the caching allocator must not hand the workspace to another stream
            # while this merge may still read it
            self._ws.record_stream(current)
            if rc == L.LM_OK:
                self._last = torch.cuda.Event()
                self._last.record(current)
        L.check(rc)


def merge_int8_stack(targets: Sequence[StackTarget], *, stochastic: bool = True) -> None:
    """Merge many per-row symmetric INT8 weights in place with one grouped launch."""
    if not targets:
        return
    merge_once(targets, "int8", stochastic=stochastic)


def merge_once(targets: Sequence[StackTarget], kind: str, *, stochastic: bool) -> None:
    """One grouped merge of ``targets`` with their own seeds, through a plan used once."""
    StackPlan(targets, kind).merge([t.seed for t in targets], stochastic=stochastic)


def merge_nvfp4_stack(targets: Sequence[StackTarget], *, stochastic: bool = True) -> None:
    """Merge many NVFP4 weights in place with grouped launches over all targets."""
    if not targets:
        return
    merge_once(targets, "nvfp4", stochastic=stochastic)
