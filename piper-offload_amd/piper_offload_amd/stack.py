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

__all__ = ["StackPlan", "StackTarget", "check_stack_status", "merge_int8_stack", "merge_nvfp4_stack"]


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
    """Items of one grouped launch must not share storage: a fused NVFP4 launch quantizes one item while
    others are still being read, so two items over the same bytes (one weight twice, views of one fused
    tensor, one shared per-tensor scale) would give results that depend on scheduling."""
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

    NVFP4 merges may run as one fused launch whose quant units wait, bounded,
    for their item's amax units.  A unit that gives up stores nothing and sets
    the workspace's status word.  After each NVFP4 merge the word is copied to
    pinned host memory on the merge's stream; the next :meth:`merge` checks the
    copy once it has arrived, and :meth:`synchronize` waits for it.  Either
    raises ``RuntimeError`` if the word was set.  No host synchronization is
    added to a merge.
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
        # the workspace's status word (written only by fused NVFP4 launches), zeroed once here
        off = self._ws_ptr - self._ws.data_ptr() + int(L.lib().lm_stack_status_offset(len(self.targets)))
        self._status_dev = self._ws[off:off + 4].view(torch.int32)
        self._status_host: torch.Tensor | None = None
        self._status_evt: torch.cuda.Event | None = None  # the copy of the word after the last NVFP4 merge
        if kind == "nvfp4":
            self._status_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
            with torch.cuda.device(self.device):
                self._status_dev.zero_()

    def _check_status(self, wait: bool) -> None:
        """Raise if a finished NVFP4 merge's fused launch gave up a wait; ``wait`` blocks until the
        last merge's copy of the status word has arrived."""
        evt = self._status_evt
        if evt is None or (not wait and not evt.query()):
            return
        evt.synchronize()
        self._status_evt = None
        assert self._status_host is not None
        if int(self._status_host[0]) != 0:
            with torch.cuda.device(self.device):
                self._status_dev.zero_()
            self._status_host.zero_()
            raise RuntimeError("NVFP4 stack merge incomplete: a quantization unit of the fused launch gave up "
                               "waiting for its tensor's amax pass and stored nothing; the merged weights of that "
                               "call are not valid")

    def synchronize(self) -> None:
        """Wait for the last merge and raise ``RuntimeError`` if it was incomplete."""
        if self._last is not None:
            self._last.synchronize()
        self._check_status(wait=True)

    def merge(self, seeds: Sequence[int] | None = None, *, stochastic: bool = True) -> None:
        """Merge every target once; ``seeds`` (one per target) replace the targets' seeds."""
        if seeds is not None:
            if len(seeds) != len(self.targets):
                raise ValueError("one seed per target is required")
            for it, seed in zip(self._arr, seeds):
                it.seed = int(seed)
        self._check_status(wait=False)
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
            if rc == L.LM_OK and self.kind == "nvfp4":
                if self._status_evt is not None:  # an earlier copy still in flight: it lands first
                    self._status_evt.synchronize()
                    self._check_status(wait=True)
                self._status_host.copy_(self._status_dev, non_blocking=True)
                self._status_evt = torch.cuda.Event()
                self._status_evt.record(current)
            if rc == L.LM_OK:
                self._last = torch.cuda.Event()
                self._last.record(current)
        L.check(rc)


def merge_int8_stack(targets: Sequence[StackTarget], *, stochastic: bool = True) -> None:
    """Merge many per-row symmetric INT8 weights in place with one grouped launch."""
    if not targets:
        return
    merge_once(targets, "int8", stochastic=stochastic)


_pending: list[StackPlan] = []  # one-shot NVFP4 merges whose status word has not been checked yet


def check_stack_status(wait: bool = True) -> None:
    """Check the one-shot NVFP4 stack merges issued so far (``merge_nvfp4_stack``): raise ``RuntimeError`` if
    one of them was incomplete.  ``wait=False`` checks only those that have finished."""
    keep = []
    try:
        while _pending:
            plan = _pending.pop(0)
            if not wait and plan._status_evt is not None and not plan._status_evt.query():
                keep.append(plan)
                continue
            plan._check_status(wait=True)
    finally:
        _pending[:0] = keep


def merge_once(targets: Sequence[StackTarget], kind: str, *, stochastic: bool) -> None:
    """One grouped merge of ``targets`` with their own seeds, through a plan used once.  An NVFP4 plan is kept
    until its status word has been checked: by the next one-shot merge once it has finished, or by
    :func:`check_stack_status`."""
    check_stack_status(wait=False)
    plan = StackPlan(targets, kind)
    plan.merge([t.seed for t in targets], stochastic=stochastic)
    if kind == "nvfp4":
        _pending.append(plan)


def merge_nvfp4_stack(targets: Sequence[StackTarget], *, stochastic: bool = True) -> None:
    """Merge many NVFP4 weights in place with grouped launches over all targets.

    Asynchronous, like every merge here: a fused launch that gave up a wait is reported by the next
    one-shot stack merge once that merge has finished, or by :func:`check_stack_status`."""
    if not targets:
        return
    merge_once(targets, "nvfp4", stochastic=stochastic)
