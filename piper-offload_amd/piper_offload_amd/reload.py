"""Merge on reload: the offloader's post-copy LoRA hook, pipelined on MI355X.

In piper-offload's merge mode every managed weight gets a post-copy hook
(P/model_offloader.py:245-288): when a block is reloaded from pinned host
memory into its device target (P/pinned_module.py:259-293), the hook runs
``LoRATransform.apply_weight`` on the freshly copied weight
(P/pinned_module.py:682-695), so every reload merges the pristine stored
weight again with the next merge index (``derive_seed(param_path,
merge_index)``).

:class:`ReloadMergePipeline` is that path for per-row INT8 layers:

* the stored weights stay in pinned host memory, the LoRA factors on the GPU;
* a reload copies one layer into a device slot on a copy stream, and the
  layer's grouped stack merge (one launch for all its weights,
  :class:`~piper_offload_amd.stack.StackPlan`) runs on a merge stream as soon
  as that copy has landed, so the next layer's copy overlaps this merge;
* slots are reused round-robin; a slot is copied into again only after its
  previous merge has finished and after the consumer of its previous contents
  has called :meth:`ReloadMergePipeline.release` (if it did).

All streams keep the default priority.  Results equal
``merge_int8_stack`` on copies of the stored weights with the same seeds.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from .formats import Int8Weight
from .seeding import derive_seed
from .stack import StackPlan, StackTarget

__all__ = ["HostInt8Target", "ReloadMergePipeline", "Reloaded"]


@dataclass(slots=True)
class HostInt8Target:
    """One stored weight: per-row symmetric INT8 codes and fp32/bf16 scales in
    pinned host memory, its LoRA factors on the GPU, and its parameter path
    (the key of its rounding seeds)."""

    path: str
    qdata: torch.Tensor  # int8 [M, N], pinned
    scale: torch.Tensor  # [M, 1], pinned
    b: torch.Tensor      # [M, r] on the GPU
    a: torch.Tensor      # [r, N] on the GPU
    strength: float = 1.0


@dataclass(slots=True)
class Reloaded:
    """A layer reloaded and merged into a device slot; ``ready`` is recorded
    on the merge stream after the merge."""

    layer: int
    slot: int
    weights: list[Int8Weight]
    ready: torch.cuda.Event

    def wait(self, stream: torch.cuda.Stream | None = None) -> None:
        """Make ``stream`` (default: the current stream) wait for the merge."""
        (stream or torch.cuda.current_stream()).wait_event(self.ready)


class ReloadMergePipeline:
    """Reload-and-merge of INT8 layers through ``slots`` device buffers."""

    def __init__(self, layers: Sequence[Sequence[HostInt8Target]], *, device: torch.device | str = "cuda",
                 slots: int = 2, stochastic: bool = True) -> None:
        if not layers or any(not layer for layer in layers):
            raise ValueError("every layer needs at least one target")
        if slots < 1:
            raise ValueError("at least one device slot is required")
        self.device = torch.device(device)
        shapes = [[(t.qdata.shape, t.scale.shape, t.scale.dtype) for t in layer] for layer in layers]
        if any(s != shapes[0] for s in shapes):
            raise ValueError("all layers must have the same weight shapes (one slot layout)")
        for layer in layers:
            for t in layer:
                if t.qdata.dtype is not torch.int8 or t.qdata.ndim != 2:
                    raise ValueError(f"{t.path}: reload merge expects int8 [M, N] codes")
                if not (t.qdata.is_pinned() and t.scale.is_pinned()):
                    raise ValueError(f"{t.path}: stored weights must be in pinned host memory")
                if t.b.device.type != "cuda" or t.a.device.type != "cuda":
                    raise ValueError(f"{t.path}: LoRA factors must be on the GPU")
        self.layers = [list(layer) for layer in layers]
        self.stochastic = stochastic
        self.copy_stream = torch.cuda.Stream(self.device)
        self.merge_stream = torch.cuda.Stream(self.device)
        # slot buffers and one stack plan per (slot, layer): the plan's factor
        # pointers are the layer's, its weight pointers the slot's
        self._slots: list[list[Int8Weight]] = []
        for _ in range(slots):
            bufs = []
            for t in self.layers[0]:
                q = torch.empty(t.qdata.shape, dtype=torch.int8, device=self.device)
                s = torch.empty(t.scale.shape, dtype=t.scale.dtype, device=self.device)
                bufs.append(Int8Weight(q, s, (1, t.qdata.shape[1]), torch.bfloat16))
            self._slots.append(bufs)
        self._plans: dict[tuple[int, int], StackPlan] = {}
        self._free: list[torch.cuda.Event | None] = [None] * slots   # consumer's release of the slot
        self._merged: list[torch.cuda.Event | None] = [None] * slots  # the slot's last merge
        self._next_slot = 0

    def _plan(self, slot: int, layer: int) -> StackPlan:
        key = (slot, layer)
        if key not in self._plans:
            targets = [StackTarget(w, t.b, t.a, t.strength) for w, t in zip(self._slots[slot], self.layers[layer])]
            self._plans[key] = StackPlan(targets, "int8")
        return self._plans[key]

    def reload(self, layer: int, merge_index: int) -> Reloaded:
        """Copy ``layer`` into the next slot and merge it with ``merge_index``'s seeds (asynchronous)."""
        slot = self._next_slot
        self._next_slot = (slot + 1) % len(self._slots)
        bufs = self._slots[slot]
        # never overwrite a slot before its previous merge has finished, nor
        # before its consumer released it (when it did)
        for ev in (self._merged[slot], self._free[slot]):
            if ev is not None:
                self.copy_stream.wait_event(ev)
        with torch.cuda.stream(self.copy_stream):
            for w, t in zip(bufs, self.layers[layer]):
                w.qdata.copy_(t.qdata, non_blocking=True)
                w.scale.copy_(t.scale, non_blocking=True)
            copied = torch.cuda.Event()
            copied.record(self.copy_stream)
        self.merge_stream.wait_event(copied)
        with torch.cuda.stream(self.merge_stream):
            seeds = [derive_seed(t.path, merge_index) for t in self.layers[layer]]
            self._plan(slot, layer).merge(seeds, stochastic=self.stochastic)
            ready = torch.cuda.Event()
            ready.record(self.merge_stream)
        self._free[slot] = None
        self._merged[slot] = ready
        return Reloaded(layer, slot, bufs, ready)

    def release(self, reloaded: Reloaded, stream: torch.cuda.Stream | None = None) -> None:
        """The consumer on ``stream`` (default: current) is done with ``reloaded``'s slot.

        A slot that is not released is copied into again once its previous
        merge has finished, which may be while a consumer still reads it."""
        ev = torch.cuda.Event()
        ev.record(stream or torch.cuda.current_stream())
        self._free[reloaded.slot] = ev
