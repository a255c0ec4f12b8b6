"""Merge on reload: the offloader's post-copy LoRA hook, pipelined on MI355X.

In piper-offload's merge mode every managed weight gets a post-copy hook
(P/model_offloader.py:245-288): when a block is reloaded from pinned host
memory into its device target (P/pinned_module.py:259-293), the hook runs
``LoRATransform.apply_weight`` on the freshly copied weight
(P/pinned_module.py:682-695), so every reload merges the pristine stored
weight again with the next merge index (``derive_seed(param_path,
merge_index)``).

:class:`ReloadMergePipeline` is that path for layers of per-row INT8,
per-row scaled FP8 and NVFP4 weights (the reference's hook re-merges every
adapter format through ``adapter.merge_lora_``):

* the stored weights stay in pinned host memory, the LoRA factors on the GPU;
* a reload copies one layer into a device slot on a copy stream, and the
  layer's merge runs on a merge stream as soon as that copy has landed, so
  the next layer's copy overlaps this merge: one grouped stack launch for the
  layer's INT8 weights and one for its NVFP4 weights
  (:class:`~piper_offload_amd.stack.StackPlan`), and the fused per-row FP8
  kernel for each FP8 weight;
* slots are reused round-robin; a slot is copied into again only after its
  previous merge has finished and after the consumer of its previous contents
  has called :meth:`ReloadMergePipeline.release` (if it did).

All streams keep the default priority.  Results equal the stack and
single-weight merges of copies of the stored weights with the same seeds.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from . import kernels as K
from .formats import Float8Weight, Int8Weight, NVFP4Weight
from .seeding import derive_seed
from .stack import StackPlan, StackTarget

__all__ = ["HostFloat8Target", "HostInt8Target", "HostNvfp4Target", "ReloadMergePipeline", "Reloaded"]


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
class HostFloat8Target:
    """One stored per-row scaled-FP8 weight (TorchAO ``Float8Tensor`` layout): fp8 codes and fp32 row scales
    in pinned host memory, its LoRA factors on the GPU."""

    path: str
    qdata: torch.Tensor  # float8_e4m3fn / float8_e5m2 [M, N], pinned
    scale: torch.Tensor  # float32 [M, 1], pinned
    b: torch.Tensor
    a: torch.Tensor
    strength: float = 1.0


@dataclass(slots=True)
class HostNvfp4Target:
    """One stored NVFP4 weight (TorchAO ``NVFP4Tensor`` layout): packed e2m1 codes, e4m3 block scales and the
    optional fp32 per-tensor scale in pinned host memory, its LoRA factors on the GPU."""

    path: str
    qdata: torch.Tensor                    # uint8 [M, N/2], pinned
    scale: torch.Tensor                    # float8_e4m3fn block scales (plain or swizzled), pinned
    per_tensor_scale: torch.Tensor | None  # float32 scalar, pinned (two-level) or None
    b: torch.Tensor
    a: torch.Tensor
    strength: float = 1.0
    is_swizzled_scales: bool = False


HostTarget = HostInt8Target | HostFloat8Target | HostNvfp4Target


def _stored(t: HostTarget) -> list[torch.Tensor]:
    """The pinned tensors of one stored weight, in copy order."""
    pts = getattr(t, "per_tensor_scale", None)
    return [t.qdata, t.scale] + ([pts] if pts is not None else [])


def _layout(t: HostTarget) -> tuple:
    return (type(t).__name__,) + tuple((x.shape, x.dtype) for x in _stored(t)) + \
        (bool(getattr(t, "is_swizzled_scales", False)),)


def _device_weight(t: HostTarget, device: torch.device) -> Int8Weight | Float8Weight | NVFP4Weight:
    """Empty device buffers with ``t``'s storage layout."""
    q = torch.empty(t.qdata.shape, dtype=t.qdata.dtype, device=device)
    s = torch.empty(t.scale.shape, dtype=t.scale.dtype, device=device)
    if isinstance(t, HostInt8Target):
        return Int8Weight(q, s, (1, t.qdata.shape[1]), torch.bfloat16)
    if isinstance(t, HostFloat8Target):
        return Float8Weight(q, s, (1, t.qdata.shape[1]), torch.bfloat16)
    pts = None if t.per_tensor_scale is None else torch.empty((), dtype=torch.float32, device=device)
    return NVFP4Weight(q, s, pts, 16, torch.bfloat16, t.is_swizzled_scales)


def _device_tensors(w: Int8Weight | Float8Weight | NVFP4Weight) -> list[torch.Tensor]:
    pts = getattr(w, "per_tensor_scale", None)
    return [w.qdata, w.scale] + ([pts] if pts is not None else [])


@dataclass(slots=True)
class Reloaded:
    """A layer reloaded and merged into a device slot; ``ready`` is recorded
    on the merge stream after the merge."""

    layer: int
    slot: int
    weights: list[Int8Weight | Float8Weight | NVFP4Weight]
    ready: torch.cuda.Event

    def wait(self, stream: torch.cuda.Stream | None = None) -> None:
        """Make ``stream`` (default: the current stream) wait for the merge."""
        (stream or torch.cuda.current_stream()).wait_event(self.ready)


class ReloadMergePipeline:
    """Reload-and-merge of INT8 / FP8 / NVFP4 layers through ``slots`` device buffers."""

    def __init__(self, layers: Sequence[Sequence[HostTarget]], *, device: torch.device | str = "cuda",
                 slots: int = 2, stochastic: bool = True) -> None:
        if not layers or any(not layer for layer in layers):
            raise ValueError("every layer needs at least one target")
        if slots < 1:
            raise ValueError("at least one device slot is required")
        self.device = torch.device(device)
        layouts = [[_layout(t) for t in layer] for layer in layers]
        if any(lay != layouts[0] for lay in layouts):
            raise ValueError("all layers must have the same weight formats and shapes (one slot layout)")
        for layer in layers:
            for t in layer:
                if isinstance(t, HostInt8Target):
                    if t.qdata.dtype is not torch.int8 or t.qdata.ndim != 2:
                        raise ValueError(f"{t.path}: reload merge expects int8 [M, N] codes")
                elif isinstance(t, HostFloat8Target):
                    if t.qdata.dtype not in (torch.float8_e4m3fn, torch.float8_e5m2) or t.qdata.ndim != 2:
                        raise ValueError(f"{t.path}: reload merge expects fp8 [M, N] codes")
                    if t.scale.dtype is not torch.float32 or tuple(t.scale.shape) != (t.qdata.shape[0], 1):
                        raise ValueError(f"{t.path}: reload merge expects float32 per-row scales [M, 1]")
                elif isinstance(t, HostNvfp4Target):
                    if t.qdata.dtype is not torch.uint8 or t.qdata.ndim != 2:
                        raise ValueError(f"{t.path}: reload merge expects packed uint8 [M, N/2] NVFP4 codes")
                else:
                    raise ValueError(f"unsupported stored weight {type(t).__name__}")
                if not all(x.is_pinned() for x in _stored(t)):
                    raise ValueError(f"{t.path}: stored weights must be in pinned host memory")
                if t.b.device.type != "cuda" or t.a.device.type != "cuda":
                    raise ValueError(f"{t.path}: LoRA factors must be on the GPU")
        self.layers = [list(layer) for layer in layers]
        self.stochastic = stochastic
        self.copy_stream = torch.cuda.Stream(self.device)
        self.merge_stream = torch.cuda.Stream(self.device)
        # slot buffers and, per (slot, layer), one stack plan per grouped
        # format: the plans' factor pointers are the layer's, their weight
        # pointers the slot's
        self._slots = [[_device_weight(t, self.device) for t in self.layers[0]] for _ in range(slots)]
        self._plans: dict[tuple[int, int], list[tuple[StackPlan, list[int]]]] = {}
        self._free: list[torch.cuda.Event | None] = [None] * slots   # consumer's release of the slot
        self._merged: list[torch.cuda.Event | None] = [None] * slots  # the slot's last merge
        self._next_slot = 0

    def _group_plans(self, slot: int, layer: int) -> list[tuple[StackPlan, list[int]]]:
        key = (slot, layer)
        if key not in self._plans:
            plans = []
            for kind, cls in (("int8", HostInt8Target), ("nvfp4", HostNvfp4Target)):
                idx = [i for i, t in enumerate(self.layers[layer]) if isinstance(t, cls)]
                if idx:
                    targets = [StackTarget(self._slots[slot][i], self.layers[layer][i].b, self.layers[layer][i].a,
                                           self.layers[layer][i].strength) for i in idx]
                    plans.append((StackPlan(targets, kind), idx))
            self._plans[key] = plans
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
                for dst, src in zip(_device_tensors(w), _stored(t)):
                    dst.copy_(src, non_blocking=True)
            copied = torch.cuda.Event()
            copied.record(self.copy_stream)
        self.merge_stream.wait_event(copied)
        targets = self.layers[layer]
        seeds = [derive_seed(t.path, merge_index) for t in targets]
        with torch.cuda.stream(self.merge_stream):
            for plan, idx in self._group_plans(slot, layer):
                plan.merge([seeds[i] for i in idx], stochastic=self.stochastic)
            for i, (w, t) in enumerate(zip(bufs, targets)):
                if isinstance(t, HostFloat8Target):
                    K.merge_float8_lora_into(w.qdata, w.scale, w.block_size, t.b, t.a, t.strength,
                                             rounding_seed=seeds[i] if self.stochastic else None,
                                             out_qdata=w.qdata, out_scale=w.scale)
            ready = torch.cuda.Event()
            ready.record(self.merge_stream)
        self._free[slot] = None
        self._merged[slot] = ready
        return Reloaded(layer, slot, bufs, ready)

    def synchronize(self) -> None:
        """Wait for every issued merge."""
        self.merge_stream.synchronize()

    def release(self, reloaded: Reloaded, stream: torch.cuda.Stream | None = None) -> None:
        """The consumer on ``stream`` (default: current) is done with ``reloaded``'s slot.

        A slot that is not released is copied into again once its previous
        merge has finished, which may be while a consumer still reads it."""
        ev = torch.cuda.Event()
        ev.record(stream or torch.cuda.current_stream())
        self._free[reloaded.slot] = ev
