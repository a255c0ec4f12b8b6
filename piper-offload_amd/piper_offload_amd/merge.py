"""Permanent LoRA merge into model weights (P/merge.py:54-214).

``merge_lora(model, [(lora, strength), ...], stochastic_rounding=True)``:
rejects duplicate LoRA instances, drops exact-zero strengths, resolves every
target to a model parameter, groups factors per tensor identity (rejecting
tied aliases), preflights every operation, then applies them and returns the
number of unique parameters modified.  Each weight gets its own
stochastic-rounding seed ``derive_seed(target_key, merge_index)``.
"""

from __future__ import annotations

import logging
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Any

import torch
from torch import nn

from .lora import LoRA, LoRATransform, ScaledLoRAFactor
from .registry import param_representation, param_tensor_id
from .stack import StackPlan, StackTarget

logger = logging.getLogger(__name__)

__all__ = ["merge_lora"]


@dataclass(slots=True, frozen=True)
class _MergeOp:
    weight: nn.Parameter
    bias: nn.Parameter | None
    transform: LoRATransform

    def validate(self) -> None:
        self.transform.validate_target(self.weight, self.bias)

    def apply(self) -> None:
        self.transform.apply(self.weight, self.bias)


def merge_lora(model: nn.Module, loras: Sequence[tuple[LoRA, float]], *, stochastic_rounding: bool = True) -> int:
    """Merge LoRAs into ``model`` in place; returns the number of unique parameters modified."""
    if len({id(lora) for lora, _s in loras}) != len(loras):
        raise ValueError("merge_lora() does not accept the same LoRA instance more than once")
    for lora, _s in loras:
        if not isinstance(lora, LoRA):
            raise TypeError("merge_lora() expects LoRA instances")
    active = [(lora, s) for lora, s in loras if s != 0.0]
    params = dict(model.named_parameters(remove_duplicate=False))
    missing = sorted({k for lora, _s in active for k in lora.targets if k not in params})
    if missing:
        sample = sorted(params)[:3]
        raise ValueError(
            f"LoRA targets are not parameters in the model: {missing}. LoRA target keys must match the model's "
            f"parameter names exactly. Sample model parameter keys: {sample} ..."
        )
    ops = _build_merge_ops(params, active, stochastic_rounding=stochastic_rounding)
    for op in ops:  # preflight everything before mutating anything
        op.validate()
    _apply_all(ops)
    modified = {param_tensor_id(op.weight) for op in ops}
    modified.update(param_tensor_id(op.bias) for op in ops if op.bias is not None)
    logger.info("merge_lora: merged %d unique parameters (%d weights, %d biases) from %d LoRA targets",
                len(modified), len(ops), sum(op.bias is not None for op in ops),
                sum(len(lora.targets) for lora, _s in active))
    return len(modified)


def _apply_all(ops: list[_MergeOp]) -> None:
    """Apply every validated op.  Weights that a grouped kernel can merge
    (per-row INT8, NVFP4) are merged together, one grouped launch per
    compatible group, instead of one launch each (P/merge.py:124-125 loops);
    the rest, and all biases, are applied one by one.  Targets are distinct
    tensors (tied aliases are rejected), so the order does not change any
    result, and each grouped target keeps its own seed."""
    groups: dict[tuple, list[tuple[_MergeOp, StackTarget]]] = {}
    single: list[_MergeOp] = []
    for op in ops:
        st = op.transform.stack_target(op.weight)
        if st is None:
            single.append(op)
        else:
            groups.setdefault(st[0], []).append((op, st[1]))
    for key, members in groups.items():
        if len(members) == 1:  # one tensor: its own launch is the tuned path
            single.append(members[0][0])
            continue
        StackPlan([t for _op, t in members], key[0]).merge(stochastic=key[-1])
        for op, _t in members:
            op.transform.advance()
            if op.bias is not None:
                op.transform.apply_bias(op.bias)
    for op in single:
        op.apply()


def _sibling(name: str, leaf: str) -> str:
    prefix, _, _ = name.rpartition(".")
    return f"{prefix}.{leaf}" if prefix else leaf


def _build_merge_ops(params: dict[str, nn.Parameter], loras: Sequence[tuple[LoRA, float]], *,
                     stochastic_rounding: bool) -> list[_MergeOp]:
    groups: dict[tuple[Any, ...], tuple[str, nn.Parameter, list[ScaledLoRAFactor]]] = {}
    for lora, strength in loras:
        arenas: dict[torch.device, Any] = {}  # this LoRA's factors on each GPU: one copy per device
        for key, factor in lora.targets.items():
            weight = params[key]
            device = param_representation(weight).device
            staged = None
            if device.type == "cuda":
                if device not in arenas:
                    arenas[device] = lora.stage_on(device)
                arena = arenas[device]
                if arena is not None:
                    sa, sb = arena.view(factor.a), arena.view(factor.b)
                    staged = None if sa is None or sb is None else (sa, sb)
            tid = param_tensor_id(weight)
            group = groups.get(tid)
            if group is None:
                group = (key, weight, [])
                groups[tid] = group
            elif group[0] != key:
                raise ValueError(
                    f"LoRA targets {group[0]!r} and {key!r} resolve to the same tied parameter backing. Apply only "
                    "one name for a tied weight in a single merge_lora() call; otherwise the same base weight would "
                    "receive multiple logical updates."
                )
            group[2].append(factor.scaled(strength, staged))
    ops: list[_MergeOp] = []
    bias_owner: dict[tuple[Any, ...], str] = {}
    for key, weight, factors in groups.values():
        transform = LoRATransform(factors, stochastic_rounding=stochastic_rounding, target_key=key)
        bias = None
        if transform.has_bias:
            bias_key = _sibling(key, "bias")
            bias = params.get(bias_key)
            if bias is None:
                raise ValueError(f"Cannot merge legacy LoRA bias for {key!r}: the model has no base bias parameter "
                                 f"{bias_key!r}. Use routed LoRA for a bias-less base layer.")
            prev = bias_owner.setdefault(param_tensor_id(bias), key)
            if prev != key:
                raise ValueError(f"LoRA targets {prev!r} and {key!r} resolve to the same tied base-bias backing. "
                                 "Apply only one logical target for a tied bias.")
        ops.append(_MergeOp(weight, bias, transform))
    return ops
