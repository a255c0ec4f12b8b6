"""Permanent LoRA merge into model weights (interface and semantics of P/merge.py:54-214).

``merge_lora(model, [(lora, strength), ...], stochastic_rounding=True)``
returns the number of distinct parameters it modified.  A call runs in four
phases, and nothing is written before the last one:

1. the request: every LoRA object at most once, exact-zero strengths dropped,
   every target key a parameter name of the model;
2. the plan (``_Planner``): one ``_Target`` per distinct weight tensor
   (adapter tensor identity), collecting every scaled factor aimed at it.  A
   tensor reached through two different names (a tied weight) is rejected,
   and so is a base bias claimed by two targets.  Each LoRA's factors are
   copied to each GPU once and targets use device views of that copy;
3. the preflight: every target's transform validates its weight and bias;
4. the apply: weights that a grouped kernel merges (per-row INT8, NVFP4) go
   through one grouped launch per compatible group, the rest one by one.

Each weight gets its own stochastic-rounding seed
``derive_seed(target_key, merge_index)``.
"""

from __future__ import annotations

import logging
from collections.abc import Sequence
from dataclasses import dataclass, field
from typing import Any

import torch
from torch import nn

from .lora import LoRA, LoRATransform, ScaledLoRAFactor
from .registry import param_representation, param_tensor_id
from .stack import StackTarget, merge_once

logger = logging.getLogger(__name__)

__all__ = ["merge_lora"]


@dataclass(slots=True)
class _Target:
    """One distinct weight tensor: the first key that named it, its parameter, the scaled factors
    aimed at it in request order, and (once planned) its transform and base bias."""

    key: str
    weight: nn.Parameter
    factors: list[ScaledLoRAFactor] = field(default_factory=list)
    transform: LoRATransform | None = None
    bias: nn.Parameter | None = None


class _Planner:
    def __init__(self, params: dict[str, nn.Parameter], stochastic: bool) -> None:
        self.params = params
        self.stochastic = stochastic
        self.targets: dict[tuple[Any, ...], _Target] = {}  # by tensor identity, in first-seen order
        self.bias_claims: dict[tuple[Any, ...], str] = {}  # base-bias identity -> claiming target key

    def add(self, lora: LoRA, strength: float) -> None:
        copies: dict[torch.device, Any] = {}  # this LoRA's factors, one copy per GPU
        for key, factor in lora.targets.items():
            weight = self.params[key]
            target = self._target(key, weight)
            target.factors.append(factor.scaled(strength, _device_views(lora, factor, weight, copies)))

    def _target(self, key: str, weight: nn.Parameter) -> _Target:
        target = self.targets.setdefault(param_tensor_id(weight), _Target(key, weight))
        if target.key != key:
            raise ValueError(
                f"LoRA targets {target.key!r} and {key!r} resolve to the same tied parameter backing. Apply only one "
                "name for a tied weight in a single merge_lora() call; otherwise the same base weight would receive "
                "multiple logical updates."
            )
        return target

    def finish(self) -> list[_Target]:
        for target in self.targets.values():
            target.transform = LoRATransform(target.factors, stochastic_rounding=self.stochastic,
                                             target_key=target.key)
            if target.transform.has_bias:
                target.bias = self._claim_bias(target.key)
        return list(self.targets.values())

    def _claim_bias(self, key: str) -> nn.Parameter:
        parent, _, _ = key.rpartition(".")
        bias_key = f"{parent}.bias" if parent else "bias"
        bias = self.params.get(bias_key)
        if bias is None:
            raise ValueError(f"Cannot merge legacy LoRA bias for {key!r}: the model has no base bias parameter "
                             f"{bias_key!r}. Use routed LoRA for a bias-less base layer.")
        owner = self.bias_claims.setdefault(param_tensor_id(bias), key)
        if owner != key:
            raise ValueError(f"LoRA targets {owner!r} and {key!r} resolve to the same tied base-bias backing. "
                             "Apply only one logical target for a tied bias.")
        return bias


def _device_views(lora: LoRA, factor: Any, weight: nn.Parameter,  # noqa: ANN401
                  copies: dict[torch.device, Any]) -> tuple[torch.Tensor, torch.Tensor] | None:
    """(A, B) as views of this LoRA's one copy on the weight's GPU, or None (CPU weight, no copy)."""
    device = param_representation(weight).device
    if device.type != "cuda":
        return None
    if device not in copies:
        copies[device] = lora.stage_on(device)
    arena = copies[device]
    if arena is None:
        return None
    a, b = arena.view(factor.a), arena.view(factor.b)
    return None if a is None or b is None else (a, b)


def _active(loras: Sequence[tuple[LoRA, float]]) -> list[tuple[LoRA, float]]:
    seen: set[int] = set()
    for lora, _strength in loras:
        if id(lora) in seen:
            raise ValueError("merge_lora() does not accept the same LoRA instance more than once")
        seen.add(id(lora))
    if any(not isinstance(lora, LoRA) for lora, _strength in loras):
        raise TypeError("merge_lora() expects LoRA instances")
    return [(lora, strength) for lora, strength in loras if strength != 0.0]


def merge_lora(model: nn.Module, loras: Sequence[tuple[LoRA, float]], *, stochastic_rounding: bool = True) -> int:
    """Merge LoRAs into ``model`` in place; returns the number of distinct parameters modified."""
    active = _active(loras)
    params = dict(model.named_parameters(remove_duplicate=False))
    unknown = sorted({key for lora, _s in active for key in lora.targets} - params.keys())
    if unknown:
        raise ValueError(
            f"LoRA targets are not parameters in the model: {unknown}. LoRA target keys must match the model's "
            f"parameter names exactly. Sample model parameter keys: {sorted(params)[:3]} ..."
        )
    planner = _Planner(params, stochastic_rounding)
    for lora, strength in active:
        planner.add(lora, strength)
    targets = planner.finish()
    for target in targets:  # preflight: everything is checked before anything is written
        target.transform.validate_target(target.weight, target.bias)
    _apply(targets)
    touched = {param_tensor_id(t.weight) for t in targets}
    touched |= {param_tensor_id(t.bias) for t in targets if t.bias is not None}
    logger.info("merge_lora: merged %d unique parameters (%d weights, %d biases) from %d LoRA targets",
                len(touched), len(targets), sum(t.bias is not None for t in targets),
                sum(len(lora.targets) for lora, _s in active))
    return len(touched)


def _apply(targets: list[_Target]) -> None:
    """Write every validated target.  Weights that a grouped kernel can merge go
    through one grouped launch per compatible group (same format, device, scale
    layout, factor dtype, rank bucket and rounding); a group of one, every other
    weight and every bias use the target's own adapter call.  Targets are
    distinct tensors, so the order changes no result, and each grouped weight
    keeps its own seed."""
    groups: dict[tuple, list[tuple[_Target, StackTarget]]] = {}
    alone: list[_Target] = []
    for target in targets:
        grouped = target.transform.stack_target(target.weight)
        if grouped is None:
            alone.append(target)
        else:
            groups.setdefault(grouped[0], []).append((target, grouped[1]))
    for (kind, *rest), members in groups.items():
        if len(members) == 1:  # one tensor: its single-target launch is the tuned path
            alone.append(members[0][0])
            continue
        merge_once([st for _t, st in members], kind, stochastic=rest[-1])
        for target, _st in members:
            target.transform.advance()
            if target.bias is not None:
                target.transform.apply_bias(target.bias)
    for target in alone:
        target.transform.apply(target.weight, target.bias)
