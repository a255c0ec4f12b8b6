"""LoRA resources and the per-weight merge transform.

Mirrors the merge half of P/lora.py (P/ = the reference's src/piper_offload/):

* :class:`LoRAFactor` / :class:`ScaledLoRAFactor` -- host-backed A/B (+bias)
  factors, strength bound extrinsically (P/lora.py:116-245);
* :class:`LoRA` -- pairs ``*.lora_A.weight`` / ``*.lora_B.weight`` (+
  ``*.lora_B.bias``) keys of a flat state dict into pinned host factors
  (P/lora.py:264-311, 940-1095);
* :class:`LoRATransform` -- validates a target, stages B/A on the target
  device in its compute dtype, packs several LoRAs along the rank with the
  strength folded into A, derives the stochastic-rounding seed
  ``derive_seed(target_key, merge_index)`` and calls the adapter's
  ``merge_lora_`` (P/lora.py:314-724).

Routed LoRA (forward hooks) and DTensor shard slicing are outside this
build's hot path.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from types import MappingProxyType
from typing import Any

import torch
from torch import nn

from .registry import param_representation, select_adapter
from .seeding import derive_seed
from .stack import StackTarget

__all__ = ["LoRA", "LoRAFactor", "LoRATransform", "ScaledLoRAFactor"]


def _host_copy(t: torch.Tensor, dtype: torch.dtype | None, pin: bool) -> torch.Tensor:
    t = t.detach().to("cpu")
    if dtype is not None and t.dtype is not dtype:
        t = t.to(dtype)
    t = t.contiguous()
    if pin and torch.cuda.is_available():
        t = t.pin_memory()
    return t


@dataclass(slots=True, frozen=True)
class LoRAFactor:
    """Host tensors for one target: ``a`` (rank, in), ``b`` (out, rank), optional ``bias`` (out,)."""

    a: torch.Tensor
    b: torch.Tensor
    bias: torch.Tensor | None = None

    @property
    def cache_bytes(self) -> int:
        total = self.a.numel() * self.a.element_size() + self.b.numel() * self.b.element_size()
        if self.bias is not None:
            total += self.bias.numel() * self.bias.element_size()
        return total

    def scaled(self, strength: float, staged: tuple | None = None) -> ScaledLoRAFactor:
        return ScaledLoRAFactor(self.a, self.b, strength, self.bias, staged)


@dataclass(slots=True, frozen=True)
class ScaledLoRAFactor:
    """Host factors bound to an application ``strength``; contributes ``strength * (b @ a)``."""

    a: torch.Tensor
    b: torch.Tensor
    strength: float
    bias: torch.Tensor | None = None
    # (a, b) already on a GPU, same values and dtype as the host tensors: the
    # staging then copies nothing (see LoRA.stage_on)
    staged: tuple[torch.Tensor, torch.Tensor] | None = None

    def __post_init__(self) -> None:
        if self.a.ndim != 2 or self.b.ndim != 2 or self.a.shape[0] != self.b.shape[1]:
            raise ValueError(
                f"LoRA factor shape mismatch: A shape is {tuple(self.a.shape)}, B shape is {tuple(self.b.shape)}."
            )
        if self.bias is not None and (self.bias.ndim != 1 or self.bias.shape[0] != self.b.shape[0]):
            raise ValueError(
                f"LoRA bias shape mismatch: bias shape is {tuple(self.bias.shape)}, B shape is "
                f"{tuple(self.b.shape)}. Expected bias=(out_dim,)."
            )

    @classmethod
    def from_tensors(cls, a: torch.Tensor, b: torch.Tensor, strength: float,
                     bias: torch.Tensor | None = None) -> ScaledLoRAFactor:
        return cls(_host_copy(a, None, True), _host_copy(b, None, True), strength,
                   None if bias is None else _host_copy(bias, None, True))

    @property
    def rank(self) -> int:
        return self.a.shape[0]

    @property
    def produced_shape(self) -> tuple[int, int]:
        return (self.b.shape[0], self.a.shape[1])


class LoRA:
    """Reusable immutable host-backed LoRA resource (P/lora.py:224-311).

    ``from_state_dict`` with pinned host backing packs every factor into one
    pinned arena (each tensor 256-byte aligned), so :meth:`stage_on` moves all
    of a LoRA's factors to a GPU with one copy.
    """

    def __init__(self, targets: Mapping[str, LoRAFactor], *, arena: torch.Tensor | None = None) -> None:
        self._targets = MappingProxyType(dict(targets))
        self._cache_bytes = sum(f.cache_bytes for f in self._targets.values())
        self._arena = arena

    def stage_on(self, device: torch.device) -> _DeviceArena | None:
        """The whole arena on ``device`` after one asynchronous copy, or None without an arena."""
        if self._arena is None or device.type != "cuda":
            return None
        return _DeviceArena(self._arena, self._arena.to(device, non_blocking=True))

    @classmethod
    def from_state_dict(cls, state_dict: dict[str, torch.Tensor], *, dtype: torch.dtype | None = None,
                        host_backing: str = "pinned") -> LoRA:
        if host_backing not in ("pinned", "adopt"):
            raise ValueError(f"host_backing must be 'pinned' or 'adopt', got {host_backing!r}")
        if dtype is not None and not dtype.is_floating_point:
            raise ValueError(f"LoRA dtype must be floating-point, got {dtype}.")
        a_t, b_t, bias_t = _split_factor_tensors(state_dict)
        if not a_t and not b_t:
            raise ValueError("LoRA state_dict contains no factor pairs")
        a_only, b_only = set(a_t) - set(b_t), set(b_t) - set(a_t)
        if a_only or b_only:
            raise ValueError(
                f"Unpaired LoRA factors: A-only={sorted(a_only)}, B-only={sorted(b_only)}. Each target needs both "
                ".lora_A.weight and .lora_B.weight."
            )
        bias_only = set(bias_t) - set(a_t)
        if bias_only:
            raise ValueError(f"Unpaired LoRA biases: {sorted(bias_only)}. Each .lora_B.bias must accompany a "
                             "complete .lora_A.weight / .lora_B.weight pair.")
        targets: dict[str, LoRAFactor] = {}
        pin = host_backing == "pinned"
        for base, a in a_t.items():
            b, bias = b_t[base], bias_t.get(base)
            _validate_factor_pair(f"{base}.weight", a, b, bias)
            if host_backing == "adopt" and dtype is not None and (a.dtype is not dtype or b.dtype is not dtype):
                raise ValueError("adopted LoRA host backing cannot convert factor dtype without copying.")
        if not pin:
            return cls({f"{base}.weight": LoRAFactor(a, b_t[base], bias_t.get(base)) for base, a in a_t.items()})
        # one pinned arena holds every factor (P/lora.py:940-975 pins each tensor separately)
        items = [(base, role, t.detach()) for base, a in a_t.items()
                 for role, t in (("a", a), ("b", b_t[base]), ("bias", bias_t.get(base))) if t is not None]
        sizes = [t.numel() * (dtype.itemsize if dtype is not None else t.element_size()) for _b, _r, t in items]
        offsets, total = [], 0
        for n in sizes:
            offsets.append(total)
            total += (n + 255) // 256 * 256
        arena = torch.empty(max(total, 256), dtype=torch.uint8, pin_memory=torch.cuda.is_available())
        placed: dict[tuple[str, str], torch.Tensor] = {}
        for (base, role, t), off, n in zip(items, offsets, sizes):
            dt = dtype if dtype is not None else t.dtype
            view = arena[off:off + n].view(dt).view(t.shape)
            view.copy_(t.to("cpu"))
            placed[(base, role)] = view
        for base in a_t:
            targets[f"{base}.weight"] = LoRAFactor(placed[(base, "a")], placed[(base, "b")], placed.get((base, "bias")))
        return cls(targets, arena=arena)

    @property
    def targets(self) -> Mapping[str, LoRAFactor]:
        return self._targets

    @property
    def cache_bytes(self) -> int:
        return self._cache_bytes


class _DeviceArena:
    """A LoRA's host arena and its copy on one GPU: device views of host factor tensors."""

    __slots__ = ("dev", "host")

    def __init__(self, host: torch.Tensor, dev: torch.Tensor) -> None:
        self.host, self.dev = host, dev

    def view(self, t: torch.Tensor) -> torch.Tensor | None:
        """The device tensor holding ``t``'s values, or None when ``t`` is not in the arena."""
        off = t.data_ptr() - self.host.data_ptr()
        n = t.numel() * t.element_size()
        if not t.is_contiguous() or off < 0 or off + n > self.host.numel():
            return None
        return self.dev[off:off + n].view(t.dtype).view(t.shape)


@dataclass(slots=True, frozen=True)
class _WeightPlan:
    adapter: Any
    staging_shape: tuple[int, ...]
    compute_dtype: torch.dtype


class LoRATransform:
    """LoRA factors applied to one base weight and optional base bias (P/lora.py:314-724)."""

    __slots__ = ("_factors", "_merge_index", "_staged", "_stochastic_rounding", "_target_key", "_weight_plan")

    def __init__(self, factors: list[ScaledLoRAFactor], *, stochastic_rounding: bool = False,
                 target_key: str = "") -> None:
        if stochastic_rounding and not target_key:
            raise ValueError("Stochastic LoRATransform requires a non-empty target_key.")
        self._factors = factors
        self._stochastic_rounding = stochastic_rounding
        self._target_key = target_key
        self._merge_index = 0
        self._weight_plan: _WeightPlan | None = None
        # staged (B, A, strength) per (device, dtype, shape), valid while the
        # host factors are unmodified (their in-place version counters)
        self._staged: dict[tuple, tuple] = {}

    @property
    def merge_index(self) -> int:
        return self._merge_index

    def _rounding_seed(self) -> int | None:
        if not self._stochastic_rounding:
            return None
        return derive_seed(self._target_key, self._merge_index)

    @property
    def has_bias(self) -> bool:
        return any(f.bias is not None for f in self._factors)

    # -- validation -------------------------------------------------------
    def validate_target(self, weight: nn.Parameter | torch.Tensor, bias: nn.Parameter | None = None) -> None:
        self._weight_plan = None
        plan = self._build_weight_plan(weight)
        if self.has_bias:
            if bias is None:
                raise ValueError("LoRA transform contains a bias but no base bias target was provided.")
            self.validate_bias_target(bias)
        self._weight_plan = plan

    def validate_weight_target(self, param: nn.Parameter | torch.Tensor) -> None:
        self._weight_plan = None
        self._weight_plan = self._build_weight_plan(param)

    def _build_weight_plan(self, param: torch.Tensor) -> _WeightPlan:
        data = param_representation(param)
        try:
            adapter = select_adapter(data)
        except NotImplementedError as exc:
            raise ValueError(
                f"Tensor type {type(data).__name__} has no registered tensor adapter. "
                "Merge requires a tensor adapter with LoRA merge support."
            ) from exc
        if not callable(getattr(adapter, "merge_lora_", None)):
            raise ValueError(f"{type(adapter).__name__} does not support LoRA merge. Use routed LoRA for this tensor type.")
        compute_dtype = adapter.compute_dtype(data)
        if not compute_dtype.is_floating_point:
            raise ValueError(f"LoRA merge requires a floating-point compute dtype, got {compute_dtype}.")
        shape = tuple(adapter.logical_shape(data))
        for f in self._factors:
            if f.produced_shape != shape:
                raise ValueError(f"LoRA factor shape mismatch: B@A produces {f.produced_shape}, target shape is {shape}.")
        for f in self._factors:
            if type(f.a) is not torch.Tensor or type(f.b) is not torch.Tensor or f.a.device.type != "cpu" \
                    or f.b.device.type != "cpu":
                raise ValueError("LoRA merge requires plain CPU torch.Tensor factors; wrapped factor "
                                 "representations are unsupported.")
        validate = getattr(adapter, "validate_lora_merge", None)
        if callable(validate):
            b, a, strength, prepared = self._stage(data, adapter, shape, compute_dtype)
            hook = getattr(adapter, "validate_prepared_lora_merge", None) if prepared else validate
            hook(data, b, a, strength, rounding_seed=self._rounding_seed())
        return _WeightPlan(adapter, shape, compute_dtype)

    def validate_bias_target(self, param: torch.Tensor) -> None:
        if not self.has_bias:
            raise ValueError("LoRA bias merge requires at least one bias")
        target = param_representation(param)
        if type(target) is not torch.Tensor:
            raise ValueError(f"LoRA bias merge requires a plain dense base bias; got {type(target).__name__}.")
        if not target.is_floating_point():
            raise ValueError(f"LoRA bias merge requires a floating-point base bias; got {target.dtype}.")
        if target.dim() != 1:
            raise ValueError(f"LoRA bias merge requires a rank-one base bias; got shape {tuple(target.shape)}.")
        for f in self._factors:
            if f.bias is not None and tuple(f.bias.shape) != tuple(target.shape):
                raise ValueError(f"LoRA bias shape mismatch: adapter bias shape is {tuple(f.bias.shape)}, "
                                 f"base bias shape is {tuple(target.shape)}.")

    # -- application ------------------------------------------------------
    def apply(self, weight: nn.Parameter | torch.Tensor, bias: nn.Parameter | None = None) -> None:
        if self.has_bias and bias is None:
            raise ValueError("LoRA transform contains a bias but no base bias target was provided.")
        self.apply_weight(weight)
        if self.has_bias and bias is not None:
            self.apply_bias(bias)

    def apply_weight(self, param: nn.Parameter | torch.Tensor) -> None:
        plan = self._weight_plan
        if plan is None:
            raise RuntimeError("LoRA weight target must be validated before application.")
        data = param_representation(param)
        seed = self._rounding_seed()
        b, a, strength, prepared = self._stage(data, plan.adapter, plan.staging_shape, plan.compute_dtype)
        if prepared:
            plan.adapter.merge_prepared_lora_(data, b, a, strength, rounding_seed=seed)
        else:
            plan.adapter.merge_lora_(data, b, a, strength, rounding_seed=seed)
        self._merge_index += 1

    def stack_target(self, param: nn.Parameter | torch.Tensor) -> tuple[tuple, StackTarget] | None:
        """This weight's merge as one target of a grouped launch, with its group key, or None.

        Only weights whose adapter names a grouped kernel (``stack_key``) and
        whose factors need no adapter-specific staging qualify; the grouped
        kernels give the same bytes as :meth:`apply_weight` with the same
        seed.  The caller merges the group and then calls :meth:`advance`.
        """
        plan = self._weight_plan
        if plan is None:
            raise RuntimeError("LoRA weight target must be validated before application.")
        key_of = getattr(plan.adapter, "stack_key", None)
        if not callable(key_of):
            return None
        data = param_representation(param)
        key = key_of(data)
        if key is None:
            return None
        b, a, strength, prepared = self._stage(data, plan.adapter, plan.staging_shape, plan.compute_dtype)
        rank = a.shape[0]
        if prepared or a.dtype not in (torch.bfloat16, torch.float16) or not 0 < rank <= 64:
            return None
        bucket = 16 if rank <= 16 else 32 if rank <= 32 else 64  # one rank padding per launch
        seed = self._rounding_seed()
        return ((*key, a.dtype, bucket, self._stochastic_rounding),
                StackTarget(data, b, a, strength, 0 if seed is None else seed))

    def advance(self) -> None:
        """Count one merge applied outside :meth:`apply_weight` (the next merge's seed index)."""
        self._merge_index += 1

    def apply_bias(self, param: torch.Tensor) -> None:
        target = param_representation(param)
        delta = torch.zeros_like(target)
        for f in self._factors:
            if f.bias is not None:
                delta.add_(f.bias.to(device=target.device, dtype=target.dtype, non_blocking=True), alpha=f.strength)
        target.add_(delta)

    # -- staging (P/lora.py:595-724) ------------------------------------------
    def staged_update(self, data: torch.Tensor, compute_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor, float]:
        """Public form of the ordinary staging: (B, A, strength) on ``data``'s device."""
        shape = (self._factors[0].b.shape[0], self._factors[0].a.shape[1])
        return self._stage_single_or_packed(data, shape, compute_dtype)

    def _stage(self, data: torch.Tensor, adapter: Any, shape: tuple[int, ...],  # noqa: ANN401
               compute_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor, float, bool]:
        stage = getattr(adapter, "stage_lora_factors", None)
        if callable(stage):
            prepared = stage(data, tuple((f.strength, f.a, f.b) for f in self._factors), logical_shape=shape,
                             compute_dtype=compute_dtype)
            if prepared is not None:
                b, a, s = prepared
                return b, a, s, True
        b, a, s = self._stage_single_or_packed(data, shape, compute_dtype)
        return b, a, s, False

    def _stage_single_or_packed(self, data: torch.Tensor, shape: tuple[int, ...],
                                compute_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor, float]:
        """(B, A, strength) on ``data``'s device in ``compute_dtype`` (P/lora.py:595-626, 684-724).

        The reference stages the factors on every validate and every apply.
        Here they land once, straight from the (pinned) host factors, in one
        device buffer holding A then B, and later validates and applies
        reuse it until a host factor is modified in place.  Several factors
        are packed along the rank with each A slice scaled by its strength in
        ``compute_dtype`` on the device, as the reference does.
        """
        device = data.device
        key = (device, compute_dtype, tuple(shape))
        versions = tuple(v for f in self._factors for v in (f.a._version, f.b._version))
        hit = self._staged.get(key)
        if hit is not None and hit[0] == versions:
            return hit[1], hit[2], hit[3]
        factors = self._factors
        total = sum(f.a.shape[0] for f in factors)
        rows, cols = shape[0], shape[1]
        def src(f: ScaledLoRAFactor) -> tuple[torch.Tensor, torch.Tensor]:
            # the GPU copy made for this merge when there is one, else the host tensors
            if f.staged is not None and f.staged[0].device == device:
                return f.staged
            return f.a, f.b

        if len(factors) == 1 and factors[0].staged is not None and factors[0].staged[0].device == device \
                and factors[0].a.dtype is compute_dtype and factors[0].b.dtype is compute_dtype:
            b, a = factors[0].staged[1], factors[0].staged[0]  # already there, in the compute dtype
            self._staged[key] = (versions, b, a, factors[0].strength)
            return b, a, factors[0].strength
        buf = torch.empty(total * cols + rows * total, dtype=compute_dtype, device=device)
        a = buf[: total * cols].view(total, cols)
        b = buf[total * cols:].view(rows, total)
        if len(factors) == 1:
            f = factors[0]
            fa, fb = src(f)
            a.copy_(fa, non_blocking=True)
            b.copy_(fb, non_blocking=True)
            strength = f.strength
        else:
            off = 0
            for f in factors:
                nxt = off + f.a.shape[0]
                fa, fb = src(f)
                a[off:nxt].copy_(fa, non_blocking=True)
                b[:, off:nxt].copy_(fb, non_blocking=True)
                if f.strength != 1.0:
                    a[off:nxt].mul_(f.strength)
                off = nxt
            strength = 1.0
        self._staged[key] = (versions, b, a, strength)
        return b, a, strength


def _split_factor_tensors(state_dict: dict[str, torch.Tensor]
                          ) -> tuple[dict[str, torch.Tensor], dict[str, torch.Tensor], dict[str, torch.Tensor]]:
    a_t: dict[str, torch.Tensor] = {}
    b_t: dict[str, torch.Tensor] = {}
    bias_t: dict[str, torch.Tensor] = {}
    for key, t in state_dict.items():
        if key.endswith(".lora_A.weight"):
            a_t[key[: -len(".lora_A.weight")]] = t
        elif key.endswith(".lora_B.weight"):
            b_t[key[: -len(".lora_B.weight")]] = t
        elif key.endswith(".lora_B.bias"):
            bias_t[key[: -len(".lora_B.bias")]] = t
    return a_t, b_t, bias_t


def _validate_factor_pair(key: str, a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None) -> None:
    if not a.is_floating_point() or not b.is_floating_point():
        raise ValueError(f"LoRA factors for {key!r}: must be floating-point; got A.dtype={a.dtype}, B.dtype={b.dtype}.")
    if a.dim() != 2 or b.dim() != 2 or a.shape[0] != b.shape[1]:
        raise ValueError(
            f"LoRA factor shape mismatch for {key!r}: A.shape={tuple(a.shape)}, B.shape={tuple(b.shape)}. "
            "Expected A=(rank, in_dim), B=(out_dim, rank) with A.shape[0] == B.shape[1]."
        )
    if bias is not None:
        if not bias.is_floating_point():
            raise ValueError(f"LoRA bias for {key!r} must be floating-point; got dtype={bias.dtype}.")
        if bias.dim() != 1 or bias.shape[0] != b.shape[0]:
            raise ValueError(f"LoRA bias shape mismatch for {key!r}: bias.shape={tuple(bias.shape)}, "
                             f"B.shape={tuple(b.shape)}. Expected bias=(out_dim,) with bias.shape[0] == B.shape[0].")


def factors_for(loras: Sequence[tuple[LoRA, float]], target_key: str) -> list[ScaledLoRAFactor]:
    return [lora.targets[target_key].scaled(s) for lora, s in loras if target_key in lora.targets]
