"""Host-side merge orchestration on CPU models (P/merge.py:54-214,
P/lora.py:264-724), mirroring the reference's tests/test_merged_lora.py.

On CPU the reference merges plain weights with ``addmm_``
(P/tensor_adapters.py:686-696) -- config 1 of the benchmark is exactly that --
so these tests run the real orchestration end to end without a GPU; the HIP
kernels are covered by the ``gpu`` tests.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from piper_offload_amd import LoRA, derive_seed, merge_lora
from piper_offload_amd.lora import LoRATransform, ScaledLoRAFactor
from piper_offload_amd.registry import register_adapter


def _lora(targets: dict[str, tuple[int, int]], rank: int, seed: int, *, bias: bool = False,
          dtype: torch.dtype = torch.float32) -> LoRA:
    g = torch.Generator().manual_seed(seed)
    sd = {}
    for name, (out_f, in_f) in targets.items():
        sd[f"{name}.lora_A.weight"] = (torch.randn(rank, in_f, generator=g) / rank).to(dtype)
        sd[f"{name}.lora_B.weight"] = (torch.randn(out_f, rank, generator=g) * 0.01).to(dtype)
        if bias:
            sd[f"{name}.lora_B.bias"] = (torch.randn(out_f, generator=g) * 0.1).to(dtype)
    return LoRA.from_state_dict(sd)


class Block(nn.Module):
    def __init__(self, dim: int, dtype: torch.dtype = torch.float32, bias: bool = False) -> None:
        super().__init__()
        self.attn = nn.Linear(dim, dim, bias=bias, dtype=dtype)
        self.mlp = nn.Linear(dim, 2 * dim, bias=bias, dtype=dtype)
        self.requires_grad_(False)


def test_config1_cpu_bf16_merge_equals_addmm() -> None:
    # CPU bf16 [4096, 4096], rank 16, strength 1.0
    m = nn.Module()
    m.proj = nn.Linear(4096, 4096, bias=False, dtype=torch.bfloat16)
    m.requires_grad_(False)
    lora = _lora({"proj": (4096, 4096)}, 16, 0, dtype=torch.bfloat16)
    expected = m.proj.weight.detach().clone()
    f = lora.targets["proj.weight"]
    expected.addmm_(f.b, f.a, alpha=1.0)
    assert merge_lora(m, [(lora, 1.0)]) == 1
    assert torch.equal(m.proj.weight, expected)


def test_returns_unique_parameter_count_and_merges_every_target() -> None:
    m = Block(16)
    lora = _lora({"attn": (16, 16), "mlp": (32, 16)}, 4, 1)
    before = {k: v.detach().clone() for k, v in m.named_parameters()}
    assert merge_lora(m, [(lora, 0.5)]) == 2
    for name in ("attn", "mlp"):
        f = lora.targets[f"{name}.weight"]
        want = before[f"{name}.weight"].clone().addmm_(f.b, f.a, alpha=0.5)
        assert torch.equal(getattr(m, name).weight, want)


def test_zero_strength_is_skipped() -> None:
    m = Block(16)
    before = m.attn.weight.detach().clone()
    assert merge_lora(m, [(_lora({"attn": (16, 16)}, 4, 2), 0.0)]) == 0
    assert torch.equal(m.attn.weight, before)


def test_rejects_duplicate_instances_and_non_loras() -> None:
    m = Block(16)
    lora = _lora({"attn": (16, 16)}, 4, 3)
    with pytest.raises(ValueError, match="same LoRA instance"):
        merge_lora(m, [(lora, 1.0), (lora, 0.5)])
    with pytest.raises(TypeError, match="LoRA instances"):
        merge_lora(m, [("not a lora", 1.0)])  # type: ignore[list-item]


def test_rejects_unknown_targets_without_mutation() -> None:
    m = Block(16)
    before = {k: v.detach().clone() for k, v in m.named_parameters()}
    lora = _lora({"missing.attn": (16, 16), "attn": (16, 16)}, 4, 4)
    with pytest.raises(ValueError, match="not parameters in the model"):
        merge_lora(m, [(lora, 1.0)])
    for k, v in m.named_parameters():
        assert torch.equal(v, before[k])


def test_tied_aliases_are_rejected_before_mutation() -> None:
    m = nn.Module()
    m.embed = nn.Linear(16, 16, bias=False)
    m.head = nn.Linear(16, 16, bias=False)
    m.head.weight = m.embed.weight
    m.requires_grad_(False)
    before = m.embed.weight.detach().clone()
    lora = _lora({"embed": (16, 16), "head": (16, 16)}, 4, 5)
    with pytest.raises(ValueError, match="same tied parameter backing"):
        merge_lora(m, [(lora, 1.0)])
    assert torch.equal(m.embed.weight, before)


def test_multiple_loras_on_one_target_pack_along_rank() -> None:
    m = Block(8)
    base = m.attn.weight.detach().clone()
    l1, l2 = _lora({"attn": (8, 8)}, 2, 6), _lora({"attn": (8, 8)}, 3, 7)
    assert merge_lora(m, [(l1, 0.5), (l2, -1.25)]) == 1
    f1, f2 = l1.targets["attn.weight"], l2.targets["attn.weight"]
    a = torch.cat([f1.a * 0.5, f2.a * -1.25])
    b = torch.cat([f1.b, f2.b], dim=1)
    assert torch.equal(m.attn.weight, base.clone().addmm_(b, a))


def test_bias_factors_merge_into_the_base_bias() -> None:
    m = Block(8, bias=True)
    bias_before = m.attn.bias.detach().clone()
    lora = _lora({"attn": (8, 8)}, 2, 8, bias=True)
    assert merge_lora(m, [(lora, 2.0)]) == 2  # weight + bias
    torch.testing.assert_close(m.attn.bias, bias_before + 2.0 * lora.targets["attn.weight"].bias)


def test_factor_shape_mismatch_is_reported() -> None:
    m = Block(16)
    lora = _lora({"attn": (16, 8)}, 4, 9)
    with pytest.raises(ValueError, match="B@A produces"):
        merge_lora(m, [(lora, 1.0)])


def test_state_dict_validation() -> None:
    with pytest.raises(ValueError, match="no factor pairs"):
        LoRA.from_state_dict({"x.weight": torch.zeros(2, 2)})
    with pytest.raises(ValueError, match="Unpaired"):
        LoRA.from_state_dict({"x.lora_A.weight": torch.zeros(2, 4)})
    with pytest.raises(ValueError, match="shape mismatch"):
        LoRA.from_state_dict({"x.lora_A.weight": torch.zeros(2, 4), "x.lora_B.weight": torch.zeros(4, 3)})
    with pytest.raises(ValueError, match="floating-point"):
        LoRA.from_state_dict({"x.lora_A.weight": torch.zeros(2, 4, dtype=torch.int32),
                              "x.lora_B.weight": torch.zeros(4, 2)})
    with pytest.raises(ValueError, match="Unpaired LoRA biases"):
        LoRA.from_state_dict({"x.lora_A.weight": torch.zeros(2, 4), "x.lora_B.weight": torch.zeros(4, 2),
                              "y.lora_B.bias": torch.zeros(4)})


class _Recorded(torch.Tensor):
    """A tensor type with its own adapter, recording the seeds the merge passes."""


class _RecordingAdapter:
    seeds: list[int | None] = []

    @staticmethod
    def matches(t: torch.Tensor) -> bool:
        return isinstance(t, _Recorded)

    @staticmethod
    def tensor_id(t: torch.Tensor) -> tuple:
        return ("recorded", id(t))

    @staticmethod
    def compute_dtype(t: torch.Tensor) -> torch.dtype:
        return torch.bfloat16

    @staticmethod
    def logical_shape(t: torch.Tensor) -> tuple[int, ...]:
        return tuple(t.shape)

    @classmethod
    def merge_lora_(cls, target: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                    rounding_seed: int | None = None) -> None:
        assert b.dtype is torch.bfloat16 and a.dtype is torch.bfloat16
        cls.seeds.append(rounding_seed)


def test_stochastic_seed_is_derived_per_target_and_merge_index() -> None:
    remove = register_adapter(_RecordingAdapter)
    try:
        _RecordingAdapter.seeds = []
        t = torch.Tensor._make_subclass(_Recorded, torch.zeros(8, 8), False)
        g = torch.Generator().manual_seed(10)
        f = ScaledLoRAFactor(torch.randn(2, 8, generator=g), torch.randn(8, 2, generator=g), 1.0)
        tr = LoRATransform([f], stochastic_rounding=True, target_key="layers.3.mlp.weight")
        tr.validate_weight_target(t)
        tr.apply_weight(t)
        tr.apply_weight(t)
        assert _RecordingAdapter.seeds == [derive_seed("layers.3.mlp.weight", 0),
                                           derive_seed("layers.3.mlp.weight", 1)]
        assert tr.merge_index == 2
        rtn = LoRATransform([f], stochastic_rounding=False, target_key="k")
        rtn.validate_weight_target(t)
        rtn.apply_weight(t)
        assert _RecordingAdapter.seeds[-1] is None
        with pytest.raises(ValueError, match="non-empty target_key"):
            LoRATransform([f], stochastic_rounding=True, target_key="")
        with pytest.raises(RuntimeError, match="validated before application"):
            LoRATransform([f], target_key="k").apply_weight(t)
    finally:
        remove()


def test_reload_pipeline_rejects_unpinned_weights() -> None:
    from piper_offload_amd.reload import HostInt8Target, ReloadMergePipeline

    t = HostInt8Target("w", torch.zeros(4, 8, dtype=torch.int8), torch.ones(4, 1), torch.zeros(4, 2),
                       torch.zeros(2, 8))
    with pytest.raises(ValueError, match="pinned host memory"):
        ReloadMergePipeline([[t]])
    with pytest.raises(ValueError, match="at least one target"):
        ReloadMergePipeline([[]])


def test_factor_staging_is_one_buffer_reused_until_a_factor_changes() -> None:
    # one host buffer holds A then B; validate and every apply reuse it, and an
    # in-place change of a host factor restages (P/lora.py:595-626 stages on each)
    g = torch.Generator().manual_seed(11)
    f = ScaledLoRAFactor(torch.randn(4, 24, generator=g), torch.randn(16, 4, generator=g), 0.75)
    tr = LoRATransform([f], target_key="w")
    data = torch.zeros(16, 24, dtype=torch.bfloat16)
    b, a, s = tr.staged_update(data, torch.bfloat16)
    assert s == 0.75 and b.dtype is torch.bfloat16 and a.dtype is torch.bfloat16
    assert torch.equal(a, f.a.to(torch.bfloat16)) and torch.equal(b, f.b.to(torch.bfloat16))
    assert a.is_contiguous() and b.is_contiguous()
    assert b.data_ptr() == a.data_ptr() + a.numel() * a.element_size()
    b2, a2, _ = tr.staged_update(data, torch.bfloat16)
    assert a2.data_ptr() == a.data_ptr() and b2.data_ptr() == b.data_ptr()
    f.a.mul_(2.0)
    b3, a3, _ = tr.staged_update(data, torch.bfloat16)
    assert torch.equal(a3, f.a.to(torch.bfloat16)) and torch.equal(b3, b)
    # another compute dtype is its own entry
    _b4, a4, _ = tr.staged_update(data, torch.float32)
    assert a4.dtype is torch.float32 and torch.equal(a4, f.a)


def test_packed_staging_folds_strength_into_a_in_the_compute_dtype() -> None:
    # k factors: concatenated along rank, each A slice times its strength in the
    # compute dtype, strength 1.0 (P/lora.py:684-724)
    g = torch.Generator().manual_seed(12)
    f1 = ScaledLoRAFactor(torch.randn(3, 40, generator=g), torch.randn(24, 3, generator=g), 0.3)
    f2 = ScaledLoRAFactor(torch.randn(5, 40, generator=g), torch.randn(24, 5, generator=g), -1.7)
    f3 = ScaledLoRAFactor(torch.randn(2, 40, generator=g), torch.randn(24, 2, generator=g), 1.0)
    tr = LoRATransform([f1, f2, f3], target_key="w")
    b, a, s = tr.staged_update(torch.zeros(24, 40, dtype=torch.bfloat16), torch.bfloat16)
    assert s == 1.0 and a.shape == (10, 40) and b.shape == (24, 10)
    want_a = torch.cat([f.a.to(torch.bfloat16) * f.strength if f.strength != 1.0 else f.a.to(torch.bfloat16)
                        for f in (f1, f2, f3)])
    assert want_a.dtype is torch.bfloat16
    assert torch.equal(a, want_a)
    assert torch.equal(b, torch.cat([f.b for f in (f1, f2, f3)], dim=1).to(torch.bfloat16))
    # folding in float32 first would round differently for some elements
    assert not torch.equal(a[3:8], (f2.a * f2.strength).to(torch.bfloat16))


def test_pinned_lora_factors_share_one_arena():
    # from_state_dict packs every factor into one host buffer (256-byte aligned),
    # so a merge stages a whole LoRA with one copy per GPU
    from piper_offload_amd.lora import _DeviceArena

    lora = _lora({"attn": (16, 24), "mlp": (32, 24)}, 4, 13, bias=True, dtype=torch.bfloat16)
    arena = lora._arena
    assert arena is not None and arena.dtype is torch.uint8
    base = arena.data_ptr()
    for f in lora.targets.values():
        for t in (f.a, f.b, f.bias):
            off = t.data_ptr() - base
            assert off % 256 == 0 and 0 <= off < arena.numel()
    assert lora.stage_on(torch.device("cpu")) is None  # GPUs only
    # a device arena maps every factor to the same values (a CPU copy stands in for the GPU one)
    dev = _DeviceArena(arena, arena.clone())
    for f in lora.targets.values():
        for t in (f.a, f.b, f.bias):
            v = dev.view(t)
            assert v is not None and v.dtype is t.dtype and torch.equal(v, t) and v.data_ptr() != t.data_ptr()
    assert dev.view(torch.zeros(4)) is None
    # the converted dtype is what the arena holds
    lora32 = _lora({"attn": (16, 24)}, 4, 14, dtype=torch.float32)
    f32 = LoRA.from_state_dict({"attn.lora_A.weight": lora32.targets["attn.weight"].a,
                                "attn.lora_B.weight": lora32.targets["attn.weight"].b}, dtype=torch.bfloat16)
    assert f32.targets["attn.weight"].a.dtype is torch.bfloat16
    assert torch.equal(f32.targets["attn.weight"].a, lora32.targets["attn.weight"].a.to(torch.bfloat16))


# ---- stack plans: items must not share buffers ---------------------------------
def _nv_cpu(rows: int, cols: int, pts: torch.Tensor | None = None, q: torch.Tensor | None = None):  # noqa: ANN202
    from piper_offload_amd import NVFP4Weight

    q = torch.zeros(rows, cols // 2, dtype=torch.uint8) if q is None else q
    s = torch.zeros(rows, cols // 16, dtype=torch.uint8).view(torch.float8_e4m3fn)
    return NVFP4Weight(q, s, pts, 16, torch.bfloat16, False)


@pytest.mark.parametrize("case", ["same_weight", "shared_global", "fused_view", "int8_same"])
def test_stack_plan_rejects_items_that_share_buffers(case: str) -> None:
    from piper_offload_amd import Int8Weight
    from piper_offload_amd.stack import StackPlan, StackTarget

    b = torch.zeros(32, 16, dtype=torch.bfloat16)
    a = torch.zeros(16, 64, dtype=torch.bfloat16)
    if case == "same_weight":
        w = _nv_cpu(32, 64, torch.ones(()))
        targets, kind = [StackTarget(w, b, a, 1.0), StackTarget(w, b, a, 1.0)], "nvfp4"
    elif case == "shared_global":
        g = torch.ones(())
        targets, kind = [StackTarget(_nv_cpu(32, 64, g), b, a, 1.0), StackTarget(_nv_cpu(32, 64, g), b, a, 1.0)], "nvfp4"
    elif case == "fused_view":
        fused = torch.zeros(64, 32, dtype=torch.uint8)  # two views over one fused q/k tensor, overlapping by a row
        targets = [StackTarget(_nv_cpu(32, 64, torch.ones(()), fused[:32]), b, a, 1.0),
                   StackTarget(_nv_cpu(32, 64, torch.ones(()), fused[31:63]), b, a, 1.0)]
        kind = "nvfp4"
    else:
        q = torch.zeros(32, 64, dtype=torch.int8)
        s = torch.ones(32, 1)
        w = Int8Weight(q, s, (1, 64), torch.bfloat16)
        targets, kind = [StackTarget(w, b, a, 1.0), StackTarget(Int8Weight(q, torch.ones(32, 1), (1, 64), torch.bfloat16),
                                                                 b, a, 1.0)], "int8"
    with pytest.raises(ValueError, match="must not share buffers"):
        StackPlan(targets, kind)


def test_stack_plan_overlap_check_passes_disjoint_views() -> None:
    # adjacent, non-overlapping views of one buffer are fine (the check stops at the ValueError stage on CPU)
    from piper_offload_amd.stack import StackTarget, _reject_shared_buffers

    fused = torch.zeros(64, 32, dtype=torch.uint8)
    b = torch.zeros(32, 16, dtype=torch.bfloat16)
    a = torch.zeros(16, 64, dtype=torch.bfloat16)
    _reject_shared_buffers([StackTarget(_nv_cpu(32, 64, torch.ones(()), fused[:32]), b, a, 1.0),
                            StackTarget(_nv_cpu(32, 64, torch.ones(()), fused[32:]), b, a, 1.0)])
