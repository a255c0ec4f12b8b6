"""TorchAO INT8 ``act_pre_scale`` in the merge path (T/test_int8_adapter.py:455-560, P/int8_adapter.py:59-141).

TorchAO multiplies activations by ``act_pre_scale`` before the weight matmul,
so a permanent merge must add ``B @ ((strength * A) / p)`` to the stored
weight.  Only a scalar or one value per input feature (singleton leading
dimensions) is accepted; anything else, and non-finite, zero or integer
scales, raise ``ValueError`` before any storage is touched.  All of this
happens on the host, before the HIP kernel, so it is tested on the CPU; the
merged codes are checked against the oracle on the GPU
(tests/test_gpu_int8.py).
"""

from __future__ import annotations

import pytest
import torch

from helpers import int8_initial, normal_bf16
from piper_offload_amd import Int8Adapter, Int8Weight

ROWS, COLS, RANK = 8, 16, 3


def _weight(pre_scale: torch.Tensor | None) -> Int8Weight:
    q, s = int8_initial(normal_bf16((ROWS, COLS), 0.02, 3))
    return Int8Weight(q, s, (1, COLS), torch.bfloat16, act_pre_scale=pre_scale)


@pytest.mark.parametrize("shape", [(), (1,), (16,), (1, 16), (1, 1, 16)])
def test_scalar_and_per_input_pre_scales_are_accepted(shape: tuple[int, ...]) -> None:
    qt = _weight(torch.full(shape, 0.75))
    Int8Adapter.validate_lora_merge(qt, torch.ones(ROWS, 1), torch.ones(1, COLS), 1.0)
    stored, strength = Int8Adapter._stored_coordinates(qt, torch.ones(1, COLS, dtype=torch.bfloat16), 0.5)
    assert strength == 1.0
    assert stored.shape == (1, COLS) and stored.dtype is torch.bfloat16
    assert torch.equal(stored.float(), torch.full((1, COLS), 0.5 / 0.75).to(torch.bfloat16).float())


@pytest.mark.parametrize(("kind", "match"), [("integer", "floating-point"),
                                             ("wrong-features", "scalar or one value per input feature"),
                                             ("batch-dependent", "scalar or one value per input feature"),
                                             ("zero", "non-zero"), ("nan", "finite"), ("infinite", "finite")])
def test_invalid_pre_scales_are_rejected_before_mutation(kind: str, match: str) -> None:
    if kind == "integer":
        pre = torch.ones(COLS, dtype=torch.int32)
    elif kind == "wrong-features":
        pre = torch.ones(COLS - 1)
    elif kind == "batch-dependent":
        pre = torch.ones(2, COLS)
    else:
        pre = torch.ones(COLS)
        pre[3] = {"zero": 0.0, "nan": float("nan"), "infinite": float("inf")}[kind]
    qt = _weight(pre)
    before = (qt.qdata.clone(), qt.scale.clone())
    b, a = torch.randn(ROWS, RANK), torch.randn(RANK, COLS)
    with pytest.raises(ValueError, match=match):
        Int8Adapter.validate_lora_merge(qt, b, a, 0.5)
    with pytest.raises(ValueError, match=match):
        Int8Adapter.merge_lora_(qt, b, a, 0.5)
    with pytest.raises(ValueError, match=match):
        Int8Adapter.stage_lora_factors(qt, ((0.5, a, b),), logical_shape=(ROWS, COLS), compute_dtype=torch.bfloat16)
    assert torch.equal(qt.qdata, before[0]) and torch.equal(qt.scale, before[1])


@pytest.mark.parametrize(("pre_scale", "a_value", "strength"), [(1e-40, 1.0, 0.0), (1e-40, 1.0, 1e-40),
                                                                (1e30, 1e10, 1e30)])
def test_strength_is_folded_in_before_the_division(pre_scale: float, a_value: float, strength: float) -> None:
    # A / p alone overflows (or p * strength underflows); (strength * A) / p in
    # float64 stays finite, so validation passes and the stored factor is exact
    qt = _weight(torch.full((COLS,), pre_scale))
    a = torch.full((RANK, COLS), a_value)
    Int8Adapter.validate_lora_merge(qt, torch.randn(ROWS, RANK), a, strength)
    stored, unit = Int8Adapter._stored_coordinates(qt, a, strength)
    assert unit == 1.0
    want = torch.full((RANK, COLS), a_value, dtype=torch.float64).mul(strength).div(
        torch.tensor(pre_scale, dtype=torch.float32).double()).float()
    assert torch.equal(stored, want)
    assert torch.isfinite(stored).all()


def test_overflowing_stored_factors_are_rejected() -> None:
    qt = _weight(torch.full((COLS,), 1e-40))
    with pytest.raises(ValueError, match="stored-coordinate LoRA factors must be finite|non-finite stored-coordinate"):
        Int8Adapter.validate_lora_merge(qt, torch.ones(ROWS, RANK), torch.ones(RANK, COLS), 1.0)


def test_staged_factors_fold_every_strength_before_the_division() -> None:
    pre = torch.linspace(0.5, 2.0, COLS)
    qt = _weight(pre)
    a1, b1 = torch.randn(2, COLS), torch.randn(ROWS, 2)
    a2, b2 = torch.randn(3, COLS), torch.randn(ROWS, 3)
    b, a, strength = Int8Adapter.stage_lora_factors(qt, ((0.5, a1, b1), (-1.25, a2, b2)), logical_shape=(ROWS, COLS),
                                                    compute_dtype=torch.bfloat16)
    assert strength == 1.0
    want_a = torch.cat([a1.double() * 0.5 / pre.double(), a2.double() * -1.25 / pre.double()]).to(torch.bfloat16)
    assert torch.equal(a, want_a)
    assert torch.equal(b, torch.cat([b1, b2], dim=1).to(torch.bfloat16))
