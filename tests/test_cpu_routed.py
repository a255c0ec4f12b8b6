"""Routed-LoRA residual: the oracle pinned on the CPU, and the host API's checks.

The oracle restates _routed_residual (P/lora.py:801-829):
``out = y + sum_i (((x @ a.T) * s) @ b.T + bias * s)`` with every op's result
in the output dtype.  It is pinned by
  * exact cases: small-integer inputs, where every sum is exact, equal the
    closed form computed in float64;
  * the reference's own expression run by torch's CPU bf16/fp16 kernels
    (fp32 accumulation, a different summation order): equal except for rare
    one-ulp differences where a sum sits at a rounding boundary.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

import oracle as O
from helpers import bf16_np
from piper_offload_amd import install_routed_residual_hook, routed_residual
from piper_offload_amd.routed import RoutedFactor


def _bits(t: torch.Tensor) -> np.ndarray:
    return bf16_np(t) if t.dtype is torch.bfloat16 else t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _torch_reference(x, y, factors):  # the reference's expression (P/lora.py:812-828), on the CPU
    total = None
    for a, b, bias, s in factors:
        part = ((x @ a.T) * s) @ b.T
        if bias is not None:
            part = part + bias * s
        total = part if total is None else total + part
    return y + total


@pytest.mark.parametrize("dtype,dt", [(torch.bfloat16, O.DT_BF16), (torch.float16, O.DT_F16)])
def test_exact_small_integers(dtype, dt):
    g = torch.Generator().manual_seed(0)
    T, K, N = 5, 24, 12
    x = torch.randint(-2, 3, (T, K), generator=g).to(dtype)
    y = torch.randint(-8, 9, (T, N), generator=g).to(dtype)
    fs = [(torch.randint(-1, 2, (r, K), generator=g).to(dtype), torch.randint(-1, 2, (N, r), generator=g).to(dtype),
           bias, s) for r, bias, s in [(3, None, 0.5), (2, torch.randint(-3, 4, (N,), generator=g).to(dtype), 2.0)]]
    out = O.routed_residual(_bits(x), _bits(y), [(_bits(a), _bits(b), None if c is None else _bits(c), s)
                                                 for a, b, c, s in fs], dt=dt)
    xd, yd = x.double(), y.double()
    exact = yd.clone()
    for a, b, bias, s in fs:
        exact += ((xd @ a.double().T) * s) @ b.double().T + (0 if bias is None else bias.double() * s)
    assert np.array_equal(out, _bits(exact.to(dtype)))
    assert np.array_equal(out, _bits(_torch_reference(x, y, fs)))


@pytest.mark.parametrize("dtype,dt", [(torch.bfloat16, O.DT_BF16), (torch.float16, O.DT_F16)])
@pytest.mark.parametrize("ranks,bias", [([16], False), ([5, 32], True), ([64], False)])
def test_oracle_matches_torch_cpu_kernels(dtype, dt, ranks, bias):
    g = torch.Generator().manual_seed(sum(ranks))
    T, K, N = 9, 256, 96
    x = (torch.randn(T, K, generator=g)).to(dtype)
    y = (torch.randn(T, N, generator=g) * 0.5).to(dtype)
    fs = []
    for i, r in enumerate(ranks):
        fs.append(((torch.randn(r, K, generator=g) / r).to(dtype), (torch.randn(N, r, generator=g) * 0.05).to(dtype),
                   (torch.randn(N, generator=g) * 0.01).to(dtype) if bias else None, [0.75, -1.5][i % 2]))
    out = O.routed_residual(_bits(x), _bits(y), [(_bits(a), _bits(b), None if c is None else _bits(c), s)
                                                 for a, b, c, s in fs], dt=dt)
    ref = _torch_reference(x, y, fs)
    got = torch.from_numpy(out.view(np.int16)).view(dtype).float()
    diff = (got - ref.float()).abs()
    ulp = torch.finfo(dtype).eps * ref.float().abs().clamp_min(torch.finfo(dtype).tiny)
    # summation order only (measured: identical on these inputs)
    assert int((diff > 2 * ulp).sum()) == 0
    assert float((diff > 0).float().mean()) <= 0.01


def test_host_api_checks():
    with pytest.raises(ValueError, match="at least one factor"):
        install_routed_residual_hook(nn.Linear(4, 4), [])
    with pytest.raises(ValueError, match="at least one factor"):
        routed_residual(torch.zeros(1, 4), [], torch.zeros(1, 4))
    f = RoutedFactor(torch.zeros(2, 4), torch.zeros(4, 2), 1.0)
    with pytest.raises(ValueError, match="bfloat16 and float16"):
        routed_residual(torch.zeros(1, 4), [f], torch.zeros(1, 4))
    with pytest.raises(ValueError, match="one GPU"):
        routed_residual(torch.zeros(1, 4, dtype=torch.bfloat16), [f], torch.zeros(1, 4, dtype=torch.bfloat16))


def test_hook_removal_is_idempotent_and_restores_the_module():
    lin = nn.Linear(4, 3, bias=False)
    from piper_offload_amd.lora import ScaledLoRAFactor
    remove = install_routed_residual_hook(lin, [ScaledLoRAFactor(torch.zeros(2, 4), torch.zeros(3, 2), 1.0)])
    assert len(lin._forward_hooks) == 1 and not lin._forward_pre_hooks
    remove()
    remove()
    assert not lin._forward_hooks and not lin._forward_pre_hooks
    x = torch.randn(2, 4)
    assert torch.equal(lin(x), x @ lin.weight.T)
