"""Routed-LoRA residual on the GPU (lm_routed_residual) vs the oracle and a torch fp32 reference.

Contract: out = dt(y + sum_i part_i) with the reference's roundings
(P/lora.py:801-829).  The MFMA sums x A^T and (x A^T s) B^T in a
hardware-defined order, so an intermediate can land one ulp away from the
oracle's at a rounding boundary.  The output must equal the oracle on all
but a small fraction of elements (ROUTED_MISMATCH), and differ by no more
than what one-ulp flips of the intermediates can cause: 2 ulps of the
output, one ulp of the residual, and for every rank r one ulp of p_r and of
p_r s carried through |b[n, r]| (the bf16 intermediate p = x A^T is coarse
when K is large, so one flip can move the residual by several of its own
ulps).  It must also agree with an fp32 computation of the same expression.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

import oracle as O

pytestmark = pytest.mark.gpu

K_ = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import install_routed_residual_hook, routed_residual  # noqa: E402
from piper_offload_amd.lora import ScaledLoRAFactor  # noqa: E402
from piper_offload_amd.routed import RoutedFactor  # noqa: E402

DEV = "cuda"
ROUTED_MISMATCH = 0.02
DT = {torch.bfloat16: O.DT_BF16, torch.float16: O.DT_F16}


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _case(T, K, N, ranks, bias, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, K, generator=g).to(dtype)
    y = (torch.randn(T, N, generator=g) * 0.5).to(dtype)
    fs = [RoutedFactor((torch.randn(r, K, generator=g) / r).to(dtype), (torch.randn(N, r, generator=g) * 0.05).to(dtype),
                       [1.0, 0.5, -1.25][i % 3], (torch.randn(N, generator=g) * 0.02).to(dtype) if bias else None)
          for i, r in enumerate(ranks)]
    return x, y, fs


def _check(got: torch.Tensor, x, y, fs, dtype):
    ref = O.routed_residual(_bits(x), _bits(y), [(_bits(f.a), _bits(f.b), None if f.bias is None else _bits(f.bias),
                                                  f.strength) for f in fs], dt=DT[dtype])
    o = torch.from_numpy(ref.view(np.int16)).view(dtype).float()
    gv = got.float().cpu()
    # fp32 reference of the same expression
    x32, y32 = x.float(), y.float()
    res32 = sum(((x32 @ f.a.float().T) * f.strength) @ f.b.float().T + (0 if f.bias is None else f.bias.float() *
                                                                         f.strength) for f in fs)
    eps = torch.finfo(dtype).eps
    ulp_out = eps * o.abs().clamp_min(torch.finfo(dtype).tiny)
    ulp_res = eps * res32.abs()
    flips = sum(2 * eps * abs(f.strength) * ((x32 @ f.a.float().T).abs() @ f.b.float().abs().T) for f in fs)
    diff = (gv - o).abs()
    bound = 2 * ulp_out + ulp_res + flips + torch.finfo(dtype).tiny
    if not bool((diff <= bound).all()):
        idx = int(torch.argmax(diff - bound))
        t_, n_ = divmod(idx, o.shape[1])
        print(f"worst ({t_},{n_}): gpu {float(gv.view(-1)[idx])} oracle {float(o.view(-1)[idx])} "
              f"fp32 {float((y32 + res32).view(-1)[idx])} y {float(y32.view(-1)[idx])} res {float(res32.view(-1)[idx])} "
              f"bound {float(bound.view(-1)[idx])} n_bad {int((diff > bound).sum())}", flush=True)
    assert float((diff > 0).float().mean()) <= ROUTED_MISMATCH
    assert bool((diff <= bound).all())
    assert bool(((gv - (y32 + res32)).abs() <= 2 * bound + 2 * eps * (y32 + res32).abs()).all())


@pytest.mark.parametrize("T,K,N,ranks,bias", [
    (1, 4096, 4096, [16], False),        # decode
    (37, 512, 1000, [5], False),         # ragged T and N, odd rank
    (64, 256, 384, [16, 32], True),      # two factors with biases
    (200, 1024, 2048, [64], False),      # rank 64
    (16, 4100, 96, [8, 8, 8], True),     # K not a multiple of 16, three factors
    (8, 1024, 2048, [64, 16], True),     # one launch (T <= 16): five rank chunks
    (3, 256, 100, [16], False),          # one launch, N not a multiple of 8
    (17, 512, 256, [16], False),         # one token past the single-launch path
    (40, 512, 512, [8, 12], False),      # row-streaming up kernel: ranks 8 and 12, partial token tile
    (300, 2048, 14336 // 8, [16], False),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_routed_residual_matches_oracle(T, K, N, ranks, bias, dtype):
    x, y, fs = _case(T, K, N, ranks, bias, dtype, T + K)
    dfs = [RoutedFactor(f.a.to(DEV), f.b.to(DEV), f.strength, None if f.bias is None else f.bias.to(DEV)) for f in fs]
    with torch.no_grad():
        got = routed_residual(x.to(DEV), dfs, y.to(DEV))
    assert got.shape == y.shape and got.dtype is dtype
    _check(got, x, y, fs, dtype)


def test_routed_batched_shapes_and_empty():
    x, y, fs = _case(24, 256, 128, [16], True, torch.bfloat16, 3)
    dfs = [RoutedFactor(f.a.to(DEV), f.b.to(DEV), f.strength, f.bias.to(DEV)) for f in fs]
    with torch.no_grad():
        got = routed_residual(x.to(DEV).view(2, 12, 256), dfs, y.to(DEV).view(2, 12, 128))
        assert got.shape == (2, 12, 128)
        _check(got.view(24, 128), x, y, fs, torch.bfloat16)
        empty = routed_residual(torch.zeros(0, 256, dtype=torch.bfloat16, device=DEV), dfs,
                                torch.zeros(0, 128, dtype=torch.bfloat16, device=DEV))
        assert empty.shape == (0, 128)


def test_routed_rejects_unsupported():
    x, y, fs = _case(4, 64, 32, [4], False, torch.bfloat16, 5)
    dfs = [RoutedFactor(f.a.to(DEV), f.b.to(DEV), f.strength) for f in fs]
    with torch.no_grad():
        with pytest.raises(ValueError, match="bfloat16 and float16"):
            routed_residual(x.to(DEV), dfs, y.float().to(DEV))
        with pytest.raises(ValueError, match="shapes"):
            routed_residual(x.to(DEV)[:, :32], dfs, y.to(DEV))
    xr = x.to(DEV).requires_grad_(True)
    with pytest.raises(NotImplementedError, match="inference-only"):
        routed_residual(xr, dfs, y.to(DEV))


def test_routed_hook_on_a_linear_layer():
    g = torch.Generator().manual_seed(9)
    lin = nn.Linear(512, 768, bias=True, dtype=torch.bfloat16).to(DEV)
    lin.requires_grad_(False)
    f1 = ScaledLoRAFactor((torch.randn(16, 512, generator=g) / 16).to(torch.bfloat16).pin_memory(),
                          (torch.randn(768, 16, generator=g) * 0.05).to(torch.bfloat16).pin_memory(), 0.8)
    f2 = ScaledLoRAFactor((torch.randn(8, 512, generator=g) / 8).to(torch.bfloat16),
                          (torch.randn(768, 8, generator=g) * 0.05).to(torch.bfloat16), -0.5,
                          (torch.randn(768, generator=g) * 0.02).to(torch.bfloat16))
    x = torch.randn(3, 7, 512, generator=g).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        y = F.linear(x, lin.weight, lin.bias)
        remove = install_routed_residual_hook(lin, [f1, f2])
        out = lin(x)
        out_again = lin(input=x)  # keyword input, staged factors reused
        remove()
        plain = lin(x)
    assert torch.equal(plain, y)
    assert torch.equal(out, out_again)
    fs = [RoutedFactor(f.a, f.b, f.strength, f.bias) for f in (f1, f2)]
    _check(out.view(21, 768), x.view(21, 512).cpu(), y.view(21, 768).cpu(), fs, torch.bfloat16)
    # an in-place change of a host factor is picked up by the next call
    with torch.no_grad():
        remove = install_routed_residual_hook(lin, [f2])
        before = lin(x)
        f2.b.mul_(2.0)
        after = lin(x)
        remove()
    assert not torch.equal(before, after)
    _check(after.view(21, 768), x.view(21, 512).cpu(), y.view(21, 768).cpu(),
           [RoutedFactor(f2.a, f2.b, f2.strength, f2.bias)], torch.bfloat16)
