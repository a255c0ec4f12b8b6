"""The reference's portable INT8 merge path in torch CPU ops: the CPU baseline.

TEST AND BENCHMARK INFRASTRUCTURE.  Only ``tests/`` and ``bench.py``'s
``cpu_baseline`` leg use this module; the product path never does.

The reference merges a TorchAO INT8 weight without its Triton kernel as
(P/int8_adapter.py:349-411 with the fused path unavailable):

* dequantize to the compute dtype (``Int8Tensor.dequantize``,
  P/_torchao_int8.py:113-116): bf16(q * s);
* ``addmm_(b, a, alpha=strength)`` on the dense weight
  (RegularAdapter.merge_lora_, P/tensor_adapters.py:686-696);
* requantize with fresh per-row scales (``Int8Tensor.from_hp``,
  P/_torchao_int8.py:119-173), whose arithmetic the Triton kernel restates
  (P/_triton_int8_lora.py:123-236): s = bf16(max(bf16(amax / 127.5), 2^-23)),
  q = clamp(rint(v * (1 / s)), -128, 127);
* with a rounding seed, replace only the codes by stochastic rounding of
  v / s with a ``torch.rand`` stream from a CPU generator seeded by it
  (P/_torchao_int8.py:176-213, P/_stochastic_quantization.py:6-60).

TorchAO is not importable here, so its ``from_hp`` is restated from that
recipe.  The stochastic codes use torch's CPU generator (the reference's
portable stream), not the Philox stream of the HIP kernels: only the
deterministic codes are comparable bit for bit with the oracle.
"""

from __future__ import annotations

import torch

EPS = torch.finfo(torch.float32).eps


def int8_dequant(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16(q * s) for per-row fp32 scales [M, 1]."""
    return (q.to(torch.float32) * scale).to(torch.bfloat16)


def int8_requant(dense: torch.Tensor, *, rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric INT8 codes and fp32 scales [M, 1] of a bf16 weight."""
    v = dense.to(torch.float32)
    amax = v.abs().amax(dim=1, keepdim=True)
    scale = (amax / torch.full_like(amax, 127.5)).to(torch.bfloat16).to(torch.float32)
    scale = scale.clamp_min(EPS).to(torch.bfloat16).to(torch.float32)
    q = torch.round(v * (1.0 / scale)).clamp_(-128, 127)
    if rounding_seed is not None:
        y = (v / scale).clamp(-128, 127)
        lower = torch.floor(y)
        p = y - lower
        g = torch.Generator(device="cpu").manual_seed(int(rounding_seed) % (1 << 63))
        u = torch.rand(y.shape, generator=g, dtype=torch.float32)
        interior = (y > -128) & (y < 127) & (p > 0)
        q = torch.where(interior, lower + (u < p).to(torch.float32), q)
    return q.to(torch.int8), scale


def int8_merge(q: torch.Tensor, scale: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float, *,
               rounding_seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One portable merge: dequantize, addmm_, requantize (codes and scales)."""
    dense = int8_dequant(q, scale)
    dense.addmm_(b, a, alpha=strength)
    return int8_requant(dense, rounding_seed=rounding_seed)
