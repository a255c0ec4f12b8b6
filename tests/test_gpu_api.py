"""merge_lora() end to end on a GPU model whose weights are packed formats.

The drop-in API (P/merge.py:54-87) resolves each target, stages its factors
once (one host buffer, one host-to-device copy, reused between validate and
apply), packs several LoRAs along the rank with each A slice scaled by its
strength in bf16 (P/lora.py:684-724) and calls the adapter's merge with the
target's seed ``derive_seed(target_key, 0)`` (P/lora.py:356-359); weights a
grouped kernel can merge (per-row INT8, NVFP4) go through one grouped launch
per compatible group.  Every weight must end up byte-identical to the
one-by-one adapter merge of the same weight with factors packed
independently here, and equal the oracle: its requant of the GPU dense merge
of the original weight with those factors and seed (codes and scales bit for
bit), or for the plain bf16 weight the oracle's dense merge within the
floating-point contract.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

import oracle as O
from helpers import assert_merged_close, bf16_np, fp8_initial, int8_initial, mismatch_report, normal_bf16, u8_np

pytestmark = pytest.mark.gpu

K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import (  # noqa: E402
    Float8Adapter, Float8Weight, GGUFWeight, GgufAdapter, Int8Adapter, Int8Weight, LoRA, NVFP4Weight, Nvfp4Adapter,
    RegularAdapter, derive_seed, merge_lora)
from piper_offload_amd.registry import param_representation  # noqa: E402

DEV = "cuda"


def _holder(w: torch.Tensor) -> nn.Module:
    h = nn.Module()
    h.weight = nn.Parameter(w, requires_grad=False)
    return h


def _model() -> nn.Module:
    m = nn.Module()
    q, s = int8_initial(normal_bf16((256, 512), 0.02, 1))
    m.q = _holder(Int8Weight(q.to(DEV), s.to(DEV), (1, 512), torch.bfloat16))
    q, s = fp8_initial(normal_bf16((128, 512), 0.02, 2))
    m.k = _holder(Float8Weight(q.to(DEV), s.to(DEV), (1, 512), torch.bfloat16))
    nq, ns, npt = O.nvfp4_requant(bf16_np(normal_bf16((256, 512), 0.02, 3)))
    m.up = _holder(NVFP4Weight(torch.from_numpy(nq).to(DEV), torch.from_numpy(ns).view(torch.float8_e4m3fn).to(DEV),
                               torch.from_numpy(npt.reshape(())).to(DEV), 16, torch.bfloat16, False))
    q, s = int8_initial(normal_bf16((64, 256), 0.02, 6))
    m.o = _holder(Int8Weight(q.to(DEV), s.to(DEV), (1, 256), torch.bfloat16))
    nq, ns, _ = O.nvfp4_requant(bf16_np(normal_bf16((128, 256), 0.02, 7)), two_level=False)
    m.dn = _holder(NVFP4Weight(torch.from_numpy(nq).to(DEV), torch.from_numpy(ns).view(torch.float8_e4m3fn).to(DEV),
                               None, 16, torch.bfloat16, False))
    packed = O.q8_0_requant(bf16_np(normal_bf16((64, 512), 0.02, 4)))
    m.g = _holder(GGUFWeight(torch.from_numpy(packed).to(DEV), quant_type=8))
    m.d = nn.Linear(512, 256, bias=False, dtype=torch.bfloat16, device=DEV)
    m.d.weight.data.copy_(normal_bf16((256, 512), 0.02, 5).to(DEV))
    m.requires_grad_(False)
    return m


_SHAPES = {"q.weight": (256, 512), "o.weight": (64, 256), "k.weight": (128, 512), "up.weight": (256, 512),
           "dn.weight": (128, 256), "g.weight": (64, 512), "d.weight": (256, 512)}
_ADAPTERS = {"q.weight": Int8Adapter, "o.weight": Int8Adapter, "k.weight": Float8Adapter, "up.weight": Nvfp4Adapter,
             "dn.weight": Nvfp4Adapter, "g.weight": GgufAdapter, "d.weight": RegularAdapter}


def _lora(keys: list[str], rank: int, seed: int) -> LoRA:
    g = torch.Generator().manual_seed(seed)
    sd = {}
    for key in keys:
        rows, cols = _SHAPES[key]
        name = key.rsplit(".", 1)[0]
        sd[f"{name}.lora_A.weight"] = (torch.randn(rank, cols, generator=g) / rank).to(torch.bfloat16)
        sd[f"{name}.lora_B.weight"] = (torch.randn(rows, rank, generator=g) * 0.01).to(torch.bfloat16)
    return LoRA.from_state_dict(sd)


def _bytes(p: torch.Tensor) -> list[np.ndarray]:
    if isinstance(p, (Int8Weight, Float8Weight, NVFP4Weight)):
        return [u8_np(t.reshape(-1)) for t in p.inner_tensors()]
    if isinstance(p, GGUFWeight):
        return [u8_np(p.as_subclass(torch.Tensor))]
    return [u8_np(p.detach())]


def _oracle_errors(key: str, got: torch.Tensor, fresh: torch.Tensor, b: torch.Tensor, a: torch.Tensor,
                   strength: float, seed: int | None) -> list[str]:
    """Compare one merged weight with the oracle; fresh is the same weight before the merge."""
    sr = O.SR_PHILOX8 if seed is not None else O.SR_OFF
    seed = seed or 0
    g, f = param_representation(got), param_representation(fresh)
    lora = (b, a, strength)
    if isinstance(f, Int8Weight):
        cols = f.qdata.shape[1]
        dense = K.dequantize_int8(f.qdata, f.scale, None, (1, cols), lora=lora)
        rq, rs, _ = O.int8_requant(bf16_np(dense), cols, sr_mode=sr, seed=seed)
        pairs = [(g.qdata.cpu().numpy(), rq), (g.scale.cpu().numpy().reshape(-1), rs)]
    elif isinstance(f, Float8Weight):
        cols = f.qdata.shape[1]
        dense = K.dequantize_float8(f.qdata, f.scale, tuple(f.block_size), lora=lora)
        rq, rs = O.fp8_requant(bf16_np(dense), cols, sr_mode=sr, seed=seed)
        pairs = [(u8_np(g.qdata), rq), (g.scale.cpu().numpy().reshape(-1), rs)]
    elif isinstance(f, NVFP4Weight):
        dense = K.dequantize_nvfp4(f.qdata, f.scale, f.per_tensor_scale, lora=lora)
        rq, rs, rp = O.nvfp4_requant(bf16_np(dense), two_level=f.per_tensor_scale is not None, sr_mode=sr, seed=seed)
        pairs = [(u8_np(g.qdata), rq), (u8_np(g.scale), rs)]
        if rp is not None:
            pairs.append((g.per_tensor_scale.cpu().numpy().reshape(-1), rp))
    elif isinstance(f, GGUFWeight):
        packed = f.as_subclass(torch.Tensor)
        dense = K.dequantize_gguf(packed, 8, lora=lora)
        pairs = [(u8_np(g.as_subclass(torch.Tensor)), O.q8_0_requant(bf16_np(dense), sr_mode=sr, seed=seed))]
    else:  # plain bf16: the oracle's dense merge, within the floating-point contract
        base = bf16_np(f.detach())
        assert_merged_close(bf16_np(g.detach()), O.merge_dense(base, bf16_np(b), bf16_np(a), strength), base)
        return []
    return [f"{key}: {m}" for m in (mismatch_report(x, y, "vs oracle", 64) for x, y in pairs) if m]


@pytest.mark.parametrize("stochastic", [False, True])
def test_merge_lora_equals_adapter_merges_with_packed_factors(stochastic):
    l1 = _lora(list(_SHAPES), 16, 10)
    # q/o (INT8) and up/dn (NVFP4) end up with rank 24 each: two grouped launches
    l2 = _lora(["q.weight", "o.weight", "up.weight", "dn.weight", "d.weight"], 8, 11)
    strengths = (0.5, -1.25)
    expected_model = _model()
    packed = {}
    for key in _SHAPES:
        facs = [(lora.targets[key], s) for lora, s in zip((l1, l2), strengths) if key in lora.targets]
        if len(facs) == 1:
            f, s = facs[0]
            b, a, strength = f.b.to(DEV), f.a.to(DEV), s
        else:  # packed along the rank, A slices scaled in bf16, unit strength
            a = torch.cat([f.a.to(DEV) * s if s != 1.0 else f.a.to(DEV) for f, s in facs])
            b = torch.cat([f.b.to(DEV) for f, _s in facs], dim=1).contiguous()
            strength = 1.0
        assert a.dtype is torch.bfloat16
        packed[key] = (b, a, strength)
        data = param_representation(dict(expected_model.named_parameters())[key])
        _ADAPTERS[key].merge_lora_(data, b, a, strength,
                                   rounding_seed=derive_seed(key, 0) if stochastic else None)
    model = _model()
    assert merge_lora(model, [(l1, strengths[0]), (l2, strengths[1])], stochastic_rounding=stochastic) == 7
    torch.cuda.synchronize()
    got = dict(model.named_parameters())
    want = dict(expected_model.named_parameters())
    for key in _SHAPES:
        for x, y in zip(_bytes(got[key]), _bytes(want[key])):
            assert np.array_equal(x, y), key
    # and every weight equals the oracle
    fresh_params = dict(_model().named_parameters())
    errors = []
    for key in _SHAPES:
        b, a, strength = packed[key]
        errors += _oracle_errors(key, got[key], fresh_params[key], b, a, strength,
                                 derive_seed(key, 0) if stochastic else None)
    assert not errors, "\n".join(errors)
    # the grouped path was taken for the INT8 and NVFP4 pairs
    keys = {}
    for key in ("q.weight", "o.weight", "up.weight", "dn.weight"):
        w = param_representation(got[key])
        keys[key] = _ADAPTERS[key].stack_key(w)
    assert keys["q.weight"] == keys["o.weight"] is not None
    assert keys["up.weight"] == keys["dn.weight"] is not None
    # the merge changed every weight
    fresh = dict(_model().named_parameters())
    for key in _SHAPES:
        assert any(not np.array_equal(x, y) for x, y in zip(_bytes(got[key]), _bytes(fresh[key]))), key
