"""Grouped (stack) merges equal per-target merges with the same seeds, bit for bit.

The stack entries (lm_int8_merge_stack / lm_nvfp4_merge_stack) replace the
per-target loop of merge_lora() (P/merge.py:121-125) with one grouped launch
per pass; every target keeps its own seed, so each target's codes, scales and
global scale must equal the single-target merge of the same inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import bf16_np, int8_initial, lora_factors, normal_bf16, u8_np

pytestmark = pytest.mark.gpu

K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import Int8Weight, NVFP4Weight, derive_seed  # noqa: E402
from piper_offload_amd.stack import StackTarget, merge_int8_stack, merge_nvfp4_stack  # noqa: E402

DEV = "cuda"


def _int8_targets(shapes, rank, seed0):  # noqa: ANN001, ANN202
    out = []
    for i, (rows, cols) in enumerate(shapes):
        q, s = int8_initial(normal_bf16((rows, cols), 0.02, seed0 + i))
        b, a = lora_factors(rows, cols, rank, seed0 + 100 + i)
        out.append((q, s, b, a, [1.0, 0.5, -0.75][i % 3], derive_seed(f"layers.{i}.weight", 3)))
    return out


@pytest.mark.parametrize("shapes", [[(64, 256), (40, 512), (128, 128), (16, 64)],   # fast kernel (N % 64 == 0)
                                    [(64, 256), (40, 14336), (16, 8192), (24, 4096)],  # + long rows (second launch)
                                    [(64, 256), (24, 96)],                           # generic kernel
                                    # one 8B layer at full size: q, k, v, o, gate, up, down
                                    [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096),
                                     (14336, 4096), (4096, 14336)]])
@pytest.mark.parametrize("sr", [False, True])
def test_int8_stack_equals_per_target_merges(shapes, sr):
    tg = _int8_targets(shapes, 16, 10)
    expected = []
    for q, s, b, a, strength, seed in tg:
        eq, es, _ = K.merge_int8_lora(q.to(DEV), s.to(DEV), None, (1, q.shape[1]), b.to(DEV), a.to(DEV), strength,
                                      asymmetric=False, reduce_range=False, rounding_seed=seed if sr else None)
        expected.append((eq.cpu(), es.cpu()))
    targets = []
    for q, s, b, a, strength, seed in tg:
        w = Int8Weight(q.clone().to(DEV), s.clone().to(DEV), (1, q.shape[1]), torch.bfloat16)
        targets.append(StackTarget(w, b.to(DEV), a.to(DEV), strength, seed))
    merge_int8_stack(targets, stochastic=sr)
    for t, (eq, es) in zip(targets, expected):
        assert torch.equal(t.weight.qdata.cpu(), eq)
        assert torch.equal(t.weight.scale.cpu().reshape(-1), es.reshape(-1))


def _nvfp4_weight(rows, cols, seed, two_level, swizzled):  # noqa: ANN001, ANN202
    q, s, pts = O.nvfp4_requant(bf16_np(normal_bf16((rows, cols), 0.02, seed)), swizzled=swizzled,
                                two_level=two_level)
    pt = None if pts is None else torch.from_numpy(pts.reshape(())).to(DEV)
    return NVFP4Weight(torch.from_numpy(q).to(DEV), torch.from_numpy(s).view(torch.float8_e4m3fn).to(DEV), pt, 16,
                       torch.bfloat16, swizzled)


@pytest.mark.parametrize("shapes", [[(64, 256), (40, 512), (16, 128), (128, 1024)],  # fast kernels (N % 128 == 0)
                                    [(32, 256), (16, 96)],                           # per-target block kernels
                                    # one 8B layer at full size: q, k, v, o, gate, up, down
                                    [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096),
                                     (14336, 4096), (4096, 14336)]])
@pytest.mark.parametrize("swizzled", [False, True])
@pytest.mark.parametrize("sr", [False, True])
def test_nvfp4_stack_equals_per_target_merges(shapes, swizzled, sr):
    specs = []
    for i, (rows, cols) in enumerate(shapes):
        two = i % 3 != 2  # mix two-level and single-level tensors
        b, a = lora_factors(rows, cols, 16, 200 + i)
        specs.append((rows, cols, two, b.to(DEV), a.to(DEV), [1.0, 0.5, 2.0][i % 3],
                      derive_seed(f"model.layers.{i}.mlp.weight", 0)))
    expected = []
    for i, (rows, cols, two, b, a, strength, seed) in enumerate(specs):
        w = _nvfp4_weight(rows, cols, 300 + i, two, swizzled)
        eq, es, ep = K.merge_nvfp4_lora(w.qdata, w.scale, w.per_tensor_scale, 16, swizzled, b, a, strength,
                                        rounding_seed=seed if sr else None)
        expected.append((u8_np(eq), u8_np(es), None if ep is None else ep.cpu().numpy().reshape(-1)))
    targets = []
    for i, (rows, cols, two, b, a, strength, seed) in enumerate(specs):
        targets.append(StackTarget(_nvfp4_weight(rows, cols, 300 + i, two, swizzled), b, a, strength, seed))
    merge_nvfp4_stack(targets, stochastic=sr)
    for t, (eq, es, ep) in zip(targets, expected):
        assert np.array_equal(u8_np(t.weight.qdata), eq)
        assert np.array_equal(u8_np(t.weight.scale), es)
        if ep is not None:
            assert np.array_equal(t.weight.per_tensor_scale.cpu().numpy().reshape(-1), ep)


def test_stack_plan_reuse_equals_repeated_per_target_merges():
    from piper_offload_amd.stack import StackPlan

    tg = _int8_targets([(64, 256), (32, 512), (16, 128)], 16, 40)
    expected = []
    for i, (q, s, b, a, strength, _seed) in enumerate(tg):
        cq, cs = q.to(DEV), s.to(DEV)
        for step in range(2):
            cq, cs, _ = K.merge_int8_lora(cq, cs, None, (1, q.shape[1]), b.to(DEV), a.to(DEV), strength,
                                          asymmetric=False, reduce_range=False,
                                          rounding_seed=derive_seed(f"w{i}", step))
        expected.append((cq.cpu(), cs.cpu()))
    targets = [StackTarget(Int8Weight(q.clone().to(DEV), s.clone().to(DEV), (1, q.shape[1]), torch.bfloat16),
                           b.to(DEV), a.to(DEV), strength, 0) for q, s, b, a, strength, _ in tg]
    plan = StackPlan(targets, "int8")
    for step in range(2):
        plan.merge([derive_seed(f"w{i}", step) for i in range(len(targets))])
    torch.cuda.synchronize()
    for t, (eq, es) in zip(targets, expected):
        assert torch.equal(t.weight.qdata.cpu(), eq)
        assert torch.equal(t.weight.scale.cpu().reshape(-1), es.reshape(-1))
