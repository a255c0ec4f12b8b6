"""Grouped (stack) merges against the oracle, bit for bit.

The stack entries (lm_int8_merge_stack / lm_nvfp4_merge_stack) replace the
per-target loop of merge_lora() (P/merge.py:121-125) with one grouped launch
per pass; every target keeps its own seed.  Each target's expected codes and
scales are the oracle's requant of the GPU's dense merge of that target
(dequantize + LoRA, the same seed), so a failure names the side that is
wrong: the grouped kernels, the single-target kernels, or both.  The dense
merge itself is checked against the oracle within the floating-point
contract in the per-format tests.

Two tests run config 5 at full size: all 224 targets of the
32-layer 8B-shaped stack in one grouped call, sampled targets against the
oracle and every target against its single-target merge and by properties
computed with torch on the GPU (code range, the scale recipe, two-neighbour
rounding).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import bf16_np, int8_initial, lora_factors, mismatch_report, normal_bf16, u8_np

pytestmark = pytest.mark.gpu

K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import Int8Weight, NVFP4Weight, derive_seed  # noqa: E402
from piper_offload_amd.stack import StackPlan, StackTarget, merge_int8_stack, merge_nvfp4_stack  # noqa: E402

DEV = "cuda"
LAYER = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096), (4096, 14336)]
LAYER_NAMES = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
               "mlp.up_proj", "mlp.down_proj"]


def _sr(sr: bool) -> int:
    return O.SR_PHILOX8 if sr else O.SR_OFF


# ---- INT8 ---------------------------------------------------------------------
def _int8_targets(shapes, rank, seed0):  # noqa: ANN001, ANN202
    out = []
    for i, (rows, cols) in enumerate(shapes):
        q, s = int8_initial(normal_bf16((rows, cols), 0.02, seed0 + i))
        b, a = lora_factors(rows, cols, rank, seed0 + 100 + i)
        out.append((q, s, b.to(DEV), a.to(DEV), [1.0, 0.5, -0.75][i % 3], derive_seed(f"layers.{i}.weight", 3)))
    return out


def _int8_oracle(q: torch.Tensor, s: torch.Tensor, b, a, strength, seed, sr):  # noqa: ANN001, ANN202
    """Oracle requant of the GPU dense merge of one per-row INT8 target."""
    cols = q.shape[1]
    dense = K.dequantize_int8(q.to(DEV), s.to(DEV), None, (1, cols), lora=(b, a, strength))
    rq, rs, _ = O.int8_requant(bf16_np(dense), cols, sr_mode=_sr(sr), seed=seed if sr else 0)
    return rq, rs


@pytest.mark.parametrize("shapes", [[(64, 256), (40, 512), (128, 128), (16, 64)],   # fast kernel (N % 64 == 0)
                                    [(64, 256), (40, 14336), (16, 8192), (24, 4096)],  # + long rows (second launch)
                                    [(64, 256), (24, 96)],                           # generic kernel
                                    # rows all 4096 wide (every tile in the register cache) with ragged
                                    # last groups, more 16-row groups than workgroups resident at once
                                    [(24, 4096), (8200, 4096), (40, 4096), (1000, 4096)],
                                    LAYER])                                          # one 8B layer at full size
@pytest.mark.parametrize("sr", [False, True])
def test_int8_stack_and_per_target_merges_equal_the_oracle(shapes, sr):
    tg = _int8_targets(shapes, 16, 10)
    errors = []
    targets = []
    for i, (q, s, b, a, strength, seed) in enumerate(tg):
        rq, rs = _int8_oracle(q, s, b, a, strength, seed, sr)
        pq, ps, _ = K.merge_int8_lora(q.to(DEV), s.to(DEV), None, (1, q.shape[1]), b, a, strength,
                                      asymmetric=False, reduce_range=False, rounding_seed=seed if sr else None)
        errors += [f"per-target item {i} {m}" for m in (mismatch_report(pq.cpu().numpy(), rq, "codes", 64),
                                                         mismatch_report(ps.cpu().numpy().reshape(-1), rs, "scales", 1))
                   if m]
        w = Int8Weight(q.clone().to(DEV), s.clone().to(DEV), (1, q.shape[1]), torch.bfloat16)
        targets.append((StackTarget(w, b, a, strength, seed), rq, rs))
    merge_int8_stack([t for t, _, _ in targets], stochastic=sr)
    for i, (t, rq, rs) in enumerate(targets):
        errors += [f"stack item {i} {m}" for m in (
            mismatch_report(t.weight.qdata.cpu().numpy(), rq, "codes", 64),
            mismatch_report(t.weight.scale.cpu().numpy().reshape(-1), rs, "scales", 1)) if m]
    assert not errors, "\n".join(errors)


@pytest.mark.parametrize("shapes", [[(64, 256), (40, 512), (128, 128), (16, 64)],
                                    [(64, 256), (40, 14336), (16, 8192), (24, 4096)],
                                    [(24, 4096), (8200, 4096), (40, 4096), (1000, 4096)],
                                    LAYER])
@pytest.mark.parametrize("sr", [False, True])
def test_int8_stack_with_bf16_scales_equals_the_oracle(shapes, sr):
    """bf16 qparams (TorchAO keeps scales in the model dtype): the fast row kernels round the quantize step's
    v * RN(1 / s) to bf16 (P/_triton_int8_lora.py:190-236) and store bf16 scales."""
    tg = _int8_targets(shapes, 16, 60)
    errors = []
    targets = []
    for i, (q, s, b, a, strength, seed) in enumerate(tg):
        s = s.to(torch.bfloat16)
        cols = q.shape[1]
        dense = K.dequantize_int8(q.to(DEV), s.to(DEV), None, (1, cols), lora=(b, a, strength))
        rq, rs, _ = O.int8_requant(bf16_np(dense), cols, scale_dt=O.DT_BF16, sr_mode=_sr(sr), seed=seed if sr else 0)
        pq, ps, _ = K.merge_int8_lora(q.to(DEV), s.to(DEV), None, (1, cols), b, a, strength, asymmetric=False,
                                      reduce_range=False, rounding_seed=seed if sr else None)
        errors += [f"per-target item {i} {m}" for m in (mismatch_report(pq.cpu().numpy(), rq, "codes", 64),
                                                         mismatch_report(bf16_np(ps).reshape(-1), rs, "scales", 1))
                   if m]
        w = Int8Weight(q.clone().to(DEV), s.clone().to(DEV), (1, cols), torch.bfloat16)
        targets.append((StackTarget(w, b, a, strength, seed), rq, rs))
    merge_int8_stack([t for t, _, _ in targets], stochastic=sr)
    for i, (t, rq, rs) in enumerate(targets):
        assert t.weight.scale.dtype is torch.bfloat16
        errors += [f"stack item {i} {m}" for m in (
            mismatch_report(t.weight.qdata.cpu().numpy(), rq, "codes", 64),
            mismatch_report(bf16_np(t.weight.scale).reshape(-1), rs, "scales", 1)) if m]
    assert not errors, "\n".join(errors)


def test_stack_plan_reuse_equals_the_oracle_twice():
    tg = _int8_targets([(64, 256), (32, 512), (16, 128)], 16, 40)
    targets = [StackTarget(Int8Weight(q.clone().to(DEV), s.clone().to(DEV), (1, q.shape[1]), torch.bfloat16),
                           b, a, strength, 0) for q, s, b, a, strength, _ in tg]
    plan = StackPlan(targets, "int8")
    current = [(q, s) for q, s, *_ in tg]
    for step in range(2):
        seeds = [derive_seed(f"w{i}", step) for i in range(len(targets))]
        expected = [_int8_oracle(cq, cs, b, a, strength, seed, True)
                    for (cq, cs), (_, _, b, a, strength, _), seed in zip(current, tg, seeds)]
        plan.merge(seeds)
        torch.cuda.synchronize()
        for i, (t, (rq, rs)) in enumerate(zip(targets, expected)):
            m = mismatch_report(t.weight.qdata.cpu().numpy(), rq, f"step {step} item {i} codes", 64)
            assert not m, m
            assert np.array_equal(t.weight.scale.cpu().numpy().reshape(-1), rs)
        current = [(t.weight.qdata.cpu(), t.weight.scale.cpu()) for t in targets]


# ---- NVFP4 --------------------------------------------------------------------
def _nvfp4_weight(rows, cols, seed, two_level, swizzled):  # noqa: ANN001, ANN202
    q, s, pts = O.nvfp4_requant(bf16_np(normal_bf16((rows, cols), 0.02, seed)), swizzled=swizzled,
                                two_level=two_level)
    pt = None if pts is None else torch.from_numpy(pts.reshape(())).to(DEV)
    return NVFP4Weight(torch.from_numpy(q).to(DEV), torch.from_numpy(s).view(torch.float8_e4m3fn).to(DEV), pt, 16,
                       torch.bfloat16, swizzled)


def _nvfp4_oracle(w: NVFP4Weight, b, a, strength, seed, sr):  # noqa: ANN001, ANN202
    """Oracle requant of the GPU dense merge of one NVFP4 target (same levels and layout)."""
    swz = bool(w.is_swizzled_scales)
    dense = K.dequantize_nvfp4(w.qdata, w.scale, w.per_tensor_scale, swizzled=swz, lora=(b, a, strength))
    return O.nvfp4_requant(bf16_np(dense), swizzled=swz, two_level=w.per_tensor_scale is not None,
                           sr_mode=_sr(sr), seed=seed if sr else 0)


def _nvfp4_errors(side: str, i: int, q, s, pts, expected) -> list[str]:  # noqa: ANN001
    rq, rs, rpts = expected
    out = [mismatch_report(u8_np(q), rq, "codes", 64), mismatch_report(u8_np(s), rs, "scales", 8)]
    if rpts is not None:
        out.append(mismatch_report(pts.cpu().numpy().reshape(-1), rpts, "global scale", 1))
    return [f"{side} item {i} {m}" for m in out if m]


@pytest.mark.parametrize("shapes", [[(64, 256), (40, 512), (16, 128), (128, 1024)],  # fast kernels (N % 128 == 0)
                                    [(32, 256), (16, 96)],                           # per-target block kernels
                                    # plain-layout block scales staged in LDS up to 128 macro tiles per row:
                                    # the limit itself with ragged row groups, then one item past it
                                    [(40, 16384), (33, 4096), (17, 128)],
                                    [(24, 16512), (40, 256)],
                                    LAYER])                                          # one 8B layer at full size
@pytest.mark.parametrize("swizzled", [False, True])
@pytest.mark.parametrize("sr", [False, True])
def test_nvfp4_stack_and_per_target_merges_equal_the_oracle(shapes, swizzled, sr):
    errors = []
    targets = []
    for i, (rows, cols) in enumerate(shapes):
        two = i % 3 != 2  # mix two-level and single-level tensors
        b, a = lora_factors(rows, cols, 16, 200 + i)
        b, a = b.to(DEV), a.to(DEV)
        strength = [1.0, 0.5, 2.0][i % 3]
        seed = derive_seed(f"model.layers.{i}.mlp.weight", 0)
        w = _nvfp4_weight(rows, cols, 300 + i, two, swizzled)
        expected = _nvfp4_oracle(w, b, a, strength, seed, sr)
        pq, ps, ppts = K.merge_nvfp4_lora(w.qdata, w.scale, w.per_tensor_scale, 16, swizzled, b, a, strength,
                                          rounding_seed=seed if sr else None)
        errors += _nvfp4_errors("per-target", i, pq, ps, ppts, expected)
        targets.append((StackTarget(w, b, a, strength, seed), expected))
    merge_nvfp4_stack([t for t, _ in targets], stochastic=sr)
    for i, (t, expected) in enumerate(targets):
        errors += _nvfp4_errors("stack", i, t.weight.qdata, t.weight.scale, t.weight.per_tensor_scale, expected)
    assert not errors, "\n".join(errors)


# ---- config 5 at full size: 224 targets in one grouped call --------------------
def _gpu_normal(shape, std, seed):  # noqa: ANN001, ANN202
    g = torch.Generator(device=DEV).manual_seed(seed % (1 << 63))
    return (torch.randn(shape, generator=g, device=DEV) * std).to(torch.bfloat16)


def _config5_specs():  # noqa: ANN202
    for layer in range(32):
        for name, (rows, cols) in zip(LAYER_NAMES, LAYER):
            yield f"model.layers.{layer}.{name}.weight", rows, cols


def _int8_properties(q: torch.Tensor, s: torch.Tensor, dense: torch.Tensor, sr: bool) -> str:
    """Torch statement of the per-row symmetric recipe (P/_triton_int8_lora.py:123-236): the scale is
    bf16(max(bf16(amax / 127.5), 2^-23)); a stochastic code is a neighbour of v / s and unbiased, a
    round-to-nearest code is rint(v * RN(1 / s))."""
    d = dense.float()
    amax = d.abs().amax(dim=1)
    # a tensor divisor: IEEE division (a Python-number divisor multiplies by its reciprocal)
    scale = (amax / torch.full_like(amax, 127.5)).to(torch.bfloat16).float()
    scale = scale.clamp_min(2.0 ** -23).to(torch.bfloat16).float()
    if not torch.equal(s.reshape(-1), scale):
        return "scale recipe"
    y = d / scale[:, None]
    lo, hi = torch.floor(y).clamp(-128, 127), torch.ceil(y).clamp(-128, 127)
    qf = q.float()
    if not sr:
        y = d * (1.0 / scale)[:, None]
    if sr:
        if not bool(((qf == lo) | (qf == hi)).all()):
            return "stochastic code outside the two neighbours"
        frac = (y - torch.floor(y)).clamp(0, 1)
        bias = float(((qf - torch.floor(y)) - frac).mean())
        if abs(bias) > 2e-3:
            return f"stochastic rounding biased by {bias}"
    elif not torch.equal(qf, torch.round(y).clamp(-128, 127)):
        return "round-to-nearest code"
    return ""


@pytest.mark.parametrize("sr", [False, True])
def test_config5_int8_stack_224_targets(sr):
    targets, paths, originals = [], [], []
    for path, rows, cols in _config5_specs():
        w = _gpu_normal((rows, cols), 0.02, derive_seed(path, 0)).float()
        s = (w.abs().amax(dim=1, keepdim=True) / 127.0).clamp_min(torch.finfo(torch.float32).eps)
        q = torch.round(w / s).clamp_(-128, 127).to(torch.int8)
        del w
        b = _gpu_normal((rows, 16), 0.01, derive_seed(path, 2))
        a = _gpu_normal((16, cols), 1.0 / 16, derive_seed(path, 1))
        originals.append((q.clone(), s.clone()))
        targets.append(StackTarget(Int8Weight(q, s, (1, cols), torch.bfloat16), b, a, 1.0, derive_seed(path, 7)))
        paths.append(path)
    assert len(targets) == 224
    merge_int8_stack(targets, stochastic=sr)
    sampled = {0, 4, 111, 223}  # q, gate (layer 0), o (layer 15), down (layer 31)
    errors = []
    for i, (t, (q0, s0)) in enumerate(zip(targets, originals)):
        pq, ps, _ = K.merge_int8_lora(q0, s0, None, (1, q0.shape[1]), t.b, t.a, 1.0, asymmetric=False,
                                      reduce_range=False, rounding_seed=t.seed if sr else None)
        if not (torch.equal(pq, t.weight.qdata) and torch.equal(ps, t.weight.scale)):
            errors.append(f"{paths[i]}: stack differs from its single-target merge")
        dense = K.dequantize_int8(q0, s0, None, (1, q0.shape[1]), lora=(t.b, t.a, 1.0))
        bad = _int8_properties(t.weight.qdata, t.weight.scale, dense, sr)
        if bad:
            errors.append(f"{paths[i]}: {bad}")
        if i in sampled:
            rq, rs, _ = O.int8_requant(bf16_np(dense), q0.shape[1], sr_mode=_sr(sr), seed=t.seed if sr else 0)
            for m in (mismatch_report(t.weight.qdata.cpu().numpy(), rq, "codes", 64),
                      mismatch_report(t.weight.scale.cpu().numpy().reshape(-1), rs, "scales", 1)):
                if m:
                    errors.append(f"{paths[i]} vs oracle: {m}")
        del dense, pq, ps
    assert not errors, "\n".join(errors[:20])


E2M1_GRID = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def _nvfp4_properties(w: NVFP4Weight, dense: torch.Tensor, sr: bool) -> str:
    """Torch statement of two-level NVFP4 (P/_triton_nvfp4_lora.py:251-366, 437-512): the global scale is
    max(amax / 2688, 2^-23), and every element's code is one of the two e2m1 grid neighbours of
    x = v * ((1 / g) / s_block) (the nearest one with round-to-nearest, up to ties), with the sign of v."""
    d = dense.float()
    # scalar steps in numpy float32 (IEEE division; torch divides a tensor by
    # a Python number as a multiplication by its reciprocal)
    g = max(np.float32(float(d.abs().amax())) / np.float32(2688.0), np.float32(2.0 ** -23))
    if np.float32(float(w.per_tensor_scale)) != g:
        return f"global scale {float(w.per_tensor_scale)} != {float(g)}"
    rows, cols = d.shape
    q = w.qdata
    codes = torch.stack([q & 15, q >> 4], dim=-1).reshape(rows, cols).long()
    grid = E2M1_GRID.to(d.device)
    mag = grid[codes & 7]
    # RN(RN(1 / g) / s) for each of the 256 e4m3 block-scale codes
    e4m3 = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    with np.errstate(divide="ignore", invalid="ignore"):
        table = (np.float32(1.0) / g) / e4m3.astype(np.float32)
    sc = w.scale.view(torch.uint8).reshape(rows, cols // 16).long()
    recip = torch.from_numpy(table.astype(np.float32)).to(d.device)[sc]
    x = (d.reshape(rows, cols // 16, 16) * recip[..., None]).reshape(rows, cols).abs().clamp(max=6.0)
    idx = torch.bucketize(x, grid, right=True).clamp(1, 7) - 1  # grid[idx] <= x < grid[idx + 1]
    lo, hi = grid[idx], grid[(idx + 1).clamp(max=7)]
    on_grid = (mag == lo) | (mag == hi)
    neg = (codes & 8) != 0
    sign_ok = (neg == (d < 0)) | (mag == 0) | (d == 0)
    if not bool((on_grid & sign_ok).all()):
        return "code outside the two grid neighbours (or sign)"
    if not sr:
        nearest = torch.where((x - lo) <= (hi - x), lo, hi)
        tie = (x - lo) == (hi - x)
        if not bool(((mag == nearest) | tie).all()):
            return "round-to-nearest code"
    return ""


@pytest.mark.parametrize("sr", [False, True])
def test_config5_nvfp4_stack_224_targets(sr):
    targets, paths, originals = [], [], []
    for path, rows, cols in _config5_specs():
        q, s, pts = K.requantize_nvfp4(_gpu_normal((rows, cols), 0.02, derive_seed(path, 0)), two_level=True)
        b = _gpu_normal((rows, 16), 0.01, derive_seed(path, 2))
        a = _gpu_normal((16, cols), 1.0 / 16, derive_seed(path, 1))
        originals.append((q.clone(), s.clone(), pts.clone()))
        targets.append(StackTarget(NVFP4Weight(q, s, pts.reshape(()), 16), b, a, 1.0, derive_seed(path, 7)))
        paths.append(path)
    assert len(targets) == 224
    merge_nvfp4_stack(targets, stochastic=sr)
    sampled = {0, 4, 111, 223}
    errors = []
    for i, (t, (q0, s0, p0)) in enumerate(zip(targets, originals)):
        pq, ps, pp = K.merge_nvfp4_lora(q0, s0, p0, 16, False, t.b, t.a, 1.0, rounding_seed=t.seed if sr else None)
        same = torch.equal(pq, t.weight.qdata) and torch.equal(ps.view(torch.uint8), t.weight.scale.view(torch.uint8))
        if not (same and torch.equal(pp.reshape(()), t.weight.per_tensor_scale.reshape(()))):
            errors.append(f"{paths[i]}: stack differs from its single-target merge")
        dense = K.dequantize_nvfp4(q0, s0, p0, lora=(t.b, t.a, 1.0))
        bad = _nvfp4_properties(t.weight, dense, sr)
        if bad:
            errors.append(f"{paths[i]}: {bad}")
        if i in sampled:
            rq, rs, rp = O.nvfp4_requant(bf16_np(dense), sr_mode=_sr(sr), seed=t.seed if sr else 0)
            for m in (mismatch_report(u8_np(t.weight.qdata), rq, "codes", 64),
                      mismatch_report(u8_np(t.weight.scale), rs, "scales", 8),
                      mismatch_report(t.weight.per_tensor_scale.cpu().numpy().reshape(-1), rp, "global", 1)):
                if m:
                    errors.append(f"{paths[i]} vs oracle: {m}")
        del dense, pq, ps
    assert not errors, "\n".join(errors[:20])


def test_stack_plan_merges_on_two_streams_run_in_order():
    # one plan, one workspace: a merge issued on a second stream must wait for
    # the first one (its completion event), or it would overwrite the factor
    # layouts and descriptors the first launch still reads
    tg = _int8_targets([(4096, 4096), (1024, 4096)], 16, 80)
    targets = [StackTarget(Int8Weight(q.clone().to(DEV), s.clone().to(DEV), (1, q.shape[1]), torch.bfloat16),
                           b, a, strength, 0) for q, s, b, a, strength, _ in tg]
    plan = StackPlan(targets, "int8")
    side = torch.cuda.Stream()
    seeds = [[derive_seed(f"two.{i}", step) for i in range(len(targets))] for step in range(2)]
    plan.merge(seeds[0])  # default stream
    with torch.cuda.stream(side):
        plan.merge(seeds[1])  # no host synchronization in between
    torch.cuda.synchronize()
    current = [(q, s) for q, s, *_ in tg]
    for step in range(2):
        nxt = []
        for (cq, cs), (_, _, b, a, strength, _), seed in zip(current, tg, seeds[step]):
            rq, rs = _int8_oracle(cq, cs, b, a, strength, seed, True)
            nxt.append((torch.from_numpy(rq), torch.from_numpy(rs).reshape(-1, 1)))
        current = nxt
    for i, (t, (rq, rs)) in enumerate(zip(targets, current)):
        m = mismatch_report(t.weight.qdata.cpu().numpy(), rq.numpy(), f"item {i} codes", 64)
        assert not m, m
        assert torch.equal(t.weight.scale.cpu().reshape(-1), rs.reshape(-1))


# ---- the pruned per-tensor amax of two-level NVFP4 ---------------------------------
def _pruned_case(case: str, swizzled: bool):  # noqa: ANN202
    """(weight, b, a, strength) of one two-level target that stresses the pruned amax (bound, seed, refine)."""
    if case == "wide":  # more than 1024 tile columns: the bound pass takes its column norms in strips
        rows, cols = 20, 1026 * 128
        b, a = lora_factors(rows, cols, 16, 41)
        return _nvfp4_weight(rows, cols, 42, True, swizzled), b.to(DEV), a.to(DEV), 1.0
    if case == "loose":
        # The tile of rows 0-15, columns 0-127 has the largest bound (||B_i|| ||A_j|| = 1) but a zero delta
        # (B_i and A_j are orthogonal), so the seed merges it and finds only its base values; the largest
        # merged value is in rows 16-31, columns 128-255 (base weights x3), which only the refine pass sees.
        rows, cols = 64, 512
        w = normal_bf16((rows, cols), 0.02, 43)
        w[16:32, 128:256] *= 3
        q, sc, pts = O.nvfp4_requant(bf16_np(w), swizzled=swizzled, two_level=True)
        wt = NVFP4Weight(torch.from_numpy(q).to(DEV), torch.from_numpy(sc).view(torch.float8_e4m3fn).to(DEV),
                         torch.from_numpy(pts.reshape(())).to(DEV), 16, torch.bfloat16, swizzled)
        b = torch.zeros((rows, 16), dtype=torch.bfloat16)
        a = torch.zeros((16, cols), dtype=torch.bfloat16)
        b[:16, 0] = 1.0
        a[1, :128] = 1.0
        return wt, b.to(DEV), a.to(DEV), 1.0
    # "delta": the update dominates the base weights, so the bounds are loose everywhere and many tiles
    # are merged exactly; negative strength
    rows, cols = 96, 1024
    b, a = lora_factors(rows, cols, 16, 44, a_std=0.5, b_std=0.5)
    return _nvfp4_weight(rows, cols, 45, True, swizzled), b.to(DEV), a.to(DEV), -30.0


@pytest.mark.parametrize("case", ["wide", "loose", "delta"])
@pytest.mark.parametrize("swizzled", [False, True])
@pytest.mark.parametrize("sr", [False, True])
def test_nvfp4_pruned_amax_edge_cases(case, swizzled, sr):
    w, b, a, strength = _pruned_case(case, swizzled)
    seed = derive_seed(f"pruned.{case}.weight", 3)
    expected = _nvfp4_oracle(w, b, a, strength, seed, sr)
    pq, ps, ppts = K.merge_nvfp4_lora(w.qdata, w.scale, w.per_tensor_scale, 16, swizzled, b, a, strength,
                                      rounding_seed=seed if sr else None)
    errors = _nvfp4_errors("per-target", 0, pq, ps, ppts, expected)
    # the same target in a stack, after a regular one
    w0 = _nvfp4_weight(64, 256, 46, True, swizzled)
    b0, a0 = (x.to(DEV) for x in lora_factors(64, 256, 16, 47))
    exp0 = _nvfp4_oracle(w0, b0, a0, 1.0, seed + 1, sr)
    merge_nvfp4_stack([StackTarget(w0, b0, a0, 1.0, seed + 1), StackTarget(w, b, a, strength, seed)], stochastic=sr)
    errors += _nvfp4_errors("stack", 0, w0.qdata, w0.scale, w0.per_tensor_scale, exp0)
    errors += _nvfp4_errors("stack", 1, w.qdata, w.scale, w.per_tensor_scale, expected)
    assert not errors, "\n".join(errors)
