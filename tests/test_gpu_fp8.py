"""Scaled FP8 (e4m3fn / e5m2) per-row and per-tensor merge vs the oracle (same contract as INT8; per-group layouts are in test_gpu_groups.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_merged_close, bf16_np, fp8_initial, lora_factors, normal_bf16, u8_np

pytestmark = pytest.mark.gpu

K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import Float8Adapter, Float8Weight, derive_seed  # noqa: E402

DEV = "cuda"
FMT = {torch.float8_e4m3fn: O.DT_E4M3, torch.float8_e5m2: O.DT_E5M2}


@pytest.mark.parametrize("shape", [(24, 69), (64, 8192), (16, 1000)])
@pytest.mark.parametrize("fp8", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("sr", [False, True])
@pytest.mark.parametrize("per_tensor", [False, True])
def test_fp8_requant_bit_exact(shape, fp8, sr, per_tensor):
    dense = normal_bf16(shape, 0.02, 7)
    dense[1] = 0
    dense[2, :3] = torch.tensor([1e-30, -3.0, 0.5], dtype=torch.bfloat16)
    dense[3, 0] = -0.0
    block = shape if per_tensor else (1, shape[1])
    group = shape[0] * shape[1] if per_tensor else shape[1]
    seed = derive_seed("fp8.requant", shape[1]) if sr else None
    q, s = K.requantize_float8(dense.to(DEV), block, fp8_dtype=fp8, rounding_seed=seed)
    oq, os_ = O.fp8_requant(bf16_np(dense), group, fmt=FMT[fp8], sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF,
                            seed=seed or 0)
    assert np.array_equal(u8_np(q), oq)
    assert np.array_equal(s.cpu().numpy().reshape(-1), os_)


# (24, 14336) r16: 16-wave rows with tiles in registers, in LDS and merged twice
@pytest.mark.parametrize("shape,rank,strength", [((64, 8192), 64, 1.0), ((24, 69), 5, 0.75), ((32, 1024), 16, 0.5),
                                                 ((24, 14336), 16, 1.0)])
@pytest.mark.parametrize("sr", [False, True])
def test_fp8_fused_equals_requant_of_gpu_dense(shape, rank, strength, sr):
    rows, cols = shape
    w = normal_bf16(shape, 0.02, 0)
    q, s = fp8_initial(w)
    b, a = lora_factors(rows, cols, rank, 2)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    base = K.dequantize_float8(qd, sd, (1, cols))
    obase = O.fp8_dequant(u8_np(q), s.numpy(), cols)
    assert np.array_equal(bf16_np(base), obase)
    dense = K.dequantize_float8(qd, sd, (1, cols), lora=(bd, ad, strength))
    omerged = O.merge_dense(obase, bf16_np(b), bf16_np(a), strength)
    assert_merged_close(bf16_np(dense), omerged, obase)
    seed = derive_seed("fp8.fused", rows) if sr else None
    oq, os_ = K.merge_float8_lora(qd, sd, (1, cols), bd, ad, strength, rounding_seed=seed)
    rq, rs = O.fp8_requant(bf16_np(dense), cols, sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(u8_np(oq), rq)
    assert np.array_equal(os_.cpu().numpy().reshape(-1), rs)


# two-pass long rows (rank above 32, rows of more than 4096 columns): rows that
# end inside a 64-row wave tile, a column count that leaves the last wave of a
# row a partial tile range, and the same merge in place (outputs aliasing the
# inputs, so the row scales are overwritten while other column ranges still
# need them)
@pytest.mark.parametrize("shape,rank", [((70, 8256), 64), ((130, 4160), 48), ((16, 12288), 64)])
@pytest.mark.parametrize("fp8", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("sr", [False, True])
def test_fp8_two_pass_rows_and_in_place(shape, rank, fp8, sr):
    rows, cols = shape
    w = normal_bf16(shape, 0.02, 11)
    q, s = fp8_initial(w, fp8)
    b, a = lora_factors(rows, cols, rank, 12)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    dense = K.dequantize_float8(qd, sd, (1, cols), lora=(bd, ad, 0.75))
    obase = O.fp8_dequant(u8_np(q), s.numpy(), cols, fmt=FMT[fp8])
    assert_merged_close(bf16_np(dense), O.merge_dense(obase, bf16_np(b), bf16_np(a), 0.75), obase)
    seed = derive_seed("fp8.two-pass", rows) if sr else None
    oq, os_ = K.merge_float8_lora(qd, sd, (1, cols), bd, ad, 0.75, rounding_seed=seed)
    rq, rs = O.fp8_requant(bf16_np(dense), cols, fmt=FMT[fp8], sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF,
                           seed=seed or 0)
    assert np.array_equal(u8_np(oq), rq)
    assert np.array_equal(os_.cpu().numpy().reshape(-1), rs)
    K.merge_float8_lora_into(qd, sd, (1, cols), bd, ad, 0.75, rounding_seed=seed, out_qdata=qd, out_scale=sd)
    assert np.array_equal(u8_np(qd), rq)
    assert np.array_equal(sd.cpu().numpy().reshape(-1), rs)


def test_fp8_per_tensor_and_adapter_in_place():
    rows, cols, rank = 32, 512, 16
    w = normal_bf16((rows, cols), 0.02, 1)
    wf = w.float()
    st = (wf.abs().max() / 448.0).reshape(1, 1)
    q = (wf / st).clamp(-448, 448).to(torch.float8_e4m3fn)
    b, a = lora_factors(rows, cols, rank, 3)
    target = Float8Weight(q.clone().to(DEV), st.clone().to(DEV), (rows, cols), torch.bfloat16)
    ptr = target.qdata.data_ptr()
    Float8Adapter.merge_lora_(target, b.to(DEV), a.to(DEV), 1.0)
    dense = K.dequantize_float8(q.to(DEV), st.to(DEV), (rows, cols), lora=(b.to(DEV), a.to(DEV), 1.0))
    rq, rs = O.fp8_requant(bf16_np(dense), rows * cols)
    assert target.qdata.data_ptr() == ptr
    assert np.array_equal(u8_np(target.qdata), rq)
    assert np.array_equal(target.scale.cpu().numpy().reshape(-1), rs)


def test_fp8_sr_two_neighbours_and_unbiased():
    rows, cols = 64, 4096
    dense = torch.full((rows, cols), 0.3, dtype=torch.bfloat16)
    dense[:, 0] = 448 * 0.3 / 0.3  # fixes the row scale at 1.0 (amax 448)
    q, s = K.requantize_float8(dense.to(DEV), (1, cols), rounding_seed=derive_seed("fp8-unbiased", 0))
    vals = q.float().cpu()[:, 1:]
    x = float(torch.tensor(0.3, dtype=torch.bfloat16).float()) / float(s[0, 0])
    neighbours = sorted({float(v) for v in vals.unique()})
    assert len(neighbours) == 2 and min(neighbours) <= x <= max(neighbours)
    assert float(vals.mean()) == pytest.approx(x, abs=1e-3)


def test_fp8_negative_zero_keeps_sign_and_zero_rows_get_eps():
    dense = torch.zeros(16, 64, dtype=torch.bfloat16)
    dense[0, 0] = -0.0
    dense[1, 1] = 1.0
    q, s = K.requantize_float8(dense.to(DEV), (1, 64), rounding_seed=derive_seed("negzero", 0))
    assert u8_np(q)[0, 0] == 0x80
    assert float(s[0, 0]) == torch.finfo(torch.float32).eps


def test_fp8_config3_full_size():
    """Config 3: W [8192, 8192] e4m3, r=64, strength 1.0, stochastic and nearest.
    The fused merge's codes and scales are compared with the oracle's requant of
    the GPU dense merge; the dense merge itself with the oracle on a row sample
    (the oracle's full GEMM is slow on the CPU)."""
    rows, cols, rank = 8192, 8192, 64
    w = normal_bf16((rows, cols), 0.02, 5)
    q, s = fp8_initial(w)
    b, a = lora_factors(rows, cols, rank, 6)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    dense = K.dequantize_float8(qd, sd, (1, cols), lora=(bd, ad, 1.0))
    dense_np = bf16_np(dense)
    for seed in (derive_seed("model.layers.0.self_attn.o_proj.weight", 0), None):
        oq, os_ = K.merge_float8_lora(qd, sd, (1, cols), bd, ad, 1.0, rounding_seed=seed)
        rq, rs = O.fp8_requant(dense_np, cols, sr_mode=O.SR_PHILOX8 if seed else O.SR_OFF, seed=seed or 0)
        assert np.array_equal(u8_np(oq), rq)
        assert np.array_equal(os_.cpu().numpy().reshape(-1), rs)
    idx = np.arange(0, rows, 101)
    obase = O.fp8_dequant(u8_np(q)[idx], s.numpy()[idx], cols)
    omerged = O.merge_dense(obase, bf16_np(b)[idx], bf16_np(a), 1.0)
    assert_merged_close(dense_np[idx], omerged, obase)
