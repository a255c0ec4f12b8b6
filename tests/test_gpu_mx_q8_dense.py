"""MX (MXFP4 / MXFP8, four scale modes), GGUF Q8_0 and dense bf16 merges vs the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_merged_close, bf16_np, lora_factors, normal_bf16, u8_np

pytestmark = pytest.mark.gpu

K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import GGUFWeight, GgufAdapter, MXWeight, MxAdapter, RegularAdapter, derive_seed  # noqa: E402

DEV = "cuda"
FP4 = getattr(torch, "float4_e2m1fn_x2", None)
ELEMS = {"fp4": (FP4, O.DT_E2M1), "e4m3": (torch.float8_e4m3fn, O.DT_E4M3), "e5m2": (torch.float8_e5m2, O.DT_E5M2)}


@pytest.mark.parametrize("elem", ["fp4", "e4m3", "e5m2"])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("swizzled", [False, True])
@pytest.mark.parametrize("sr", [False, True])
def test_mx_requant_bit_exact(elem, mode, swizzled, sr):
    tdt, fmt = ELEMS[elem]
    shape = (40, 256)
    dense = normal_bf16(shape, 0.02, 3)
    dense[0, :32] = 0
    dense[1, 32:64] *= 1e4
    seed = derive_seed("mx.requant", mode) if sr else None
    q, s = K.requantize_mx(dense.to(DEV), tdt, scaling_mode=mode, swizzled=swizzled, rounding_seed=seed)
    oq, os_ = O.mx_requant(bf16_np(dense), fmt, mode, swizzled=swizzled, sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF,
                           seed=seed or 0)
    assert np.array_equal(u8_np(q), oq)
    assert np.array_equal(u8_np(s), os_)


@pytest.mark.parametrize("elem", ["fp4", "e4m3", "e5m2"])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("swizzled", [False, True])
@pytest.mark.parametrize("sr", [False, True])
@pytest.mark.parametrize("shape,rank,strength", [((128, 4096), 16, 1.0), ((24, 96), 5, 1.0), ((40, 256), 32, 0.75),
                                                 ((16, 128), 64, -0.5)])
def test_mx_fused_equals_requant_of_gpu_dense(elem, mode, swizzled, sr, shape, rank, strength):
    tdt, fmt = ELEMS[elem]
    rows, cols = shape
    w = normal_bf16(shape, 0.02, 4)
    q, s = O.mx_requant(bf16_np(w), fmt, mode, swizzled=swizzled)
    b, a = lora_factors(rows, cols, rank, 5)
    qd = torch.from_numpy(q).to(DEV)
    sd = torch.from_numpy(s).to(DEV)
    base = K.dequantize_mx(qd, sd, tdt, cols, swizzled=swizzled)
    obase = O.mx_dequant(q, s, fmt, cols, swizzled=swizzled)
    assert np.array_equal(bf16_np(base), obase)
    dense = K.dequantize_mx(qd, sd, tdt, cols, swizzled=swizzled, lora=(b.to(DEV), a.to(DEV), strength))
    assert_merged_close(bf16_np(dense), O.merge_dense(obase, bf16_np(b), bf16_np(a), strength), obase)
    seed = derive_seed("mx.fused", rows) if sr else None
    qstore = qd.clone() if elem == "fp4" else qd.clone().view(tdt)
    K.merge_mx_lora_(qstore, sd, tdt, 32, torch.bfloat16, b.to(DEV), a.to(DEV), strength, scaling_mode=mode,
                     swizzled=swizzled, rounding_seed=seed)
    rq, rs = O.mx_requant(bf16_np(dense), fmt, mode, swizzled=swizzled, sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF,
                          seed=seed or 0)
    assert np.array_equal(u8_np(qstore), rq)
    assert np.array_equal(u8_np(sd), rs)


def test_mx_zero_update_is_identity_and_code0_subnormal():
    """Zero-update merges keep bytes exactly (T/test_mx_adapter.py:565-604)."""
    rows, cols = 32, 128
    w = normal_bf16((rows, cols), 0.02, 8)
    q, s = O.mx_requant(bf16_np(w), O.DT_E4M3, 0)
    s[0, 0] = 0  # code 0 = 2^-127 (T/test_mx_adapter.py:621-660)
    t = MXWeight(torch.from_numpy(q).view(torch.float8_e4m3fn).to(DEV), torch.from_numpy(s).to(DEV),
                 torch.float8_e4m3fn, 32, torch.bfloat16, False, "floor")
    b = torch.zeros(rows, 16, dtype=torch.bfloat16, device=DEV)
    a = torch.zeros(16, cols, dtype=torch.bfloat16, device=DEV)
    MxAdapter.merge_lora_(t, b, a, 1.0)
    dense = O.mx_dequant(q, s, O.DT_E4M3, cols)
    rq, rs = O.mx_requant(dense, O.DT_E4M3, 0)
    assert np.array_equal(u8_np(t.qdata), rq)
    assert np.array_equal(u8_np(t.scale), rs)


# N % 128 == 0 with bf16 factors takes the one-block-per-lane kernel (k_q8_fast);
# the other shapes take the generic block kernel.  Rank <= 16 with an even
# number of 16-row groups rounds to nearest two groups per item ((30, 256):
# a short last group; (47, 384): three groups, one per item).
@pytest.mark.parametrize("shape,rank,strength", [
    ((13824 // 64, 5120), 16, 1.0), ((48, 96), 5, 1.0), ((33, 64), 16, 1.0),
    ((37, 384), 32, 0.5), ((40, 256), 64, -1.25), ((17, 128), 16, 2.0),
    ((30, 256), 12, 1.0), ((47, 384), 16, 0.75)])
@pytest.mark.parametrize("sr", [False, True])
def test_q8_0_merge(shape, rank, strength, sr):
    rows, cols = shape
    w = normal_bf16(shape, 0.02, 1)
    packed = O.q8_0_requant(bf16_np(w))
    b, a = lora_factors(rows, cols, rank, 2)
    pd = torch.from_numpy(packed).to(DEV)
    base = K.dequantize_gguf(pd, 8)
    obase = O.q8_0_dequant(packed, cols)
    assert np.array_equal(bf16_np(base), obase)
    dense = K.dequantize_gguf(pd, 8, lora=(b.to(DEV), a.to(DEV), strength))
    assert_merged_close(bf16_np(dense), O.merge_dense(obase, bf16_np(b), bf16_np(a), strength), obase)
    seed = derive_seed("q8.fused", rows) if sr else None
    out = K.merge_q8_0_lora(pd, b.to(DEV), a.to(DEV), strength, rounding_seed=seed)
    ref = O.q8_0_requant(bf16_np(dense), sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(u8_np(out), ref)
    rq = K.requantize_q8_0(dense, rounding_seed=seed)
    assert np.array_equal(u8_np(rq), ref)
    # in place (the output aliases the input) gives the same bytes
    K.merge_q8_0_lora(pd, b.to(DEV), a.to(DEV), strength, rounding_seed=seed, out=pd)
    assert np.array_equal(u8_np(pd), ref)


@pytest.mark.parametrize("sr", [False, True])
def test_q8_0_merge_config4_full_size(sr):
    # [13824, 5120] rank 16, strength 1.0, RTN (and SR): every
    # wave of the persistent kernel walks many items
    rows, cols = 13824, 5120
    packed = O.q8_0_requant(bf16_np(normal_bf16((rows, cols), 0.02, 11)))
    b, a = lora_factors(rows, cols, 16, 12)
    pd = torch.from_numpy(packed).to(DEV)
    dense = K.dequantize_gguf(pd, 8, lora=(b.to(DEV), a.to(DEV), 1.0))
    seed = derive_seed("model.layers.0.mlp.down_proj.weight", 0) if sr else None
    out = K.merge_q8_0_lora(pd, b.to(DEV), a.to(DEV), 1.0, rounding_seed=seed)
    ref = O.q8_0_requant(bf16_np(dense), sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(u8_np(out), ref)


def test_gguf_adapter_in_place():
    rows, cols = 32, 256
    packed = O.q8_0_requant(bf16_np(normal_bf16((rows, cols), 0.02, 3)))
    t = GGUFWeight(torch.from_numpy(packed).to(DEV), quant_type=8)
    ptr = t.data_ptr()
    assert GgufAdapter.logical_shape(t) == (rows, cols)
    b, a = lora_factors(rows, cols, 16, 4)
    dense = K.dequantize_gguf(torch.from_numpy(packed).to(DEV), 8, lora=(b.to(DEV), a.to(DEV), 1.0))
    GgufAdapter.merge_lora_(t, b.to(DEV), a.to(DEV), 1.0)
    assert t.data_ptr() == ptr
    assert np.array_equal(u8_np(t.as_subclass(torch.Tensor)), O.q8_0_requant(bf16_np(dense)))


@pytest.mark.parametrize("shape,rank,strength", [((4096, 4096), 16, 1.0), ((24, 69), 5, 0.5), ((64, 1000), 64, 0.75)])
def test_dense_bf16_merge(shape, rank, strength):
    rows, cols = shape
    w = normal_bf16(shape, 0.02, 0)
    b, a = lora_factors(rows, cols, rank, 1, a_std=1.0 / rank)
    wd = w.to(DEV)
    RegularAdapter.merge_lora_(wd, b.to(DEV), a.to(DEV), strength)
    ref = O.merge_dense(bf16_np(w), bf16_np(b), bf16_np(a), strength)
    assert_merged_close(bf16_np(wd), ref, bf16_np(w))
