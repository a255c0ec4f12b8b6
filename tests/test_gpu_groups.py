"""Per-group INT8 and scaled-FP8 layouts (TorchAO block_size (1, g), g < N) on the GPU vs the oracle.

The reference handles them with the per-row recipe applied to each group of
g consecutive elements of a row, one qparam per group, stored [M, N / g]
(P/_triton_int8_lora.py:251-264, P/float8_adapter.py:63-98).  Contract as for
per-row: requant bit-exact, dense merge within the stated tolerance, fused
merge bit-exact against the requant of the GPU's own dense merge.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_merged_close, bf16_np, lora_factors, normal_bf16, u8_np

pytestmark = pytest.mark.gpu

K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import Float8Adapter, Float8Weight, Int8Adapter, Int8Weight, derive_seed  # noqa: E402

DEV = "cuda"
FP8 = {"e4m3": (torch.float8_e4m3fn, O.DT_E4M3), "e5m2": (torch.float8_e5m2, O.DT_E5M2)}


def _scale_np(s: torch.Tensor) -> np.ndarray:
    s = s.detach().cpu().contiguous()
    return bf16_np(s).reshape(-1) if s.dtype is torch.bfloat16 else s.numpy().reshape(-1)


def _dense(shape, seed):
    d = normal_bf16(shape, 0.02, seed)
    d[1] = 0                       # all-zero groups -> eps scale
    d[2, :5] *= 50                 # a group with a large amax
    d[3, : shape[1] // 2] = d[3, : shape[1] // 2].abs()  # non-negative groups (asymmetric zero points)
    return d


def _int8_encode(dense, g, scale_dtype, asym):
    sdt = O.DT_F32 if scale_dtype is torch.float32 else O.DT_BF16
    q, s, z = O.int8_requant(bf16_np(dense), g, scale_dt=sdt, asymmetric=asym)
    rows, cols = dense.shape
    st = torch.from_numpy(s.reshape(rows, cols // g))
    if scale_dtype is torch.bfloat16:
        st = st.view(torch.bfloat16)
    return torch.from_numpy(q), st, torch.from_numpy(z.reshape(rows, cols // g)) if asym else None


@pytest.mark.parametrize("shape,g", [((40, 256), 16), ((40, 256), 32), ((33, 512), 64), ((16, 1024), 128),
                                     ((20, 1024), 256), ((24, 96), 32), ((17, 4096), 512)])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("sr", [False, True])
def test_int8_group_requant_bit_exact(shape, g, scale_dtype, asym, sr):
    rows, cols = shape
    dense = _dense(shape, 3)
    seed = derive_seed("int8.group.requant", g) if sr else None
    q, s, z = K.requantize_int8(dense.to(DEV), (1, g), scale_dtype=scale_dtype, asymmetric=asym, rounding_seed=seed)
    assert tuple(s.shape) == (rows, cols // g)
    sdt = O.DT_F32 if scale_dtype is torch.float32 else O.DT_BF16
    oq, os_, oz = O.int8_requant(bf16_np(dense), g, scale_dt=sdt, asymmetric=asym,
                                 sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(_scale_np(s), os_)
    if asym:
        assert np.array_equal(z.cpu().numpy().reshape(-1), oz)


@pytest.mark.parametrize("shape,g,rank,strength", [((40, 256), 16, 16, 1.0), ((40, 256), 32, 32, 0.5),
                                                   ((33, 512), 64, 16, 1.0), ((16, 1024), 128, 64, -0.75),
                                                   ((24, 96), 32, 5, 1.0), ((20, 2048), 256, 16, 1.0)])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("sr", [False, True])
def test_int8_group_fused_equals_requant_of_gpu_dense(shape, g, rank, strength, scale_dtype, asym, sr):
    rows, cols = shape
    q, s, z = _int8_encode(_dense(shape, 4), g, scale_dtype, asym)
    b, a = lora_factors(rows, cols, rank, 5)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    zd = None if z is None else z.to(DEV)
    sdt = O.DT_F32 if scale_dtype is torch.float32 else O.DT_BF16
    base = K.dequantize_int8(qd, sd, zd, (1, g))
    obase = O.int8_dequant(q.numpy(), _scale_np(s) if scale_dtype is torch.float32 else _scale_np(s).view(np.uint16),
                           None if z is None else z.numpy(), g, scale_dt=sdt)
    assert np.array_equal(bf16_np(base), obase)
    dense = K.dequantize_int8(qd, sd, zd, (1, g), lora=(bd, ad, strength))
    assert_merged_close(bf16_np(dense), O.merge_dense(obase, bf16_np(b), bf16_np(a), strength), obase)
    seed = derive_seed("int8.group.fused", g) if sr else None
    oq, os_, oz = K.merge_int8_lora(qd, sd, zd, (1, g), bd, ad, strength, asymmetric=asym, reduce_range=False,
                                    rounding_seed=seed)
    rq, rs, rz = O.int8_requant(bf16_np(dense), g, scale_dt=sdt, asymmetric=asym,
                                sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(oq.cpu().numpy(), rq)
    assert np.array_equal(_scale_np(os_), rs)
    if asym:
        assert np.array_equal(oz.cpu().numpy().reshape(-1), rz)


def test_int8_group_reduce_range_and_fp16():
    rows, cols, g = 24, 512, 64
    dense = _dense((rows, cols), 6).to(torch.float16)
    seed = derive_seed("int8.group.rr", 0)
    q, s, _ = K.requantize_int8(dense.to(DEV), (1, g), reduce_range=True, rounding_seed=seed)
    oq, os_, _ = O.int8_requant(dense.view(torch.int16).numpy().view(np.uint16), g, cd=O.DT_F16, reduce_range=True,
                                sr_mode=O.SR_PHILOX8, seed=seed)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(_scale_np(s), os_)
    assert q.min() >= -64 and q.max() <= 63


def test_int8_group_adapter_in_place():
    rows, cols, g = 48, 1024, 128
    q, s, _ = _int8_encode(_dense((rows, cols), 7), g, torch.float32, False)
    b, a = lora_factors(rows, cols, 16, 8)
    t = Int8Weight(q.clone().to(DEV), s.clone().to(DEV), (1, g), torch.bfloat16)
    ptrs = (t.qdata.data_ptr(), t.scale.data_ptr())
    Int8Adapter.validate_lora_merge(t, b.to(DEV), a.to(DEV), 1.0)
    seed = derive_seed("layers.0.mlp.weight", 0)
    dense = K.dequantize_int8(q.to(DEV), s.to(DEV), None, (1, g), lora=(b.to(DEV), a.to(DEV), 1.0))
    Int8Adapter.merge_lora_(t, b.to(DEV), a.to(DEV), 1.0, rounding_seed=seed)
    assert (t.qdata.data_ptr(), t.scale.data_ptr()) == ptrs
    rq, rs, _ = O.int8_requant(bf16_np(dense), g, sr_mode=O.SR_PHILOX8, seed=seed)
    assert np.array_equal(t.qdata.cpu().numpy(), rq)
    assert np.array_equal(_scale_np(t.scale), rs)


@pytest.mark.parametrize("elem", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape,g,rank,strength", [((40, 256), 32, 16, 1.0), ((16, 1024), 128, 64, 0.5),
                                                   ((24, 96), 16, 5, 1.0), ((33, 512), 64, 32, -1.0)])
@pytest.mark.parametrize("sr", [False, True])
def test_fp8_group_fused_equals_requant_of_gpu_dense(elem, shape, g, rank, strength, sr):
    tdt, fmt = FP8[elem]
    rows, cols = shape
    oq0, os0 = O.fp8_requant(bf16_np(_dense(shape, 9)), g, fmt=fmt)
    q = torch.from_numpy(oq0).view(tdt)
    s = torch.from_numpy(os0.reshape(rows, cols // g))
    b, a = lora_factors(rows, cols, rank, 10)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    base = K.dequantize_float8(qd, sd, (1, g))
    obase = O.fp8_dequant(oq0, os0, g, fmt=fmt)
    assert np.array_equal(bf16_np(base), obase)
    dense = K.dequantize_float8(qd, sd, (1, g), lora=(bd, ad, strength))
    assert_merged_close(bf16_np(dense), O.merge_dense(obase, bf16_np(b), bf16_np(a), strength), obase)
    seed = derive_seed("fp8.group.fused", g) if sr else None
    mq, ms = K.merge_float8_lora(qd, sd, (1, g), bd, ad, strength, rounding_seed=seed)
    rq, rs = O.fp8_requant(bf16_np(dense), g, fmt=fmt, sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(u8_np(mq), rq)
    assert np.array_equal(ms.cpu().numpy().reshape(-1), rs)
    rq2, rs2 = K.requantize_float8(dense, (1, g), fp8_dtype=tdt, rounding_seed=seed)
    assert np.array_equal(u8_np(rq2), rq)
    assert np.array_equal(rs2.cpu().numpy().reshape(-1), rs)


def test_fp8_group_adapter_in_place():
    rows, cols, g = 32, 512, 128
    oq0, os0 = O.fp8_requant(bf16_np(_dense((rows, cols), 11)), g)
    t = Float8Weight(torch.from_numpy(oq0).view(torch.float8_e4m3fn).to(DEV),
                     torch.from_numpy(os0.reshape(rows, cols // g)).to(DEV), (1, g), torch.bfloat16)
    b, a = lora_factors(rows, cols, 16, 12)
    dense = K.dequantize_float8(t.qdata.clone(), t.scale.clone(), (1, g), lora=(b.to(DEV), a.to(DEV), 1.0))
    Float8Adapter.validate_lora_merge(t, b.to(DEV), a.to(DEV), 1.0)
    Float8Adapter.merge_lora_(t, b.to(DEV), a.to(DEV), 1.0)
    rq, rs = O.fp8_requant(bf16_np(dense), g)
    assert np.array_equal(u8_np(t.qdata), rq)
    assert np.array_equal(t.scale.cpu().numpy().reshape(-1), rs)


def test_group_layouts_rejected_cleanly():
    q = torch.zeros(16, 192, dtype=torch.int8, device=DEV)
    s = torch.ones(16, 4, device=DEV)
    b = torch.zeros(16, 16, dtype=torch.bfloat16, device=DEV)
    a = torch.zeros(16, 192, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="per-group"):
        K.merge_int8_lora(q, s, None, (1, 48), b, a, 1.0, asymmetric=False, reduce_range=False)
    with pytest.raises(ValueError, match="per-group"):
        K.merge_float8_lora(q.view(torch.float8_e4m3fn), s, (1, 48), b, a, 1.0)
