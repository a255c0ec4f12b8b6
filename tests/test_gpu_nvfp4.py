"""NVFP4 (two-level and single-level, regular and swizzled scales) merge vs the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_merged_close, bf16_np, lora_factors, normal_bf16, u8_np

pytestmark = pytest.mark.gpu

K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import NVFP4Weight, Nvfp4Adapter, derive_seed  # noqa: E402

DEV = "cuda"


def _encode(w: torch.Tensor, two_level: bool, swizzled: bool):
    """Initial NVFP4 encode of a bf16 weight with the oracle (the reference's requant recipe)."""
    q, s, pts = O.nvfp4_requant(bf16_np(w), swizzled=swizzled, two_level=two_level)
    qt = torch.from_numpy(q)
    st = torch.from_numpy(s).view(torch.float8_e4m3fn)
    pt = None if pts is None else torch.from_numpy(pts.reshape(()))
    return qt, st, pt


@pytest.mark.parametrize("shape", [(16, 64), (200, 1024), (128, 4096), (33, 96)])
@pytest.mark.parametrize("two_level", [True, False])
@pytest.mark.parametrize("swizzled", [False, True])
@pytest.mark.parametrize("sr", [False, True])
def test_nvfp4_requant_bit_exact(shape, two_level, swizzled, sr):
    dense = normal_bf16(shape, 0.02, 9)
    dense[0, :16] = 0
    dense[1, 16:32] = torch.tensor([-0.0] * 16, dtype=torch.bfloat16)
    seed = derive_seed("nvfp4.requant", shape[1]) if sr else None
    q, s, pts = K.requantize_nvfp4(dense.to(DEV), two_level=two_level, swizzled=swizzled, rounding_seed=seed)
    oq, os_, opts = O.nvfp4_requant(bf16_np(dense), swizzled=swizzled, two_level=two_level,
                                    sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(u8_np(q), oq)
    assert np.array_equal(u8_np(s), os_)
    if two_level:
        assert np.array_equal(pts.cpu().numpy().reshape(-1), opts)


@pytest.mark.parametrize("shape,rank", [((128, 4096), 16), ((48, 256), 32), ((16, 64), 5), ((40, 384), 64), ((300, 256), 16)])
@pytest.mark.parametrize("two_level", [True, False])
@pytest.mark.parametrize("swizzled", [False, True])
@pytest.mark.parametrize("sr", [False, True])
def test_nvfp4_fused_equals_requant_of_gpu_dense(shape, rank, two_level, swizzled, sr):
    rows, cols = shape
    w = normal_bf16(shape, 0.02, 1)
    q, s, pts = _encode(w, two_level, swizzled)
    b, a = lora_factors(rows, cols, rank, 2)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    ptsd = None if pts is None else pts.to(DEV)
    base = K.dequantize_nvfp4(qd, sd, ptsd, swizzled=swizzled)
    obase = O.nvfp4_dequant(q.numpy(), u8_np(s), None if pts is None else pts.numpy(), swizzled=swizzled)
    assert np.array_equal(bf16_np(base), obase)
    dense = K.dequantize_nvfp4(qd, sd, ptsd, swizzled=swizzled, lora=(bd, ad, 1.0))
    omerged = O.merge_dense(obase, bf16_np(b), bf16_np(a), 1.0, keep_zero_update=True)
    assert_merged_close(bf16_np(dense), omerged, obase)
    seed = derive_seed("nvfp4.fused", rows) if sr else None
    oq, os_, opts = K.merge_nvfp4_lora(qd, sd, ptsd, 16, swizzled, bd, ad, 1.0, rounding_seed=seed)
    rq, rs, rpts = O.nvfp4_requant(bf16_np(dense), swizzled=swizzled, two_level=two_level,
                                   sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(u8_np(oq), rq)
    assert np.array_equal(u8_np(os_), rs)
    if two_level:
        assert np.array_equal(opts.cpu().numpy().reshape(-1), rpts)


def test_nvfp4_adapter_in_place_and_replay():
    rows, cols, rank = 64, 512, 16
    w = normal_bf16((rows, cols), 0.02, 5)
    q, s, pts = _encode(w, True, True)
    b, a = lora_factors(rows, cols, rank, 6)
    outs = []
    for key in ("a.weight", "a.weight", "b.weight"):
        t = NVFP4Weight(q.clone().to(DEV), s.clone().to(DEV), pts.clone().to(DEV), 16, torch.bfloat16, True)
        ptr = t.qdata.data_ptr()
        Nvfp4Adapter.merge_lora_(t, b.to(DEV), a.to(DEV), 0.75, rounding_seed=derive_seed(key, 0))
        assert t.qdata.data_ptr() == ptr
        outs.append(t)
    assert torch.equal(outs[0].qdata, outs[1].qdata) and not torch.equal(outs[0].qdata, outs[2].qdata)
    assert torch.equal(outs[0].scale.view(torch.uint8), outs[2].scale.view(torch.uint8))
    assert torch.equal(outs[0].per_tensor_scale, outs[2].per_tensor_scale)


def test_nvfp4_zero_weight_global_scale_is_eps():
    rows, cols = 16, 64
    q = torch.zeros(rows, cols // 2, dtype=torch.uint8, device=DEV)
    s = torch.zeros(rows, cols // 16, dtype=torch.float8_e4m3fn, device=DEV)
    pts = torch.ones((), device=DEV)
    b = torch.zeros(rows, 16, dtype=torch.bfloat16, device=DEV)
    a = torch.zeros(16, cols, dtype=torch.bfloat16, device=DEV)
    oq, _os, opts = K.merge_nvfp4_lora(q, s, pts, 16, False, b, a, 1.0)
    assert float(opts) == torch.finfo(torch.float32).eps
    assert not oq.any()


def test_nvfp4_sr_two_neighbours_and_unbiased():
    rows, cols = 64, 1024
    dense = torch.full((rows, cols), 0.8, dtype=torch.bfloat16)
    dense[:, ::16] = 6.0  # block amax 6 -> block scale 1 (single level)
    x = float(torch.tensor(0.8, dtype=torch.bfloat16).float())
    samples = []
    for i in range(4):
        q, _s, _ = K.requantize_nvfp4(dense.to(DEV), two_level=False, rounding_seed=derive_seed("nvfp4-sr", i))
        codes = np.stack([u8_np(q) & 15, u8_np(q) >> 4], axis=-1).reshape(rows, cols)
        mask = np.ones(cols, bool)
        mask[::16] = False
        samples.append(O.E2M1_VALUES[codes[:, mask]])
    vals = np.concatenate([v.reshape(-1) for v in samples])
    assert set(np.unique(vals).tolist()) == {0.5, 1.0}
    assert float(vals.mean()) == pytest.approx(x, abs=3e-3)


@pytest.mark.parametrize("two_level", [True, False])
@pytest.mark.parametrize("sr", [False, True])
def test_nvfp4_zero_update_rows_keep_signed_zero_codes(two_level, sr):
    # B rows of zeros make delta == 0 exactly: the reference keeps the base
    # there, including -0.0 (code 8), where base + 0 would give +0.0
    # (P/_triton_nvfp4_lora.py:183-186)
    rows, cols, rank = 64, 512, 16
    w = normal_bf16((rows, cols), 0.02, 21)
    q, s, pts = _encode(w, two_level, False)
    assert ((u8_np(q) & 15) == 8).any() or ((u8_np(q) >> 4) == 8).any()
    b, a = lora_factors(rows, cols, rank, 22)
    b[::3] = 0.0
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    ptsd = None if pts is None else pts.to(DEV)
    dense = K.dequantize_nvfp4(qd, sd, ptsd, lora=(bd, ad, 1.0))
    seed = derive_seed("nvfp4.zero_rows", 0) if sr else None
    oq, os_, opts = K.merge_nvfp4_lora(qd, sd, ptsd, 16, False, bd, ad, 1.0, rounding_seed=seed)
    rq, rs, rpts = O.nvfp4_requant(bf16_np(dense), two_level=two_level, sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF,
                                   seed=seed or 0)
    assert np.array_equal(u8_np(oq), rq)
    assert np.array_equal(u8_np(os_), rs)


@pytest.mark.parametrize("two_level", [True, False])
@pytest.mark.parametrize("sr", [False, True])
def test_nvfp4_isolated_zero_updates_keep_signed_zero_codes(two_level, sr):
    # One column per 16-element block gets an exactly zero update (its A
    # column is zero) while the other 15 do not, so only the per-element rule
    # keeps -0.0 (code 8) there (P/_triton_nvfp4_lora.py:183-186).  This is
    # the pattern of the two elements (737, 3340) and (6519, 2489) of the
    # 8B layer's up_proj whose codes once differed between launches.
    rows, cols, rank = 1024, 4096, 16
    w = normal_bf16((rows, cols), 0.02, 31)
    q, s, pts = _encode(w, two_level, False)
    b, a = lora_factors(rows, cols, rank, 32)
    a[:, 5::16] = 0.0
    codes = np.stack([u8_np(q) & 15, u8_np(q) >> 4], axis=-1).reshape(rows, cols)
    assert (codes[:, 5::16] == 8).sum() > 100  # many -0 bases under a zero update
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    ptsd = None if pts is None else pts.to(DEV)
    dense = K.dequantize_nvfp4(qd, sd, ptsd, lora=(bd, ad, 2.0))
    seed = derive_seed("nvfp4.isolated_zero", 0) if sr else None
    rq, rs, rpts = O.nvfp4_requant(bf16_np(dense), two_level=two_level, sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF,
                                   seed=seed or 0)
    oq, os_, opts = K.merge_nvfp4_lora(qd, sd, ptsd, 16, False, bd, ad, 2.0, rounding_seed=seed)
    assert np.array_equal(u8_np(oq), rq)
    assert np.array_equal(u8_np(os_), rs)
    from piper_offload_amd.stack import StackTarget, merge_nvfp4_stack

    t = StackTarget(NVFP4Weight(qd.clone(), sd.clone(), None if ptsd is None else ptsd.clone(), 16, torch.bfloat16,
                                False), bd, ad, 2.0, seed or 0)
    merge_nvfp4_stack([t], stochastic=sr)
    assert np.array_equal(u8_np(t.weight.qdata), rq)
    assert np.array_equal(u8_np(t.weight.scale), rs)
