"""INT8 per-row / per-tensor merge on the GPU vs the CPU oracle.

Contract (the same for every format):
  * requant of a given dense tensor is bit-exact (codes, scales, zero points),
    for round-to-nearest and for stochastic rounding (same Philox stream);
  * the dense merged weight agrees with the oracle within 1 bf16 ulp on at
    most 1e-3 of the elements (the MFMA sums B@A in a hardware-defined order);
  * the fused merge equals the oracle requant of the GPU's own dense merge,
    bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_merged_close, bf16_np, int8_initial, lora_factors, normal_bf16, np_bf16

pytestmark = pytest.mark.gpu

K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import Int8Adapter, Int8Weight, derive_seed  # noqa: E402

DEV = "cuda"
MISMATCH_FRACTION = 1e-3  # dense merged values allowed to differ by 1 bf16 ulp


def _scale_np(s: torch.Tensor) -> np.ndarray:
    s = s.detach().cpu().contiguous()
    if s.dtype is torch.bfloat16:
        return bf16_np(s).reshape(-1)
    return s.numpy().reshape(-1)


def _dense(shape, seed, std=0.02):
    d = normal_bf16(shape, std, seed)
    if shape[0] > 3:
        d[1] = 0  # an all-zero row -> eps scale
        d[2, : min(5, shape[1])] *= 50  # a row with a large amax
    return d


@pytest.mark.parametrize("shape", [(24, 69), (64, 4096), (33, 256), (16, 1024)])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("sr", [False, True])
def test_int8_requant_bit_exact(shape, scale_dtype, asym, sr):
    dense = _dense(shape, 11)
    seed = derive_seed("int8.requant", shape[0]) if sr else None
    q, s, z = K.requantize_int8(dense.to(DEV), (1, shape[1]), scale_dtype=scale_dtype, asymmetric=asym,
                                rounding_seed=seed)
    oq, os_, oz = O.int8_requant(bf16_np(dense), shape[1], scale_dt=O.DT_F32 if scale_dtype is torch.float32 else O.DT_BF16,
                                 asymmetric=asym, sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(_scale_np(s), os_)
    if asym:
        assert np.array_equal(z.cpu().numpy().reshape(-1), oz)


@pytest.mark.parametrize("reduce_range", [False, True])
@pytest.mark.parametrize("per_tensor", [False, True])
def test_int8_requant_reduce_range_and_per_tensor(reduce_range, per_tensor):
    shape = (40, 96)
    dense = _dense(shape, 5)
    block = shape if per_tensor else (1, shape[1])
    group = shape[0] * shape[1] if per_tensor else shape[1]
    q, s, _ = K.requantize_int8(dense.to(DEV), block, reduce_range=reduce_range)
    oq, os_, _ = O.int8_requant(bf16_np(dense), group, reduce_range=reduce_range)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(_scale_np(s), os_)
    lo, hi = (-64, 63) if reduce_range else (-128, 127)
    assert q.min().item() >= lo and q.max().item() <= hi


def _int8_case(rows, cols, rank, seed=0, scale_dtype=torch.float32):
    w = normal_bf16((rows, cols), 0.02, seed)
    q, s = int8_initial(w)
    s = s.to(scale_dtype)
    b, a = lora_factors(rows, cols, rank, seed + 1)
    return q, s, b, a


@pytest.mark.parametrize("shape,rank", [((64, 4096), 32), ((24, 69), 5), ((48, 640), 16), ((32, 512), 64)])
def test_int8_dequant_and_dense_merge(shape, rank):
    rows, cols = shape
    q, s, b, a = _int8_case(rows, cols, rank)
    base = K.dequantize_int8(q.to(DEV), s.to(DEV), None, (1, cols))
    obase = O.int8_dequant(q.numpy(), s.numpy(), None, cols)
    assert np.array_equal(bf16_np(base), obase)
    merged = K.dequantize_int8(q.to(DEV), s.to(DEV), None, (1, cols), lora=(b.to(DEV), a.to(DEV), 0.5))
    omerged = O.merge_dense(obase, bf16_np(b), bf16_np(a), 0.5)
    assert_merged_close(bf16_np(merged), omerged, obase)


# long rows (more 64-column tiles per wave than the 8-tile register cache):
# rank 16 takes 16-wave workgroups with 4 more tiles per wave in LDS (40 x 14336
# also merges its last tiles twice, 17 x 12288 fills registers and LDS
# exactly), rank 32 RTN and rank 64 the 16-tile cache, rank 32 SR recomputes
# the surplus tiles
@pytest.mark.parametrize("shape,rank,strength", [((64, 4096), 32, 0.5), ((24, 69), 5, 0.75), ((40, 1024), 16, 1.0),
                                                 ((32, 2048), 64, 1.0), ((16, 8192), 32, 0.5),
                                                 ((40, 14336), 16, 1.0), ((17, 12288), 16, 0.5),
                                                 ((20, 8192), 64, 0.75), ((16400, 4608), 64, 1.0),
                                                 ((16400, 1024), 16, 0.5)])
@pytest.mark.parametrize("sr", [False, True])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_int8_fused_equals_requant_of_gpu_dense(shape, rank, strength, sr, scale_dtype):
    rows, cols = shape
    q, s, b, a = _int8_case(rows, cols, rank, scale_dtype=scale_dtype)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    seed = derive_seed("int8.fused", rows) if sr else None
    oq, os_, oz = K.merge_int8_lora(qd, sd, None, (1, cols), bd, ad, strength, asymmetric=False, reduce_range=False,
                                    rounding_seed=seed)
    dense = K.dequantize_int8(qd, sd, None, (1, cols), lora=(bd, ad, strength))
    rq, rs, _ = O.int8_requant(bf16_np(dense), cols, scale_dt=O.DT_F32 if scale_dtype is torch.float32 else O.DT_BF16,
                               sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(oq.cpu().numpy(), rq)
    assert np.array_equal(_scale_np(os_), rs)
    assert not oz.any()


# The 8-wave row kernels read the dequantized base from a per-row table of the
# 256 code bytes built from the row's scale (entries for negative codes are the
# negated positive ones).  Scales of exactly 0, negative scales and full-range
# codes (-128 included) against the dense merge, which converts and scales each
# code: rank 16 and rank 32 take the table, 14336 columns the 16-wave kernel.
@pytest.mark.parametrize("shape,rank", [((40, 1024), 16), ((64, 4096), 32), ((33, 14336), 16)])
@pytest.mark.parametrize("sr", [False, True])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_int8_fused_table_edge_scales(shape, rank, sr, scale_dtype):
    rows, cols = shape
    q, s, b, a = _int8_case(rows, cols, rank, seed=7, scale_dtype=scale_dtype)
    g = torch.Generator().manual_seed(11)
    q[3] = torch.randint(-128, 128, (cols,), generator=g, dtype=torch.int8)  # every code byte
    q[3, :4] = torch.tensor([-128, 127, 0, -1], dtype=torch.int8)
    s[3] = -s[3]          # a negative scale
    s[5] = 0.0            # a zero scale with non-zero codes
    s[rows - 1] = -0.0    # a negative zero
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    seed = derive_seed("int8.table", rows) if sr else None
    oq, os_, _ = K.merge_int8_lora(qd, sd, None, (1, cols), bd, ad, 1.0, asymmetric=False, reduce_range=False,
                                   rounding_seed=seed)
    dense = K.dequantize_int8(qd, sd, None, (1, cols), lora=(bd, ad, 1.0))
    rq, rs, _ = O.int8_requant(bf16_np(dense), cols, scale_dt=O.DT_F32 if scale_dtype is torch.float32 else O.DT_BF16,
                               sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    assert np.array_equal(oq.cpu().numpy(), rq)
    assert np.array_equal(_scale_np(os_), rs)


# two-pass long rows (rank above 32, rows of more than 4096 columns): rows that
# end inside a 64-row wave tile and a partial last tile range, merged out of
# place and then in place (outputs aliasing the inputs)
@pytest.mark.parametrize("shape,rank", [((70, 8256), 64), ((130, 4160), 48)])
@pytest.mark.parametrize("sr", [False, True])
def test_int8_two_pass_rows_and_in_place(shape, rank, sr):
    rows, cols = shape
    q, s, b, a = _int8_case(rows, cols, rank, seed=21)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    seed = derive_seed("int8.two-pass", rows) if sr else None
    dense = K.dequantize_int8(qd, sd, None, (1, cols), lora=(bd, ad, 0.5))
    rq, rs, _ = O.int8_requant(bf16_np(dense), cols, sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    oq, os_, oz = K.merge_int8_lora(qd, sd, None, (1, cols), bd, ad, 0.5, asymmetric=False, reduce_range=False,
                                    rounding_seed=seed)
    assert np.array_equal(oq.cpu().numpy(), rq)
    assert np.array_equal(_scale_np(os_), rs)
    K.merge_int8_lora_into(qd, sd, None, (1, cols), bd, ad, 0.5, asymmetric=False, reduce_range=False,
                           rounding_seed=seed, out_qdata=qd, out_scale=sd, out_zero_point=None)
    assert np.array_equal(qd.cpu().numpy(), rq)
    assert np.array_equal(_scale_np(sd), rs)


def test_int8_fused_sr_two_neighbours_and_unbiased():
    """The fused merge's stochastic codes (Philox4x32-7 draws) over 64 seeds:
    every code is floor or ceil of merged / scale, and the mean code is
    merged / scale within 0.005 overall and within 0.01 in each tenth of the
    fractional part (the reference's contract: E[code] = x, P(up) = frac)."""
    rows, cols, rank = 64, 4096, 16
    q, s, b, a = _int8_case(rows, cols, rank, seed=31)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    dense = K.dequantize_int8(qd, sd, None, (1, cols), lora=(bd, ad, 0.5))
    acc = np.zeros((rows, cols), np.float64)
    n_seeds = 64
    for i in range(n_seeds):
        oq, os_, _ = K.merge_int8_lora(qd, sd, None, (1, cols), bd, ad, 0.5, asymmetric=False, reduce_range=False,
                                       rounding_seed=derive_seed("int8.sr-stats", i))
        if i == 0:
            y = O.bf16_to_f32(bf16_np(dense)).astype(np.float64) / _scale_np(os_).astype(np.float64)[:, None]
            yc = np.clip(y, -128, 127)
        qf = oq.cpu().numpy().astype(np.float64)
        assert np.all((qf == np.floor(yc)) | (qf == np.ceil(yc)))
        acc += qf
    interior = (y > -128) & (y < 127) & (y != np.floor(y))
    err = (acc / n_seeds - y)[interior]
    assert abs(err.mean()) < 0.005
    frac = (y - np.floor(y))[interior]
    for lo in np.arange(0.0, 1.0, 0.1):
        sel = (frac >= lo) & (frac < lo + 0.1)
        assert abs(err[sel].mean()) < 0.01, (lo, err[sel].mean())


def test_int8_fused_vs_oracle_pipeline():
    rows, cols, rank = 64, 4096, 32
    q, s, b, a = _int8_case(rows, cols, rank)
    oq, os_, _ = K.merge_int8_lora(q.to(DEV), s.to(DEV), None, (1, cols), b.to(DEV), a.to(DEV), 0.5,
                                   asymmetric=False, reduce_range=False)
    dense = O.merge_dense(O.int8_dequant(q.numpy(), s.numpy(), None, cols), bf16_np(b), bf16_np(a), 0.5)
    rq, rs, _ = O.int8_requant(dense, cols)
    mism = (oq.cpu().numpy() != rq)
    assert mism.mean() <= MISMATCH_FRACTION
    got = oq.cpu().float() * os_.cpu().float()
    want = torch.from_numpy(rq.astype(np.float32)) * torch.from_numpy(rs).reshape(-1, 1)
    step = float(torch.from_numpy(rs).max())
    assert float((got - want).abs().max()) <= 1.01 * step


def test_int8_asymmetric_merge():
    rows, cols, rank = 32, 256, 16
    w = normal_bf16((rows, cols), 0.02, 3) + 0.01
    wf = w.float()
    mn, mx = wf.amin(1, keepdim=True).clamp(max=0), wf.amax(1, keepdim=True).clamp(min=0)
    s = ((mx - mn) / 255).clamp_min(1e-6)
    zp = (-128 - torch.round(mn / s)).clamp(-128, 127).to(torch.int8)
    q = (torch.round(wf / s) + zp.float()).clamp(-128, 127).to(torch.int8)
    b, a = lora_factors(rows, cols, rank, 4)
    oq, os_, oz = K.merge_int8_lora(q.to(DEV), s.to(DEV), zp.to(DEV), (1, cols), b.to(DEV), a.to(DEV), 1.0,
                                    asymmetric=True, reduce_range=False)
    dense = K.dequantize_int8(q.to(DEV), s.to(DEV), zp.to(DEV), (1, cols), lora=(b.to(DEV), a.to(DEV), 1.0))
    rq, rs, rz = O.int8_requant(bf16_np(dense), cols, asymmetric=True)
    assert np.array_equal(oq.cpu().numpy(), rq)
    assert np.array_equal(os_.cpu().numpy().reshape(-1), rs)
    assert np.array_equal(oz.cpu().numpy().reshape(-1), rz)


def test_int8_per_tensor_merge():
    rows, cols, rank = 48, 384, 16
    q, s, b, a = _int8_case(rows, cols, rank)
    s_t = s.max().reshape(1, 1)
    oq, os_, _ = K.merge_int8_lora(q.to(DEV), s_t.to(DEV), None, (rows, cols), b.to(DEV), a.to(DEV), 1.0,
                                   asymmetric=False, reduce_range=False)
    dense = K.dequantize_int8(q.to(DEV), s_t.to(DEV), None, (rows, cols), lora=(b.to(DEV), a.to(DEV), 1.0))
    rq, rs, _ = O.int8_requant(bf16_np(dense), rows * cols)
    assert np.array_equal(oq.cpu().numpy(), rq)
    assert np.array_equal(os_.cpu().numpy().reshape(-1), rs)


def test_int8_adapter_merges_in_place():
    rows, cols, rank = 32, 512, 16
    q, s, b, a = _int8_case(rows, cols, rank)
    target = Int8Weight(q.clone().to(DEV), s.clone().to(DEV), (1, cols), torch.bfloat16)
    ptr_q, ptr_s = target.qdata.data_ptr(), target.scale.data_ptr()
    seed = derive_seed("layer.0.weight", 0)
    Int8Adapter.merge_lora_(target, b.to(DEV), a.to(DEV), 0.5, rounding_seed=seed)
    ref_q, ref_s, _ = K.merge_int8_lora(q.to(DEV), s.to(DEV), None, (1, cols), b.to(DEV), a.to(DEV), 0.5,
                                        asymmetric=False, reduce_range=False, rounding_seed=seed)
    assert target.qdata.data_ptr() == ptr_q and target.scale.data_ptr() == ptr_s
    assert torch.equal(target.qdata, ref_q) and torch.equal(target.scale, ref_s)


def test_int8_sr_replay_and_seed_independent_scales():
    rows, cols, rank = 24, 300, 5
    q, s, b, a = _int8_case(rows, cols, rank)
    outs = []
    for key in ("triton.weight", "triton.weight", "triton.other_weight"):
        outs.append(K.merge_int8_lora(q.to(DEV), s.to(DEV), None, (1, cols), b.to(DEV), a.to(DEV), 0.75,
                                      asymmetric=False, reduce_range=False, rounding_seed=derive_seed(key, 0)))
    (q1, s1, _), (q2, s2, _), (q3, s3, _) = outs
    assert torch.equal(q1, q2) and not torch.equal(q1, q3)
    assert torch.equal(s1, s2) and torch.equal(s1, s3)


def test_int8_sr_probability_uses_fp32_quotient():
    """Port of the reference's probability check (T/test_stochastic_quantized_merge.py:711-742)."""
    rows, cols = 16, 8192
    qdata = torch.zeros(rows, cols, device=DEV, dtype=torch.int8)
    scale = torch.ones(rows, 1, device=DEV, dtype=torch.bfloat16)
    b = torch.ones(rows, 1, device=DEV, dtype=torch.bfloat16)
    a = torch.full((1, cols), 128.0, device=DEV, dtype=torch.bfloat16)
    a[0, -1] = 254.0
    out, final_scale, _ = K.merge_int8_lora(qdata, scale, None, (1, cols), b, a, 1.0, asymmetric=False,
                                            reduce_range=False, rounding_seed=derive_seed("int8-bfloat16-probability.weight", 0))
    samples = out[:, :-1]
    assert bool(((samples == 64) | (samples == 65)).all())
    expected = 128.0 / float(final_scale[0, 0]) - 64.0
    observed = float((samples == 65).float().mean())
    assert observed == pytest.approx(expected, abs=0.01)


def test_int8_zero_weight_gives_eps_scale():
    rows, cols = 16, 256
    q = torch.zeros(rows, cols, dtype=torch.int8, device=DEV)
    s = torch.ones(rows, 1, device=DEV)
    b = torch.zeros(rows, 16, dtype=torch.bfloat16, device=DEV)
    a = torch.zeros(16, cols, dtype=torch.bfloat16, device=DEV)
    oq, os_, _ = K.merge_int8_lora(q, s, None, (1, cols), b, a, 1.0, asymmetric=False, reduce_range=False)
    assert not oq.any()
    assert torch.all(os_ == torch.finfo(torch.float32).eps)


def test_int8_rejects_bad_inputs():
    q = torch.zeros(16, 64, dtype=torch.int8, device=DEV)
    s = torch.ones(16, 1, device=DEV)
    b = torch.zeros(16, 4, dtype=torch.bfloat16, device=DEV)
    a = torch.zeros(4, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="do not match"):
        K.merge_int8_lora(q, s, None, (1, 64), b, a[:, :32], 1.0, asymmetric=False, reduce_range=False)
    with pytest.raises(ValueError, match="per-tensor, per-row and per-group"):  # 2-D blocks
        K.merge_int8_lora(q, torch.ones(8, 2, device=DEV), None, (2, 32), b, a, 1.0, asymmetric=False,
                          reduce_range=False)
    with pytest.raises(ValueError, match="scale shape"):  # a per-group layout with per-row scales
        K.merge_int8_lora(q, s, None, (1, 32), b, a, 1.0, asymmetric=False, reduce_range=False)
    with pytest.raises(ValueError, match="int8"):
        K.merge_int8_lora(q.float(), s, None, (1, 64), b, a, 1.0, asymmetric=False, reduce_range=False)


def test_int8_config2_full_size_properties():
    """W [14336, 4096], r=32, strength 0.5, RTN and SR."""
    rows, cols, rank = 14336, 4096, 32
    w = normal_bf16((rows, cols), 0.02, 0)
    q, s = int8_initial(w)
    b, a = lora_factors(rows, cols, rank, 1)
    qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
    dense = K.dequantize_int8(qd, sd, None, (1, cols), lora=(bd, ad, 0.5))
    dense_np = bf16_np(dense)
    for seed in (None, derive_seed("model.layers.0.mlp.gate_proj.weight", 0)):
        oq, os_, _ = K.merge_int8_lora(qd, sd, None, (1, cols), bd, ad, 0.5, asymmetric=False, reduce_range=False,
                                       rounding_seed=seed)
        rq, rs, _ = O.int8_requant(dense_np, cols, sr_mode=O.SR_PHILOX8 if seed else O.SR_OFF, seed=seed or 0)
        assert np.array_equal(oq.cpu().numpy(), rq)
        assert np.array_equal(os_.cpu().numpy().reshape(-1), rs)
    # dense merge vs oracle on a row sample (the oracle's full GEMM is slow on the CPU)
    idx = np.arange(0, rows, 97)
    obase = O.int8_dequant(q.numpy()[idx], s.numpy()[idx], None, cols)
    omerged = O.merge_dense(obase, bf16_np(b)[idx], bf16_np(a), 0.5)
    assert_merged_close(dense_np[idx], omerged, obase)


@pytest.mark.parametrize("pre_shape", [(), (512,), (1, 1, 512)])
@pytest.mark.parametrize("sr", [False, True])
def test_int8_act_pre_scale_merge_equals_the_oracle(pre_shape, sr):
    # TorchAO applies act_pre_scale p to the activation, so the merge adds
    # B @ ((strength * A) / p) to the stored weight, the fold done in float64
    # and rounded to the factor dtype (P/int8_adapter.py:103-141); the adapter's
    # result must equal the oracle requant of the dense merge with that factor
    rows, cols, rank, strength = 64, 512, 16, 0.75
    q, s = int8_initial(normal_bf16((rows, cols), 0.02, 71))
    b, a = lora_factors(rows, cols, rank, 72)
    pre = torch.linspace(0.5, 2.0, cols).reshape(pre_shape) if pre_shape else torch.tensor(1.5)
    stored = (a.double() * strength / pre.reshape(1, -1).double()).to(torch.bfloat16)
    qd, sd, bd = q.to(DEV), s.to(DEV), b.to(DEV)
    dense = K.dequantize_int8(qd, sd, None, (1, cols), lora=(bd, stored.to(DEV), 1.0))
    seed = derive_seed("int8.act_pre_scale", 0) if sr else None
    rq, rs, _ = O.int8_requant(bf16_np(dense), cols, sr_mode=O.SR_PHILOX8 if sr else O.SR_OFF, seed=seed or 0)
    w = Int8Weight(qd.clone(), sd.clone(), (1, cols), torch.bfloat16, act_pre_scale=pre.to(DEV))
    Int8Adapter.validate_lora_merge(w, bd, a.to(DEV), strength)
    Int8Adapter.merge_lora_(w, bd, a.to(DEV), strength, rounding_seed=seed)
    assert np.array_equal(w.qdata.cpu().numpy(), rq)
    assert np.array_equal(w.scale.cpu().numpy().reshape(-1), rs)
    assert Int8Adapter.stack_key(w) is None  # the grouped launch would skip the pre-scale: kept out of it
