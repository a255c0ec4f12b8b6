"""Requantization recipes of the CPU oracle against independent torch / numpy
restatements of the reference's formulas, plus the invariants the reference's
own tests assert.

* INT8 per-row / per-group, symmetric and affine (P/_triton_int8_lora.py:123-236)
* scaled FP8 per-row (P/_triton_float8_lora.py:253-301)
* NVFP4 single- and two-level (P/_triton_nvfp4_lora.py:251-346, 437-512)
* MXFP4 / MXFP8 zero-update idempotence (tests/test_mx_adapter.py:565-604 of
  the reference)
* GGUF Q8_0 against the public ggml quantize_row_q8_0 recipe
* the dense merge against torch's fp32 matmul
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_merged_close, bf16_np, np_bf16

EPS = 1.1920928955078125e-07


def _bf16r(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).float()


def _dense(M: int, N: int, seed: int, std: float = 0.02) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(M, N, generator=g) * std).to(torch.bfloat16)


# ---------------------------------------------------------------------------
# INT8
# ---------------------------------------------------------------------------
def _int8_torch(dense: torch.Tensor, group: int, asymmetric: bool, reduce_range: bool):  # noqa: ANN202
    qmin, qmax = (-64, 63) if reduce_range else (-128, 127)
    v = dense.float().reshape(-1, group)
    mn = _bf16r(torch.minimum(v, torch.zeros(())).amin(dim=1))
    mx = _bf16r(torch.maximum(v, torch.zeros(())).amax(dim=1))
    if asymmetric:
        scale = _bf16r(mx - mn) / float(qmax - qmin)
    else:
        scale = torch.maximum(-mn, mx) / ((qmax - qmin) / 2.0)
    scale = _bf16r(torch.clamp_min(_bf16r(scale), EPS))
    zp = torch.zeros_like(scale, dtype=torch.int64)
    if asymmetric:
        ratio = _bf16r(mn / scale)
        zp = torch.clamp(qmin - torch.round(ratio).long(), qmin, qmax)
    inv = 1.0 / scale
    q = torch.round(v * inv[:, None]).long() + zp[:, None]
    q = torch.clamp(q, qmin, qmax)
    return q.reshape(dense.shape).to(torch.int8), scale, zp.to(torch.int8)


@pytest.mark.parametrize("group", [4096, 128, 32])
@pytest.mark.parametrize("asymmetric", [False, True])
@pytest.mark.parametrize("reduce_range", [False, True])
def test_int8_rtn_matches_closed_form(group: int, asymmetric: bool, reduce_range: bool) -> None:
    dense = _dense(24, 4096, 1)
    dense[3] = 0.0  # an all-zero row
    dense[5, :7] = torch.tensor([1.0, -3.0, 2.5, 0.0, -0.0, 1e-30, -2.0], dtype=torch.bfloat16)
    q, s, zp = O.int8_requant(bf16_np(dense), group, asymmetric=asymmetric, reduce_range=reduce_range)
    tq, ts, tzp = _int8_torch(dense, group, asymmetric, reduce_range)
    assert np.array_equal(s, ts.numpy())
    assert np.array_equal(q, tq.numpy())
    if asymmetric:
        assert np.array_equal(zp, tzp.numpy())


def test_int8_zero_rows_get_eps_scale_and_zero_codes() -> None:
    dense = torch.zeros(4, 256, dtype=torch.bfloat16)
    q, s, _ = O.int8_requant(bf16_np(dense), 256)
    assert (q == 0).all()
    assert np.all(s == np.float32(_bf16r(torch.tensor(EPS)).item()))


@pytest.mark.parametrize("reduce_range", [False, True])
def test_int8_codes_stay_in_range(reduce_range: bool) -> None:
    dense = _dense(64, 1024, 2, std=3.0)
    for sr in (O.SR_OFF, O.SR_PHILOX8):
        q, _, _ = O.int8_requant(bf16_np(dense), 1024, reduce_range=reduce_range, sr_mode=sr, seed=5)
        lo, hi = (-64, 63) if reduce_range else (-128, 127)
        assert q.min() >= lo and q.max() <= hi


def test_int8_stochastic_picks_a_neighbour_and_is_unbiased() -> None:
    dense = _dense(16, 512, 3)
    _, s_rtn, _ = O.int8_requant(bf16_np(dense), 512)
    y = dense.float().numpy() / s_rtn[:, None]  # fp32 true division, as the reference
    acc = np.zeros_like(y, dtype=np.float64)
    n_seeds = 200
    for seed in range(n_seeds):
        q, s, _ = O.int8_requant(bf16_np(dense), 512, sr_mode=O.SR_PHILOX8, seed=O.derive_seed("w", seed))
        assert np.array_equal(s, s_rtn)  # scales are final before stochastic coding
        qf = q.astype(np.float64)
        yc = np.clip(y, -128, 127)  # saturated values keep the clamped RTN code
        assert np.all((qf == np.floor(yc)) | (qf == np.ceil(yc)))
        acc += qf
    interior = (y > -128) & (y < 127)
    err = (acc / n_seeds - y)[interior]
    assert abs(err.mean()) < 0.005
    assert np.abs(err).max() < 0.2  # 200 Bernoulli draws: 0.2 is > 5 sigma


# ---------------------------------------------------------------------------
# FP8 per row
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("fmt,limit,tdt", [(O.DT_E4M3, 448.0, torch.float8_e4m3fn),
                                           (O.DT_E5M2, 57344.0, torch.float8_e5m2)])
def test_fp8_rtn_matches_closed_form(fmt: int, limit: float, tdt: torch.dtype) -> None:
    dense = _dense(32, 2048, 4)
    dense[7] = 0.0
    q, s = O.fp8_requant(bf16_np(dense), 2048, fmt=fmt)
    v = dense.float()
    scale = _bf16r(v.abs().amax(dim=1) / limit)
    scale = torch.where(scale == 0.0, torch.tensor(EPS), scale)
    codes = torch.clamp(v / scale[:, None], -limit, limit).to(tdt)
    assert np.array_equal(s, scale.numpy())
    assert np.array_equal(q, codes.view(torch.uint8).numpy())


def test_fp8_stochastic_neighbours_and_bias() -> None:
    dense = _dense(8, 1024, 5)
    q0, s0 = O.fp8_requant(bf16_np(dense), 1024, fmt=O.DT_E4M3)
    x = (dense.float() / torch.from_numpy(s0)[:, None]).numpy()
    acc = np.zeros(x.shape)
    n = 200
    for seed in range(n):
        q, s = O.fp8_requant(bf16_np(dense), 1024, fmt=O.DT_E4M3, sr_mode=O.SR_PHILOX8, seed=seed)
        assert np.array_equal(s, s0)
        vals = O.fp8_to_f32(q).astype(np.float64)
        # a neighbour of x on the e4m3 grid: within one grid step (2^(e-3), at least 2^-9)
        step = np.maximum(2.0 ** (np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -6))) - 3), 2.0 ** -9)
        assert np.all(np.abs(vals - x) <= step)
        acc += vals
    # bias in units of the local grid step (a 16-bit uniform leaves < 2^-16 of a step)
    err = (acc / n - x) / step
    assert abs(err.mean()) < 0.005


# ---------------------------------------------------------------------------
# NVFP4
# ---------------------------------------------------------------------------
def _e2m1_codes(x: torch.Tensor) -> torch.Tensor:
    mags = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=torch.float64)
    m = x.double().abs().clamp(max=6.0)
    dist = (m[..., None] - mags).abs()
    best = dist.min(dim=-1, keepdim=True).values
    cand = dist == best
    even = torch.arange(8) % 2 == 0
    tie = cand.sum(-1) > 1
    code = torch.where(tie, (cand & even).double().argmax(-1), cand.double().argmax(-1))
    sign = torch.signbit(x).long() << 3
    return code | sign


def _nvfp4_torch(dense: torch.Tensor, two_level: bool):  # noqa: ANN202
    M, N = dense.shape
    v = dense.float()
    blocks = v.reshape(M, N // 16, 16)
    bs = blocks.abs().amax(dim=-1) / 6.0
    if two_level:
        g = torch.clamp_min(v.abs().max() / 2688.0, EPS)
        fp8 = torch.clamp(bs / g, 0.015625, 448.0).to(torch.float8_e4m3fn).float()
        normalized = blocks * ((1.0 / g) / fp8)[..., None]
    else:
        g = None
        fp8 = torch.clamp(bs, 0.015625, 448.0).to(torch.float8_e4m3fn).float()
        normalized = blocks / fp8[..., None]
    codes = _e2m1_codes(torch.clamp(normalized, -6.0, 6.0)).reshape(M, N)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8)
    return packed, fp8.to(torch.float8_e4m3fn).view(torch.uint8), g


@pytest.mark.parametrize("two_level", [True, False])
def test_nvfp4_rtn_matches_closed_form(two_level: bool) -> None:
    dense = _dense(32, 256, 6)
    dense[4, :16] = 0.0  # an all-zero block
    q, s, pts = O.nvfp4_requant(bf16_np(dense), two_level=two_level)
    tq, ts, tg = _nvfp4_torch(dense, two_level)
    assert np.array_equal(s, ts.numpy())
    assert np.array_equal(q, tq.numpy())
    if two_level:
        assert np.float32(pts[0]) == np.float32(tg.item())


def test_nvfp4_zero_weight_gets_eps_global_scale() -> None:
    q, s, pts = O.nvfp4_requant(np.zeros((16, 64), np.uint16), two_level=True)
    assert pts[0] == np.float32(EPS)
    assert (q == 0).all()


def test_blocked_scale_offsets_are_a_bijection() -> None:
    for M, cols in ((128, 4), (256, 8), (300, 13), (17, 3)):
        rows_p, cols_p = O.blocked_scale_shape(M, cols * 16, 16, True)
        seen = set()
        for r in range(M):
            for c in range(cols):
                off = O.blocked_scale_offset(r, c, cols, True)
                assert 0 <= off < rows_p * cols_p
                seen.add(off)
        assert len(seen) == M * cols


def test_nvfp4_dequant_of_requant_is_within_half_a_code_step() -> None:
    dense = _dense(16, 512, 7)
    q, s, pts = O.nvfp4_requant(bf16_np(dense), two_level=True)
    back = O.bf16_to_f32(O.nvfp4_dequant(q, s, pts[0]))
    v = dense.float().numpy()
    scale = O.fp8_to_f32(s).repeat(16, axis=1) * pts[0]
    # largest e2m1 gap is 2 (between 4 and 6): half a gap, times the block scale, plus bf16 rounding
    assert np.all(np.abs(back - v) <= scale * 1.0 + np.abs(v) * 2.0 ** -7)


# ---------------------------------------------------------------------------
# MX: dequantize -> requantize reproduces the codes (zero LoRA update)
# ---------------------------------------------------------------------------
# FLOOR (the default) and EVEN re-derive the same shared exponent from the
# dequantized block; CEIL / RCEIL need not (a block max of 130 * 2^e in e4m3
# dequantizes to 128 * 2^e, one binade lower), so they are not idempotent.
@pytest.mark.parametrize("fmt", [O.DT_E2M1, O.DT_E4M3, O.DT_E5M2])
@pytest.mark.parametrize("mode", [O.MX_FLOOR, O.MX_EVEN])
@pytest.mark.parametrize("swizzled", [False, True])
def test_mx_zero_update_is_bit_exact(fmt: int, mode: int, swizzled: bool) -> None:
    dense = _dense(64, 256, 8)
    q, s = O.mx_requant(bf16_np(dense), fmt, mode, swizzled=swizzled)
    back = O.mx_dequant(q, s, fmt, 256, swizzled=swizzled)
    q2, s2 = O.mx_requant(back, fmt, mode, swizzled=swizzled)
    assert np.array_equal(q, q2)
    assert np.array_equal(s, s2)


# ---------------------------------------------------------------------------
# GGUF Q8_0 (public ggml recipe, the reference has no requant)
# ---------------------------------------------------------------------------
def _ggml_q8_0(x: np.ndarray) -> np.ndarray:
    M, N = x.shape
    blocks = x.reshape(M, N // 32, 32).astype(np.float32)
    amax = np.abs(blocks).max(axis=-1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    y = (blocks * inv[..., None]).astype(np.float32).astype(np.float64)
    q = np.where(y >= 0, np.floor(y + 0.5), np.ceil(y - 0.5)).astype(np.int8)  # roundf: half away from zero
    out = np.empty((M, N // 32, 34), np.uint8)
    out[..., :2] = d.astype(np.float16).view(np.uint8).reshape(M, N // 32, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(M, N // 32 * 34)


def test_q8_0_requant_matches_ggml() -> None:
    dense = _dense(16, 512, 9)
    dense[2, :32] = 0.0
    packed = O.q8_0_requant(bf16_np(dense))
    assert np.array_equal(packed, _ggml_q8_0(dense.float().numpy()))


def test_q8_0_dequant_closed_form() -> None:
    packed = _ggml_q8_0(_dense(8, 256, 10).float().numpy())
    got = O.q8_0_dequant(packed, 256)
    blocks = packed.reshape(8, 8, 34)
    d = torch.from_numpy(blocks[..., :2].copy().view(np.float16).astype(np.float32))
    q = torch.from_numpy(blocks[..., 2:].copy().view(np.int8).astype(np.float32))
    want = (_bf16r(d) * q).to(torch.bfloat16).reshape(8, 256)  # P/gguf_dequant.py:57-61
    assert np.array_equal(got, bf16_np(want))


# ---------------------------------------------------------------------------
# dense merge
# ---------------------------------------------------------------------------
def test_merge_dense_matches_torch_within_contract() -> None:
    M, N, r = 64, 512, 16
    base = _dense(M, N, 11)
    g = torch.Generator().manual_seed(12)
    a = (torch.randn(r, N, generator=g) / r).to(torch.bfloat16)
    b = (torch.randn(M, r, generator=g) * 0.01).to(torch.bfloat16)
    got = O.merge_dense(bf16_np(base), bf16_np(b), bf16_np(a), 0.75)
    want = (base.float() + 0.75 * (b.float() @ a.float())).to(torch.bfloat16)
    assert_merged_close(got, bf16_np(want), bf16_np(base))


def test_merge_dense_exact_on_integer_inputs() -> None:
    # integers with small sums are exact in every summation order
    g = torch.Generator().manual_seed(13)
    base = torch.randint(-8, 9, (32, 64), generator=g).to(torch.bfloat16)
    a = torch.randint(-3, 4, (16, 64), generator=g).to(torch.bfloat16)
    b = torch.randint(-3, 4, (32, 16), generator=g).to(torch.bfloat16)
    got = O.merge_dense(bf16_np(base), bf16_np(b), bf16_np(a), 0.5)
    want = (base.float() + 0.5 * (b.float() @ a.float())).to(torch.bfloat16)
    assert np.array_equal(got, bf16_np(want))


def test_merge_dense_strength_zero_and_rank_padding() -> None:
    base = _dense(16, 64, 14)
    g = torch.Generator().manual_seed(15)
    a = torch.randn(5, 64, generator=g).to(torch.bfloat16)
    b = torch.randn(16, 5, generator=g).to(torch.bfloat16)
    assert np.array_equal(O.merge_dense(bf16_np(base), bf16_np(b), bf16_np(a), 0.0), bf16_np(base))
    back = np_bf16(O.merge_dense(bf16_np(base), bf16_np(b), bf16_np(a), 1.0))
    assert back.shape == base.shape


# ---- per-group layouts: the per-row recipe on each group ---------------------
# A per-group quantization of [M, N] with group g is the per-row quantization
# of the same memory viewed as [M N / g, g]: every group is one row of the
# view and keeps its flat element offsets, so the stochastic draws are the
# same.  This pins the oracle's per-group path to its per-row path.
@pytest.mark.parametrize("g", [16, 32, 64, 128])
@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("sr", [O.SR_OFF, O.SR_PHILOX8])
def test_int8_group_is_per_row_of_the_group_view(g, asym, sr):
    rng = np.random.default_rng(g)
    dense = O.f32_to_bf16((rng.standard_normal((12, 256)) * 0.02).astype(np.float32))
    dense[3, :g] = 0
    q, s, z = O.int8_requant(dense, g, asymmetric=asym, sr_mode=sr, seed=77)
    view = dense.reshape(-1, g)
    rq, rs, rz = O.int8_requant(view, g, asymmetric=asym, sr_mode=sr, seed=77)
    assert np.array_equal(q.reshape(-1, g), rq)
    assert np.array_equal(s, rs)
    if asym:
        assert np.array_equal(z, rz)
    deq = O.int8_dequant(q, s, z if asym else None, g)
    assert np.array_equal(deq.reshape(-1, g), O.int8_dequant(rq, rs, rz if asym else None, g))


@pytest.mark.parametrize("g", [16, 64])
@pytest.mark.parametrize("fmt", [O.DT_E4M3, O.DT_E5M2])
@pytest.mark.parametrize("sr", [O.SR_OFF, O.SR_PHILOX8])
def test_fp8_group_is_per_row_of_the_group_view(g, fmt, sr):
    rng = np.random.default_rng(g + fmt)
    dense = O.f32_to_bf16((rng.standard_normal((8, 128)) * 0.05).astype(np.float32))
    q, s = O.fp8_requant(dense, g, fmt=fmt, sr_mode=sr, seed=5)
    rq, rs = O.fp8_requant(dense.reshape(-1, g), g, fmt=fmt, sr_mode=sr, seed=5)
    assert np.array_equal(q.reshape(-1, g), rq)
    assert np.array_equal(s, rs)


def _to_blocked(scales: torch.Tensor) -> torch.Tensor:
    """TorchAO's 128x4 block-scaling layout (torchao 0.18.0, ``to_blocked``; the layout cuBLAS
    documents for block-scaled GEMMs), written as tensor reshapes: pad rows to 128 and columns to 4,
    cut into 128x4 tiles in row-major tile order, then inside a tile store element (32 g + l, c) at
    16 l + 4 g + c.  The flat result is the memory of the [ceil(M/128) * 32, ceil(C/4) * 16] scale
    tensor."""
    rows, cols = scales.shape
    rb, cb = -(-rows // 128), -(-cols // 4)
    padded = torch.zeros((rb * 128, cb * 4), dtype=scales.dtype)
    padded[:rows, :cols] = scales
    tiles = padded.view(rb, 128, cb, 4).permute(0, 2, 1, 3)            # [rb, cb, 128, 4]
    inner = tiles.reshape(rb * cb, 4, 32, 4).transpose(1, 2)            # [tile, l, g, c]
    return inner.reshape(-1).reshape(rb * 32, cb * 16)


@pytest.mark.parametrize("rows,cols", [(128, 64), (256, 512), (300, 208), (17, 48), (1000, 4096)])
def test_nvfp4_swizzled_scales_are_torchao_to_blocked_of_the_plain_ones(rows: int, cols: int) -> None:
    # the same weight encoded with plain and with swizzled scales: equal codes, and the swizzled
    # scale array is the block layout of the plain one (P/_triton_nvfp4_lora.py:88-104); a swapped
    # row-lane / row-group stride, or a wrong tile order, fails here (bijectivity alone does not)
    dense = bf16_np(_dense(rows, cols, 40 + rows))
    q0, s0, p0 = O.nvfp4_requant(dense, two_level=True, swizzled=False)
    q1, s1, p1 = O.nvfp4_requant(dense, two_level=True, swizzled=True)
    assert np.array_equal(q0, q1) and np.array_equal(p0, p1)
    want = _to_blocked(torch.from_numpy(s0)).numpy()
    assert s1.shape == want.shape
    assert np.array_equal(s1, want)
    # and the offset function agrees element by element
    for r in range(0, rows, max(1, rows // 37)):
        for c in range(0, cols // 16, max(1, cols // 16 // 11)):
            assert s1.reshape(-1)[O.blocked_scale_offset(r, c, cols // 16, True)] == s0[r, c]


@pytest.mark.parametrize("fmt", [O.DT_E2M1, O.DT_E4M3])
@pytest.mark.parametrize("rows,cols", [(128, 128), (300, 640), (33, 256)])
def test_mx_swizzled_scales_are_torchao_to_blocked_of_the_plain_ones(fmt: int, rows: int, cols: int) -> None:
    # MX's e8m0 block-32 scales use the same layout (P/_triton_mx_lora.py:97-112)
    dense = bf16_np(_dense(rows, cols, 60 + rows))
    q0, s0 = O.mx_requant(dense, fmt, swizzled=False)
    q1, s1 = O.mx_requant(dense, fmt, swizzled=True)
    assert np.array_equal(q0, q1)
    assert np.array_equal(s1, _to_blocked(torch.from_numpy(s0)).numpy())
