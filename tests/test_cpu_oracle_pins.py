"""Pins for three oracle functions that the GPU parity tests lean on:

* ``lmo_nvfp4_dequant``: the reference's dequant chain
  ``bf16(code * bf16(bf16(e4m3) * g))`` (P/_triton_nvfp4_lora.py:133-163);
* ``lmo_fp8_dequant``: ``cd(fp32(q) * s)`` (P/_triton_float8_lora.py:80-85);
* ``lmo_merge_dense(keep_zero_update=1)``: ``update == 0 ? base : base + update``
  with ``update = acc * strength`` (P/_triton_nvfp4_lora.py:183-186).

Each is compared with a torch restatement written in the reference's order,
with an explicit ``.to(torch.bfloat16)`` at every rounding step, over every
code and every scale code.  Each test also builds the plausible mistakes (one
rounding dropped, a rounding moved, nibbles swapped, the rule left out) and
asserts that every one of them differs from the oracle somewhere on the same
inputs, so the comparison is known to catch them.  Where a rounding is exact
for every input (bf16 of an e4m3 value; the single-level NVFP4 product), the
test asserts that fact instead, since no mistake there can change a value.
The same three mistakes planted in ``oracle/lm_oracle.c`` itself (the
``bf16(bs * g)`` rounding dropped, the FP8 scale rounded to the compute dtype,
the zero rule tested on the delta instead of ``delta * strength``) each fail
a test here.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
# global scales: 1, the eps floor 2^-23, the configs' typical amax/2688, and assorted fp32 values
GLOBALS = [1.0, 2.0 ** -23, 0.02 * 4.5 / 2688.0, 3.3e-3, 0.7, 1.37, 255.5, 7.3e-6] + \
    [float(x) for x in np.random.default_rng(7).uniform(1e-6, 1e-2, 24).astype(np.float32)]


def _bf16r(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).float()


def _canon(x: np.ndarray) -> np.ndarray:
    """fp32 bit patterns with every NaN mapped to one pattern (signed zeros stay distinct)."""
    x = np.asarray(x, np.float32).copy()
    x[np.isnan(x)] = np.float32("nan")
    return x.view(np.uint32)


def _same(x: np.ndarray, y: np.ndarray) -> bool:
    return np.array_equal(_canon(x), _canon(y))


def _oracle_f32(out: np.ndarray, cd: int) -> np.ndarray:
    if cd == O.DT_BF16:
        return O.bf16_to_f32(out)
    if cd == O.DT_F16:
        return O.f16_to_f32(out)
    return out.astype(np.float32)


# ---------------------------------------------------------------------------
# NVFP4 dequant
# ---------------------------------------------------------------------------
def _all_codes_and_scales() -> tuple[np.ndarray, np.ndarray, torch.Tensor]:
    """256 rows (one per e4m3 scale code) x 32 columns: both 16-element blocks of a row carry
    all 16 e2m1 codes, the second block in reverse order; every scale code appears twice."""
    codes = np.tile(np.concatenate([np.arange(16), np.arange(15, -1, -1)]), (256, 1)).astype(np.uint8)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    scale = np.stack([np.arange(256), (np.arange(256) * 37 + 11) % 256], axis=1).astype(np.uint8)
    return packed, scale, torch.from_numpy(codes.astype(np.int64))


def _nvfp4_torch(codes: torch.Tensor, scale: np.ndarray, g: float | None, bf16: bool,
                 mistake: str = "") -> torch.Tensor:
    """P/_triton_nvfp4_lora.py:133-163 in torch, with optional planted mistakes."""
    if mistake == "swap_nibbles":
        codes = codes.view(codes.shape[0], -1, 2).flip(-1).reshape(codes.shape)
    v = E2M1[codes & 7] * torch.where((codes & 8) != 0, -1.0, 1.0)
    bs = torch.from_numpy(scale).view(torch.float8_e4m3fn).float()
    if bf16:
        bs = _bf16r(bs)
    if g is not None:
        gt = torch.tensor(g, dtype=torch.float32)
        if mistake == "fold_global_last":   # code * bs first, then * g, one rounding at the end
            base = v * bs.repeat_interleave(16, dim=1)
            base = base * gt
            return _bf16r(base) if bf16 else base
        bs = bs * gt
        if bf16 and mistake != "drop_global_rounding":
            bs = _bf16r(bs)
    base = v * bs.repeat_interleave(16, dim=1)
    if bf16 and mistake != "drop_base_rounding":
        base = _bf16r(base)
    return base


def test_bf16_of_every_e4m3_value_is_exact() -> None:
    # the first rounding of the chain, bf16(e4m3), can never change a value: state it, so that a
    # restatement that drops it is known to lose nothing
    e = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    finite = ~torch.isnan(e)
    assert torch.equal(_bf16r(e)[finite], e[finite])
    assert int((~finite).sum()) == 2  # 0x7f and 0xff


@pytest.mark.parametrize("cd", [O.DT_BF16, O.DT_F32])
def test_nvfp4_dequant_two_level_every_code_and_scale(cd: int) -> None:
    packed, scale, codes = _all_codes_and_scales()
    bf16 = cd == O.DT_BF16
    missed = {"drop_global_rounding": [], "drop_base_rounding": [], "fold_global_last": [], "swap_nibbles": []}
    for g in GLOBALS:
        got = _oracle_f32(O.nvfp4_dequant(packed, scale, g, cd=cd), cd)
        want = _nvfp4_torch(codes, scale, g, bf16).numpy()
        assert _same(got, want), f"global scale {g!r}"
        for m in missed:
            missed[m].append(_same(got, _nvfp4_torch(codes, scale, g, bf16, m).numpy()))
    caught = {m: not all(v) for m, v in missed.items()}
    if bf16:
        assert all(caught.values()), caught
    else:  # fp32 compute has no bf16 steps: only the nibble order can go wrong
        assert caught["swap_nibbles"]


@pytest.mark.parametrize("cd", [O.DT_BF16, O.DT_F32])
def test_nvfp4_dequant_single_level_every_code_and_scale(cd: int) -> None:
    packed, scale, codes = _all_codes_and_scales()
    got = _oracle_f32(O.nvfp4_dequant(packed, scale, None, cd=cd), cd)
    want = _nvfp4_torch(codes, scale, None, cd == O.DT_BF16).numpy()
    assert _same(got, want)
    # single level: code * e4m3 has at most 2 + 4 significant bits within bf16's exponent range,
    # so the bf16 rounding is exact; only decoding and nibble order can be wrong
    assert _same(got, _nvfp4_torch(codes, scale, None, False).numpy())
    assert not _same(got, _nvfp4_torch(codes, scale, None, cd == O.DT_BF16, "swap_nibbles").numpy())


def test_nvfp4_dequant_swizzled_reads_the_blocked_layout() -> None:
    from test_cpu_requant import _to_blocked

    rng = np.random.default_rng(3)
    M, N = 300, 128
    packed = rng.integers(0, 256, (M, N // 2), dtype=np.uint8)
    scale = rng.integers(0, 0x7e, (M, N // 16), dtype=np.uint8)  # finite, non-negative e4m3 codes
    sw = _to_blocked(torch.from_numpy(scale)).numpy()
    for g in (None, 3.3e-3):
        plain = O.nvfp4_dequant(packed, scale, g)
        assert np.array_equal(O.nvfp4_dequant(packed, sw, g, swizzled=True), plain)


# ---------------------------------------------------------------------------
# FP8 dequant
# ---------------------------------------------------------------------------
_FP8 = {O.DT_E4M3: torch.float8_e4m3fn, O.DT_E5M2: torch.float8_e5m2}
_CD = {O.DT_BF16: torch.bfloat16, O.DT_F16: torch.float16, O.DT_F32: torch.float32}


def _fp8_torch(q: np.ndarray, scale: np.ndarray, group: int, fmt: int, cd: int, mistake: str = "") -> np.ndarray:
    """P/_triton_float8_lora.py:80-85: base = q.to(fp32) * scale, then .to(compute dtype)."""
    v = torch.from_numpy(q).view(_FP8[fmt]).float().reshape(-1)
    s = torch.from_numpy(scale).repeat_interleave(group)
    if mistake == "scale_in_cd":       # the NVFP4 habit of rounding the scale to the compute dtype first
        s = s.to(_CD[cd]).float()
    if mistake == "exact_product":     # one rounding of the exact product instead of fp32 then cd
        base = torch.from_numpy(_round_once(v.double().numpy() * s.double().numpy(), cd))
    else:
        base = v * s
        if mistake != "drop_cd_rounding":
            base = base.to(_CD[cd]).float()
    return base.reshape(q.shape).numpy()


def _round_once(x: np.ndarray, cd: int) -> np.ndarray:
    """float64 -> the nearest cd value (ties to even) in one rounding, for the normal range
    (torch's double -> bf16/fp16 cast goes through fp32, which rounds twice)."""
    bits = 8 if cd == O.DT_BF16 else 11
    m, e = np.frexp(x)
    return np.ldexp(np.rint(m * 2.0 ** bits), e - bits).astype(np.float32)


def _double_rounding_scales(fmt: int, cd: int, want: int = 8) -> np.ndarray:
    """fp32 scales s for which cd(fp32(v * s)) differs from cd(v * s) for some code value v: the
    fp32 product lands on a cd rounding midpoint the exact product lies beyond (found by a seeded
    search; about one product in 2^15 is such a case)."""
    vals = torch.arange(256, dtype=torch.uint8).view(_FP8[fmt]).float()
    vals = vals[torch.isfinite(vals) & (vals > 0)]
    g = torch.Generator().manual_seed(5 + cd)
    s = (torch.rand(1 << 14, generator=g) * 2 + 0.25)
    hits = torch.zeros(s.numel(), dtype=torch.bool)
    for v in vals:
        two = (v * s).to(_CD[cd]).float().numpy()
        one = _round_once(v.double().numpy() * s.double().numpy(), cd)
        hits |= torch.from_numpy((two != one) & np.isfinite(two) & np.isfinite(one))
    found = s[hits][:want].numpy()
    assert found.size >= 2
    return found


@pytest.mark.parametrize("fmt", [O.DT_E4M3, O.DT_E5M2])
@pytest.mark.parametrize("cd", [O.DT_BF16, O.DT_F16, O.DT_F32])
def test_fp8_dequant_every_code_many_scales(fmt: int, cd: int) -> None:
    rng = np.random.default_rng(11 + fmt)
    # 256 codes per row, one row per scale: fixed values plus random fp32 scales over many binades
    fixed = np.array([1.0, 2.0 ** -23, 0.02 / 448, 1.0 / 3.0, 0.1, 7.0, 2.0 ** 10], np.float32)
    scales = np.concatenate([fixed, (2.0 ** rng.uniform(-30, 8, 500) * (1 + rng.random(500))).astype(np.float32)])
    if cd != O.DT_F32:
        scales = np.concatenate([scales, _double_rounding_scales(fmt, cd)])
    M = scales.size
    q = np.tile(np.arange(256, dtype=np.uint8), (M, 1))
    got = _oracle_f32(O.fp8_dequant(q, scales, 256, fmt=fmt, cd=cd), cd)
    assert _same(got, _fp8_torch(q, scales, 256, fmt, cd))
    # per tensor and per group of 32 read the scale of their group
    q2 = q[:64].copy()
    s_tensor = np.array([0.37], np.float32)
    assert _same(_oracle_f32(O.fp8_dequant(q2, s_tensor, q2.size, fmt=fmt, cd=cd), cd),
                 _fp8_torch(q2, s_tensor, q2.size, fmt, cd))
    s_group = np.resize(scales, q2.size // 32).astype(np.float32)
    assert _same(_oracle_f32(O.fp8_dequant(q2, s_group, 32, fmt=fmt, cd=cd), cd),
                 _fp8_torch(q2, s_group, 32, fmt, cd))
    if cd != O.DT_F32:
        for mistake in ("scale_in_cd", "drop_cd_rounding", "exact_product"):
            assert not _same(got, _fp8_torch(q, scales, 256, fmt, cd, mistake)), mistake


# ---------------------------------------------------------------------------
# The "update == 0 keeps the base" rule of the NVFP4 merge
# ---------------------------------------------------------------------------
def _zero_rule_case() -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """A [8, 16] bf16 base with +-0 and ordinary values, and rank-2 factors whose products are exact
    in fp32: rows 0-3 get an exactly zero update (B row zero), column 5 too (A column zero), row 6
    gets the smallest fp32 subnormal 2^-149 as its delta, and the rest ordinary deltas."""
    base = torch.tensor([[0.0, -0.0, 1.0, -2.5, 0.0, -0.0, 3.0, -0.0] * 2] * 8, dtype=torch.bfloat16)
    b = torch.tensor([[0, 0], [0, 0], [0, 0], [0, 0], [0.5, -1], [2, 0.25], [2.0 ** -75, 0], [-1, 1]],
                     dtype=torch.bfloat16)
    a = torch.ones(2, 16, dtype=torch.bfloat16) * 0.5
    a[0, 3] = 2.0 ** -74
    a[:, 5] = 0.0
    base[6, 3] = -0.0
    return base, b, a


def _zero_rule_torch(base: torch.Tensor, b: torch.Tensor, a: torch.Tensor, strength: float,
                     rule: bool = True) -> torch.Tensor:
    acc = (b.float()[:, :, None] * a.float()[None, :, :]).sum(1)  # elementwise: no BLAS flush of subnormals
    update = acc * torch.tensor(strength, dtype=torch.float32)
    merged = base.float() + update
    if rule:
        merged = torch.where(update == 0.0, base.float(), merged)
    return merged.to(torch.bfloat16)


@pytest.mark.parametrize("strength", [1.0, 0.75, 0.25, -0.75])
def test_zero_update_keeps_the_base(strength: float) -> None:
    from helpers import bf16_np

    base, b, a = _zero_rule_case()
    got = O.merge_dense(bf16_np(base), bf16_np(b), bf16_np(a), strength, keep_zero_update=True)
    want = bf16_np(_zero_rule_torch(base, b, a, strength))
    assert np.array_equal(got, want)
    if strength < 0:  # a zero update is then -0, and -0 + -0 = -0: the rule cannot show
        return
    # without the rule a -0 base under a zero update turns into +0
    assert not np.array_equal(got, bf16_np(_zero_rule_torch(base, b, a, strength, rule=False)))
    # -0 bases under exactly zero updates keep their sign bit
    zero_upd = (b.float()[:, :, None] * a.float()[None, :, :]).sum(1) * strength == 0
    neg0 = (bf16_np(base) == 0x8000) & zero_upd.numpy()
    assert neg0.any() and (got[neg0] == 0x8000).all()
    if strength == 0.25:
        # 2^-149 * 0.25 underflows to 0: the update is zero although the delta is not
        assert (got[6, 3] == bf16_np(base)[6, 3]) and bf16_np(base)[6, 3] == 0x8000
