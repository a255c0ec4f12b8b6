"""Stochastic-rounding selections of the CPU oracle.

Mirrors the reference's statistical and structural checks
(tests/test_stochastic_rounding.py:101-199 and
tests/test_stochastic_quantized_merge.py of the reference): only the two
neighbouring codes are ever chosen, the mean is unbiased, exact endpoints,
saturated and non-finite inputs keep the round-to-nearest code, a value half
way to the smallest subnormal rounds up half of the time, and -0.0 keeps its
sign bit.  The selections follow P/_triton_stochastic_quantization.py:25-177.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

SHAPE = (256, 512)


def _u(seed_key: str = "layers.0.weight", n: int = SHAPE[0] * SHAPE[1], merge_index: int = 0) -> np.ndarray:
    return O.uniforms(O.derive_seed(seed_key, merge_index), 0, n)


def test_integer_grid_selection_is_unbiased() -> None:
    x = np.full(SHAPE, 0.3, np.float32).ravel()
    q = O.sr_int(x, np.zeros(x.size, np.int32), _u(), -2, 2)
    assert set(np.unique(q).tolist()) == {0, 1}
    assert q.mean() == pytest.approx(0.3, abs=0.005)


def test_integer_grid_negative_values() -> None:
    x = np.full(SHAPE, -1.75, np.float32).ravel()
    q = O.sr_int(x, np.full(x.size, -2, np.int32), _u(), -128, 127)
    assert set(np.unique(q).tolist()) == {-2, -1}
    assert q.mean() == pytest.approx(-1.75, abs=0.005)


def test_integer_endpoints_nonfinite_and_saturation_keep_deterministic_codes() -> None:
    x = np.array([-np.inf, -2.0, 0.0, 2.0, np.inf, np.nan, 5.5, -7.25], np.float32)
    det = np.array([41, 42, 43, 44, 45, 46, 47, 48], np.int32)
    q = O.sr_int(x, det, _u(n=x.size), -2, 2)
    assert np.array_equal(q, det)


def test_e2m1_selection_between_codebook_neighbours() -> None:
    # 2.5 lies half way from 2 to 3, 0.3 sits 60% of the way from 0 to 0.5, 5.0 half way from 4 to 6
    for value, lo, hi, p_up in ((2.5, 4, 5, 0.5), (0.3, 0, 1, 0.6), (5.0, 6, 7, 0.5), (-1.25, 2, 3, 0.5)):
        x = np.full(SHAPE, value, np.float32).ravel()
        det = O.f32_to_e2m1(x)
        codes = O.sr_e2m1(x, det, _u())
        mags = np.unique(codes & 7).tolist()
        assert set(mags) == {lo, hi}
        assert ((codes & 7) == hi).mean() == pytest.approx(p_up, abs=0.01)
        if value < 0:
            assert np.all(codes & 8)


def test_e2m1_exact_and_saturated_keep_deterministic_codes() -> None:
    x = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -6.0, -0.5], np.float32)
    det = O.f32_to_e2m1(x)
    assert np.array_equal(O.sr_e2m1(x, det, _u(n=x.size)), det)


@pytest.mark.parametrize("fmt", [O.DT_E4M3, O.DT_E5M2])
def test_fp8_rounds_across_smallest_subnormal(fmt: int) -> None:
    smallest = 2.0 ** -9 if fmt == O.DT_E4M3 else 2.0 ** -16
    x = np.full(SHAPE, smallest / 2, np.float32).ravel()
    limit = 448.0 if fmt == O.DT_E4M3 else 57344.0
    codes = O.sr_fp8(x, _u(), fmt, limit)
    vals = O.fp8_to_f32(codes, fmt)
    assert set(np.unique(vals).tolist()) == {0.0, smallest}
    assert (vals > 0).mean() == pytest.approx(0.5, abs=0.01)


@pytest.mark.parametrize("fmt", [O.DT_E4M3, O.DT_E5M2])
def test_fp8_two_neighbours_and_unbiased_in_normal_range(fmt: int) -> None:
    x = np.full(SHAPE, 1.3, np.float32).ravel()
    limit = 448.0 if fmt == O.DT_E4M3 else 57344.0
    vals = O.fp8_to_f32(O.sr_fp8(x, _u(), fmt, limit), fmt)
    lo, hi = (1.25, 1.375) if fmt == O.DT_E4M3 else (1.25, 1.5)
    assert set(np.unique(vals).tolist()) == {lo, hi}
    assert vals.astype(np.float64).mean() == pytest.approx(1.3, abs=0.002)


def test_fp8_exact_negative_zero_keeps_sign_bit() -> None:
    codes = O.sr_fp8(np.array([-0.0], np.float32), _u(n=1), O.DT_E4M3, 448.0)
    assert codes[0] == 0x80


def test_fp8_saturated_and_exact_values_keep_rtn_code() -> None:
    x = np.array([448.0, -448.0, 1.0, -2.0, 0.015625, 0.0], np.float32)
    codes = O.sr_fp8(x, _u(n=x.size), O.DT_E4M3, 448.0)
    assert np.array_equal(codes, O.f32_to_fp8(x, O.DT_E4M3))


def test_requant_streams_are_independent_of_target_and_merge_index() -> None:
    rng = np.random.default_rng(0)
    dense = O.f32_to_bf16((rng.standard_normal((64, 256)) * 0.02).astype(np.float32))
    runs = {}
    for key, idx in (("a.weight", 0), ("a.weight", 1), ("b.weight", 0)):
        q, _, _ = O.int8_requant(dense, 256, sr_mode=O.SR_PHILOX8, seed=O.derive_seed(key, idx))
        runs[(key, idx)] = q
    q_again, _, _ = O.int8_requant(dense, 256, sr_mode=O.SR_PHILOX8, seed=O.derive_seed("a.weight", 0))
    assert np.array_equal(q_again, runs[("a.weight", 0)])  # replay
    assert not np.array_equal(runs[("a.weight", 0)], runs[("a.weight", 1)])
    assert not np.array_equal(runs[("a.weight", 0)], runs[("b.weight", 0)])


# ---- the integer rule on the 13-bit grid (INT8, Q8_0; gfx950 v_cvt_sr_f16_f32) ----
def test_sr_int13_is_the_reference_rule_with_13_bit_u_and_p() -> None:
    # on values with 13 fraction bits and s = 1, sr_int13 is the reference's
    # selection (P/_triton_stochastic_quantization.py:25-40) with u = (h >> 3) 2^-13
    rng = np.random.default_rng(3)
    n = 200_000
    y = (rng.integers(-130 * 8192, 130 * 8192, n) / 8192.0).astype(np.float32)
    h = rng.integers(0, 65536, n).astype(np.uint32)
    got = O.sr_int13(y, 1.0, 0.0, h, -128, 127)
    det = np.clip(np.rint(y), -128, 127).astype(np.int32)
    want = np.clip(O.sr_int(y, det, (h >> 3).astype(np.float32) / 8192.0, -128, 127), -128, 127)
    assert np.array_equal(got, want)


def test_sr_int13_up_probability_is_exactly_the_13_bit_fraction() -> None:
    # over every 16-bit draw, the up-count of a fraction F * 2^-13 is exactly 8 F
    h = np.arange(65536, dtype=np.uint32)
    for frac13 in (0, 1, 2, 1000, 4096, 8191):
        v = np.full(h.size, 3.0 + frac13 / 8192.0, np.float32)
        up = O.sr_int13(v, 1.0, 0.0, h, -128, 127) - 3
        assert set(np.unique(up).tolist()) <= {0, 1}
        assert int(up.sum()) == 8 * frac13


def test_sr_int13_neighbours_unbiased_and_clamped() -> None:
    rng = np.random.default_rng(5)
    n = 1_000_000
    s = np.float32(0.00037)
    v = (rng.standard_normal(n) * 0.02).astype(np.float32)
    rcp = np.float32(1.0) / s
    h = O.sr_h16(O.derive_seed("sr13", 0), 0, n)
    q = O.sr_int13(v, rcp, 0.0, h, -128, 127)
    y = np.clip(v.astype(np.float64) / np.float64(s), -128, 127)
    assert np.all((q == np.floor(y)) | (q == np.ceil(y)))
    assert abs(float(np.mean(q - y))) < 2e-3
    assert O.sr_int13(np.float32([1e30, -1e30, np.nan]), 1.0, 0.0, 12345, -128, 127).tolist() == [127, -128, -128]
    assert O.sr_int13(np.float32([5.0, -7.0]), 1.0, 0.0, 0, -128, 127).tolist() == [5, -7]  # integers stay
    # reduce_range and a zero point shift the grid, not the rule
    # (h = 0 is u = 0: any fraction rounds up; h = 65535 is u = 8191 / 8192: only a fraction above it does)
    assert O.sr_int13(np.float32([70.0, 10.25]), 1.0, np.float32([0.0, 3.0]), 0, -64, 63).tolist() == [63, 14]
    assert O.sr_int13(np.float32([70.0, 10.25]), 1.0, np.float32([0.0, 3.0]), 65535, -64, 63).tolist() == [63, 13]
