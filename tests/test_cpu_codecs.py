"""Element codecs of the CPU oracle against library routines and brute force.

bf16 / fp16 / e4m3fn / e5m2 / e8m0 are checked against torch's and numpy's
conversions (exhaustively where the input space is 2^16), e2m1 against a
brute-force nearest-value search with ties to the even code (the threshold
chain of P/_triton_nvfp4_lora.py:55-85 is exactly that), and the MX shared
exponent against a math.frexp restatement of P/_triton_mx_lora.py:115-159.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O

ALL_BF16 = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)


def _bf16_inputs_f32() -> np.ndarray:
    x = O.bf16_to_f32(ALL_BF16)
    return x[np.isfinite(x)]


def _torch_bits(t: torch.Tensor, np_dtype) -> np.ndarray:  # noqa: ANN001
    return t.contiguous().view({np.uint16: torch.int16, np.uint8: torch.uint8}[np_dtype]).numpy().view(np_dtype)


def _random_f32(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 1.0, -1.0, 3.3895314e38, 1e-45, -1e-45, 1.17549435e-38],
                        dtype=np.float32)
    # exact ties between neighbouring bf16 values, both parities
    ties = (np.arange(1, 2000, dtype=np.uint32) << 15 | 0x3F800000 | 0x8000).view(np.float32)
    return np.concatenate([x[np.isfinite(x)], specials, ties, -ties])


def test_bf16_rne_matches_torch() -> None:
    x = _random_f32(1 << 18, 1)
    got = O.f32_to_bf16(x)
    want = _torch_bits(torch.from_numpy(x).to(torch.bfloat16), np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(O.bf16_to_f32(got), torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_f16_rne_matches_numpy() -> None:
    x = _random_f32(1 << 18, 2)
    got = O.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    allh = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    dec = O.f16_to_f32(allh)
    ref = allh.view(np.float16).astype(np.float32)
    same = (dec == ref) | (np.isnan(dec) & np.isnan(ref))
    assert same.all()


@pytest.mark.parametrize("fmt,tdt,limit", [(O.DT_E4M3, torch.float8_e4m3fn, 448.0),
                                           (O.DT_E5M2, torch.float8_e5m2, 57344.0)])
def test_fp8_encode_exhaustive_over_bf16(fmt: int, tdt: torch.dtype, limit: float) -> None:
    # the merge kernels clamp to the finite range before the cast (P/_triton_float8_lora.py:295-299)
    x = np.clip(_bf16_inputs_f32(), -limit, limit)
    got = O.f32_to_fp8(x, fmt)
    want = _torch_bits(torch.from_numpy(x).to(tdt), np.uint8)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt,tdt,limit", [(O.DT_E4M3, torch.float8_e4m3fn, 448.0),
                                           (O.DT_E5M2, torch.float8_e5m2, 57344.0)])
def test_fp8_encode_random_f32(fmt: int, tdt: torch.dtype, limit: float) -> None:
    x = np.clip(_random_f32(1 << 17, 3), -limit, limit)
    got = O.f32_to_fp8(x, fmt)
    want = _torch_bits(torch.from_numpy(x).to(tdt), np.uint8)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt,tdt", [(O.DT_E4M3, torch.float8_e4m3fn), (O.DT_E5M2, torch.float8_e5m2)])
def test_fp8_decode_all_codes(fmt: int, tdt: torch.dtype) -> None:
    codes = np.arange(256, dtype=np.uint8)
    got = O.fp8_to_f32(codes, fmt)
    want = torch.from_numpy(codes).view(tdt).float().numpy()
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    assert np.array_equal(np.signbit(got[~np.isnan(got)]), np.signbit(want[~np.isnan(want)]))


def test_e8m0_decode_all_codes() -> None:
    codes = np.arange(256, dtype=np.uint8)
    got = O.e8m0_to_f32(codes)
    want = torch.from_numpy(codes).view(torch.float8_e8m0fnu).float().numpy()
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    assert got[127] == 1.0 and np.isnan(got[255])


def _e2m1_brute(x: np.ndarray) -> np.ndarray:
    mags = O.E2M1_VALUES[:8].astype(np.float64)
    m = np.minimum(np.abs(x.astype(np.float64)), 6.0)
    dist = np.abs(m[:, None] - mags[None, :])
    best = dist.min(axis=1, keepdims=True)
    cand = dist == best
    # ties go to the even code (even mantissa); there are never more than two candidates
    code = np.where(cand.sum(axis=1) > 1, np.argmax(cand & (np.arange(8) % 2 == 0)[None, :], axis=1),
                    np.argmax(cand, axis=1))
    sign = np.signbit(x).astype(np.uint8) << 3
    return code.astype(np.uint8) | sign


def test_e2m1_encode_exhaustive_over_bf16() -> None:
    x = np.clip(_bf16_inputs_f32(), -6.0, 6.0)
    assert np.array_equal(O.f32_to_e2m1(x), _e2m1_brute(x))


def test_e2m1_encode_midpoints_and_signed_zero() -> None:
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float32)
    x = np.concatenate([mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 7), [0.0, -0.0]]).astype(np.float32)
    got = O.f32_to_e2m1(x)
    assert np.array_equal(got, _e2m1_brute(x))
    assert list(got[:7]) == [0, 2, 2, 4, 4, 6, 6]  # ties to even
    assert got[-1] == 0x8  # -0.0 keeps its sign bit


def _mx_reference(amax: float, emax: int, fmax: float, mbits: int, mode: int) -> tuple[int, float]:
    """Shared exponent code and 1/scale (P/_triton_mx_lora.py:115-159), from math.frexp."""
    if math.isnan(amax):
        return 255, float("nan")
    if mode == O.MX_RCEIL:
        # ceil(log2(fp32(amax / max_pos))) clamped to [-127, 127]; 1/scale is 1.0 for code 0
        d = float(np.float32(np.float32(amax) / np.float32(fmax)))
        if d == 0.0:
            unb = -127
        else:
            m, e = math.frexp(d)  # d = m * 2^e, m in [0.5, 1)
            unb = e - 1 if m == 0.5 else e
        unb = max(-127, min(127, unb))
        return unb + 127, (1.0 if unb == -127 else 2.0 ** -unb)
    if amax == 0.0 or amax < 2.0 ** -126:
        e_floor, frac = -127, amax * 2.0 ** 126  # biased exponent 0: mantissa read as the fraction
    else:
        m, e = math.frexp(amax)
        e_floor, frac = e - 1, 2.0 * m - 1.0
    if mode == O.MX_FLOOR:
        e_unb = e_floor
    elif mode == O.MX_CEIL:
        e_unb = e_floor + (1 if frac > 0.0 else 0)
    else:  # EVEN: round the significand to mbits, carry into the exponent
        e_unb = e_floor + (1 if (e_floor > -127 and frac >= 1.0 - 2.0 ** -(mbits + 1)) else 0)
    unb = max(-127, min(128, e_unb - emax))
    scale = max(2.0 ** unb if unb > -127 else 0.0, 2.0 ** -126)
    return unb + 127, (0.0 if unb == 128 else 1.0 / scale)


@pytest.mark.parametrize("fmt,emax,fmax,mbits", [(O.DT_E2M1, 2, 6.0, 1), (O.DT_E4M3, 8, 448.0, 3),
                                                (O.DT_E5M2, 15, 57344.0, 2)])
@pytest.mark.parametrize("mode", [O.MX_FLOOR, O.MX_RCEIL, O.MX_CEIL, O.MX_EVEN])
def test_mx_shared_exponent(fmt: int, emax: int, fmax: float, mbits: int, mode: int) -> None:
    rng = np.random.default_rng(11)
    pow2 = (2.0 ** np.arange(-149, 128)).astype(np.float32)
    amax = np.concatenate([
        np.abs(_random_f32(4000, 5)).astype(np.float32),
        pow2, np.nextafter(pow2, np.float32(np.inf)), np.nextafter(pow2, np.float32(0)),
        np.array([0.0, 6.0, 448.0, 57344.0, 3.0, 1.5 * 2 ** -130, 1.875, 1.9375, 1.75], dtype=np.float32),
        rng.uniform(0, 10, 500).astype(np.float32),
    ])
    amax = amax[np.isfinite(amax)]
    codes, inv = O.mx_scale(amax, fmt, mode)
    for a, c, i in zip(amax.tolist(), codes.tolist(), inv.tolist()):
        wc, wi = _mx_reference(a, emax, fmax, mbits, mode)
        assert c == wc, (a, c, wc)
        assert i == np.float32(wi), (a, i, wi)
