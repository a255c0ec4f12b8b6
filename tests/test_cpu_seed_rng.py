"""Seeds and the stochastic-rounding random stream (CPU oracle).

Pins: the reference's derive_seed known answer and error contract
(tests/test_stochastic_rounding.py:23-39 of the reference), the published
Random123 Philox4x32-10 and Philox4x32-7 vectors, and the stream properties the reference's
tests assert of its uniforms (replay, range, decorrelation by target path
and merge index, launch-geometry independence; P/_stochastic_quantization.py
and P/_triton_stochastic_quantization.py).
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle as O
from piper_offload_amd import seeding

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))


def _hex(v: str) -> int:
    return int(v, 16)


@pytest.mark.parametrize("case", GOLDEN["derive_seed"], ids=lambda c: repr(c["parts"]))
def test_derive_seed_known_answer(case: dict) -> None:
    assert O.derive_seed(*case["parts"]) == _hex(case["value"])
    assert seeding.derive_seed(*case["parts"]) == _hex(case["value"])


def test_derive_seed_typed_encoding_and_range() -> None:
    for fn in (O.derive_seed, seeding.derive_seed):
        assert fn("1") != fn(1)
        assert fn("ab", "c") != fn("a", "bc")
        assert 0 <= fn(0, (1 << 64) - 1) < 1 << 64
        with pytest.raises(ValueError, match="unsigned 64-bit"):
            fn(-1)
        with pytest.raises(ValueError, match="unsigned 64-bit"):
            fn(1 << 64)
        with pytest.raises(TypeError, match="strings or unsigned 64-bit"):
            fn(True)
        with pytest.raises(TypeError, match="strings or unsigned 64-bit"):
            fn(1.5)  # type: ignore[arg-type]


def test_package_and_oracle_seeds_agree() -> None:
    rng = np.random.default_rng(7)
    for i in range(200):
        key = f"model.layers.{i}.mlp.gate_proj.weight"
        idx = int(rng.integers(0, 1 << 63))
        assert seeding.derive_seed(key, idx) == O.derive_seed(key, idx)


@pytest.mark.parametrize("rounds,case", [(10, c) for c in GOLDEN["philox4x32_10"]]
                         + [(7, c) for c in GOLDEN["philox4x32_7"]], ids=lambda v: str(v) if isinstance(v, int) else v["ctr"][0])
def test_philox_known_answers(rounds: int, case: dict) -> None:
    ctr = tuple(_hex(v) for v in case["ctr"])
    key = tuple(_hex(v) for v in case["key"])
    assert O.philox4x32(ctr, key, rounds=rounds) == tuple(_hex(v) for v in case["out"])


@pytest.mark.parametrize("rounds", [10, 7])
def test_philox_round_count_matters(rounds: int) -> None:
    # a dropped or extra round must not reproduce the published vectors
    case = GOLDEN[f"philox4x32_{rounds}"][2]
    ctr = tuple(_hex(v) for v in case["ctr"])
    key = tuple(_hex(v) for v in case["key"])
    want = tuple(_hex(v) for v in case["out"])
    assert O.philox4x32(ctr, key, rounds=rounds - 1) != want
    assert O.philox4x32(ctr, key, rounds=rounds + 1) != want


def test_sr_stream_uses_seven_rounds() -> None:
    assert O.sr_rounds() == 7


def test_stream_layout_eight_halfwords_per_philox_call() -> None:
    # element i uses word j>>1 (j = i & 7) of Philox4x32-7(counter = i >> 3, key = seed),
    # complemented when j>>1 is odd: its high half for even j, low half for odd j; u = h * 2^-16
    seed = O.derive_seed("layers.0.weight", 0)
    key = (seed & 0xFFFFFFFF, seed >> 32)
    start = (1 << 33) + 5  # counter above 2^32 exercises the high counter word
    u = O.uniforms(seed, start, 64)
    for k in range(64):
        idx = start + k
        ctr = idx >> 3
        words = O.philox4x32((ctr & 0xFFFFFFFF, ctr >> 32, 0, 0), key, rounds=7)
        j = idx & 7
        w = words[j >> 1] ^ (0xFFFFFFFF if (j >> 1) & 1 else 0)
        h = (w >> (16 * (1 - (j & 1)))) & 0xFFFF
        assert u[k] == np.float32(h / 65536.0)


def test_uniforms_replay_range_and_geometry_independence() -> None:
    seed = O.derive_seed("layers.0.weight", 0)
    a = O.uniforms(seed, 0, 64 * 128)
    b = O.uniforms(seed, 0, 64 * 128)
    assert np.array_equal(a, b)
    assert (a >= 0).all() and (a < 1).all()
    # any sub-range drawn on its own equals the same slice of a longer draw
    for lo, n in ((1, 7), (13, 100), (4096, 333)):
        assert np.array_equal(O.uniforms(seed, lo, n), a[lo:lo + n])


def test_target_path_and_merge_index_decorrelate() -> None:
    base = O.uniforms(O.derive_seed("layers.0.weight", 0), 0, 8192)
    other_path = O.uniforms(O.derive_seed("layers.1.weight", 0), 0, 8192)
    other_merge = O.uniforms(O.derive_seed("layers.0.weight", 1), 0, 8192)
    assert not np.array_equal(base, other_path)
    assert not np.array_equal(base, other_merge)
    # and are statistically unrelated
    assert abs(np.corrcoef(base, other_path)[0, 1]) < 0.05
    assert abs(np.corrcoef(base, other_merge)[0, 1]) < 0.05


def test_uniforms_are_uniform_on_the_16_bit_grid() -> None:
    u = O.uniforms(O.derive_seed("stats", 3), 0, 1 << 18)
    h = np.round(u * 65536.0)
    assert np.array_equal(h / 65536.0, u.astype(np.float64))  # exactly on the 2^-16 grid
    counts = np.bincount((u * 16).astype(np.int64), minlength=16)
    expected = u.size / 16
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 45.0  # 15 dof; p ~ 1e-4
    assert abs(float(u.mean()) - (0.5 - 2.0 ** -17)) < 0.003


def test_sr_stream_has_no_serial_correlation() -> None:
    # Philox4x32-7 draws: neighbouring elements (same call, next half-word,
    # next word, next call) are uncorrelated at the 2^18-sample level
    u = O.uniforms(O.derive_seed("serial", 0), 0, 1 << 18).astype(np.float64) - 0.5
    for lag in (1, 2, 3, 4, 7, 8, 9, 16):
        r = float(np.dot(u[:-lag], u[lag:]) / np.dot(u, u))
        assert abs(r) < 0.01, (lag, r)

