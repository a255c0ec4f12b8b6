"""The torch CPU port of the reference's portable INT8 merge (oracle/portable.py), which bench.py
times as its CPU baseline, against the C oracle: dequantize and round-to-nearest requant bit for
bit, the addmm_ merge within the floating-point contract, stochastic codes on the two neighbours."""

from __future__ import annotations

import numpy as np
import torch

import oracle as O
from helpers import assert_merged_close, bf16_np, int8_initial, lora_factors, normal_bf16
from oracle import portable as P


def test_dequant_and_rtn_requant_equal_the_oracle() -> None:
    dense = normal_bf16((96, 512), 0.02, 1)
    dense[3] = 0  # eps scale
    dense[5, :7] *= 40
    q, s = P.int8_requant(dense)
    oq, os_, _ = O.int8_requant(bf16_np(dense), 512)
    assert np.array_equal(q.numpy(), oq)
    assert np.array_equal(s.numpy().reshape(-1), os_)
    assert np.array_equal(bf16_np(P.int8_dequant(q, s)), O.int8_dequant(q.numpy(), s.numpy(), None, 512))


def test_addmm_merge_is_within_the_dense_contract() -> None:
    q, s = int8_initial(normal_bf16((64, 256), 0.02, 2))
    b, a = lora_factors(64, 256, 16, 3)
    dense = P.int8_dequant(q, s)
    base = bf16_np(dense).copy()  # bf16_np of a CPU tensor is a view: keep the pre-merge values
    dense.addmm_(b, a, alpha=0.5)
    assert_merged_close(bf16_np(dense), O.merge_dense(base, bf16_np(b), bf16_np(a), 0.5), base)


def test_stochastic_codes_are_neighbours_and_replay() -> None:
    q, s = int8_initial(normal_bf16((64, 256), 0.02, 4))
    b, a = lora_factors(64, 256, 16, 5)
    q1, s1 = P.int8_merge(q, s, b, a, 1.0, rounding_seed=7)
    q2, _ = P.int8_merge(q, s, b, a, 1.0, rounding_seed=7)
    q3, _ = P.int8_merge(q, s, b, a, 1.0, rounding_seed=8)
    assert torch.equal(q1, q2) and not torch.equal(q1, q3)
    dense = P.int8_dequant(q, s)
    dense.addmm_(b, a, alpha=1.0)
    y = dense.float() / s1
    assert bool(((q1.float() == torch.floor(y).clamp(-128, 127)) | (q1.float() == torch.ceil(y).clamp(-128, 127))).all())
