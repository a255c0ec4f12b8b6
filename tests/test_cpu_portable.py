"""The torch CPU ports of the reference's portable merges (oracle/portable.py), which bench.py times as
its CPU baselines, against the C oracle: dequantize and round-to-nearest requant bit for bit for INT8,
FP8, NVFP4, MXFP4 and Q8_0, the addmm_ merge within the floating-point contract, stochastic codes on
the two neighbours."""

from __future__ import annotations

import numpy as np
import pytest
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


# ---- the other formats' portable merges (the CPU baselines of their bench workloads) ----
def _mag_edges(dense: torch.Tensor) -> torch.Tensor:
    dense = dense.clone()
    dense[1] = 0  # eps scales
    dense[2, :32] = torch.tensor([0.0, -0.0] * 16, dtype=torch.bfloat16)
    dense[4, :8] *= 50
    return dense


def test_fp8_portable_equals_the_oracle() -> None:
    dense = _mag_edges(normal_bf16((64, 512), 0.02, 11))
    q, s = P.fp8_requant(dense)
    oq, os_ = O.fp8_requant(bf16_np(dense), 512)
    assert np.array_equal(q.numpy(), oq)
    assert np.array_equal(s.numpy().reshape(-1), os_)
    assert np.array_equal(bf16_np(P.fp8_dequant(q, s)), O.fp8_dequant(q.numpy(), s.numpy(), 512))
    q1, _ = P.fp8_requant(dense, rounding_seed=3)
    x = dense.float() / s
    lo = torch.from_numpy(oq).view(torch.float8_e4m3fn).float()
    got = q1.view(torch.float8_e4m3fn).float()
    # stochastic codes are the round-to-nearest code or its neighbour on the far side of x
    assert bool(((got == lo) | ((got - x).sign() != (lo - x).sign()) | (got == x)).all())


@pytest.mark.parametrize("two_level", [True, False])
def test_nvfp4_portable_equals_the_oracle(two_level: bool) -> None:
    dense = _mag_edges(normal_bf16((48, 256), 0.02, 12))
    q, s, g = P.nvfp4_requant(dense, two_level=two_level)
    oq, os_, og = O.nvfp4_requant(bf16_np(dense), two_level=two_level)
    assert np.array_equal(q.numpy(), oq)
    assert np.array_equal(s.numpy(), os_)
    if two_level:
        assert np.array_equal(g.numpy(), og)
    assert np.array_equal(bf16_np(P.nvfp4_dequant(q, s, g)), O.nvfp4_dequant(oq, os_, og))
    q1, s1, _ = P.nvfp4_requant(dense, two_level=two_level, rounding_seed=5)
    assert torch.equal(s1, s)  # stochastic rounding replaces codes only


def test_mxfp4_portable_equals_the_oracle() -> None:
    dense = _mag_edges(normal_bf16((32, 512), 0.02, 13))
    q, s = P.mxfp4_requant(dense)
    oq, os_ = O.mx_requant(bf16_np(dense), O.DT_E2M1, O.MX_FLOOR)
    assert np.array_equal(q.numpy(), oq)
    assert np.array_equal(s.numpy(), os_)
    assert np.array_equal(bf16_np(P.mxfp4_dequant(q, s)), O.mx_dequant(oq, os_, O.DT_E2M1, 512))


def test_q8_0_portable_equals_the_oracle() -> None:
    dense = _mag_edges(normal_bf16((16, 1024), 0.02, 14))
    # values whose x = v / d sits just below a half (x + 0.5 would round up in fp32)
    dense[6, :32] = torch.tensor([127.0] + [0.5 - 2.0 ** -9] * 31, dtype=torch.bfloat16)
    packed = P.q8_0_requant(dense)
    opacked = O.q8_0_requant(bf16_np(dense))
    assert np.array_equal(packed.numpy().reshape(-1), opacked.reshape(-1))
    assert np.array_equal(bf16_np(P.q8_0_dequant(packed, 1024)), O.q8_0_dequant(opacked, 1024))


def test_portable_merges_run_and_replay() -> None:
    b, a = lora_factors(32, 512, 16, 15)
    dense = normal_bf16((32, 512), 0.02, 16)
    q, s = P.fp8_requant(dense)
    assert torch.equal(P.fp8_merge(q, s, b, a, 1.0, rounding_seed=9)[0], P.fp8_merge(q, s, b, a, 1.0, rounding_seed=9)[0])
    nq, ns, ng = P.nvfp4_requant(dense)
    assert torch.equal(P.nvfp4_merge(nq, ns, ng, b, a, 1.0, rounding_seed=9)[0],
                       P.nvfp4_merge(nq, ns, ng, b, a, 1.0, rounding_seed=9)[0])
    mq, ms = P.mxfp4_requant(dense)
    assert P.mxfp4_merge(mq, ms, b, a, 1.0)[0].shape == mq.shape
    pk = P.q8_0_requant(dense)
    assert P.q8_0_merge(pk, 512, b, a, 1.0, rounding_seed=2).shape == pk.shape
