"""GGUF dequantize oracle (every type of P/gguf_dequant.py:278-294), pinned
without importing the reference.

The oracle (oracle/lm_oracle.c, lmo_gguf_dequant) follows the reference's
torch-op formulation: tensor splits, reshapes and shifts.  The pin below is a
second statement of each format, written from the public ggml reference
decoders (ggml-quants.c ``dequantize_row_q4_0`` ... ``dequantize_row_iq4_xs``,
MIT).  Those decoders walk each block with explicit loops (pointer bumps,
shift counters, the 12-byte K-quant scale unpacking by ``get_scale_min_k4``
and the Q3_K ``kmask`` shuffle), so a wrong nibble order, bit index or
scale-slot mapping in the oracle disagrees with them.  Both apply the
reference's precision rule: each op in fp32, rounded to the output dtype
(numpy's float32->float16 RNE and torch's float32->bfloat16 RNE are the
rounding routines here).  In fp32 output the ggml loops are exactly ggml's
own float arithmetic.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import gguf_blocks

F32 = np.float32
KVALUES = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
TYPES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10, "Q3_K": 11,
         "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23, "BF16": 30}
SIZES = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         20: (32, 18), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
         23: (256, 136)}  # ggml's GGML_QUANT_SIZES


def _rounder(dt: int):
    if dt == O.DT_F32:
        return lambda x: F32(x)
    if dt == O.DT_F16:
        def f16(x):
            with np.errstate(over="ignore"):  # overflow to inf is the fp16 result
                return F32(np.float16(F32(x)))
        return f16
    return lambda x: F32(torch.tensor([float(F32(x))], dtype=torch.float32).to(torch.bfloat16).item())


def _f16(b: np.ndarray, off: int) -> np.float32:
    return F32(b[off:off + 2].copy().view(np.float16)[0])


def _scale_min_k4(j: int, q: np.ndarray) -> tuple[int, int]:
    if j < 4:
        return int(q[j]) & 63, int(q[j + 4]) & 63
    return (int(q[j + 4]) & 0xF) | ((int(q[j - 4]) >> 6) << 4), (int(q[j + 4]) >> 4) | ((int(q[j]) >> 6) << 4)


def ggml_dequant_block(t: int, x: np.ndarray, r) -> list:
    """One block, in the order and loop structure of ggml's dequantize_row_* (r = output rounding)."""
    y: list = []
    if t in (0, 1, 30):
        if t == 0:
            v = F32(x.copy().view(np.float32)[0])
        elif t == 1:
            v = _f16(x, 0)
        else:
            v = F32(np.array([int(x[0]) | (int(x[1]) << 8)], np.uint32).__lshift__(16).view(np.float32)[0])
        return [r(v)]
    if t == 8:  # block_q8_0 {d; qs[32]}
        d = r(_f16(x, 0))
        return [r(d * F32(int(np.int8(x[2 + j])))) for j in range(32)]
    if t in (2, 3, 20):  # block_q4_0 {d; qs[16]}, block_q4_1 {d; m; qs[16]}, block_iq4_nl {d; qs[16]}
        d = r(_f16(x, 0))
        qs = x[4:] if t == 3 else x[2:]
        y = [F32(0)] * 32
        for j in range(16):
            lo, hi = int(qs[j]) & 0x0F, int(qs[j]) >> 4
            if t == 2:
                y[j], y[j + 16] = r(F32(lo - 8) * d), r(F32(hi - 8) * d)
            elif t == 20:
                y[j], y[j + 16] = r(d * F32(KVALUES[lo])), r(d * F32(KVALUES[hi]))
            else:
                m = r(_f16(x, 2))
                y[j], y[j + 16] = r(r(F32(lo) * d) + m), r(r(F32(hi) * d) + m)
        return y
    if t in (6, 7):  # block_q5_0 {d; qh[4]; qs[16]}, block_q5_1 {d; m; qh[4]; qs[16]}
        d = r(_f16(x, 0))
        off = 4 if t == 7 else 2
        qh = int(x[off]) | (int(x[off + 1]) << 8) | (int(x[off + 2]) << 16) | (int(x[off + 3]) << 24)
        qs = x[off + 4:]
        y = [F32(0)] * 32
        for j in range(16):
            xh0 = ((qh >> j) << 4) & 0x10
            xh1 = (qh >> (j + 12)) & 0x10
            x0, x1 = (int(qs[j]) & 0x0F) | xh0, (int(qs[j]) >> 4) | xh1
            if t == 6:
                y[j], y[j + 16] = r(F32(x0 - 16) * d), r(F32(x1 - 16) * d)
            else:
                m = r(_f16(x, 2))
                y[j], y[j + 16] = r(r(F32(x0) * d) + m), r(r(F32(x1) * d) + m)
        return y
    if t == 10:  # block_q2_K {scales[16]; qs[64]; d; dmin}
        d, mn = r(_f16(x, 80)), r(_f16(x, 82))
        q0, is_ = 16, 0
        for _n in range(0, 256, 128):
            shift = 0
            for _j in range(4):
                for half in (0, 16):
                    sc = int(x[is_])
                    is_ += 1
                    dl, ml = r(d * F32(sc & 0xF)), r(mn * F32(sc >> 4))
                    for l in range(16):
                        y.append(r(r(dl * F32((int(x[q0 + l + half]) >> shift) & 3)) - ml))
                shift += 2
            q0 += 32
        return y
    if t == 11:  # block_q3_K {hmask[32]; qs[64]; scales[12]; d}
        d_all = r(_f16(x, 108))
        aux = x[96:108].copy().view(np.uint32).astype(np.uint64)
        k1, k2 = 0x03030303, 0x0F0F0F0F
        tmp = int(aux[2])
        a0, a1 = int(aux[0]), int(aux[1])
        aux2 = ((a0 >> 4) & k2) | (((tmp >> 4) & k1) << 4)
        aux3 = ((a1 >> 4) & k2) | (((tmp >> 6) & k1) << 4)
        aux0 = (a0 & k2) | (((tmp >> 0) & k1) << 4)
        aux1 = (a1 & k2) | (((tmp >> 2) & k1) << 4)
        scales = np.array([aux0, aux1, aux2, aux3], np.uint32).view(np.int8)
        q0, m, is_ = 32, 1, 0
        for _n in range(0, 256, 128):
            shift = 0
            for _j in range(4):
                for half in (0, 16):
                    dl = r(d_all * F32(int(scales[is_]) - 32))
                    is_ += 1
                    for l in range(16):
                        q = int(np.int8((int(x[q0 + l + half]) >> shift) & 3)) - (0 if int(x[l + half]) & m else 4)
                        y.append(r(dl * F32(q)))
                shift += 2
                m <<= 1
            q0 += 32
        return y
    if t in (12, 13):  # block_q4_K {d; dmin; scales[12]; qs[128]}, block_q5_K {...; qh[32]; qs[128]}
        d, mn = r(_f16(x, 0)), r(_f16(x, 2))
        sc12 = x[4:16]
        ql0 = 48 if t == 13 else 16
        is_, u1, u2 = 0, 1, 2
        for _j in range(0, 256, 64):
            s1, m1 = _scale_min_k4(is_, sc12)
            s2, m2 = _scale_min_k4(is_ + 1, sc12)
            d1, mm1, d2, mm2 = r(d * F32(s1)), r(mn * F32(m1)), r(d * F32(s2)), r(mn * F32(m2))
            for l in range(32):
                q = int(x[ql0 + l]) & 0xF
                if t == 13:
                    q += 16 if int(x[16 + l]) & u1 else 0
                y.append(r(r(d1 * F32(q)) - mm1))
            for l in range(32):
                q = int(x[ql0 + l]) >> 4
                if t == 13:
                    q += 16 if int(x[16 + l]) & u2 else 0
                y.append(r(r(d2 * F32(q)) - mm2))
            ql0 += 32
            is_ += 2
            u1 <<= 2
            u2 <<= 2
        return y
    if t == 14:  # block_q6_K {ql[128]; qh[64]; scales[16]; d}
        d = r(_f16(x, 208))
        y = [F32(0)] * 256
        for n in range(2):
            ql, qh, sc, yb = 64 * n, 128 + 32 * n, 192 + 8 * n, 128 * n
            for l in range(32):
                is_ = l // 16
                q1 = int(np.int8((int(x[ql + l]) & 0xF) | (((int(x[qh + l]) >> 0) & 3) << 4))) - 32
                q2 = int(np.int8((int(x[ql + l + 32]) & 0xF) | (((int(x[qh + l]) >> 2) & 3) << 4))) - 32
                q3 = int(np.int8((int(x[ql + l]) >> 4) | (((int(x[qh + l]) >> 4) & 3) << 4))) - 32
                q4 = int(np.int8((int(x[ql + l + 32]) >> 4) | (((int(x[qh + l]) >> 6) & 3) << 4))) - 32
                for k, q in enumerate((q1, q2, q3, q4)):
                    y[yb + l + 32 * k] = r(r(d * F32(int(np.int8(x[sc + is_ + 2 * k])))) * F32(q))
        return y
    if t == 23:  # block_iq4_xs {d; scales_h; scales_l[4]; qs[128]}
        d = r(_f16(x, 0))
        sh = int(x[2]) | (int(x[3]) << 8)
        for ib in range(8):
            ls = ((int(x[4 + ib // 2]) >> 4 * (ib % 2)) & 0xF) | (((sh >> 2 * ib) & 3) << 4)
            dl = r(d * F32(ls - 32))
            qs = x[8 + 16 * ib:]
            blk = [F32(0)] * 32
            for j in range(16):
                blk[j] = r(dl * F32(KVALUES[int(qs[j]) & 0xF]))
                blk[j + 16] = r(dl * F32(KVALUES[int(qs[j]) >> 4]))
            y.extend(blk)
        return y
    raise AssertionError(t)


def _bits(vals: list, dt: int) -> np.ndarray:
    a = np.array(vals, np.float32)
    if dt == O.DT_F32:
        return a.view(np.uint32)
    if dt == O.DT_F16:
        with np.errstate(over="ignore"):
            return a.astype(np.float16).view(np.uint16)
    u = a.view(np.uint32)
    assert not np.any(u & 0xFFFF), "bf16 step left low bits set"
    return (u >> 16).astype(np.uint16)


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("dt", [O.DT_BF16, O.DT_F16, O.DT_F32], ids=["bf16", "f16", "f32"])
def test_oracle_matches_ggml_loop_decoders(name: str, dt: int) -> None:
    t = TYPES[name]
    bs, ts = O.gguf_sizes(t)
    nblocks = {1: 96, 32: 8, 256: 3}[bs]
    raw = gguf_blocks(t, nblocks, seed=100 + t)
    got = O.gguf_dequant(raw, t, cd=dt)
    r = _rounder(dt)
    want = []
    for i in range(nblocks):
        want.extend(ggml_dequant_block(t, raw[i * ts:(i + 1) * ts], r))
    got_bits = got.view(np.uint32) if dt == O.DT_F32 else got
    assert np.array_equal(got_bits, _bits(want, dt))


def test_sizes_match_the_ggml_table() -> None:
    from piper_offload_amd import gguf_dequant as G
    from piper_offload_amd.kernels import GGUF_DEQUANT_TYPES

    for t, sz in SIZES.items():
        assert O.gguf_sizes(t) == sz
        assert GGUF_DEQUANT_TYPES[t] == sz
        assert G.GGML_QUANT_SIZES[t] == sz
    assert G.SUPPORTED_QUANT_TYPES == set(SIZES)
    assert O.gguf_sizes(9) is None  # Q8_1: in the size table, not dispatched
    assert G.dequant_shape((7, 3, 10 * 144), 12) == (7, 3, 2560)
    assert G.dequant_shape((5, 68), 8) == (5, 64)


def test_known_answer_blocks() -> None:
    # Q4_0: d = 0.5, qs[j] = j | (15 - j) << 4 -> element j = (j - 8) / 2, element 16 + j = (7 - j) / 2
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:] = [j | ((15 - j) << 4) for j in range(16)]
    got = O.gguf_dequant(blk, 2, cd=O.DT_F32)
    assert got.tolist() == [(j - 8) / 2 for j in range(16)] + [(7 - j) / 2 for j in range(16)]
    # Q8_0 with a bf16-rounded scale: d = 1 + 2^-10 rounds to 1.0 in bf16, stays exact in fp16
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([1 + 2**-10], np.float16).view(np.uint8)
    blk[2:] = np.arange(32, dtype=np.int8).view(np.uint8)
    assert O.gguf_dequant(blk, 8, cd=O.DT_F32).tolist() == [j * (1 + 2**-10) for j in range(32)]
    bf = O.gguf_dequant(blk, 8, cd=O.DT_BF16)
    assert (bf.astype(np.uint32) << 16).view(np.float32).tolist() == [float(j) for j in range(32)]
    # IQ4_NL with d = 1: the code book itself
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:] = [j | (j << 4) for j in range(16)]
    assert O.gguf_dequant(blk, 20, cd=O.DT_F32).tolist() == KVALUES + KVALUES


def test_api_errors_without_a_gpu() -> None:
    from piper_offload_amd import gguf_dequant as G

    with pytest.raises(NotImplementedError, match="Unsupported GGUF quant type"):
        G.dequantize(torch.zeros(4, 36, dtype=torch.uint8), 9)
    with pytest.raises(ValueError, match="GPU tensors"):
        G.dequantize(torch.zeros(4, 34, dtype=torch.uint8), 8)
