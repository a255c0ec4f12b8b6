"""GGUF dequantize on the GPU (every type of P/gguf_dequant.py:278-294) vs the oracle, bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import gguf_blocks

pytestmark = pytest.mark.gpu

G = pytest.importorskip("piper_offload_amd.gguf_dequant")

DEV = "cuda"
TYPES = {"F32": 0, "F16": 1, "BF16": 30, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10,
         "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23}
DTYPES = {"bf16": (torch.bfloat16, O.DT_BF16), "f16": (torch.float16, O.DT_F16), "f32": (torch.float32, O.DT_F32)}


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous().reshape(-1)
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


def _oracle_bits(raw: np.ndarray, t: int, cd: int) -> np.ndarray:
    out = O.gguf_dequant(raw, t, cd=cd)
    return out.view(np.uint32) if cd == O.DT_F32 else out


def _check(raw: np.ndarray, t: int, rows: int, dtype_name: str, *, offset: int = 0) -> None:
    tdt, cd = DTYPES[dtype_name]
    bs, ts = G.GGML_QUANT_SIZES[t]
    data = raw.reshape(rows, -1)
    if offset:
        # the same bytes at an address that is not 16-byte aligned
        buf = torch.zeros(data.size + offset, dtype=torch.uint8, device=DEV)
        buf[offset:] = torch.from_numpy(data.reshape(-1)).to(DEV)
        dev = buf[offset:].view(rows, -1)
        assert dev.data_ptr() % 16 != 0
    else:
        dev = torch.from_numpy(data).to(DEV)
    got = G.dequantize(dev, t, dtype=tdt)
    assert got.dtype == tdt and tuple(got.shape) == G.dequant_shape(tuple(data.shape), t)
    assert np.array_equal(_bits(got), _oracle_bits(raw, t, cd))


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("dtype_name", list(DTYPES))
def test_dequant_bit_exact(name: str, dtype_name: str) -> None:
    t = TYPES[name]
    bs, _ = G.GGML_QUANT_SIZES[t]
    # 7 rows of a ragged number of blocks: the last 2048-element chunk is partial
    per_row = {1: 1000, 32: 44, 256: 11}[bs]
    raw = gguf_blocks(t, 7 * per_row, seed=7 + t)
    _check(raw, t, 7, dtype_name)


@pytest.mark.parametrize("name", list(TYPES))
def test_dequant_unaligned_source(name: str) -> None:
    t = TYPES[name]
    bs, _ = G.GGML_QUANT_SIZES[t]
    per_row = {1: 520, 32: 33, 256: 9}[bs]
    raw = gguf_blocks(t, 3 * per_row, seed=40 + t)
    _check(raw, t, 3, "bf16", offset=2)


@pytest.mark.parametrize("name", ["F16", "F32", "Q8_0", "Q4_K", "Q6_K"])
def test_dequant_single_block_and_leading_dims(name: str) -> None:
    t = TYPES[name]
    bs, ts = G.GGML_QUANT_SIZES[t]
    one = gguf_blocks(t, 1 if bs > 1 else 13, seed=90 + t)
    _check(one, t, 1, "bf16")
    raw = gguf_blocks(t, 2 * 3 * (4 if bs > 1 else 64), seed=91 + t)
    data = torch.from_numpy(raw.reshape(2, 3, -1)).to(DEV)
    got = G.dequantize(data, t, dtype=torch.float32)
    assert tuple(got.shape) == G.dequant_shape(tuple(data.shape), t)
    assert np.array_equal(_bits(got), _oracle_bits(raw, t, O.DT_F32))


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "Q5_0", "IQ4_XS"])
def test_dequant_large(name: str) -> None:
    # [4096, 4096] logical: 16.8 M elements, 8192 workgroups
    t = TYPES[name]
    bs, ts = G.GGML_QUANT_SIZES[t]
    raw = gguf_blocks(t, 4096 * 4096 // bs, seed=5)
    _check(raw, t, 4096, "bf16")


def test_dequant_errors() -> None:
    with pytest.raises(NotImplementedError, match="Unsupported GGUF quant type"):
        G.dequantize(torch.zeros(2, 36, dtype=torch.uint8, device=DEV), 9)
    with pytest.raises(ValueError, match="whole 144-byte blocks"):
        G.dequantize(torch.zeros(2, 100, dtype=torch.uint8, device=DEV), 12)
    with pytest.raises(ValueError, match="bf16, fp16 or fp32"):
        G.dequantize(torch.zeros(2, 34, dtype=torch.uint8, device=DEV), 8, dtype=torch.float64)
    empty = G.dequantize(torch.zeros(0, 34, dtype=torch.uint8, device=DEV), 8)
    assert tuple(empty.shape) == (0, 32)
