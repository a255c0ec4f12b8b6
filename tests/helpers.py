"""Test helpers: synthetic data and torch <-> oracle (numpy) conversions."""

from __future__ import annotations

import numpy as np
import torch

import oracle as O


def bf16_np(t: torch.Tensor) -> np.ndarray:
    """bf16 torch tensor -> uint16 numpy bit pattern."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f16_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def np_bf16(a: np.ndarray, device: str | torch.device = "cpu") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def u8_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def normal_bf16(shape: tuple[int, ...], std: float, seed: int) -> torch.Tensor:
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(torch.bfloat16)


def lora_factors(rows: int, cols: int, rank: int, seed: int, *, a_std: float | None = None, b_std: float = 0.01,
                 dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor]:
    """B ~ N(0, b_std) [rows, rank], A ~ N(0, 1/rank) [rank, cols] (std convention of the configs)."""
    g = torch.Generator("cpu").manual_seed(seed)
    a = (torch.randn((rank, cols), generator=g) * (a_std if a_std is not None else 1.0 / rank)).to(dtype)
    b = (torch.randn((rows, rank), generator=g) * b_std).to(dtype)
    return b, a


def oracle_dense_merge(base_bits: np.ndarray, b: torch.Tensor, a: torch.Tensor, strength: float, *,
                       keep_zero_update: bool = False) -> np.ndarray:
    fdt = O.DT_BF16 if b.dtype is torch.bfloat16 else O.DT_F16
    return O.merge_dense(base_bits, bf16_np(b) if fdt == O.DT_BF16 else f16_np(b),
                         bf16_np(a) if fdt == O.DT_BF16 else f16_np(a), strength, fdt=fdt,
                         keep_zero_update=keep_zero_update)


def bf16_ulp_diff(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """|ordinal(x) - ordinal(y)| for bf16 bit patterns (sign-magnitude aware)."""
    def ordinal(h: np.ndarray) -> np.ndarray:
        h = h.astype(np.int32)
        mag = h & 0x7FFF
        return np.where(h & 0x8000, -mag, mag)
    return np.abs(ordinal(x) - ordinal(y))


def int8_initial(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric absmax/127 fp32 encode of a bf16 weight (the configs' initial encode)."""
    wf = w.float()
    scale = (wf.abs().amax(dim=1, keepdim=True) / 127.0).clamp_min(torch.finfo(torch.float32).eps)
    q = torch.round(wf / scale).clamp(-128, 127).to(torch.int8)
    return q, scale


def fp8_initial(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row amax/448 fp32 encode to e4m3fn."""
    wf = w.float()
    scale = (wf.abs().amax(dim=1, keepdim=True) / 448.0).clamp_min(torch.finfo(torch.float32).eps)
    q = (wf / scale).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q, scale


MERGED_MISMATCH_FRACTION = 1e-3
MERGED_ABS_REL = 2.0 ** -18


def assert_merged_close(got: np.ndarray, ref: np.ndarray, base: np.ndarray) -> None:
    """Tolerance contract for dense merged weights (bf16 bit patterns).

    An element matches when it is within 1 bf16 ulp of the oracle, or within
    2^-18 * (|base| + |oracle - base|) absolutely: when base and delta cancel,
    the result is far smaller than its operands and a different fp32
    summation order of B@A (the MFMA's) moves it by many of its own ulps.
    At most 1e-3 of the elements may differ at all.
    """
    g, r, b = (O.bf16_to_f32(x).astype(np.float64) for x in (got, ref, base))
    ulp = bf16_ulp_diff(got, ref)
    tol = MERGED_ABS_REL * (np.abs(b) + np.abs(r - b))
    bad = (ulp > 1) & (np.abs(g - r) > tol)
    assert not bad.any(), f"{int(bad.sum())} merged values outside tolerance, first at {np.argwhere(bad)[0]}"
    assert (ulp > 0).mean() <= MERGED_MISMATCH_FRACTION
