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


def fp8_initial(w: torch.Tensor, fp8: torch.dtype = torch.float8_e4m3fn) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row amax/limit fp32 encode to e4m3fn (limit 448) or e5m2 (57344)."""
    limit = float(torch.finfo(fp8).max)
    wf = w.float()
    scale = (wf.abs().amax(dim=1, keepdim=True) / limit).clamp_min(torch.finfo(torch.float32).eps)
    q = (wf / scale).clamp(-limit, limit).to(fp8)
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


# byte offsets of the fp16 fields (d, dmin / m) in each GGUF block struct
GGUF_F16_FIELDS = {2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 20: (0,), 10: (80, 82), 11: (108,),
                   12: (0, 2), 13: (0, 2), 14: (208,), 23: (0,)}


def random_f16_bits(n: int, rng: np.random.Generator, *, with_inf: bool = False) -> np.ndarray:
    """Finite fp16 bit patterns spread over the whole range: signs, subnormals, zeros, up to 65504."""
    mag = np.exp2(rng.uniform(-25.0, 16.0, n)) * rng.uniform(1.0, 2.0, n)
    v = np.minimum(mag, 65504.0).astype(np.float16) * rng.choice(np.array([-1, 1], np.float16), n)
    bits = v.view(np.uint16).copy()
    bits[rng.random(n) < 0.03] = 0
    bits[rng.random(n) < 0.03] = 0x8000
    if with_inf:
        bits[rng.random(n) < 0.01] = 0x7C00
    return bits


def gguf_blocks(quant_type: int, nblocks: int, seed: int) -> np.ndarray:
    """`nblocks` random GGUF blocks of one type as flat bytes; fp16 fields hold finite values
    (the float types: finite values of every magnitude, fp32 subnormals included)."""
    rng = np.random.default_rng(seed)
    bs, ts = O.gguf_sizes(quant_type)
    if quant_type == 1:
        return random_f16_bits(nblocks, rng, with_inf=True).view(np.uint8).copy()
    if quant_type == 30:
        h = rng.integers(0, 1 << 16, nblocks, dtype=np.uint32).astype(np.uint16)
        nan = ((h & 0x7F80) == 0x7F80) & ((h & 0x7F) != 0)
        h[nan] &= 0xFF80  # NaN -> inf of the same sign
        return h.view(np.uint8).copy()
    if quant_type == 0:
        u = rng.integers(0, 1 << 32, nblocks, dtype=np.uint64).astype(np.uint32)
        nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x7FFFFF) != 0)
        u[nan] &= 0xFF800000
        return u.view(np.uint8).copy()
    raw = rng.integers(0, 256, (nblocks, ts), dtype=np.uint8)
    for off in GGUF_F16_FIELDS[quant_type]:
        raw[:, off:off + 2] = random_f16_bits(nblocks, rng).view(np.uint8).reshape(nblocks, 2)
    return raw.reshape(-1)


def mismatch_report(got: np.ndarray, want: np.ndarray, what: str, cols_per_tile: int) -> str:
    """'' when equal; otherwise the count and the first mismatching (row, column, tile) positions."""
    got = np.asarray(got)
    want = np.asarray(want)
    if got.shape != want.shape:
        return f"{what}: shape {got.shape} != {want.shape}"
    bad = np.argwhere(got != want) if got.ndim > 1 else np.argwhere((got != want).reshape(-1, 1))
    if bad.size == 0:
        return ""
    first = ", ".join(
        f"(row {int(r)}, col {int(c)}, tile {int(c) // cols_per_tile}: {got[r, c] if got.ndim > 1 else got[r]} "
        f"!= {want[r, c] if got.ndim > 1 else want[r]})" for r, c in bad[:6])
    return f"{what}: {len(bad)} of {want.size} differ; first {first}"
