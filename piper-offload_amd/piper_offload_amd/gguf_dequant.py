"""GGUF dequantization on MI355X: the API of P/gguf_dequant.py.

``dequantize(data, quant_type, dtype=...)`` keeps the reference's signature,
output shape (``dequant_shape``) and errors (``NotImplementedError`` for a
type it does not dispatch), and runs one HIP kernel per call instead of a
chain of torch ops.  Every type of the reference's dispatch table
(P/gguf_dequant.py:278-294) is implemented: F32, F16, BF16, Q4_0, Q4_1,
Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL and IQ4_XS.  The
result equals the reference's bit for bit in bf16, fp16 and fp32: each step
rounds to ``dtype`` in the reference's order.

``GGML_QUANT_SIZES`` is ggml's (block elements, block bytes) table, keyed by
the ``gguf.GGMLQuantizationType`` integer, as in P/gguf_dequant.py:21-23 (the
reference reads it from the ``gguf`` package; the values are fixed by the
GGUF format).

P/ = the reference's src/piper_offload/.
"""

from __future__ import annotations

import torch

from .kernels import GGUF_DEQUANT_TYPES, dequantize_gguf

__all__ = ["GGML_QUANT_SIZES", "K_SCALE_SIZE", "QK_K", "SUPPORTED_QUANT_TYPES", "dequant_shape", "dequantize"]

QK_K = 256
K_SCALE_SIZE = 12

GGML_QUANT_SIZES: dict[int, tuple[int, int]] = {
    0: (1, 4),        # F32
    1: (1, 2),        # F16
    2: (32, 18),      # Q4_0
    3: (32, 20),      # Q4_1
    6: (32, 22),      # Q5_0
    7: (32, 24),      # Q5_1
    8: (32, 34),      # Q8_0
    9: (32, 36),      # Q8_1
    10: (256, 84),    # Q2_K
    11: (256, 110),   # Q3_K
    12: (256, 144),   # Q4_K
    13: (256, 176),   # Q5_K
    14: (256, 210),   # Q6_K
    15: (256, 292),   # Q8_K
    16: (256, 66),    # IQ2_XXS
    17: (256, 74),    # IQ2_XS
    18: (256, 98),    # IQ3_XXS
    19: (256, 50),    # IQ1_S
    20: (32, 18),     # IQ4_NL
    21: (256, 110),   # IQ3_S
    22: (256, 82),    # IQ2_S
    23: (256, 136),   # IQ4_XS
    24: (1, 1),       # I8
    25: (1, 2),       # I16
    26: (1, 4),       # I32
    27: (1, 8),       # I64
    28: (1, 8),       # F64
    29: (256, 56),    # IQ1_M
    30: (1, 2),       # BF16
    34: (256, 54),    # TQ1_0
    35: (256, 66),    # TQ2_0
}

# the types dequantize() accepts (P/gguf_dequant.py:278-294)
SUPPORTED_QUANT_TYPES = frozenset(GGUF_DEQUANT_TYPES)


def dequant_shape(packed_shape: tuple[int, ...], quant_type: int) -> tuple[int, ...]:
    """Logical tensor shape from the packed byte-level shape (P/gguf_dequant.py:297-300)."""
    block_size, type_size = GGML_QUANT_SIZES[quant_type]
    return (*packed_shape[:-1], packed_shape[-1] // type_size * block_size)


def dequantize(data: torch.Tensor, quant_type: int, *, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Dequantize GGUF raw bytes on the GPU (P/gguf_dequant.py:303-331).

    Raises ``NotImplementedError`` for a type outside the reference's dispatch
    table and ``ValueError`` for CPU data or a ``dtype`` other than bf16, fp16
    or fp32 (the HIP kernels compute in those).
    """
    return dequantize_gguf(data, quant_type, dtype=dtype)
