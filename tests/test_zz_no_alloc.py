"""lm_int8_merge_noalloc against lm_int8_merge, through the C ABI.

lm_int8_merge_noalloc has no counterpart in the reference: it is
lm_int8_merge for callers that cannot allocate (code under HIP graph capture,
tight serving loops), with its scratch in a static device array of
LM_NOALLOC_SCRATCH_BYTES per GPU.  Its results must equal the workspace entry
point's bit for bit, on consecutive calls that reuse the array (the second
one smaller, so stale contents of the first would show), and shapes beyond
the array must fail before any device work.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import int8_initial, lora_factors, normal_bf16

pytestmark = pytest.mark.gpu

K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import _lib as L  # noqa: E402
from piper_offload_amd import derive_seed  # noqa: E402

DEV = "cuda"
NOALLOC_SCRATCH_BYTES = 8 << 20  # LM_NOALLOC_SCRATCH_BYTES


def _noalloc(q, s, b, a, strength, seed, q_out, s_out) -> int:  # noqa: ANN001
    lora = L.lora_struct(b, a, strength)
    rnd = L.rounding_struct(seed)
    return L.lib().lm_int8_merge_noalloc(q.data_ptr(), s.data_ptr(), None, q_out.data_ptr(), s_out.data_ptr(), None,
                                         q.shape[0], q.shape[1], q.shape[1], L.LM_F32, 0, 0, ctypes.byref(lora),
                                         ctypes.byref(rnd), L.stream_ptr(q.device))


@pytest.mark.parametrize("in_place", [False, True])
def test_noalloc_equals_the_workspace_entry_point_on_consecutive_calls(in_place):
    cases = [((1000, 8192), 64, 1.0, derive_seed("noalloc.long.weight", 0)),  # two-pass rows (row slots in scratch)
             ((300, 6144), 48, 0.5, derive_seed("noalloc.long.weight", 1)),    # smaller two-pass: stale slots would show
             ((4096, 4096), 32, 0.5, derive_seed("noalloc.first.weight", 0)),  # SR, rank 32
             ((1000, 512), 16, -0.75, None)]                                   # smaller, RTN, ragged rows
    for i, ((rows, cols), rank, strength, seed) in enumerate(cases):
        q, s = int8_initial(normal_bf16((rows, cols), 0.02, 50 + i))
        b, a = lora_factors(rows, cols, rank, 60 + i)
        qd, sd, bd, ad = q.to(DEV), s.to(DEV), b.to(DEV), a.to(DEV)
        eq, es, _ = K.merge_int8_lora(qd, sd, None, (1, cols), bd, ad, strength, asymmetric=False, reduce_range=False,
                                      rounding_seed=seed)
        q_out = qd.clone() if in_place else torch.empty_like(qd)
        s_out = sd.clone() if in_place else torch.empty_like(sd)
        src_q, src_s = (q_out, s_out) if in_place else (qd, sd)
        rc = _noalloc(src_q, src_s, bd, ad, strength, seed, q_out, s_out)
        L.check(rc)
        torch.cuda.synchronize()
        assert torch.equal(q_out, eq), f"call {i}: codes differ"
        assert torch.equal(s_out.reshape(-1), es.reshape(-1)), f"call {i}: scales differ"


def test_noalloc_rejects_shapes_beyond_its_scratch_before_device_work():
    rows, cols, rank = 16, 64, 64
    q = torch.zeros(rows, cols, dtype=torch.int8, device=DEV)
    s = torch.ones(rows, 1, device=DEV)
    b = torch.zeros(rows, rank, dtype=torch.bfloat16, device=DEV)
    a = torch.zeros(rank, cols, dtype=torch.bfloat16, device=DEV)
    big_rows = 40000  # (rows + cols) * 64 * 2 bytes of relayout > 8 MiB
    assert L.lib().lm_workspace_size(big_rows, 40000, rank) > NOALLOC_SCRATCH_BYTES
    lora = L.LoraStruct(b.data_ptr(), a.data_ptr(), 40000, 40000, rank, L.LM_BF16, 1.0, 0)
    rnd = L.rounding_struct(None)
    rc = L.lib().lm_int8_merge_noalloc(q.data_ptr(), s.data_ptr(), None, q.data_ptr(), s.data_ptr(), None, big_rows,
                                       40000, 40000, L.LM_F32, 0, 0, ctypes.byref(lora), ctypes.byref(rnd),
                                       L.stream_ptr(q.device))
    assert rc == L.LM_EWORKSPACE
    assert b"static array" in L.lib().lm_last_error()
    assert not q.any()  # nothing ran
