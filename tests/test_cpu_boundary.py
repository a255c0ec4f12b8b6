"""The C-ABI drop-in boundary, checked without a GPU.

* ``libpiper_lora_merge.so`` loads and exports every function that
  ``include/lora_merge.h`` declares, and the Python binding binds each one;
* the ctypes mirrors of ``lm_lora`` / ``lm_rounding`` / ``lm_stack_item``
  have the layout a C compiler gives the header;
* argument validation is host-side and loud (status + message, mapped to
  ValueError), and the product path refuses to run without a GPU instead of
  falling back to the CPU.
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
import tempfile

import pytest
import torch

from piper_offload_amd import _lib as L
from piper_offload_amd import kernels as K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lora_merge.h")


def _declared() -> list[str]:
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|size_t|const char\*)\s+(lm_\w+)\(", text, re.M)))


def test_header_declares_the_entry_points() -> None:
    names = _declared()
    assert len(names) >= 20
    for must in ("lm_int8_merge", "lm_fp8_merge", "lm_nvfp4_merge", "lm_mx_merge", "lm_q8_0_merge",
                 "lm_gguf_dequant", "lm_dense_merge", "lm_int8_merge_stack", "lm_nvfp4_merge_stack",
                 "lm_last_error", "lm_version"):
        assert must in names


def test_library_exports_every_declared_symbol() -> None:
    handle = L.load_library()
    for name in _declared():
        assert hasattr(handle, name), name
    assert set(_declared()) == set(L.exported_symbols())


def test_nm_lists_the_symbols_as_exported_functions() -> None:
    out = subprocess.run(["nm", "-D", "--defined-only", L.library_path()], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in _declared() if n not in exported]
    assert not missing, missing


def test_struct_layout_matches_a_c_compiler() -> None:
    src = r'''
#include <stdio.h>
#include <stddef.h>
#include "lora_merge.h"
#define F(T, m) printf(#T "." #m " %zu\n", offsetof(T, m));
int main(void) {
  printf("lm_lora %zu\n", sizeof(lm_lora));
  F(lm_lora, b) F(lm_lora, a) F(lm_lora, ldb) F(lm_lora, lda) F(lm_lora, rank) F(lm_lora, dtype)
  F(lm_lora, strength) F(lm_lora, reserved)
  printf("lm_rounding %zu\n", sizeof(lm_rounding));
  F(lm_rounding, mode) F(lm_rounding, reserved) F(lm_rounding, seed)
  printf("lm_stack_item %zu\n", sizeof(lm_stack_item));
  F(lm_stack_item, q) F(lm_stack_item, scale) F(lm_stack_item, aux) F(lm_stack_item, q_out)
  F(lm_stack_item, scale_out) F(lm_stack_item, aux_out) F(lm_stack_item, M) F(lm_stack_item, N)
  F(lm_stack_item, lora) F(lm_stack_item, seed)
  return 0;
}
'''
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HEADER), c, "-o", exe], check=True)
        lines = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    c_layout = dict(line.rsplit(" ", 1) for line in lines if line)
    for cname, ctype in (("lm_lora", L.LoraStruct), ("lm_rounding", L.RoundingStruct),
                         ("lm_stack_item", L.StackItem)):
        assert int(c_layout[cname]) == ctypes.sizeof(ctype), cname
        for field, _t in ctype._fields_:
            assert int(c_layout[f"{cname}.{field}"]) == getattr(ctype, field).offset, (cname, field)


def test_version_and_workspace_queries_need_no_gpu() -> None:
    h = L.load_library()
    text = open(HEADER).read()
    assert h.lm_version() == int(re.search(r"#define LM_ABI_VERSION (\d+)", text).group(1))
    small = h.lm_workspace_size(16, 64, 16)
    big = h.lm_workspace_size(14336, 4096, 64)
    assert 256 <= small < big
    assert h.lm_workspace_size(4096, 4096, 16) % 256 == 0
    assert h.lm_stack_workspace_extra(224) > h.lm_stack_workspace_extra(1)
    # routed residual: at most 16 tokens run as one launch with no workspace
    fs = (L.RoutedFactor * 2)()
    fs[0].rank, fs[1].rank = 16, 40
    assert h.lm_routed_workspace_size(1, 4096, fs, 2) == 0
    assert h.lm_routed_workspace_size(16, 4096, fs, 2) == 0
    w17 = h.lm_routed_workspace_size(17, 4096, fs, 2)
    assert w17 >= 17 * 4 * 16 * (4 + 2) and w17 % 256 == 0


def test_invalid_arguments_fail_loudly_before_any_device_work() -> None:
    h = L.load_library()
    rc = h.lm_int8_merge(None, None, None, None, None, None, 16, 64, 64, 0, 0, 0, None, None, None, 0, None)
    assert rc == L.LM_EINVAL
    assert b"non-null" in h.lm_last_error()
    with pytest.raises(ValueError, match="non-null"):
        L.check(h.lm_dense_merge(None, 16, 64, 64, None, None, 0, None))


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU refusal")
def test_product_path_refuses_to_run_without_a_gpu() -> None:
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        L.lib()
    q = torch.zeros(16, 64, dtype=torch.int8)
    s = torch.ones(16, 1)
    b = torch.zeros(16, 16, dtype=torch.bfloat16)
    a = torch.zeros(16, 64, dtype=torch.bfloat16)
    with pytest.raises((RuntimeError, ValueError)):
        K.merge_int8_lora(q, s, None, (1, 64), b, a, 1.0, asymmetric=False, reduce_range=False)
    assert torch.equal(q, torch.zeros_like(q))  # untouched: nothing ran on the CPU
