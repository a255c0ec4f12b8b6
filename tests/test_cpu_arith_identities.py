"""Exhaustive CPU checks of fp32 identities the HIP kernels use (tests/arith/identities.c):
the two-instruction round-half-away of k_q8_fast over every input of its
domain (2.5e9 floats, about 10-15 s), and the three-instruction IEEE quotient
of lm_device.h div_rn over every bf16 and every fp16 operand pair of its
domain (1e9 and 2e9 pairs, about 11 and 15 s)."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "arith", "identities.c")


@pytest.fixture(scope="module")
def binary(tmp_path_factory) -> str:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    out = str(tmp_path_factory.mktemp("arith") / "identities")
    subprocess.run([cc, "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", out, SRC, "-lm"], check=True)
    return out


@pytest.mark.parametrize("identity", ["round", "quotient_bf16", "quotient_f16"])
def test_identity_holds_on_its_whole_domain(binary: str, identity: str) -> None:
    r = subprocess.run([binary, identity], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 mismatches" in r.stdout
