"""The exact-arithmetic shortcuts of the quantize kernel (csrc/quantize.hip
commit_record), checked exhaustively on the CPU by tests/exact_shortcuts.c:
reciprocal-and-correction division by an E4M3 scale and by the code levels,
ceil(q - 0.5) rounding, the exact code*scale+offset restore and the
single-rounded BF16 sum.  The
canonical formulas are those of the oracle (quantize/kernel.cuh:120-203)."""

from __future__ import annotations

import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def results(tmp_path_factory):
    binary = str(tmp_path_factory.mktemp("shortcuts") / "exact_shortcuts")
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-o", binary,
                    os.path.join(HERE, "exact_shortcuts.c"), "-lm"], check=True)
    out = subprocess.run([binary], check=True, capture_output=True, text=True, timeout=600).stdout
    return {line.split()[0]: int(line.split()[1]) for line in out.splitlines()}


@pytest.mark.parametrize("check", ["reciprocal_division", "half_down_rounding", "code_restore", "bf16_sum",
                                   "level_division"])
def test_shortcut_is_exact(results, check):
    assert results[check] == 0
