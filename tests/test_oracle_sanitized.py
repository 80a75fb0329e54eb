"""The CPU oracle under AddressSanitizer + UndefinedBehaviorSanitizer.

The oracle restates the reference's quantize and attention math
(csrc/quantize/kernel.cuh:33-228, csrc/attention/compute.cuh:226-727) with
fixed-size stack buffers, so an access past a buffer, page or row would
silently corrupt the checker itself.  ``make -C oracle asan`` builds
oracle/sanitize_check.c with rq_oracle.c under both sanitizers (no
recovery) and runs every exported function at the shapes the tests use and
at the buffers' limits; any report aborts the run."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ORACLE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle")


def test_oracle_clean_under_asan_and_ubsan():
    if shutil.which(os.environ.get("CC", "gcc")) is None:
        pytest.skip("no C compiler")
    result = subprocess.run(["make", "-s", "-B", "-C", ORACLE, "asan"], capture_output=True, text=True, timeout=600)
    print(result.stdout[-2000:], result.stderr[-4000:])
    assert result.returncode == 0, result.stderr[-4000:]
    assert "oracle sanitizer run: ok" in result.stdout
