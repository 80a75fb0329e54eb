"""The reference's registered signature set (residualquant_amd/registry.py,
csrc/dispatch/decode_*.cu) on the CPU: its size and the page widths the
library computes for it."""

from __future__ import annotations

import ctypes

from residualquant_amd import _lib, registry
from residualquant_amd.layout import page_width


def test_reference_signature_count():
    # 2 geometries x (10 adjacent-0 + 10 anchor-0 + 7 anchor-3 schedules) x 2 page sizes x mean on/off
    assert len(registry.REFERENCE_SIGNATURES) == 216
    assert len(set(registry.REFERENCE_SIGNATURES)) == 216


def test_page_widths_of_every_signature():
    lib = _lib.lib()
    for s in registry.REFERENCE_SIGNATURES:
        bits = (ctypes.c_int * len(s.records))(*[b for b, _ in s.records])
        groups = (ctypes.c_int * len(s.records))(*[g for _, g in s.records])
        assert lib.rq_page_width(s.head_dim, len(s.records), bits, groups) == page_width(s.head_dim, s.records)
