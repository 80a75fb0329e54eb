"""The C ABI library (CPU): it loads, exports every symbol include/rq_hip.h
declares, and rejects invalid arguments on the host before any device work
with the reference's error messages (quantize/api.cpp:18-85,
attention/api.cpp:23-104, dispatch/kernel_registry.h:42-72)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from residualquant_amd import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rq_hip.h")


def _declared():
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:const\s+)?[\w\*\s]+?\b(rq_\w+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        _lib.build()
    return _lib.lib()


def test_header_declares_exactly_the_exported_list():
    assert _declared() == set(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = _declared() - exported
    assert not missing, missing
    for name in _declared():
        assert getattr(lib, name) is not None


def _schedule(records):
    bits = (ctypes.c_int * len(records))(*[r[0] for r in records])
    groups = (ctypes.c_int * len(records))(*[r[1] for r in records])
    return bits, groups


def test_page_width_known_answers_and_errors(lib):
    assert lib.rq_page_width(128, 4, *_schedule([(2, 32)] * 3 + [(4, 32)])) == 200
    assert lib.rq_page_width(128, 4, *_schedule([(2, 16)] * 3 + [(4, 32)])) == 224
    assert lib.rq_page_width(96, 4, *_schedule([(2, 16)] * 3 + [(4, 32)])) == 170
    assert lib.rq_page_width(96, 4, *_schedule([(2, 32)] * 3 + [(4, 32)])) == 152
    assert lib.rq_page_width(128, 1, *_schedule([(2, 48)])) == _lib.RQ_EINVAL
    assert b"divisible" in lib.rq_last_error()
    assert lib.rq_page_width(100, 1, *_schedule([(2, 32)])) == _lib.RQ_EINVAL


def _quantize_call(lib, records, *, head_dim=128, page_tokens=16, page_width=200, mode=0, anchor=3,
                   coefficient=2, tokens=4, input_rows=4, width_override=None, input=0x10000,
                   stride=None, rotation=None):
    count = len(records)
    fake = ctypes.c_void_p(0x10000)
    ptrs = (ctypes.c_void_p * count)(*([input] * count))
    strides = (ctypes.c_int64 * count)(*([stride or 16 * head_dim] * count))
    bits, groups = _schedule(records)
    return lib.rq_quantize(count, ctypes.cast(ptrs, ctypes.c_void_p), ctypes.cast(strides, ctypes.c_void_p),
                           ctypes.cast(ptrs, ctypes.c_void_p), ctypes.cast(strides, ctypes.c_void_p), input_rows,
                           fake, 8, 16, page_tokens, width_override or page_width, fake, tokens, head_dim,
                           rotation, rotation, None, ctypes.cast(bits, ctypes.c_void_p),
                           ctypes.cast(groups, ctypes.c_void_p), mode, anchor, coefficient, None)


G32 = [(2, 32)] * 3 + [(4, 32)]


def test_quantize_rejects_before_device_work(lib):
    assert _quantize_call(lib, G32, coefficient=7) == _lib.RQ_EINVAL
    assert lib.rq_last_error() == b"Unsupported coefficient"
    assert _quantize_call(lib, G32, input_rows=3) == _lib.RQ_EINVAL
    assert lib.rq_last_error() == b"Input has fewer rows than slot mapping"
    assert _quantize_call(lib, G32, width_override=199) == _lib.RQ_EINVAL
    assert lib.rq_last_error() == b"Packed cache width differs from records"
    assert _quantize_call(lib, G32, page_tokens=8) == _lib.RQ_ENOKERNEL
    assert lib.rq_last_error().startswith(b"No compiled packed HIP kernel for heads=16")
    assert _quantize_call(lib, G32, mode=1, anchor=3) == _lib.RQ_ENOKERNEL  # adjacent needs anchor 0
    assert _quantize_call(lib, [(3, 32)]) == _lib.RQ_ENOKERNEL
    assert _quantize_call(lib, G32, anchor=4) == _lib.RQ_ENOKERNEL
    assert _quantize_call(lib, G32, input=0x10004) == _lib.RQ_EINVAL
    assert lib.rq_last_error() == b"K/V addresses and token strides must be 8-byte aligned"
    assert _quantize_call(lib, G32, stride=16 * 128 + 2) == _lib.RQ_EINVAL
    assert _quantize_call(lib, G32, rotation=0x10008) == _lib.RQ_EINVAL
    assert lib.rq_last_error() == b"Rotation addresses must be 16-byte aligned"
    assert _quantize_call(lib, G32, tokens=0, input_rows=0) == _lib.RQ_OK  # empty slot mapping: no launch


def _attention_call(lib, *, loop=0, workspace=None, workspace_bytes=0, query_stride=16 * 128, records=G32,
                    page_width=200, query=0x10000):
    fake = 0x10000
    bits, groups = _schedule(records)
    return lib.rq_attention(query, query_stride, fake, 16 * 128, fake, 16 * 128, fake, 16 * 128, 2, 16, 128,
                            fake, 8, 16, page_width, fake, fake, 2, fake, 4, 4, None, None, None,
                            len(records), ctypes.cast(bits, ctypes.c_void_p), ctypes.cast(groups, ctypes.c_void_p),
                            0, 3, loop, workspace, workspace_bytes, None)


def test_attention_rejects_before_device_work(lib):
    assert _attention_call(lib, loop=4) == _lib.RQ_EINVAL
    assert lib.rq_last_error() == b"Invalid loop index"
    assert _attention_call(lib, page_width=201) == _lib.RQ_EINVAL
    assert lib.rq_last_error() == b"Packed cache width differs from records"
    assert _attention_call(lib, query=0x10004) == _lib.RQ_EINVAL
    assert lib.rq_last_error() == b"Q/K addresses and token strides must be 8-byte aligned"
    assert _attention_call(lib, query_stride=16 * 128 + 2) == _lib.RQ_EINVAL
    assert _attention_call(lib) == _lib.RQ_ENOSPACE
    assert lib.rq_last_error().startswith(b"Attention workspace of")


def test_workspace_size_depends_on_shapes_only(lib):
    a = lib.rq_attention_workspace_bytes(32, 16, 128, 512, 16)
    b = lib.rq_attention_workspace_bytes(32, 16, 128, 512, 16)
    assert a == b and a > 32 * 16 * 130 * 4
    assert lib.rq_attention_workspace_bytes(64, 16, 128, 512, 16) > a


def test_workspace_grows_no_faster_than_linearly_in_rows(lib):
    """The workspace bound of a call with many rows (prefill over packed
    history) is sized for the splits its row count allows: from 64 rows up
    the bytes per row never grow with the rows, and a 4096-row x 16-head
    call over 8192 history tokens needs the per-row route's one-split layout
    (query records of 272 floats plus partials of 130 floats per (row,
    head): ~105 MB), not eight multi-row splits' worth (~277 MB)."""
    rows = (64, 128, 256, 512, 1024, 2048, 4096, 8192, 32768)
    for history_pages in (64, 512, 2048):
        sizes = [lib.rq_attention_workspace_bytes(n, 16, 128, history_pages, 16) for n in rows]
        for (n_small, small), (n_large, large) in zip(zip(rows, sizes), zip(rows[1:], sizes[1:])):
            assert large * n_small <= small * n_large + 4096 * n_large, (history_pages, sizes)
    assert lib.rq_attention_workspace_bytes(4096, 16, 128, 512, 16) < 110 * 10 ** 6


def test_python_ops_mirror_reference_messages():
    cpu = torch.zeros((2, 16, 128), dtype=torch.bfloat16)
    cache = torch.zeros((2, 4, 16, 16, 200), dtype=torch.uint8)
    slots = torch.zeros(2, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="A nonempty group with one K/V input per record required"):
        ops.quantize([(cpu, cpu)] * 3, cache, slots, None, None, None, G32, "anchor", 3, "ls")
    with pytest.raises(RuntimeError, match=r"Contiguous CUDA UINT8 \[2, blocks, heads, page tokens, page width\]"):
        ops.quantize([(cpu, cpu)] * 4, cache, slots, None, None, None, G32, "anchor", 3, "ls")
    with pytest.raises(RuntimeError, match=r"BF16 \[tokens, heads, channels\] with packed trailing strides required"):
        ops.attention(cpu, cpu, cpu, cache, cpu, torch.zeros(3, dtype=torch.int32),
                      torch.zeros(2, dtype=torch.int32), torch.zeros((2, 4), dtype=torch.int32), None, None, None,
                      G32, "anchor", 3, 0)


def _prefill_call(lib, *, head_dim=128, heads_q=4, heads_k=2, query=0x10000, stride=None):
    # Every call below fails validation: the fake pointers never reach a kernel.
    fake = 0x10000
    row = stride or heads_q * head_dim
    return lib.rq_prefill_attention(query, row, fake, heads_k * head_dim, fake, heads_k * head_dim, fake, row,
                                    heads_q, heads_k, head_dim, fake, fake, 2, 64, 64, 0.1, 1, None, 0, None)


def test_prefill_rejects_before_device_work(lib):
    assert _prefill_call(lib, head_dim=64) == _lib.RQ_ENOKERNEL
    assert lib.rq_last_error().startswith(b"No compiled prefill attention kernel")
    assert _prefill_call(lib, heads_q=3) == _lib.RQ_EINVAL
    assert _prefill_call(lib, query=0x10004) == _lib.RQ_EINVAL
    assert lib.rq_last_error() == b"Q/K/V/output addresses and token strides must be 8-byte aligned"
    assert _prefill_call(lib, stride=4 * 128 + 2) == _lib.RQ_EINVAL


def test_prefill_workspace_plan(lib):
    # Query blocks merge within their workgroup: no workspace at any size.
    for args in ((2, 4, 128, 64, 64, 1, 1), (1, 16, 128, 4096, 4096, 1, 1), (1, 16, 128, 4096, 4096, 1, 0),
                 (3, 8, 96, 70000, 90000, 0, 0)):
        assert lib.rq_prefill_workspace_bytes(*args) == 0
    # Invalid shapes report 0 as well (the call itself rejects them).
    assert lib.rq_prefill_workspace_bytes(0, 16, 128, 4096, 4096, 1, 1) == 0



def test_step_ops_reject_before_device_work(lib):
    # Every call below fails validation before any launch (fake pointers never reach a kernel).
    fake = 0x10000
    assert lib.rq_rms_norm(fake, 4096, None, None, 0, None, 0, fake, fake, 4096, 2, 4096, 1e-6, None) == _lib.RQ_EINVAL
    assert b"multiple of 8 up to 2048" in lib.rq_last_error()
    assert lib.rq_rms_norm(fake, 256, None, fake, 256, None, 0, fake, fake, 256, 2, 256, 1e-6, None) == _lib.RQ_EINVAL
    assert lib.rq_rms_norm(fake + 8, 256, None, None, 0, None, 0, fake, fake, 256, 2, 256, 1e-6, None) == _lib.RQ_EINVAL
    assert b"16-byte aligned" in lib.rq_last_error()
    assert lib.rq_rms_norm(fake, 256, fake + 8, None, 0, None, 0, fake, fake, 256, 2, 256, 1e-6, None) == _lib.RQ_EINVAL
    assert b"16-byte aligned" in lib.rq_last_error()
    assert lib.rq_rms_norm(fake, 256, None, None, 0, None, 0, fake, fake, 256, 0, 256, 1e-6, None) == _lib.RQ_OK
    assert lib.rq_rope_qkv(fake, 3 * 256, fake, fake, fake, 16, 2, 127, 1, fake, 256, fake, 256, None, None, 0,
                           None) == _lib.RQ_EINVAL
    assert lib.rq_rope_qkv(fake, 2 * 256, fake, fake, fake, 16, 2, 128, 1, fake, 256, fake, 256, None, None, 0,
                           None) == _lib.RQ_EINVAL
    assert lib.rq_rope_qkv(fake, 3 * 256, fake, fake, fake, 0, 2, 128, 1, fake, 256, fake, 256, None, None, 0,
                           None) == _lib.RQ_EINVAL
    assert lib.rq_silu_mul(fake, 10, fake, 5, 1, 5, None) == _lib.RQ_EINVAL
    assert lib.rq_silu_mul(fake, 6, fake, 4, 1, 4, None) == _lib.RQ_EINVAL
    assert lib.rq_silu_mul(fake + 2, 8, fake, 4, 1, 4, None) == _lib.RQ_EINVAL
