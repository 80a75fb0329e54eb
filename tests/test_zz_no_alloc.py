"""rq_attention_noalloc (workspace in a static device array) against
rq_attention (caller workspace), both called through the C ABI on the same
inputs: the outputs must be identical, on two calls in a row with the second
one smaller, and sizes beyond the static scratch are rejected on the host."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from residualquant_amd import _lib

from .cases import OURO_G32, make_decode, oracle_attention

pytestmark = pytest.mark.gpu

_MODES = {"anchor": 0, "adjacent": 1}


def _schedule(records):
    bits = (ctypes.c_int * len(records))(*[r[0] for r in records])
    groups = (ctypes.c_int * len(records))(*[r[1] for r in records])
    return bits, groups


def _call(lib, d, device, cache, loop, noalloc, stream=None, sync=True, keep=None):
    g = d.group
    q, k, v = (t.to(device) for t in (d.query, d.key, d.value))
    out = torch.full_like(q, float("nan"))
    starts, lens, table = (t.to(device) for t in (d.query_start_loc, d.seq_lens, d.table))
    kr, vr, km = g.device_args(device)
    if keep is not None:  # the inputs must outlive a call that is not synchronized here
        keep.extend([q, k, v, starts, lens, table, kr, vr, km])
    rows, heads, dim = q.shape
    bits, groups = _schedule(g.records)
    ptr = (lambda t: None if t is None else t.data_ptr())
    stream = (stream or torch.cuda.current_stream(device)).cuda_stream
    common = [q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
              out.data_ptr(), out.stride(0), rows, heads, dim, cache.data_ptr(), cache.size(1),
              cache.size(3), cache.size(4), starts.data_ptr(), lens.data_ptr(), len(d.lengths),
              table.data_ptr(), table.stride(0), table.size(1), ptr(kr), ptr(vr), ptr(km),
              len(g.records), bits, groups, _MODES[g.mode], g.anchor, loop]
    if noalloc:
        status = lib.rq_attention_noalloc(*common, stream)
    else:
        size = lib.rq_attention_workspace_bytes(rows, heads, dim, table.size(1), cache.size(3))
        workspace = torch.empty(size, dtype=torch.uint8, device=device)
        status = lib.rq_attention(*common, workspace.data_ptr(), size, stream)
    _lib.check(status)
    if sync:
        torch.cuda.synchronize(device)
    return out


def test_noalloc_matches_workspace_entry_point(oracle, device):
    lib = _lib.lib()
    # The first call splits each (row, head) over several workgroups (arrival
    # counters and partials in the scratch); the second is smaller and
    # reuses the scratch the first one left behind; the third has 12 and 8
    # rows per request, so it runs the multi-row kernels (their split
    # partials and row shifts in the scratch); the fourth is the first again.
    cases = [([700, 300, 129, 50], 4, 61, None), ([90, 33], 4, 62, None), ([300, 120], 4, 63, [12, 8]),
             ([700, 300, 129, 50], 4, 61, None)]
    for lengths, heads, seed, rows in cases:
        print(f"[case] noalloc lengths={lengths} heads={heads} seed={seed} rows={rows}", flush=True)
        d = make_decode(lengths, heads, 128, OURO_G32, seed=seed, rows_per_request=rows)
        expected_cache = d.group.oracle_cache(oracle)
        cache = torch.from_numpy(expected_cache).to(device)
        for loop in (0, 3):
            want = _call(lib, d, device, cache, loop, noalloc=False)
            got = _call(lib, d, device, cache, loop, noalloc=True)
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"loop {loop}"
            err = np.abs(got.float().cpu().numpy() - oracle_attention(oracle, d, expected_cache, loop))
            assert err.max() <= 2e-2 and err.mean() <= 1e-3, (err.max(), err.mean())


def test_noalloc_calls_on_two_streams_are_ordered(oracle, device):
    """Back-to-back noalloc calls on two streams with no synchronization
    between them: the library makes the second stream wait for the first
    call (both share the scratch's arrival counters and partials), so each
    output equals the workspace entry point's."""
    lib = _lib.lib()
    first = make_decode([700, 300, 129, 50], 4, 128, OURO_G32, seed=71)  # split over several workgroups
    second = make_decode([600, 90, 33], 4, 128, OURO_G32, seed=72)
    caches = [torch.from_numpy(d.group.oracle_cache(oracle)).to(device) for d in (first, second)]
    for loop in (0, 3):
        print(f"[case] noalloc two streams loop={loop}", flush=True)
        want = [_call(lib, d, device, c, loop, noalloc=False) for d, c in zip((first, second), caches)]
        streams = [torch.cuda.Stream(device), torch.cuda.Stream(device)]
        keep = []
        for s in streams:
            s.wait_stream(torch.cuda.current_stream(device))
        got = [_call(lib, d, device, c, loop, noalloc=True, stream=s, sync=False, keep=keep)
               for d, c, s in zip((first, second), caches, streams)]
        torch.cuda.synchronize(device)
        for g, w in zip(got, want):
            assert torch.equal(g.view(torch.int16), w.view(torch.int16)), f"loop {loop}"


def test_noalloc_one_row_decode_at_batch_128(device):
    """A plain decode step of 128 requests x 1 row x 16 heads over 2047
    history tokens runs the per-row kernels, whose workspace (~3.3 MB) fits
    the scratch even though a multi-row call of 128 rows would not: the
    call is checked against the route it takes, and its output equals
    rq_attention's bit for bit at every loop."""
    import residualquant_amd as rq
    from residualquant_amd import workloads

    lib = _lib.lib()
    batch, heads, dim, history, pt = 128, 16, 128, 2047, 16
    print(f"[case] noalloc decode batch {batch} x {heads} heads x {history} history", flush=True)
    pages = (history + pt) // pt
    table = workloads.block_tables(batch, pages, 71, device=device)
    cache = torch.zeros((2, batch * pages, heads, pt, rq.page_width(dim, OURO_G32)), dtype=torch.uint8, device=device)
    kr = workloads.random_sign_rotation(heads, dim, 72, device=device)
    vr = workloads.random_sign_rotation(heads, dim, 73, device=device)
    km = workloads.key_means(4, heads, dim, 74, device=device)
    slots = workloads.history_slots(table, [history] * batch, pt).to(device)
    for start in range(0, slots.numel(), 32768):
        part = slots[start:start + 32768]
        pairs = workloads.loop_kv(part.numel(), heads, dim, 4, 75 + start, device=device, anchor_index=3)
        rq.quantize(pairs, cache, part, kr, vr, km, OURO_G32, "anchor", 3, "ls")
    generator = torch.Generator().manual_seed(76)
    q, k, v = (torch.randn((batch, heads, dim), generator=generator).to(torch.bfloat16) for _ in range(3))

    class Inputs:  # the fields _call reads
        pass

    d = Inputs()
    d.query, d.key, d.value = q, k, v
    d.query_start_loc = torch.arange(batch + 1, dtype=torch.int32)
    d.seq_lens = torch.full((batch,), history + 1, dtype=torch.int32)
    d.lengths = [history + 1] * batch
    d.table = table
    d.group = Inputs()
    d.group.records, d.group.mode, d.group.anchor = OURO_G32, "anchor", 3
    d.group.device_args = lambda dev: (kr, vr, km)
    assert lib.rq_attention_workspace_bytes(batch, heads, dim, pages, pt) > _lib.RQ_ATTENTION_NOALLOC_MAX_BYTES
    for loop in range(4):
        want = _call(lib, d, device, cache, loop, noalloc=False)
        got = _call(lib, d, device, cache, loop, noalloc=True)
        assert bool(torch.isfinite(want.float()).all())
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"loop {loop}"


def test_noalloc_rejects_calls_beyond_the_scratch(device):
    lib = _lib.lib()
    heads, dim, rows = 16, 128, 8192
    needed = lib.rq_attention_workspace_bytes(rows, heads, dim, 8, 16)
    assert needed > _lib.RQ_ATTENTION_NOALLOC_MAX_BYTES
    bits, groups = _schedule(OURO_G32)
    dummy = torch.zeros(16, dtype=torch.uint8, device=device).data_ptr()
    status = lib.rq_attention_noalloc(dummy, heads * dim, dummy, heads * dim, dummy, heads * dim, dummy,
                                      heads * dim, rows, heads, dim, dummy, 1, 16, 200, dummy, dummy, rows,
                                      dummy, 8, 8, None, None, None, 4, bits, groups, 0, 3, 0,
                                      torch.cuda.current_stream(device).cuda_stream)
    assert status == _lib.RQ_ENOSPACE
    assert b"static scratch" in lib.rq_last_error()
