"""The write path on the GPU: a loop group staged loop by loop
(residualquant_amd/group.py, install_model.py:17-52, packed_backend.py:101-137)
writes the same cache bytes as one quantize of every record, with the earlier
loops kept on the device or, during prefill, in pinned host memory
(prefill_offload.py, the reference's prefill_offload.py:10-200) returned in
chunks or through the lookahead ring."""

from __future__ import annotations

import pytest
import torch

import residualquant_amd as rq
from residualquant_amd import workloads
from residualquant_amd.prefill_offload import PrefillCPUOffload

pytestmark = pytest.mark.gpu

RECORDS = ((2, 32), (2, 32), (2, 32), (4, 32))
CONFIG = {"reference_mode": "anchor", "anchor_index": 3, "coefficient_method": "ls"}
HEADS, DIM, PT = 2, 128, 16


def _layer(tokens, seed, device):
    pages = (tokens + PT - 1) // PT + 1
    table = workloads.block_tables(1, pages, seed, device=device)
    slots = workloads.history_slots(table, [tokens], PT).to(device)
    pairs = workloads.loop_kv(tokens, HEADS, DIM, len(RECORDS), seed + 1, device=device, anchor_index=3)
    kr = workloads.random_sign_rotation(HEADS, DIM, seed + 2, device=device)
    vr = workloads.random_sign_rotation(HEADS, DIM, seed + 3, device=device)
    mean = torch.randn((len(RECORDS), HEADS, DIM), generator=torch.Generator().manual_seed(seed)).to(device)
    shape = (2, pages, HEADS, PT, rq.page_width(DIM, RECORDS))
    return pairs, slots, kr, vr, mean, shape


def _direct(layer, device):
    pairs, slots, kr, vr, mean, shape = layer
    cache = torch.zeros(shape, dtype=torch.uint8, device=device)
    rq.quantize(pairs, cache, slots, kr, vr, mean, RECORDS, "anchor", 3, "ls")
    return cache


def test_group_store_matches_one_quantize(device):
    layer = _layer(333, 11, device)
    pairs, slots, kr, vr, mean, shape = layer
    cache = torch.zeros(shape, dtype=torch.uint8, device=device)
    group = rq.DeferredKVGroup(CONFIG, RECORDS, PT)
    done = [group.store(k, v, cache, slots, kr, vr, mean) for k, v in pairs]
    assert done == [False, False, False, True]
    assert torch.equal(cache, _direct(layer, device))


@pytest.mark.parametrize("lookahead", [False, True], ids=["chunks", "lookahead"])
def test_prefill_offload_matches_device_staging(device, lookahead):
    layers, tokens = 3, 250  # 250 tokens in chunks of 96: 96, 96, 58
    offload = PrefillCPUOffload(96, len(RECORDS) - 1, HEADS, DIM)
    offload.lookahead_enabled = lookahead
    offload.reserve(tokens)
    chain = []
    groups = []
    for i in range(layers):
        group = rq.DeferredKVGroup(CONFIG, RECORDS, PT, prefill_offload=offload)
        if lookahead:
            group.offload_chain, group.offload_index = chain, i
            chain.append(group)
        groups.append(group)
    for call in range(2):  # the second prompt reuses the pinned buffers and rings
        print(f"offload lookahead={lookahead} call {call}", flush=True)
        data = [_layer(tokens, 100 * call + 7 * i, device) for i in range(layers)]
        caches = [torch.zeros(d[5], dtype=torch.uint8, device=device) for d in data]
        # Model order: every layer of loop 0, then of loop 1, ...
        for loop in range(len(RECORDS)):
            for i, (pairs, slots, kr, vr, mean, _) in enumerate(data):
                key, value = pairs[loop]
                done = groups[i].store(key.clone(), value.clone(), caches[i], slots, kr, vr, mean, prefill=True)
                assert done == (loop == len(RECORDS) - 1)
        for i, d in enumerate(data):
            assert torch.equal(caches[i], _direct(d, device)), (call, i)
    if lookahead:
        assert offload.prefetched == {}


def test_offload_store_round_trip(device):
    offload = PrefillCPUOffload(64, 1, HEADS, DIM)
    key = torch.randn((100, HEADS, DIM), device=device).to(torch.bfloat16)
    value = torch.randn((100, HEADS, DIM), device=device).to(torch.bfloat16)
    buffer = offload.store(key, value, None)
    assert buffer.is_pinned() and buffer.shape == (2, 100, HEADS, DIM)
    key_copy, value_copy = key.clone(), value.clone()
    key.zero_()  # the caller may reuse its tensors right away
    torch.cuda.synchronize()
    assert torch.equal(buffer[0], key_copy.cpu()) and torch.equal(buffer[1], value_copy.cpu())
    again = offload.store(value_copy, key_copy, buffer)
    torch.cuda.synchronize()
    assert again is buffer and torch.equal(buffer[0], value_copy.cpu())
