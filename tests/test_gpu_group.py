"""The write path on the GPU: a loop group staged loop by loop
(residualquant_amd/group.py, install_model.py:17-52, packed_backend.py:101-137)
writes the CPU oracle's bytes for one quantize of every record (bit-exact),
with the earlier loops kept on the device or, during prefill, spilled to
pinned host memory (residualquant_amd/prefill_offload.py, whose contract is
the reference's prefill_offload.py:10-200) and recalled in windows or through
the lookahead ring of layer slots."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import residualquant_amd as rq
from residualquant_amd import prefill_offload, workloads
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


def _expected(oracle, layer):
    """The oracle's bytes for one quantize of every record of ``layer``."""
    pairs, slots, kr, vr, mean, shape = layer
    bits = workloads.bf16_bits
    cache = np.zeros(shape, dtype=np.uint8)
    oracle.quantize([(bits(k), bits(v)) for k, v in pairs], cache, slots.cpu().numpy(), bits(kr), bits(vr),
                    mean.cpu().numpy(), RECORDS, "anchor", 3, "ls")
    return cache


def test_group_store_matches_one_quantize(oracle, device):
    layer = _layer(333, 11, device)
    pairs, slots, kr, vr, mean, shape = layer
    cache = torch.zeros(shape, dtype=torch.uint8, device=device)
    group = rq.DeferredKVGroup(CONFIG, RECORDS, PT)
    done = [group.store(k, v, cache, slots, kr, vr, mean) for k, v in pairs]
    assert done == [False, False, False, True]
    assert np.array_equal(cache.cpu().numpy(), _expected(oracle, layer))


@pytest.mark.parametrize("lookahead,layers,ring", [(False, 3, 8), (True, 3, 8), (True, 5, 2)],
                         ids=["chunks", "lookahead", "lookahead-2-slots"])
def test_prefill_offload_matches_device_staging(oracle, device, monkeypatch, lookahead, layers, ring):
    # With 2 layer slots for 5 layers, later layers are recalled as earlier
    # ones free their slot (chain order), and none waits for a slot.
    monkeypatch.setattr(prefill_offload, "RING_MAX_LAYERS", ring)
    tokens = 250  # 250 tokens in windows of 96: 96, 96, 58
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
            assert np.array_equal(caches[i].cpu().numpy(), _expected(oracle, d)), (call, i)
    if lookahead:
        assert offload.prefetched == {}
        assert offload.layers.slots == ring and sorted(offload.layers.free) == list(range(ring))
    assert sorted(offload.windows.free) == [0, 1]


def test_offload_store_round_trip(device):
    offload = PrefillCPUOffload(64, 1, HEADS, DIM)
    key = torch.randn((100, HEADS, DIM), device=device).to(torch.bfloat16)
    value = torch.randn((100, HEADS, DIM), device=device).to(torch.bfloat16)
    spill = offload.store(key, value, None)
    assert spill.block.is_pinned() and spill.block.shape == (2, 100, HEADS, DIM)
    key_copy, value_copy = key.clone(), value.clone()
    key.zero_()  # the caller may reuse its tensors right away
    torch.cuda.synchronize()
    k, v = spill.views()
    assert torch.equal(k, key_copy.cpu()) and torch.equal(v, value_copy.cpu())
    again = offload.store(value_copy[:60], key_copy[:60], spill)
    torch.cuda.synchronize()
    assert again is spill and spill.rows == 60 and torch.equal(spill.views()[0], value_copy[:60].cpu())
    longer = torch.cat([key_copy, key_copy])
    bigger = offload.store(longer, longer, spill)
    torch.cuda.synchronize()
    assert bigger is not spill and bigger.rows == 200 and torch.equal(bigger.views()[1], longer.cpu())


def test_recall_windows_returned_when_the_consumer_stops_early(device):
    offload = PrefillCPUOffload(32, 1, HEADS, DIM)
    key = torch.randn((100, HEADS, DIM), device=device).to(torch.bfloat16)
    spill = offload.store(key, key, None)
    slots = torch.arange(100, dtype=torch.int64, device=device)
    pieces = offload.chunks([spill.views(), (key, key)], slots)
    first, first_slots = next(pieces)
    assert first_slots.numel() == 32 and torch.equal(first[0][0], key[:32])
    pieces.close()
    assert sorted(offload.windows.free) == [0, 1]
