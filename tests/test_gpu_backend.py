"""The packed backend's per-call routing on the GPU (residualquant_amd/backend.py;
the reference's PackedImpl.forward and _store_kv,
src/residual_quantization/packed_backend.py:28-137).

A loop group of 4 records runs two batches through ``backend.forward``, one
call per loop: first two full prompts, then a mixed batch (one decode token
for each of those requests, followed by a new prompt).  Every output slice
must equal the op the reference routes it to, called directly on the same
inputs (prompts: causal varlen attention over raw K/V; decode: packed
attention over the cache with the current token live), and after each
group's last loop the cache must hold the bytes of one quantize of all
records."""

from __future__ import annotations

import pytest
import torch

import residualquant_amd as rq
from residualquant_amd import backend, workloads

pytestmark = pytest.mark.gpu

RECORDS = ((2, 32), (2, 32), (2, 32), (4, 32))
CONFIG = {"reference_mode": "anchor", "anchor_index": 3, "coefficient_method": "ls"}
HEADS, DIM, PT, PAGES = 4, 128, 16, 3


def _slots(table, spans):
    table = table.cpu().long()
    out = []
    for request, (begin, end) in spans:
        pos = torch.arange(begin, end, dtype=torch.int64)
        out.append(table[request, pos // PT] * PT + pos % PT)
    return torch.cat(out)


def _run_batch(layer_state, cache, meta, queries, pairs):
    outputs = []
    for loop in range(len(RECORDS)):
        layer_state.loop_index = loop
        key, value = pairs[loop]
        out = torch.empty_like(queries[loop])
        assert backend.forward(layer_state, queries[loop], key, value, cache, meta, out) is out
        outputs.append(out)
    return outputs


def test_forward_routes_prompts_and_decode_like_the_reference(device):
    table = workloads.block_tables(3, PAGES, 31, device=device)
    kr = workloads.random_sign_rotation(HEADS, DIM, 32, device=device)
    vr = workloads.random_sign_rotation(HEADS, DIM, 33, device=device)
    mean = torch.randn((len(RECORDS), HEADS, DIM), generator=torch.Generator().manual_seed(34)).to(device)
    shape = backend.kv_cache_shape(table.numel(), PT, HEADS, rq.page_width(DIM, RECORDS))
    cache = torch.zeros(shape, dtype=torch.uint8, device=device)
    group = rq.DeferredKVGroup(CONFIG, RECORDS, PT)
    layer_state = backend.PackedLayer(group=group, loop_index=0, key_rotation=kr, value_rotation=vr,
                                      key_mean=mean)
    generator = torch.Generator(device=device).manual_seed(35)
    scale = DIM ** -0.5

    def queries(tokens):
        return [torch.randn((tokens, HEADS, DIM), generator=generator, device=device).to(torch.bfloat16)
                for _ in RECORDS]

    # Batch 1: two full prompts of 20 and 37 tokens.
    slots_a = _slots(table, [(0, (0, 20)), (1, (0, 37))]).to(device)
    meta_a = backend.build_metadata(torch.tensor([0, 20, 57], dtype=torch.int32),
                                    torch.tensor([20, 37], dtype=torch.int32), table[:2], slots_a)
    q_a = queries(57)
    kv_a = workloads.loop_kv(57, HEADS, DIM, len(RECORDS), 36, device=device, anchor_index=3)
    out_a = _run_batch(layer_state, cache, meta_a, q_a, kv_a)
    cu = torch.tensor([0, 20, 57], dtype=torch.int32, device=device)
    for loop in range(len(RECORDS)):
        k, v = kv_a[loop]
        expected = rq.flash_attn_varlen_func(q_a[loop], k, v, 37, cu, 37, softmax_scale=scale, causal=True)
        assert torch.equal(out_a[loop], expected), f"prompt output, loop {loop}"
    expected_cache = torch.zeros_like(cache)
    rq.quantize(kv_a, expected_cache, slots_a, kr, vr, mean, RECORDS, "anchor", 3, "ls")
    assert torch.equal(cache, expected_cache), "cache after the prompts"

    # Batch 2: one decode token for each request, then a 9-token prompt.
    slots_b = _slots(table, [(0, (20, 21)), (1, (37, 38)), (2, (0, 9))]).to(device)
    meta_b = backend.build_metadata(torch.tensor([0, 1, 2, 11], dtype=torch.int32),
                                    torch.tensor([21, 38, 9], dtype=torch.int32), table, slots_b)
    q_b = queries(11)
    kv_b = workloads.loop_kv(11, HEADS, DIM, len(RECORDS), 37, device=device, anchor_index=3)
    cache_before = cache.clone()
    out_b = _run_batch(layer_state, cache, meta_b, q_b, kv_b)
    qsl = torch.tensor([0, 1, 2], dtype=torch.int32, device=device)
    seq = torch.tensor([21, 38], dtype=torch.int32, device=device)
    cu9 = torch.tensor([0, 9], dtype=torch.int32, device=device)
    for loop in range(len(RECORDS)):
        k, v = kv_b[loop]
        decode = torch.empty_like(q_b[loop][:2])
        rq.attention(q_b[loop][:2], k[:2], v[:2], cache_before, decode, qsl, seq, table[:2], kr, vr, mean,
                     RECORDS, "anchor", 3, loop)
        assert torch.equal(out_b[loop][:2], decode), f"decode output, loop {loop}"
        prompt = rq.flash_attn_varlen_func(q_b[loop][2:], k[2:], v[2:], 9, cu9, 9, softmax_scale=scale,
                                           causal=True)
        assert torch.equal(out_b[loop][2:], prompt), f"prompt output, loop {loop}"
        assert bool(torch.isfinite(out_b[loop].float()).all())
    expected_cache = cache_before.clone()
    rq.quantize(kv_b, expected_cache, slots_b, kr, vr, mean, RECORDS, "anchor", 3, "ls")
    assert torch.equal(cache, expected_cache), "cache after the mixed batch"


@pytest.mark.parametrize("lookahead", [False, True], ids=["chunks", "lookahead"])
def test_forward_with_prefill_offload(device, lookahead):
    """Two layers' groups with the pinned-host prefill offload driven through
    ``backend.forward`` in model order (every layer of loop 0, then loop 1,
    ...): the forward prepares the lookahead before its attention calls, and
    the caches hold the bytes of one quantize of every record."""
    from residualquant_amd.prefill_offload import PrefillCPUOffload

    layers, lens = 2, [150, 90]
    tokens = sum(lens)
    offload = PrefillCPUOffload(64, len(RECORDS) - 1, HEADS, DIM)
    offload.lookahead_enabled = lookahead
    offload.reserve(tokens)
    table = workloads.block_tables(2, PAGES * 4, 51, device=device)
    slots = _slots(table, [(0, (0, lens[0])), (1, (0, lens[1]))]).to(device)
    meta = backend.build_metadata(torch.tensor([0, lens[0], tokens], dtype=torch.int32),
                                  torch.tensor(lens, dtype=torch.int32), table, slots)
    chain, states, caches, data = [], [], [], []
    for i in range(layers):
        group = rq.DeferredKVGroup(CONFIG, RECORDS, PT, prefill_offload=offload)
        if lookahead:
            group.offload_chain, group.offload_index = chain, i
            chain.append(group)
        kr = workloads.random_sign_rotation(HEADS, DIM, 60 + i, device=device)
        vr = workloads.random_sign_rotation(HEADS, DIM, 70 + i, device=device)
        states.append(backend.PackedLayer(group=group, loop_index=0, key_rotation=kr, value_rotation=vr))
        shape = backend.kv_cache_shape(table.numel(), PT, HEADS, rq.page_width(DIM, RECORDS))
        caches.append(torch.zeros(shape, dtype=torch.uint8, device=device))
        data.append(workloads.loop_kv(tokens, HEADS, DIM, len(RECORDS), 80 + i, device=device, anchor_index=3))
    generator = torch.Generator(device=device).manual_seed(90)
    cu = torch.tensor([0, lens[0], tokens], dtype=torch.int32, device=device)
    for loop in range(len(RECORDS)):
        for i in range(layers):
            print(f"offload forward lookahead={lookahead} loop {loop} layer {i}", flush=True)
            states[i].loop_index = loop
            key, value = data[i][loop]
            q = torch.randn((tokens, HEADS, DIM), generator=generator, device=device).to(torch.bfloat16)
            out = torch.empty_like(q)
            backend.forward(states[i], q, key.clone(), value.clone(), caches[i], meta, out)
            expected = rq.flash_attn_varlen_func(q, key, value, max(lens), cu, max(lens),
                                                 softmax_scale=DIM ** -0.5, causal=True)
            assert torch.equal(out, expected)
    for i in range(layers):
        direct = torch.zeros_like(caches[i])
        rq.quantize(data[i], direct, slots, states[i].key_rotation, states[i].value_rotation, None, RECORDS,
                    "anchor", 3, "ls")
        assert torch.equal(caches[i], direct), i
    if lookahead:
        assert offload.prefetched == {}
