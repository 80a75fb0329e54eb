"""The packed backend's per-call routing on the GPU (residualquant_amd/backend.py;
the reference's PackedImpl.forward and _store_kv,
src/residual_quantization/packed_backend.py:28-137).

A loop group of 4 records runs two batches through ``backend.forward``, one
call per loop: first two full prompts, then a mixed batch (one decode token
for each of those requests, followed by a new prompt).

- After each group's last loop the cache must hold the CPU oracle's bytes
  for one quantize of every record of the batch's tokens (bit-exact).
- Prompt slices must match the oracle's float64 causal varlen attention over
  the raw K/V, and decode slices the oracle's packed attention over the cache
  as it was before the batch (2e-2 max-abs / 1e-3 mean-abs on BF16 outputs).
- Every slice must also be bit-equal to the op the reference routes it to,
  called directly on the same inputs (the routing adds no arithmetic)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import residualquant_amd as rq
from residualquant_amd import backend, workloads

pytestmark = pytest.mark.gpu

RECORDS = ((2, 32), (2, 32), (2, 32), (4, 32))
CONFIG = {"reference_mode": "anchor", "anchor_index": 3, "coefficient_method": "ls"}
HEADS, DIM, PT, PAGES = 4, 128, 16, 3
MAX_ABS, MEAN_ABS = 2e-2, 1e-3
bits = workloads.bf16_bits


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


def _oracle_quantize(oracle, cache_np, pairs, slots, kr, vr, mean):
    """The oracle's quantize of ``pairs`` at ``slots`` into a copy of ``cache_np``."""
    expected = cache_np.copy()
    oracle.quantize([(bits(k), bits(v)) for k, v in pairs], expected, slots.cpu().numpy(),
                    None if kr is None else bits(kr), None if vr is None else bits(vr),
                    None if mean is None else mean.cpu().numpy(), RECORDS, "anchor", 3, "ls")
    return expected


def _close(got, expected, what):
    err = np.abs(got.float().cpu().numpy() - expected)
    print(f"  {what}: max {err.max():.2e} mean {err.mean():.2e}", flush=True)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (what, err.max(), err.mean())


def _oracle_prompt(oracle, q, k, v, cu):
    cu = cu.cpu().numpy()
    return oracle.prefill_attention(bits(q), bits(k), bits(v), cu, cu, DIM ** -0.5, causal=True)


def test_forward_routes_prompts_and_decode_like_the_reference(oracle, device):
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
    print("[case] backend batch 1: prompts of 20 and 37 tokens", flush=True)
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
        _close(out_a[loop], _oracle_prompt(oracle, q_a[loop], k, v, cu), f"prompt loop {loop}")
    oracle_cache = _oracle_quantize(oracle, np.zeros(shape, dtype=np.uint8), kv_a, slots_a, kr, vr, mean)
    assert np.array_equal(cache.cpu().numpy(), oracle_cache), "cache after the prompts"

    # Batch 2: one decode token for each request, then a 9-token prompt.
    print("[case] backend batch 2: two decode rows and a 9-token prompt", flush=True)
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
        expected = oracle.attention(bits(q_b[loop][:2]), bits(k[:2]), bits(v[:2]), oracle_cache, qsl.cpu().numpy(),
                                    seq.cpu().numpy(), table[:2].cpu().numpy(), bits(kr), bits(vr),
                                    mean.cpu().numpy(), RECORDS, "anchor", 3, loop)
        _close(out_b[loop][:2], expected, f"decode loop {loop}")
        prompt = rq.flash_attn_varlen_func(q_b[loop][2:], k[2:], v[2:], 9, cu9, 9, softmax_scale=scale,
                                           causal=True)
        assert torch.equal(out_b[loop][2:], prompt), f"prompt output, loop {loop}"
        _close(out_b[loop][2:], _oracle_prompt(oracle, q_b[loop][2:], k[2:], v[2:], cu9), f"prompt loop {loop}")
    oracle_cache = _oracle_quantize(oracle, oracle_cache, kv_b, slots_b, kr, vr, mean)
    assert np.array_equal(cache.cpu().numpy(), oracle_cache), "cache after the mixed batch"


@pytest.mark.parametrize("lookahead", [False, True], ids=["chunks", "lookahead"])
def test_forward_with_prefill_offload(oracle, device, lookahead):
    """Two layers' groups with the pinned-host prefill offload driven through
    ``backend.forward`` in model order (every layer of loop 0, then loop 1,
    ...): the forward prepares the lookahead before its attention calls, the
    prompt outputs match the oracle's causal attention, and the caches hold
    the oracle's bytes for one quantize of every record."""
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
            print(f"[case] offload forward lookahead={lookahead} loop {loop} layer {i}", flush=True)
            states[i].loop_index = loop
            key, value = data[i][loop]
            q = torch.randn((tokens, HEADS, DIM), generator=generator, device=device).to(torch.bfloat16)
            out = torch.empty_like(q)
            backend.forward(states[i], q, key.clone(), value.clone(), caches[i], meta, out)
            expected = rq.flash_attn_varlen_func(q, key, value, max(lens), cu, max(lens),
                                                 softmax_scale=DIM ** -0.5, causal=True)
            assert torch.equal(out, expected)
            if loop in (0, len(RECORDS) - 1):
                _close(out, _oracle_prompt(oracle, q, key, value, cu), f"prompt loop {loop} layer {i}")
    for i in range(layers):
        expected = _oracle_quantize(oracle, np.zeros(caches[i].shape, dtype=np.uint8), data[i], slots,
                                    states[i].key_rotation, states[i].value_rotation, None)
        assert np.array_equal(caches[i].cpu().numpy(), expected), i
    if lookahead:
        assert offload.prefetched == {}
