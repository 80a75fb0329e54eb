"""HIP kernels at the benchmark configurations' full sizes, checked through
properties that hold at any size.

- Quantize (4096 tokens x 16 heads x D128 x 4 loops, the quantize benchmark
  shape): a token's packed bytes depend only on that token's K/V, so the
  bytes of a random sample of tokens from the full GPU call must equal the
  oracle's bytes for those tokens alone.
- Decode (B32 x 8192 history x 16 heads x D128, and B8 x 4096 x 55 heads x
  D96): a row's output depends only on its own pages, so sampled rows of the
  full GPU call must match the FP64 oracle run on those rows' pages alone
  (BF16 output: 2e-2 max-abs, 1e-3 mean-abs).

The caches are built by the GPU quantize (bit-exact against the oracle in
test_gpu_parity.py), as the benchmark builds them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import residualquant_amd as rq
from residualquant_amd import workloads

from .cases import OURO_G16, OURO_G32, make_group

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 1e-3
QUANTIZE_SCHEDULE = ((2, 16), (2, 16), (2, 32), (4, 32))


def test_quantize_full_size_sampled_tokens(oracle, device):
    print("[case] quantize 4096 tokens x 16 heads x D128, 48 sampled tokens", flush=True)
    g = make_group(4096, 16, 128, QUANTIZE_SCHEDULE, seed=4242, anchor=3, coefficient="ls", skipped=5)
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    rq.quantize([(k.to(device), v.to(device)) for k, v in g.pairs], cache, g.slots.to(device), kr, vr, km,
                g.records, g.mode, g.anchor, g.coefficient)
    gpu = cache.cpu().numpy()

    live = torch.nonzero(g.slots >= 0).flatten()
    pick = live[torch.randperm(live.numel(), generator=torch.Generator().manual_seed(7))[:48]]
    sample = make_group(1, 16, 128, QUANTIZE_SCHEDULE, seed=1, anchor=3)  # shape holder
    sample.pairs = [(k[pick], v[pick]) for k, v in g.pairs]
    sample.slots = g.slots[pick]
    sample.key_rotation, sample.value_rotation, sample.key_mean = g.key_rotation, g.value_rotation, g.key_mean
    sample.num_blocks = g.num_blocks
    # The oracle rewrites the sampled tokens' bytes in a copy of the GPU
    # cache (a page interleaves its tokens' codes and parameters, so the
    # copy keeps every other token's bytes in place): equal bytes leave the
    # copy unchanged.
    expected = sample.oracle_cache(oracle, cache=gpu.copy())
    assert np.array_equal(gpu, expected)
    # The same rewrite from zeros changes the sampled pages (the check has teeth).
    assert sample.oracle_cache(oracle).any()


def _decode_full_size(oracle, device, batch, history, heads, dim, records, rows, loops, seed):
    page_tokens = 16
    pages = history // page_tokens
    table = workloads.block_tables(batch, pages, seed, device=device)
    width = rq.page_width(dim, records)
    cache = torch.zeros((2, batch * pages, heads, page_tokens, width), dtype=torch.uint8, device=device)
    kr = workloads.random_sign_rotation(heads, dim, seed + 1, device=device)
    vr = workloads.random_sign_rotation(heads, dim, seed + 2, device=device)
    km = workloads.key_means(len(records), heads, dim, seed + 3, device=device)
    slots = workloads.history_slots(table, [history] * batch, page_tokens)
    for start in range(0, slots.numel(), 16384):
        part = slots[start:start + 16384]
        pairs = workloads.loop_kv(part.numel(), heads, dim, len(records), seed + start, device=device,
                                  anchor_index=3)
        rq.quantize(pairs, cache, part.to(device), kr, vr, km, records, "anchor", 3, "ls")
        del pairs
    generator = torch.Generator().manual_seed(seed + 4)
    q, k, v = (torch.randn((batch, heads, dim), generator=generator).to(torch.bfloat16) for _ in range(3))
    qsl = torch.arange(batch + 1, dtype=torch.int32)
    seq = torch.full((batch,), history + 1, dtype=torch.int32)

    # The sampled rows' pages alone, renumbered 0..len(rows) * pages - 1.
    rows = list(rows)
    blocks = table[rows].flatten().long()
    sub_cache = cache[:, blocks].cpu().numpy()
    sub_table = np.arange(len(rows) * pages, dtype=np.int32).reshape(len(rows), pages)
    sub_qsl = np.arange(len(rows) + 1, dtype=np.int32)
    sub_seq = np.full(len(rows), history + 1, dtype=np.int32)
    bits = workloads.bf16_bits
    for loop in loops:
        out = torch.empty((batch, heads, dim), dtype=torch.bfloat16, device=device)
        rq.attention(q.to(device), k.to(device), v.to(device), cache, out, qsl.to(device), seq.to(device), table,
                     kr, vr, km, records, "anchor", 3, loop)
        got = out.float().cpu().numpy()[rows]
        expected = oracle.attention(bits(q[rows]), bits(k[rows]), bits(v[rows]), sub_cache, sub_qsl, sub_seq,
                                    sub_table, bits(kr), bits(vr), km.cpu().numpy(), records, "anchor", 3, loop)
        err = np.abs(got - expected)
        print(f"  loop {loop}: max {err.max():.2e} mean {err.mean():.2e}", flush=True)
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (loop, err.max(), err.mean())


def test_decode_full_size_ouro_sampled_rows(oracle, device):
    print("[case] decode B32 x 8192 x 16 heads x D128, rows 0, 19 and 31, every loop", flush=True)
    _decode_full_size(oracle, device, 32, 8192, 16, 128, OURO_G32, rows=(0, 19, 31), loops=(0, 1, 2, 3), seed=8100)


def test_decode_full_size_huginn_sampled_rows(oracle, device):
    print("[case] decode B8 x 4096 x 55 heads x D96, rows 0, 5 and 7, every loop", flush=True)
    _decode_full_size(oracle, device, 8, 4096, 55, 96, OURO_G16, rows=(0, 5, 7), loops=(0, 1, 2, 3), seed=8200)
