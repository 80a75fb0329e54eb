"""BASELINE configuration 0 on the GPU: one layer of an Ouro-1.4B-shaped
cache, 16 KV heads x D128, 4 loops, batch 1, 512 history tokens, page 16,
INT4 anchor g32 (loop 3) + INT2 residuals g32, LS coefficients, seeded
random-sign Hadamard rotations, anchor K/V ~ N(0, 1) with 4 K channels x8,
earlier loops = anchor + N(0, 0.15^2), one query token ~ N(0, 1) per head.

Quantize must be bit-exact against the oracle and every loop's attention
within 2e-2 max-abs / 1e-3 mean-abs of it."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import residualquant_amd as rq

from .cases import OURO_G32, make_decode, oracle_attention

pytestmark = pytest.mark.gpu


def test_c0_quantize_and_attention(oracle, device):
    print("[case] C0 H16 D128 B1 T512", flush=True)
    d = make_decode([513], 16, 128, OURO_G32, seed=2026, mean=False)
    g = d.group
    assert len(g.slots) == 512
    expected = g.oracle_cache(oracle)
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    rq.quantize([(k.to(device), v.to(device)) for k, v in g.pairs], cache, g.slots.to(device), kr, vr, km,
                g.records, g.mode, g.anchor, g.coefficient)
    got = cache.cpu().numpy()
    assert np.array_equal(got, expected), f"{int((got != expected).sum())} bytes differ"
    for loop in range(4):
        out = torch.zeros_like(d.query, device=device)
        rq.attention(d.query.to(device), d.key.to(device), d.value.to(device), cache, out,
                     d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device), kr, vr, km,
                     g.records, g.mode, g.anchor, loop)
        err = np.abs(out.float().cpu().numpy() - oracle_attention(oracle, d, expected, loop))
        print(f"[case] C0 loop {loop}: max {err.max():.3g} mean {err.mean():.3g}", flush=True)
        assert err.max() <= 2e-2 and err.mean() <= 1e-3, loop
