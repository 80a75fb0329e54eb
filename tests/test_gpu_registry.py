"""Every packed signature the reference compiles
(residualquant_amd/registry.py, after csrc/dispatch/decode_*.cu and
dispatch/schedules.cuh:9-77), swept on the GPU with rotations on and off and
every coefficient method: quantize of two tokens is bit-exact against the
oracle, and attention with no history returns the live value exactly at
every loop (the reference's start-up warm-up, install_cache.py:187-256,
makes the same calls with zero inputs)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import residualquant_amd as rq
from residualquant_amd import registry

from .cases import make_group

pytestmark = pytest.mark.gpu

COEFFICIENTS = ("unit", "norm", "ls")


def _sweep(oracle, device, signature, rotation, coefficient, seed):
    s = signature
    g = make_group(2, s.heads, s.head_dim, s.records, seed=seed, page_tokens=s.page_tokens, mode=s.reference_mode,
                   anchor=s.anchor_index, coefficient=coefficient, rotation=rotation, mean=s.has_mean,
                   spare_blocks=0)
    expected = g.oracle_cache(oracle)
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    rq.quantize([(k.to(device), v.to(device)) for k, v in g.pairs], cache, g.slots.to(device), kr, vr, km,
                g.records, g.mode, g.anchor, g.coefficient)
    assert np.array_equal(cache.cpu().numpy(), expected), "quantize bytes"
    generator = torch.Generator(device=device).manual_seed(seed)
    q, k, v = (torch.randn((2, s.heads, s.head_dim), generator=generator, device=device).to(torch.bfloat16)
               for _ in range(3))
    starts = torch.tensor([0, 1, 2], dtype=torch.int32, device=device)
    lengths = torch.ones(2, dtype=torch.int32, device=device)
    table = torch.zeros((2, 1), dtype=torch.int32, device=device)
    for loop in range(len(s.records)):
        out = torch.full_like(q, float("nan"))
        rq.attention(q, k, v, cache, out, starts, lengths, table, kr, vr, km, g.records, g.mode, g.anchor, loop)
        assert torch.equal(out.view(torch.int16), v.view(torch.int16)), f"loop {loop}"


@pytest.mark.parametrize("geometry", [(16, 128), (55, 96)], ids=["ouro", "huginn"])
def test_every_registered_signature(oracle, device, geometry):
    cases = [s for s in registry.REFERENCE_SIGNATURES if (s.heads, s.head_dim) == geometry]
    for n, signature in enumerate(cases):
        print(f"[case] signature {n} {signature}", flush=True)
        for rotation in (False, True):
            for coefficient in COEFFICIENTS:
                _sweep(oracle, device, signature, rotation, coefficient, seed=1000 + n)


def test_warmup_runs_each_distinct_signature_once(device):
    layers = []
    for s in registry.REFERENCE_SIGNATURES[:6]:
        mean = torch.zeros((len(s.records), s.heads, s.head_dim), device=device) if s.has_mean else None
        for _ in range(2):  # duplicates are skipped
            layers.append(registry.WarmupLayer(s.heads, s.head_dim, s.records, s.page_tokens, s.reference_mode,
                                               s.anchor_index, "ls", key_mean=mean))
    assert registry.warmup(layers, device) == 6
