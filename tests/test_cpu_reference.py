"""The vectorised torch-CPU restatement used as the benchmark's CPU baseline
(oracle/cpu_reference.py) against the C oracle: restored values bit for
bit, attention within 1e-9, for every loop, with and without key means."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cpu_reference
from residualquant_amd import workloads

from .cases import OURO_G16, OURO_G32, make_decode, oracle_attention
from .test_oracle_restore_pins import bf16_bits_of


@pytest.mark.parametrize("records,dim,pt,mean", [(OURO_G32, 128, 16, False), (OURO_G16, 96, 32, True)])
def test_cpu_reference_matches_oracle(oracle, records, dim, pt, mean):
    d = make_decode([40, 1, 70], 3, dim, records, seed=dim + pt, page_tokens=pt, mean=mean)
    g = d.group
    cache = g.oracle_cache(oracle)
    cache_t = torch.from_numpy(cache)
    for loop in range(4):
        got = cpu_reference.attention(d.query, d.key, d.value, cache_t, d.query_start_loc.numpy(),
                                      d.seq_lens.numpy(), d.table.numpy(), g.key_rotation, g.value_rotation,
                                      g.key_mean, records, g.anchor, loop).numpy()
        assert np.abs(got - oracle_attention(oracle, d, cache, loop)).max() < 1e-9, loop


def test_cpu_reference_values_bit_exact(oracle):
    d = make_decode([50], 2, 128, OURO_G32, seed=5)
    g = d.group
    cache = g.oracle_cache(oracle)
    history = 49
    slots = workloads.history_slots(d.table, [history], 16).numpy()
    blocks = torch.as_tensor(d.table.numpy()[0][:4], dtype=torch.long)
    for loop in range(4):
        _, want_v = oracle.dequantize(cache, slots, 128, g.key_mean.numpy(), g.records, "anchor", 3, loop)
        _, values = cpu_reference.request_keys_values(torch.from_numpy(cache), blocks, history, 128, g.records, 3,
                                                      loop, g.key_mean)
        assert np.array_equal(bf16_bits_of(values.permute(1, 0, 2).numpy()), want_v), loop
