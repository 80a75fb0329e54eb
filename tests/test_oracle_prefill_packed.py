"""Pins of the oracle's attention of several new rows per request over the
packed history (oracle.attention_prefill, rq_oracle.c attention_rows with
causal = 1): the n rows of a request are its last n tokens, they see the
seq_len - n history tokens of the cache and, causally, the request's new
keys/values.  The reference has no such path (its scheduler forbids partial
prefill, rq/scheduler.py:11-18); the pins are:

- one row per request: identical to the decode oracle (oracle.attention);
- no history: identical to textbook causal prefill attention
  (oracle.prefill_attention, itself pinned against torch SDPA);
- any history: a float64 torch restatement (keys and values from
  oracle/cpu_reference.py, which is pinned against the decode oracle) with a
  textbook softmax over history + causal live set;
- q = 0: uniform weights over the visible history and new values.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import cpu_reference
from residualquant_amd import workloads

from .cases import OURO_G16, OURO_G32, make_decode


def _bits(t):
    return None if t is None else workloads.bf16_bits(t)


def _prefill(oracle, d, cache, loop):
    g = d.group
    return oracle.attention_prefill(
        _bits(d.query), _bits(d.key), _bits(d.value), cache, d.query_start_loc.numpy(), d.seq_lens.numpy(),
        d.table.numpy(), _bits(g.key_rotation), _bits(g.value_rotation),
        None if g.key_mean is None else g.key_mean.numpy(), g.records, g.mode, g.anchor, loop)


def _decode(oracle, d, cache, loop):
    g = d.group
    return oracle.attention(
        _bits(d.query), _bits(d.key), _bits(d.value), cache, d.query_start_loc.numpy(), d.seq_lens.numpy(),
        d.table.numpy(), _bits(g.key_rotation), _bits(g.value_rotation),
        None if g.key_mean is None else g.key_mean.numpy(), g.records, g.mode, g.anchor, loop)


def _textbook(d, cache, loop):
    g = d.group
    dim = g.dim
    qsl, sl, table = d.query_start_loc.numpy(), d.seq_lens.numpy(), d.table.numpy()
    out = np.zeros(d.query.shape)
    kr = g.key_rotation.double() if g.key_rotation is not None else None
    vr = g.value_rotation.double() if g.value_rotation is not None else None
    for b in range(len(sl)):
        first, n = int(qsl[b]), int(qsl[b + 1] - qsl[b])
        history = max(0, int(sl[b]) - n)
        pages = (history + g.page_tokens - 1) // g.page_tokens
        keys, values = cpu_reference.request_keys_values(torch.from_numpy(cache),
                                                         torch.as_tensor(table[b][:pages], dtype=torch.long),
                                                         history, dim, g.records, g.anchor, loop, g.key_mean)
        if vr is not None:
            values = torch.einsum("htd,hcd->htc", values, vr)  # back to the model's space
        for r in range(n):
            i = first + r
            q = d.query[i].double()
            rotated = (torch.einsum("hd,hde->he", q, kr) if kr is not None else q) / np.sqrt(dim)
            live_k = d.key[first:i + 1].double().transpose(0, 1)       # [heads, r + 1, D]
            live_v = d.value[first:i + 1].double().transpose(0, 1)
            scores = torch.cat([torch.einsum("he,hte->ht", rotated, keys),
                                torch.einsum("hd,htd->ht", q, live_k) / np.sqrt(dim)], -1)
            p = torch.softmax(scores, -1)
            out[i] = torch.einsum("ht,htd->hd", p, torch.cat([values, live_v], 1)).numpy()
    return out


def test_one_row_per_request_is_the_decode_oracle(oracle):
    d = make_decode([40, 1, 77], 3, 128, OURO_G32, seed=3)
    cache = d.group.oracle_cache(oracle)
    for loop in (0, 3):
        assert np.array_equal(_prefill(oracle, d, cache, loop), _decode(oracle, d, cache, loop))


def test_no_history_is_causal_prefill(oracle):
    rows = [5, 1, 9]
    d = make_decode(rows, 2, 128, OURO_G32, seed=4, rows_per_request=rows)
    cache = d.group.oracle_cache(oracle)
    cu = np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)
    want = oracle.prefill_attention(_bits(d.query), _bits(d.key), _bits(d.value), cu, cu, 1 / np.sqrt(128))
    for loop in (1, 3):
        assert np.abs(_prefill(oracle, d, cache, loop) - want).max() < 1e-12


def test_matches_textbook_softmax(oracle):
    for lengths, rows, dim, records, pt, mean in (([60, 9, 33], [4, 9, 1], 128, OURO_G32, 16, True),
                                                  ([45, 70], [6, 3], 96, OURO_G16, 32, False)):
        d = make_decode(lengths, 2, dim, records, seed=sum(lengths), page_tokens=pt, mean=mean,
                        rows_per_request=rows)
        cache = d.group.oracle_cache(oracle)
        for loop in range(4):
            got = _prefill(oracle, d, cache, loop)
            assert np.abs(got - _textbook(d, cache, loop)).max() < 1e-9, loop


def test_zero_query_averages_visible_history_and_new_values(oracle):
    lengths, rows = [30, 12], [3, 2]
    d = make_decode(lengths, 2, 128, OURO_G32, seed=9, rows_per_request=rows)
    d.query = torch.zeros_like(d.query)
    g = d.group
    cache = g.oracle_cache(oracle)
    loop = 2
    got = _prefill(oracle, d, cache, loop)
    first = 0
    for b, (length, n) in enumerate(zip(lengths, rows)):
        history = length - n
        slots = workloads.history_slots(d.table[b:b + 1], [history], 16).numpy()
        _, v = oracle.dequantize(cache, slots, 128, g.key_mean.numpy(), g.records, "anchor", 3, loop)
        v = torch.from_numpy(v.view(np.int16)).view(torch.bfloat16).double()
        for h in range(2):
            hist = g.value_rotation[h].double() @ v[:, h].sum(0)
            for r in range(n):
                live = d.value[first:first + r + 1, h].double().sum(0)
                expected = (hist + live) / (history + r + 1)
                assert np.abs(got[first + r, h] - expected.numpy()).max() < 1e-12
        first += n
