"""Pins of the oracle's decode attention (CPU).

- An independent numpy decoding of the page bytes (np.unpackbits codes,
  torch FP8 scales) rebuilt into keys as the reference decode kernel scores
  them (compute.cuh:397-505: alpha_L * (c.s+o + bf16(mu_A))_A + (c.s+o)_L,
  shift-invariant mean of the current loop) and values as its BF16 restore
  (compute.cuh:28-107), then a textbook float64 softmax.  Adjacent mode is
  pinned the same way in test_oracle_restore_pins.py.
- Closed forms: no history -> the live value exactly (merge.cuh:19-83);
  q = 0 -> uniform weights over history and live token.
- Moving a request's pages to other block ids (and the table with them)
  leaves the output unchanged.
"""

from __future__ import annotations

import numpy as np
import torch

from residualquant_amd import workloads
from residualquant_amd.layout import record_offsets

from .cases import OURO_G16, OURO_G32, make_decode, oracle_attention
from .test_oracle_restore_pins import rne_bf16


def _fp8(b):
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint8)).view(torch.float8_e4m3fn).double().numpy()


def _bf(x):
    return rne_bf16(x)


def _record(cache, plane, block, head, token, r, records, dim, pt):
    bits, group = records[r]
    cb, groups = dim * bits // 8, dim // group
    region = cache[plane, block, head].reshape(-1)[record_offsets(dim, records, pt)[r]:]
    codes = np.unpackbits(region[cb * token: cb * token + cb], bitorder="little").reshape(-1, bits) @ (1 << np.arange(bits))
    scale = np.repeat(_fp8(region[pt * cb + groups * token: pt * cb + groups * token + groups]), group)
    offset = np.repeat(_fp8(region[pt * (cb + groups) + groups * token: pt * (cb + groups) + groups * token + groups]), group)
    a = region[pt * (cb + 2 * groups) + 2 * token: pt * (cb + 2 * groups) + 2 * token + 2]
    alpha = torch.tensor([int(a[0]) | (int(a[1]) << 8)], dtype=torch.int32).to(torch.int16).view(torch.bfloat16).item()
    return codes * scale + offset, alpha


def _independent(d, cache, loop):
    g = d.group
    dim, pt, anchor, records = g.dim, g.page_tokens, g.anchor, g.records
    rk = g.key_rotation.double().numpy() if g.key_rotation is not None else None
    rv = g.value_rotation.double().numpy() if g.value_rotation is not None else None
    mu = g.key_mean.double().numpy() if g.key_mean is not None else None
    qsl, sl, table = d.query_start_loc.numpy(), d.seq_lens.numpy(), d.table.numpy()
    out = np.zeros(d.query.shape)
    for b in range(len(sl)):
        history = max(0, int(sl[b]) - 1)
        for i in range(qsl[b], qsl[b + 1]):
            for h in range(g.heads):
                q = d.query[i, h].double().numpy()
                qr = (q @ rk[h] if rk is not None else q) / np.sqrt(dim)
                keys, values = [], []
                for t in range(history):
                    block, token = table[b, t // pt], t % pt
                    ka, _ = _record(cache, 0, block, h, token, anchor, records, dim, pt)
                    va, _ = _record(cache, 1, block, h, token, anchor, records, dim, pt)
                    if loop == anchor:
                        keys.append(ka + (mu[anchor, h] if mu is not None else 0))
                        values.append(_bf(va))
                    else:
                        kl, alpha_k = _record(cache, 0, block, h, token, loop, records, dim, pt)
                        vl, alpha_v = _record(cache, 1, block, h, token, loop, records, dim, pt)
                        mean_a = _bf(mu[anchor, h]) if mu is not None else 0
                        keys.append(alpha_k * (ka + mean_a) + kl + (mu[loop, h] if mu is not None else 0))
                        values.append(_bf(alpha_v * _bf(va) + _bf(vl)))
                scores = np.array([qr @ k for k in keys] + [q @ d.key[i, h].double().numpy() / np.sqrt(dim)])
                p = np.exp(scores - scores.max())
                p /= p.sum()
                hist = (p[:-1, None] * np.array(values)).sum(0) if history else np.zeros(dim)
                if rv is not None:
                    hist = rv[h] @ hist
                out[i, h] = hist + p[-1] * d.value[i, h].double().numpy()
    return out


def test_attention_matches_independent_decoding(oracle):
    for lengths, dim, records, pt, mean in (([23, 1, 40], 128, OURO_G32, 16, True),
                                             ([35, 12], 96, OURO_G16, 32, False)):
        d = make_decode(lengths, 2, dim, records, seed=sum(lengths), page_tokens=pt, mean=mean)
        cache = d.group.oracle_cache(oracle)
        for loop in (0, 3):
            got = oracle_attention(oracle, d, cache, loop)
            assert np.abs(got - _independent(d, cache, loop)).max() < 1e-9


def test_no_history_gives_live_value(oracle):
    d = make_decode([1, 1], 3, 128, OURO_G32, seed=4)
    cache = d.group.oracle_cache(oracle)
    for loop in range(4):
        out = oracle_attention(oracle, d, cache, loop)
        assert np.array_equal(out, d.value.double().numpy())


def test_zero_query_averages_history_and_live(oracle):
    d = make_decode([30, 9], 2, 128, OURO_G32, seed=6)
    d.query = torch.zeros_like(d.query)
    g = d.group
    cache = g.oracle_cache(oracle)
    loop = 1
    out = oracle_attention(oracle, d, cache, loop)
    histories = [29, 8]
    slots = workloads.history_slots(d.table, histories, 16).numpy()
    _, v = oracle.dequantize(cache, slots, 128, g.key_mean.numpy(), g.records, "anchor", 3, loop)
    v = torch.from_numpy(v.view(np.int16)).view(torch.bfloat16).double().numpy()
    start = 0
    for b, history in enumerate(histories):
        for h in range(2):
            hist = g.value_rotation[h].double().numpy() @ v[start:start + history, h].sum(0)
            expected = (hist + d.value[b, h].double().numpy()) / (history + 1)
            assert np.abs(out[b, h] - expected).max() < 1e-12
        start += history


def test_block_table_relocation_invariance(oracle):
    d = make_decode([70, 33], 2, 128, OURO_G32, seed=8, extra_pages=3)
    cache = d.group.oracle_cache(oracle)
    before = oracle_attention(oracle, d, cache, 2)
    perm = np.random.default_rng(1).permutation(cache.shape[1])
    moved = np.zeros_like(cache)
    moved[:, perm] = cache  # block b now lives at perm[b]
    d.table = torch.from_numpy(perm[d.table.numpy()].astype(np.int32))
    after = oracle_attention(oracle, d, moved, 2)
    assert np.array_equal(before, after)
