"""Independent pins of the oracle's restore chain (anchor and adjacent mode)
and of its BF16 paged-attention baseline (CPU).

The restore chain is restated here from the reference kernels in exact
float64 arithmetic with an explicit round-to-nearest-even to BF16 after
every BF16 operation, written without the oracle's TwoSum code:

- quantizer reference, quantize/kernel.cuh:160-203: X_r = bf16(code*s + o),
  K plane: X_r = bf16(X_r + bf16(mu_r)), then for every record after the
  first of the chain X_r = bf16(X_prev * alpha_r + X_r);
- adjacent attention keys, attention/compute.cuh:120-197: the same chain
  over records 0..L, without the current loop's mean (compute.cuh:116-117).

A swapped mean/fma order, alpha taken from the wrong record, a double
rounding or a chain that skips a record changes the bits and fails here.

The BF16 baseline is pinned against torch's float64
scaled_dot_product_attention on the gathered pages plus the live token, and
by two closed forms (no history -> v_live exactly; q = 0 -> the mean of
history and live values).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from residualquant_amd import workloads
from residualquant_amd.layout import record_offsets

from .cases import OURO_G16, OURO_G32, make_decode, make_group, oracle_attention

ADJACENT_G32 = ((4, 32), (2, 32), (2, 32), (2, 32))
ADJACENT_MIXED = ((4, 16), (2, 16), (2, 32), (4, 32))


def rne_bf16(x) -> np.ndarray:
    """Round exact float64 values to the nearest BF16 (ties to even), as float64."""
    x = np.asarray(x, dtype=np.float64)
    _, e = np.frexp(x)                      # x = m * 2**e, 0.5 <= |m| < 1
    e = np.maximum(e, -125)                 # BF16 subnormals: quantum 2**-133
    quantum = np.ldexp(1.0, e - 8)          # 8 significant bits
    return np.rint(x / quantum) * quantum   # np.rint rounds half to even


def bf16_bits_of(x: np.ndarray) -> np.ndarray:
    """Bits of float64 values that are exactly BF16 numbers."""
    f = np.asarray(x, dtype=np.float32)
    assert np.array_equal(f.astype(np.float64), np.asarray(x)), "value is not a BF16 number"
    return (f.view(np.uint32) >> 16).astype(np.uint16)


def test_rne_bf16_against_exact_cases():
    one = 1.0
    ulp = 2.0 ** -7
    # halfway between 1 and 1 + ulp rounds to the even one; just above rounds up
    assert rne_bf16(one + ulp / 2) == one
    assert rne_bf16(one + ulp / 2 + 2.0 ** -40) == one + ulp
    assert rne_bf16(one + 3 * ulp / 2) == one + 2 * ulp
    # the double-rounding trap: 1 + ulp/2 + 2**-30 must round up; a float32 detour loses it
    x = one + ulp / 2 + 2.0 ** -30
    assert rne_bf16(x) == one + ulp
    assert float(torch.tensor(np.float32(x)).to(torch.bfloat16)) == one
    # agreement with torch's RNE on float32 inputs (single rounding there)
    values = np.random.default_rng(0).standard_normal(20000).astype(np.float32) * 8
    torch_bits = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf16_bits_of(rne_bf16(values.astype(np.float64))), torch_bits)
    # subnormal range keeps the 2**-133 quantum
    assert rne_bf16(2.0 ** -134 * 3) == 2.0 ** -132
    assert rne_bf16(-0.0) == 0.0 and np.signbit(rne_bf16(-0.0))


def _fp8(b) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint8)).view(torch.float8_e4m3fn).double().numpy()


def _record_fields(page: np.ndarray, token: int, r: int, records, dim: int, pt: int):
    """Codes, per-channel FP8 scale and offset, and alpha of record r for one token."""
    bits, group = records[r]
    cb, groups = dim * bits // 8, dim // group
    region = page.reshape(-1)[record_offsets(dim, records, pt)[r]:]
    raw = region[cb * token: cb * (token + 1)]
    codes = np.unpackbits(raw, bitorder="little").reshape(dim, bits) @ (1 << np.arange(bits))
    scale = np.repeat(_fp8(region[pt * cb + groups * token: pt * cb + groups * (token + 1)]), group)
    base = pt * (cb + groups) + groups * token
    offset = np.repeat(_fp8(region[base: base + groups]), group)
    a = region[pt * (cb + 2 * groups) + 2 * token: pt * (cb + 2 * groups) + 2 * token + 2]
    alpha = np.array([int(a[0]) | (int(a[1]) << 8)], dtype=np.uint16).astype(np.uint32) << 16
    return codes.astype(np.float64), scale, offset, float(alpha.view(np.float32)[0])


def restore_chain(page, token, chain, records, dim, pt, mean=None, skip_mean_of=None):
    """BF16 restore over the records of `chain` in order (float64 values)."""
    previous = None
    for i, r in enumerate(chain):
        codes, scale, offset, alpha = _record_fields(page, token, r, records, dim, pt)
        value = rne_bf16(codes * scale + offset)
        if mean is not None and r != skip_mean_of:
            value = rne_bf16(value + rne_bf16(mean[r].astype(np.float64)))
        if i > 0:
            value = rne_bf16(previous * alpha + value)
        previous = value
    return previous


def _chain(mode, anchor, loop):
    if mode == "adjacent":
        return list(range(loop + 1))
    return [anchor] if loop == anchor else [anchor, loop]


@pytest.mark.parametrize("mode,records,anchor,dim,pt,coefficient", [
    ("adjacent", ADJACENT_G32, 0, 128, 16, "ls"),
    ("adjacent", ADJACENT_MIXED, 0, 128, 32, "norm"),
    ("adjacent", ((4, 32), (2, 16), (2, 16)), 0, 96, 16, "ls"),
    ("anchor", OURO_G32, 3, 128, 16, "ls"),
    ("anchor", OURO_G16, 3, 96, 32, "unit"),
])
def test_dequantize_matches_restated_chain_bit_for_bit(oracle, mode, records, anchor, dim, pt, coefficient):
    g = make_group(40, 2, dim, records, seed=dim + pt + len(records), page_tokens=pt, mode=mode,
                   anchor=anchor, coefficient=coefficient)
    cache = g.oracle_cache(oracle)
    slots = g.slots.numpy()
    mean = g.key_mean.numpy()
    for loop in range(len(records)):
        k, v = oracle.dequantize(cache, slots, dim, mean, records, mode, anchor, loop)
        for n, slot in enumerate(slots):
            block, token = slot // pt, slot % pt
            for h in range(g.heads):
                chain = _chain(mode, anchor, loop)
                want_k = restore_chain(cache[0, block, h], token, chain, records, dim, pt, mean=mean[:, h])
                want_v = restore_chain(cache[1, block, h], token, chain, records, dim, pt)
                assert np.array_equal(k[n, h], bf16_bits_of(want_k)), (loop, n, h)
                assert np.array_equal(v[n, h], bf16_bits_of(want_v)), (loop, n, h)


def test_restated_chain_catches_plausible_mistakes(oracle):
    """The restatement is sharp: each plausible slip in the chain changes bits."""
    records, dim, pt = ADJACENT_G32, 128, 16
    g = make_group(24, 1, dim, records, seed=77, page_tokens=pt, mode="adjacent", anchor=0)
    cache = g.oracle_cache(oracle)
    slots = g.slots.numpy()
    mean = g.key_mean.numpy()
    k, _ = oracle.dequantize(cache, slots, dim, mean, records, "adjacent", 0, 3)

    def wrong(variant):
        differs = 0
        for n, slot in enumerate(slots):
            page, token = cache[0, slot // pt, 0], slot % pt
            previous = None
            for i, r in enumerate(range(4)):
                codes, scale, offset, alpha = _record_fields(page, token, r, records, dim, pt)
                value = rne_bf16(codes * scale + offset)
                if variant == "alpha_of_previous_record" and i > 0:
                    alpha = _record_fields(page, token, r - 1, records, dim, pt)[3] if r > 1 else 1.0
                if variant == "mean_after_link":
                    if i > 0:
                        value = rne_bf16(previous * alpha + value)
                    value = rne_bf16(value + rne_bf16(mean[r, 0].astype(np.float64)))
                else:
                    value = rne_bf16(value + rne_bf16(mean[r, 0].astype(np.float64)))
                    if i > 0:
                        value = rne_bf16(previous * alpha + value)
                previous = value
            differs += int(not np.array_equal(k[n, 0], bf16_bits_of(previous)))
        return differs

    assert wrong("alpha_of_previous_record") > 0
    assert wrong("mean_after_link") > 0


def _independent_adjacent(d, cache, loop):
    """Textbook float64 softmax over keys/values restored by restore_chain."""
    g = d.group
    dim, pt, records = g.dim, g.page_tokens, g.records
    rk = g.key_rotation.double().numpy() if g.key_rotation is not None else None
    rv = g.value_rotation.double().numpy() if g.value_rotation is not None else None
    mu = g.key_mean.numpy() if g.key_mean is not None else None
    qsl, sl, table = d.query_start_loc.numpy(), d.seq_lens.numpy(), d.table.numpy()
    out = np.zeros(d.query.shape)
    chain = list(range(loop + 1))
    for b in range(len(sl)):
        history = max(0, int(sl[b]) - 1)
        for i in range(qsl[b], qsl[b + 1]):
            for h in range(g.heads):
                q = d.query[i, h].double().numpy()
                qr = (q @ rk[h] if rk is not None else q) / np.sqrt(dim)
                keys, values = [], []
                for t in range(history):
                    block, token = table[b, t // pt], t % pt
                    key = restore_chain(cache[0, block, h], token, chain, records, dim, pt,
                                        mean=None if mu is None else mu[:, h], skip_mean_of=loop)
                    keys.append(key + (mu[loop, h].astype(np.float64) if mu is not None else 0))
                    values.append(restore_chain(cache[1, block, h], token, chain, records, dim, pt))
                scores = np.array([qr @ k for k in keys] + [q @ d.key[i, h].double().numpy() / np.sqrt(dim)])
                p = np.exp(scores - scores.max())
                p /= p.sum()
                hist = (p[:-1, None] * np.array(values)).sum(0) if history else np.zeros(dim)
                if rv is not None:
                    hist = rv[h] @ hist
                out[i, h] = hist + p[-1] * d.value[i, h].double().numpy()
    return out


@pytest.mark.parametrize("records,dim,pt,mean", [(ADJACENT_G32, 128, 16, True),
                                                 (((4, 32), (2, 16), (2, 16)), 96, 32, True),
                                                 (ADJACENT_MIXED, 128, 16, False)])
def test_adjacent_attention_matches_independent_decoding(oracle, records, dim, pt, mean):
    d = make_decode([21, 1, 38], 2, dim, records, seed=dim + pt, page_tokens=pt, mode="adjacent", anchor=0,
                    mean=mean)
    cache = d.group.oracle_cache(oracle)
    for loop in range(len(records)):
        got = oracle_attention(oracle, d, cache, loop)
        assert np.abs(got - _independent_adjacent(d, cache, loop)).max() < 1e-9, loop


# ------------------------------------------------------------- BF16 baseline


def _bf16_case(lengths, heads, dim, pt, seed):
    histories = [max(0, x - 1) for x in lengths]
    max_pages = max(1, max((h + pt - 1) // pt for h in histories)) + 1
    blocks = len(lengths) * max_pages
    g = torch.Generator().manual_seed(seed)
    cache = torch.randn((2, blocks, heads, pt, dim), generator=g).to(torch.bfloat16)
    table = workloads.block_tables(len(lengths), max_pages, seed + 1)
    rows = len(lengths)
    q, k, v = (torch.randn((rows, heads, dim), generator=g).to(torch.bfloat16) for _ in range(3))
    qsl = torch.arange(rows + 1, dtype=torch.int32)
    sl = torch.tensor(lengths, dtype=torch.int32)
    return cache, table, q, k, v, qsl, sl


def _bf16_oracle(oracle, cache, table, q, k, v, qsl, sl):
    bits = lambda t: workloads.bf16_bits(t)
    return oracle.paged_attention_bf16(bits(q), bits(k), bits(v), bits(cache), qsl.numpy(), sl.numpy(),
                                       table.numpy())


@pytest.mark.parametrize("lengths,heads,dim,pt", [([37, 1, 70], 3, 128, 16), ([50, 9], 2, 96, 32)])
def test_paged_attention_bf16_matches_torch_sdpa(oracle, lengths, heads, dim, pt):
    cache, table, q, k, v, qsl, sl = _bf16_case(lengths, heads, dim, pt, seed=sum(lengths))
    got = _bf16_oracle(oracle, cache, table, q, k, v, qsl, sl)
    c = cache.double()
    for b, length in enumerate(lengths):
        history = length - 1
        t = torch.arange(history)
        blocks = table[b, t // pt].long()
        keys = torch.cat([c[0, blocks, :, t % pt], k[b:b + 1].double()], 0)      # [T+1, H, D]
        values = torch.cat([c[1, blocks, :, t % pt], v[b:b + 1].double()], 0)
        expected = F.scaled_dot_product_attention(q[b].double()[:, None], keys.transpose(0, 1),
                                                  values.transpose(0, 1))[:, 0]
        assert np.abs(got[b] - expected.numpy()).max() < 1e-12


def test_paged_attention_bf16_closed_forms(oracle):
    # no history: the output is the live value exactly
    cache, table, q, k, v, qsl, sl = _bf16_case([1, 1, 1], 2, 128, 16, seed=3)
    got = _bf16_oracle(oracle, cache, table, q, k, v, qsl, sl)
    assert np.array_equal(got, v.double().numpy())
    # q = 0: uniform weights over history and the live token
    cache, table, q, k, v, qsl, sl = _bf16_case([33, 17], 2, 128, 16, seed=4)
    q = torch.zeros_like(q)
    got = _bf16_oracle(oracle, cache, table, q, k, v, qsl, sl)
    c = cache.double()
    for b, length in enumerate([33, 17]):
        t = torch.arange(length - 1)
        blocks = table[b, t // 16].long()
        total = c[1, blocks, :, t % 16].sum(0) + v[b].double()
        assert np.abs(got[b] - (total / length).numpy()).max() < 1e-12
