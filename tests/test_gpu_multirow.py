"""Several query rows per request over the packed history on the multi-row
MFMA kernels (residualquant_amd/csrc/multirow.hip) against the CPU oracle.

- ``packed_prefill_attention``: each request's rows are its last n tokens,
  seeing seq_len - n history tokens and, causally, the new ones
  (oracle.attention_prefill);
- ``attention`` with an average of 2 or more rows per request (3 in the
  anchor-only loop) routes to the same kernels with the reference's decode
  semantics (oracle.attention); fewer rows take the per-row decode kernel,
  checked against the same oracle.

Both head dims of the reference's attention registry (96 and 128) and both
reference modes: anchor mode (compute.cuh:397-505) and adjacent mode, whose
loops past 0 rebuild the BF16 restore chain (compute.cuh:120-197, :506-623).
Calls whose requests average 16 rows or fewer run on 16-row tiles
(v_mfma_f32_16x16x32), the others on 32-row tiles; the cases hold both.

Bar: within 2e-2 max-abs / 1e-3 mean-abs of the oracle, both in BF16 (the
oracle's FP64 output rounded to BF16: the BF16 quantum of outputs of
magnitude ~1 at short histories is half the mean bar by itself).
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

import residualquant_amd as rq
from residualquant_amd import workloads

from .cases import OURO_G16, OURO_G32, make_decode

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 1e-3


def _bits(t):
    return None if t is None else workloads.bf16_bits(t)


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).float().to(torch.bfloat16).double().numpy()


def _oracle(oracle, d, cache, loop, causal):
    g = d.group
    function = oracle.attention_prefill if causal else oracle.attention
    return function(_bits(d.query), _bits(d.key), _bits(d.value), cache, d.query_start_loc.numpy(),
                    d.seq_lens.numpy(), d.table.numpy(), _bits(g.key_rotation), _bits(g.value_rotation),
                    None if g.key_mean is None else g.key_mean.numpy(), g.records, g.mode, g.anchor, loop)


def _run(d, device, cache, loop, causal):
    g = d.group
    kr, vr, km = g.device_args(device)
    out = torch.full_like(d.query, float("nan"), device=device)
    function = rq.packed_prefill_attention if causal else rq.attention
    function(d.query.to(device), d.key.to(device), d.value.to(device), cache, out, d.query_start_loc.to(device),
             d.seq_lens.to(device), d.table.to(device), kr, vr, km, g.records, g.mode, g.anchor, loop)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


ADJACENT_G32 = ((4, 32), (2, 32), (2, 32), (2, 32))
ADJACENT_G16 = ((4, 32), (2, 16), (2, 16), (2, 16))

CASES = [
    # lengths (seq_len incl. the new rows), rows per request, heads, records, page tokens, mean, rotation,
    # head dim, mode
    ([100, 37, 9], [4, 1, 8], 3, OURO_G32, 16, True, True, 128, "anchor"),
    ([300], [33], 2, OURO_G32, 16, True, True, 128, "anchor"),           # two row tiles
    ([70, 200], [70, 5], 2, OURO_G16, 32, False, True, 128, "anchor"),   # the first request has no history (prefill)
    ([16, 40], [16, 3], 2, OURO_G32, 32, True, False, 128, "anchor"),    # no rotation; no history (prefill)
    ([2100], [3], 2, OURO_G32, 16, True, True, 128, "anchor"),           # eight history splits
    ([90, 51], [2, 6], 2, ((2, 16), (2, 16), (4, 32), (2, 32)), 16, True, True, 128, "anchor"),
    ([77], [5], 1, ((4, 16),), 32, True, True, 128, "anchor"),           # single-record group
    ([400, 123], [12, 20], 2, OURO_G32, 16, True, True, 128, "anchor"),  # 16 rows per request on average
    ([50, 300], [0, 33], 2, OURO_G32, 16, True, True, 128, "anchor"),    # a request with no new rows
    # D96 (the Huginn geometry: three 32-channel quarters per token)
    ([100, 37, 9], [4, 1, 8], 3, OURO_G16, 16, True, True, 96, "anchor"),
    ([300, 70], [33, 70], 2, OURO_G32, 32, True, True, 96, "anchor"),    # two row tiles; no history (prefill)
    ([2100], [3], 2, OURO_G16, 16, False, True, 96, "anchor"),           # eight history splits
    ([77, 50], [5, 0], 1, ((4, 16),), 16, True, False, 96, "anchor"),    # single-record group, no rotation
    ([300, 60, 9], [33, 1, 2], 2, OURO_G16, 32, True, True, 96, "anchor"),  # 16-row tiles, three in one request
    # 8 requests x 55 heads: 440 (request, head, tile) groups, one history split each
    ([260, 131, 99, 64, 300, 17, 180, 222], [2] * 8, 55, OURO_G16, 16, True, True, 96, "anchor"),
    # adjacent mode (every loop past 0 rebuilds the restore chain of records 0..L)
    ([100, 37, 9], [4, 1, 8], 3, ADJACENT_G32, 16, True, True, 128, "adjacent"),
    ([300, 40], [33, 2], 2, ADJACENT_G16, 32, True, True, 128, "adjacent"),
    ([2100], [3], 2, ADJACENT_G32, 16, False, False, 128, "adjacent"),   # eight history splits
    ([100, 37, 9], [4, 1, 8], 2, ADJACENT_G16, 16, True, True, 96, "adjacent"),
    ([400, 123], [12, 20], 2, ((4, 32), (2, 32), (4, 16)), 32, True, True, 96, "adjacent"),
]


def _ids(case):
    return f"n{sum(case[1])}-h{case[2]}-r{len(case[3])}-pt{case[4]}-d{case[7]}-{case[8]}"


@pytest.mark.parametrize("case", CASES, ids=_ids)
@pytest.mark.parametrize("causal", [True, False], ids=["prefill", "decode"])
def test_multirow_matches_oracle(oracle, device, case, causal):
    lengths, rows, heads, records, pt, mean, rotation, dim, mode = case
    print(f"[case] multirow causal={causal} {case}", flush=True)
    d = make_decode(lengths, heads, dim, records, seed=sum(lengths) + len(rows), page_tokens=pt, mean=mean,
                    rotation=rotation, rows_per_request=rows, mode=mode, anchor=0 if mode == "adjacent" else None)
    expected_cache = d.group.oracle_cache(oracle)
    cache = torch.from_numpy(expected_cache).to(device)
    for loop in range(len(records)):
        got = _run(d, device, cache, loop, causal)
        want = _oracle(oracle, d, expected_cache, loop, causal)
        err = np.abs(got - _bf16(want))
        print(f"[case]   loop {loop}: max {err.max():.3g} mean {err.mean():.3g}", flush=True)
        assert np.isfinite(got).all()
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (loop, err.max(), err.mean())


def _random_cases(seed: int, count: int):
    """Seeded mixes of row counts (empty requests, one row, exact and ragged
    32-row tiles), history lengths (none, one token, page-ragged, several
    splits), heads, schedules, page sizes and mean / rotation switches."""
    schedules = [OURO_G32, OURO_G16, ((2, 16), (2, 16), (4, 32), (2, 32)), ((4, 32), (2, 32)), ((2, 32), (4, 16))]
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        rows = [rng.choice([0, 1, 2, 3, 5, 16, 31, 33, 40]) for _ in range(rng.randint(1, 4))]
        if sum(rows) == 0:
            rows[0] = 2
        lengths = [max(1, r + rng.choice([0, 1, 15, 17, 100, 333, 700])) for r in rows]
        cases.append((lengths, rows, rng.choice([1, 2, 3]), rng.choice(schedules), rng.choice([16, 32]),
                      rng.random() < 0.7, rng.random() < 0.7, rng.random() < 0.5, rng.choice([96, 128]),
                      rng.choice(["anchor", "anchor", "adjacent"])))
    return cases


@pytest.mark.parametrize("index,case", list(enumerate(_random_cases(7, 16))),
                         ids=[f"c{i}" for i in range(16)])
def test_multirow_random_mixes(oracle, device, index, case):
    """Every loop of each random mix, through ``attention`` (rows routed per
    call between the per-row and multi-row kernels) or
    ``packed_prefill_attention``, at D 96 or 128, in anchor or adjacent mode."""
    lengths, rows, heads, records, pt, mean, rotation, causal, dim, mode = case
    print(f"[case] random c{index} causal={causal} {case}", flush=True)
    d = make_decode(lengths, heads, dim, records, seed=1000 + index, page_tokens=pt, mean=mean, rotation=rotation,
                    rows_per_request=rows, mode=mode, anchor=0 if mode == "adjacent" else None)
    expected_cache = d.group.oracle_cache(oracle)
    cache = torch.from_numpy(expected_cache).to(device)
    for loop in range(len(records)):
        got = _run(d, device, cache, loop, causal)
        err = np.abs(got - _bf16(_oracle(oracle, d, expected_cache, loop, causal)))
        assert np.isfinite(got).all()
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (loop, err.max(), err.mean())


def _view(t: torch.Tensor, device, extra: int, offset: int) -> torch.Tensor:
    """t as a [rows, heads, D] view with token stride heads * D + extra, starting `offset` elements in."""
    rows, heads, dim = t.shape
    width = heads * dim + extra
    flat = torch.full((rows * width + offset + 8,), float("nan"), dtype=torch.bfloat16, device=device)
    view = torch.as_strided(flat, (rows, heads, dim), (width, dim, 1), storage_offset=offset)
    view.copy_(t.to(device))
    return view


@pytest.mark.parametrize("causal", [True, False], ids=["prefill", "decode"])
def test_multirow_strided_views(oracle, device, causal):
    """Token strides and offsets the boundary allows: queries and keys 8-byte
    aligned rows (stride a multiple of 4), values and outputs 2-byte aligned
    (odd stride, odd offset), so the finish reads and writes them value by
    value instead of in 16-byte words."""
    d = make_decode([300, 123], 2, 128, OURO_G32, seed=31, rows_per_request=[40, 12])
    g = d.group
    expected_cache = g.oracle_cache(oracle)
    cache = torch.from_numpy(expected_cache).to(device)
    kr, vr, km = g.device_args(device)
    q, k = _view(d.query, device, 4, 4), _view(d.key, device, 4, 4)
    v = _view(d.value, device, 1, 1)
    out = _view(torch.zeros_like(d.query), device, 3, 1)
    function = rq.packed_prefill_attention if causal else rq.attention
    for loop in (0, 3):
        out.fill_(float("nan"))
        function(q, k, v, cache, out, d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device), kr, vr,
                 km, g.records, g.mode, g.anchor, loop)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        want = _oracle(oracle, d, expected_cache, loop, causal)
        err = np.abs(got - _bf16(want))
        print(f"[case] strided causal={causal} loop {loop}: max {err.max():.3g} mean {err.mean():.3g}", flush=True)
        assert np.isfinite(got).all()
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (loop, err.max(), err.mean())


def test_decode_rows_agree_with_single_row_calls(oracle, device):
    """The multi-row route and the per-row decode kernel give the same rows within the bar."""
    d = make_decode([500, 300], 4, 128, OURO_G32, seed=5, rows_per_request=[9, 7])
    g = d.group
    cache = torch.from_numpy(g.oracle_cache(oracle)).to(device)
    kr, vr, km = g.device_args(device)
    for loop in (0, 3):
        multi = _run(d, device, cache, loop, causal=False)
        starts = d.query_start_loc.tolist()
        for b in range(2):
            for i in range(starts[b], starts[b + 1]):
                out = torch.empty((1, 4, 128), dtype=torch.bfloat16, device=device)
                rq.attention(d.query[i:i + 1].to(device), d.key[i:i + 1].to(device), d.value[i:i + 1].to(device),
                             cache, out, torch.tensor([0, 1], dtype=torch.int32, device=device),
                             d.seq_lens[b:b + 1].to(device), d.table[b:b + 1].to(device), kr, vr, km, g.records,
                             g.mode, g.anchor, loop)
                single = out.float().cpu().numpy()[0]
                assert np.abs(multi[i] - single).max() <= MAX_ABS


def test_multirow_rejections(device):
    """Head dims outside the attention registry (96, 128) are refused before any launch."""
    d = make_decode([40], 2, 64, ((4, 32), (2, 32)), seed=2, rows_per_request=[3])
    g = d.group
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    out = torch.empty_like(d.query, device=device)
    with pytest.raises(RuntimeError, match="No compiled packed HIP"):
        rq.packed_prefill_attention(d.query.to(device), d.key.to(device), d.value.to(device), cache, out,
                                    d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device), kr, vr,
                                    km, g.records, g.mode, g.anchor, 0)


@pytest.mark.parametrize("dim,mode,records", [(96, "anchor", OURO_G16), (128, "adjacent", ADJACENT_G32),
                                              (96, "adjacent", ADJACENT_G16)])
def test_multirow_agrees_with_per_row_kernels(oracle, device, dim, mode, records):
    """At D96 and in adjacent mode, decode rows on the multi-row route agree
    with the same rows called one at a time (the per-row decode kernels:
    decode96_dma_kernel, decode_chain_kernel) within the bar, at every loop."""
    d = make_decode([500, 300], 3, dim, records, seed=6, rows_per_request=[9, 7], mode=mode,
                    anchor=0 if mode == "adjacent" else None)
    g = d.group
    cache = torch.from_numpy(g.oracle_cache(oracle)).to(device)
    kr, vr, km = g.device_args(device)
    for loop in range(len(records)):
        multi = _run(d, device, cache, loop, causal=False)
        starts = d.query_start_loc.tolist()
        for b in range(2):
            for i in range(starts[b], starts[b + 1]):
                out = torch.empty((1, 3, dim), dtype=torch.bfloat16, device=device)
                rq.attention(d.query[i:i + 1].to(device), d.key[i:i + 1].to(device), d.value[i:i + 1].to(device),
                             cache, out, torch.tensor([0, 1], dtype=torch.int32, device=device),
                             d.seq_lens[b:b + 1].to(device), d.table[b:b + 1].to(device), kr, vr, km, g.records,
                             g.mode, g.anchor, loop)
                single = out.float().cpu().numpy()[0]
                assert np.abs(multi[i] - single).max() <= MAX_ABS, (loop, i)
