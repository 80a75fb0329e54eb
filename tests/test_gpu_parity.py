"""HIP kernels against the CPU oracle on the same seeded inputs (MI355X).

Bars: packed bytes and restored BF16 K/V bit-exact; attention output within
2e-2 max-abs and 1e-3 mean-abs of the FP64 oracle (BF16 output).
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

import residualquant_amd as rq
from residualquant_amd import workloads

from .cases import OURO_G16, OURO_G32, make_decode, make_group, oracle_attention

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 1e-3

QUANTIZE_CASES = [
    # tokens, heads, dim, records, page_tokens, mode, anchor, coefficient, rotation, mean, skipped
    # (short calls give workgroups one partial pass; the long ones several passes each)
    (37, 4, 128, OURO_G32, 16, "anchor", 3, "ls", True, True, 3),
    (20, 3, 128, OURO_G16, 16, "anchor", 3, "ls", True, False, 0),
    (19, 5, 96, OURO_G16, 16, "anchor", 3, "ls", True, True, 2),
    (33, 2, 128, ((4, 32), (2, 32), (2, 32), (2, 32)), 32, "adjacent", 0, "norm", False, True, 1),
    (9, 2, 128, ((2, 32),), 16, "anchor", 0, "unit", True, True, 0),
    (17, 2, 128, ((4, 32),) * 4, 16, "anchor", 3, "unit", False, False, 0),
    (25, 3, 96, ((2, 32),) * 4, 32, "anchor", 0, "ls", True, False, 4),
    (64, 2, 128, ((4, 16), (2, 16)), 16, "adjacent", 0, "ls", True, True, 0),
    (63, 2, 128, OURO_G32, 16, "anchor", 3, "ls", True, True, 1),
    (300, 4, 128, OURO_G32, 16, "anchor", 3, "norm", True, True, 7),
    (2100, 2, 128, OURO_G32, 16, "anchor", 3, "ls", True, True, 5),
    (2048, 2, 96, OURO_G16, 16, "anchor", 3, "ls", True, True, 3),
    (2053, 1, 128, ((4, 32), (2, 32), (2, 32), (2, 32)), 32, "adjacent", 0, "norm", True, False, 1),
    (2049, 1, 128, ((4, 32), (2, 16)), 16, "anchor", 0, "unit", False, True, 2),
    (2050, 1, 96, ((2, 16), (4, 32), (2, 32)), 16, "anchor", 1, "ls", True, True, 3),
    (2048, 1, 128, ((4, 32),), 32, "anchor", 0, "unit", True, False, 0),
    (6000, 1, 128, OURO_G16, 16, "adjacent", 0, "ls", True, True, 9),  # many passes per wave
]


def _print_case(name, case):
    print(f"[case] {name} {case}", flush=True)


@pytest.mark.parametrize("case", QUANTIZE_CASES, ids=lambda c: f"{c[2]}d-{len(c[3])}r-{c[5]}-{c[7]}-pt{c[4]}")
def test_quantize_bitexact(oracle, device, case):
    _print_case("quantize", case)
    tokens, heads, dim, records, pt, mode, anchor, coef, rotation, mean, skipped = case
    g = make_group(tokens, heads, dim, records, seed=tokens * 7 + dim, page_tokens=pt, mode=mode,
                   anchor=anchor, coefficient=coef, rotation=rotation, mean=mean, skipped=skipped)
    expected = g.oracle_cache(oracle)
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    rq.quantize([(k.to(device), v.to(device)) for k, v in g.pairs], cache, g.slots.to(device), kr, vr, km,
                g.records, g.mode, g.anchor, g.coefficient)
    got = cache.cpu().numpy()
    mismatch = np.argwhere(got != expected)
    assert mismatch.size == 0, f"{len(mismatch)} bytes differ, first at {mismatch[:4].tolist()}"


def _random_quantize_cases(seed: int, count: int):
    """Seeded calls on both sides of the VALU / MFMA kernel switch at 64
    tokens: 1-2100 tokens, 1-5 heads, D96 / D128, five schedules, any anchor
    index, adjacent mode, the three coefficients, page sizes 16 / 32, up to a
    tenth of the slots skipped (-1)."""
    schedules = [OURO_G32, OURO_G16, ((2, 16), (2, 16), (4, 32), (2, 32)), ((4, 32), (2, 32)), ((2, 32), (4, 16))]
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        tokens = rng.choice([1, 7, 63, 64, 65, 130, 777, 2047, 2100])
        records = rng.choice(schedules)
        mode = rng.choice(["anchor", "adjacent"])
        cases.append((tokens, rng.randint(1, 5), rng.choice([96, 128]), records, rng.choice([16, 32]), mode,
                      rng.randrange(len(records)) if mode == "anchor" else 0, rng.choice(["ls", "norm", "unit"]),
                      rng.random() < 0.7, rng.random() < 0.7, rng.randint(0, tokens // 10)))
    return cases


@pytest.mark.parametrize("index,case", list(enumerate(_random_quantize_cases(13, 16))),
                         ids=[f"c{i}" for i in range(16)])
def test_quantize_random_calls(oracle, device, index, case):
    _print_case(f"random quantize c{index}", case)
    tokens, heads, dim, records, pt, mode, anchor, coef, rotation, mean, skipped = case
    g = make_group(tokens, heads, dim, records, seed=3000 + index, page_tokens=pt, mode=mode, anchor=anchor,
                   coefficient=coef, rotation=rotation, mean=mean, skipped=skipped)
    expected = g.oracle_cache(oracle)
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    rq.quantize([(k.to(device), v.to(device)) for k, v in g.pairs], cache, g.slots.to(device), kr, vr, km,
                g.records, g.mode, g.anchor, g.coefficient)
    mismatch = np.argwhere(cache.cpu().numpy() != expected)
    assert mismatch.size == 0, f"{len(mismatch)} bytes differ, first at {mismatch[:4].tolist()}"


def test_quantize_strided_inputs(oracle, device):
    """Token strides wider than heads*D (a [tokens, 3*heads, D] buffer view) are honoured."""
    g = make_group(21, 2, 128, OURO_G32, seed=5)
    expected = g.oracle_cache(oracle)
    pairs = []
    for k, v in g.pairs:
        wide = torch.zeros((k.size(0), 3 * k.size(1), k.size(2)), dtype=torch.bfloat16, device=device)
        wide[:, : k.size(1)] = k.to(device)
        wide[:, k.size(1): 2 * k.size(1)] = v.to(device)
        pairs.append((wide[:, : k.size(1)], wide[:, k.size(1): 2 * k.size(1)]))
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    rq.quantize(pairs, cache, g.slots.to(device), kr, vr, km, g.records, g.mode, g.anchor, g.coefficient)
    assert np.array_equal(cache.cpu().numpy(), expected)


def test_quantize_rows_eight_byte_aligned(oracle, device):
    """Rows that start 8 bytes past a 16-byte boundary, with a token stride of heads*D + 4."""
    g = make_group(37, 2, 128, OURO_G16, seed=12)
    expected = g.oracle_cache(oracle)
    pairs = []
    for k, v in g.pairs:
        width = k.size(1) * k.size(2) + 4
        flat_k = torch.zeros(k.size(0) * width + 8, dtype=torch.bfloat16, device=device)
        flat_v = torch.zeros_like(flat_k)
        view_k = flat_k[4:4 + k.size(0) * width].view(k.size(0), width)[:, : k.size(1) * k.size(2)]
        view_v = flat_v[4:4 + k.size(0) * width].view(k.size(0), width)[:, : k.size(1) * k.size(2)]
        view_k.copy_(k.reshape(k.size(0), -1).to(device))
        view_v.copy_(v.reshape(v.size(0), -1).to(device))
        pairs.append((view_k.view(k.shape), view_v.view(v.shape)))
    assert pairs[0][0].data_ptr() % 16 == 8
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    rq.quantize(pairs, cache, g.slots.to(device), kr, vr, km, g.records, g.mode, g.anchor, g.coefficient)
    assert np.array_equal(cache.cpu().numpy(), expected)


@pytest.mark.parametrize("case", QUANTIZE_CASES[:5], ids=lambda c: f"{c[2]}d-{len(c[3])}r-{c[5]}")
def test_dequantize_bitexact(oracle, device, case):
    _print_case("dequantize", case)
    tokens, heads, dim, records, pt, mode, anchor, coef, rotation, mean, skipped = case
    g = make_group(tokens, heads, dim, records, seed=tokens * 11 + dim, page_tokens=pt, mode=mode,
                   anchor=anchor, coefficient=coef, rotation=rotation, mean=mean, skipped=skipped)
    cache_np = g.oracle_cache(oracle)
    cache = torch.from_numpy(cache_np).to(device)
    km = None if g.key_mean is None else g.key_mean.to(device)
    for loop in range(len(records)):
        k_exp, v_exp = oracle.dequantize(cache_np, g.slots.numpy(), dim,
                                         None if g.key_mean is None else g.key_mean.numpy(), records, mode,
                                         anchor, loop)
        k, v = rq.dequantize(cache, g.slots.to(device), dim, km, records, mode, anchor, loop)
        assert np.array_equal(workloads.bf16_bits(k), k_exp), f"K differs at loop {loop}"
        assert np.array_equal(workloads.bf16_bits(v), v_exp), f"V differs at loop {loop}"


ATTENTION_CASES = [
    # lengths, heads, dim, records, page_tokens, rotation, mean, rows_per_request
    ([130, 1, 77, 300], 4, 128, OURO_G32, 16, True, True, None),
    ([65, 200], 3, 128, OURO_G16, 16, True, False, None),
    ([97, 33, 256], 2, 96, OURO_G16, 16, True, True, None),
    ([250, 17], 2, 128, OURO_G32, 32, False, True, None),
    ([120, 40], 2, 128, OURO_G32, 16, True, True, [2, 1]),
    ([513], 2, 128, ((4, 32),) * 4, 16, False, False, None),
    ([90, 45], 3, 96, ((2, 32),) * 4, 32, True, False, None),
]


@pytest.mark.parametrize("case", ATTENTION_CASES, ids=lambda c: f"{c[2]}d-pt{c[4]}-b{len(c[0])}")
def test_attention_matches_oracle(oracle, device, case):
    _print_case("attention", case)
    lengths, heads, dim, records, pt, rotation, mean, rows = case
    d = make_decode(lengths, heads, dim, records, seed=sum(lengths) + dim, page_tokens=pt,
                    rotation=rotation, mean=mean, rows_per_request=rows)
    g = d.group
    cache_np = g.oracle_cache(oracle)
    cache = torch.from_numpy(cache_np).to(device)
    kr, vr, km = g.device_args(device)
    for loop in range(len(records)):
        expected = oracle_attention(oracle, d, cache_np, loop)
        out = torch.zeros_like(d.query, device=device)
        rq.attention(d.query.to(device), d.key.to(device), d.value.to(device), cache, out,
                     d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device), kr, vr, km,
                     g.records, g.mode, g.anchor, loop)
        err = np.abs(out.float().cpu().numpy().astype(np.float64) - expected)
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (loop, err.max(), err.mean())


def _random_decode_cases(seed: int, count: int):
    """Seeded one-row-per-request calls: 1-8 requests with histories from none
    to several splits, 1-4 heads, D96 / D128, page sizes 16 / 32, five
    schedules, anchor and adjacent modes, mean and rotation switches."""
    schedules = [OURO_G32, OURO_G16, ((2, 16), (2, 16), (4, 32), (2, 32)), ((4, 32), (2, 32)), ((2, 32), (4, 16))]
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        lengths = [rng.choice([1, 2, 17, 33, 129, 500, 1500, 3000]) for _ in range(rng.randint(1, 8))]
        cases.append((lengths, rng.randint(1, 4), rng.choice([96, 128]), rng.choice(schedules), rng.choice([16, 32]),
                      rng.random() < 0.7, rng.random() < 0.7, rng.choice(["anchor", "adjacent"])))
    return cases


@pytest.mark.parametrize("index,case", list(enumerate(_random_decode_cases(11, 16))),
                         ids=[f"c{i}" for i in range(16)])
def test_attention_random_calls(oracle, device, index, case):
    _print_case(f"random attention c{index}", case)
    lengths, heads, dim, records, pt, rotation, mean, mode = case
    d = make_decode(lengths, heads, dim, records, seed=2000 + index, page_tokens=pt, mode=mode,
                    anchor=0 if mode == "adjacent" else None, rotation=rotation, mean=mean)
    g = d.group
    cache_np = g.oracle_cache(oracle)
    cache = torch.from_numpy(cache_np).to(device)
    kr, vr, km = g.device_args(device)
    for loop in range(len(records)):
        expected = oracle_attention(oracle, d, cache_np, loop)
        out = torch.full_like(d.query, float("nan"), device=device)
        rq.attention(d.query.to(device), d.key.to(device), d.value.to(device), cache, out,
                     d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device), kr, vr, km,
                     g.records, g.mode, g.anchor, loop)
        got = out.float().cpu().numpy().astype(np.float64)
        err = np.abs(got - expected)
        assert np.isfinite(got).all()
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (loop, err.max(), err.mean())


ADJACENT_CASES = [
    # lengths, heads, dim, records, page_tokens, rotation, mean, split target (0: default)
    ([130, 1, 77, 300], 2, 128, ((4, 32), (2, 32), (2, 32), (2, 32)), 16, True, True, 0),
    ([97, 33], 3, 96, ((4, 16), (2, 16), (4, 32), (2, 32)), 32, True, False, 0),
    ([250, 65], 2, 128, ((4, 32), (4, 16), (2, 16)), 16, False, True, 1),
]


@pytest.mark.parametrize("case", ADJACENT_CASES, ids=lambda c: f"{c[2]}d-pt{c[4]}-r{len(c[3])}-t{c[7]}")
def test_adjacent_attention_matches_oracle(oracle, device, case):
    """Adjacent mode: loop L scores and sums the BF16 restore chain of records
    0..L (compute.cuh:120-197, :506-528); loop 0 is the anchor record alone."""
    _print_case("adjacent attention", case)
    lengths, heads, dim, records, pt, rotation, mean, target = case
    d = make_decode(lengths, heads, dim, records, seed=sum(lengths) + 3 * dim, page_tokens=pt, mode="adjacent",
                    anchor=0, rotation=rotation, mean=mean)
    g = d.group
    cache_np = g.oracle_cache(oracle)
    cache = torch.from_numpy(cache_np).to(device)
    kr, vr, km = g.device_args(device)
    try:
        rq.ops.set_split_target(target)
        for loop in range(len(records)):
            expected = oracle_attention(oracle, d, cache_np, loop)
            out = torch.zeros_like(d.query, device=device)
            rq.attention(d.query.to(device), d.key.to(device), d.value.to(device), cache, out,
                         d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device), kr, vr, km,
                         g.records, g.mode, g.anchor, loop)
            err = np.abs(out.float().cpu().numpy().astype(np.float64) - expected)
            print(f"[case]   loop {loop}: max {err.max():.3g} mean {err.mean():.3g}", flush=True)
            assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (loop, err.max(), err.mean())
    finally:
        rq.ops.set_split_target(0)


def test_attention_history_zero_is_live_value(device):
    """With no history the output is the current token's value exactly (merge.cuh:19-83)."""
    d = make_decode([1, 1, 1], 4, 128, OURO_G32, seed=3)
    g = d.group
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    for loop in range(4):
        out = torch.zeros_like(d.query, device=device)
        rq.attention(d.query.to(device), d.key.to(device), d.value.to(device), cache, out,
                     d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device), kr, vr, km,
                     g.records, g.mode, g.anchor, loop)
        assert torch.equal(out.cpu(), d.value)


# Residual loops of every (bits, group) the D = 96 decode kernel compiles,
# INT4 g32 anchor.
MIXED_D96 = ((2, 16), (4, 16), (2, 32), (4, 32))


@pytest.mark.parametrize("dim,records,loops", [(128, OURO_G32, (1,)), (96, MIXED_D96, (0, 1, 2, 3))],
                         ids=["128d", "96d"])
def test_attention_split_invariance(oracle, device, dim, records, loops):
    """Different split-K counts give outputs within rounding of each other and the oracle.

    A target of one workgroup gives one split per (row, head): the decode
    launch then prepares its own query and finishes without partials.  The
    2100-token history (132 pages at 16 pages per split at least) lets the
    targets give 1, 2, 9 and 9 splits."""
    print(f"split invariance dim={dim}", flush=True)
    d = make_decode([2100, 129], 2, dim, records, seed=9 + dim)
    g = d.group
    cache_np = g.oracle_cache(oracle)
    cache = torch.from_numpy(cache_np).to(device)
    kr, vr, km = g.device_args(device)
    for loop in loops:
        expected = oracle_attention(oracle, d, cache_np, loop)
        outs = []
        try:
            for target in (1, 8, 64, 4096):
                rq.ops.set_split_target(target)
                out = torch.zeros_like(d.query, device=device)
                rq.attention(d.query.to(device), d.key.to(device), d.value.to(device), cache, out,
                             d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device), kr, vr,
                             km, g.records, g.mode, g.anchor, loop)
                outs.append(out.float().cpu().numpy())
        finally:
            rq.ops.set_split_target(0)
        for out in outs:
            err = np.abs(out - expected)
            assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (loop, err.max(), err.mean())
            assert np.abs(out - outs[0]).max() <= 2 * MAX_ABS


def test_paged_attention_bf16_matches_oracle(oracle, device):
    lengths = [300, 45, 1, 129]
    heads, dim, pt = 4, 128, 16
    max_pages = 20
    table = workloads.block_tables(len(lengths), max_pages, 77)
    generator = torch.Generator().manual_seed(78)
    blocks = len(lengths) * max_pages
    cache = torch.randn((2, blocks, heads, pt, dim), generator=generator).to(torch.bfloat16)
    rows = len(lengths)
    q = torch.randn((rows, heads, dim), generator=generator).to(torch.bfloat16)
    k = torch.randn((rows, heads, dim), generator=generator).to(torch.bfloat16)
    v = torch.randn((rows, heads, dim), generator=generator).to(torch.bfloat16)
    qsl = torch.arange(rows + 1, dtype=torch.int32)
    sl = torch.tensor(lengths, dtype=torch.int32)
    expected = oracle.paged_attention_bf16(workloads.bf16_bits(q), workloads.bf16_bits(k),
                                           workloads.bf16_bits(v), workloads.bf16_bits(cache),
                                           qsl.numpy(), sl.numpy(), table.numpy())
    out = torch.zeros_like(q, device=device)
    rq.paged_attention_bf16(q.to(device), k.to(device), v.to(device), cache.to(device), out,
                            qsl.to(device), sl.to(device), table.to(device))
    err = np.abs(out.float().cpu().numpy() - expected)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (err.max(), err.mean())


def test_gpu_quantize_then_attention(oracle, device):
    """The whole write+read path on the GPU against the oracle on the oracle's own cache."""
    d = make_decode([400, 260, 31], 4, 128, OURO_G32, seed=21)
    g = d.group
    cache_np = g.oracle_cache(oracle)
    cache = torch.zeros(g.cache_shape, dtype=torch.uint8, device=device)
    kr, vr, km = g.device_args(device)
    rq.quantize([(k.to(device), v.to(device)) for k, v in g.pairs], cache, g.slots.to(device), kr, vr, km,
                g.records, g.mode, g.anchor, g.coefficient)
    assert np.array_equal(cache.cpu().numpy(), cache_np)
    for loop in range(4):
        expected = oracle_attention(oracle, d, cache_np, loop)
        out = torch.zeros_like(d.query, device=device)
        rq.attention(d.query.to(device), d.key.to(device), d.value.to(device), cache, out,
                     d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device), kr, vr, km,
                     g.records, g.mode, g.anchor, loop)
        err = np.abs(out.float().cpu().numpy() - expected)
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (loop, err.max(), err.mean())


def test_attention_graph_replay(oracle, device):
    """Captured in a HIP graph with a fixed workspace, every replay equals eager."""
    d = make_decode([300, 190], 4, 128, OURO_G32, seed=31)
    g = d.group
    cache_np = g.oracle_cache(oracle)
    cache = torch.from_numpy(cache_np).to(device)
    kr, vr, km = g.device_args(device)
    q, k, v = d.query.to(device), d.key.to(device), d.value.to(device)
    qsl, sl, table = d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device)
    need = rq.ops.attention_workspace_bytes(q.size(0), 4, 128, table.size(1), 16)
    workspace = torch.empty(need, dtype=torch.uint8, device=device)
    eager = torch.zeros_like(q)
    rq.attention(q, k, v, cache, eager, qsl, sl, table, kr, vr, km, g.records, g.mode, g.anchor, 2,
                 workspace=workspace)
    out = torch.zeros_like(q)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        rq.attention(q, k, v, cache, out, qsl, sl, table, kr, vr, km, g.records, g.mode, g.anchor, 2,
                     workspace=workspace)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            rq.attention(q, k, v, cache, out, qsl, sl, table, kr, vr, km, g.records, g.mode, g.anchor, 2,
                         workspace=workspace)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_empty_calls_are_noops(device):
    """Zero tokens / rows through every op: nothing is launched or written."""
    g = make_group(20, 2, 128, OURO_G32, seed=77)
    kr, vr, km = g.device_args(device)
    cache = torch.full(g.cache_shape, 7, dtype=torch.uint8, device=device)
    empty = torch.empty((0, 2, 128), dtype=torch.bfloat16, device=device)
    pairs = [(empty, empty) for _ in g.records]
    rq.quantize(pairs, cache, torch.empty(0, dtype=torch.int64, device=device), kr, vr, km, g.records, "anchor",
                3, "ls")
    assert bool((cache == 7).all())
    qsl = torch.zeros(1, dtype=torch.int32, device=device)
    lens = torch.empty(0, dtype=torch.int32, device=device)
    table = torch.empty((0, 4), dtype=torch.int32, device=device)
    out = torch.empty_like(empty)
    rq.attention(empty, empty, empty, cache, out, qsl, lens, table, kr, vr, km, g.records, "anchor", 3, 1)
    k, v = rq.dequantize(cache, torch.empty(0, dtype=torch.int64, device=device), 128, km, g.records, "anchor", 3, 0)
    assert k.shape == (0, 2, 128) and v.shape == (0, 2, 128)
    cu = torch.zeros(2, dtype=torch.int32, device=device)
    res = rq.flash_attn_varlen_func(empty, empty, empty, 0, cu, 0, causal=True)
    assert res.shape == (0, 2, 128)
    torch.cuda.synchronize()
    assert bool((cache == 7).all())
