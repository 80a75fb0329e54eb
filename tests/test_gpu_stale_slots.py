"""Attention over pages whose unwritten token slots hold stale bytes.

A page's slots past a request's history are never written by quantize, so
they can hold anything; 0xFF bytes are NaN as FP8 E4M3 scales and offsets.
The kernels must not let them reach the output: the decode kernels score
only history tokens, and the multi-row kernels zero the values past the
history (their keys there produce scores that are replaced by -inf).  The
cache here starts as 0xFF everywhere and the history is quantized into it;
every history ends inside a page.

Bar: finite outputs within 2e-2 max-abs / 1e-3 mean-abs of the FP64 oracle
(which reads only history tokens) on the same bytes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import residualquant_amd as rq
from residualquant_amd import workloads

from .cases import OURO_G16, OURO_G32, make_decode

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 1e-3
ADJACENT = ((4, 32), (2, 32), (2, 32), (2, 32))


def _bits(t):
    return None if t is None else workloads.bf16_bits(t)


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).float().to(torch.bfloat16).double().numpy()


CASES = [
    # lengths, rows per request, heads, dim, records, page tokens, mode, anchor, split target (0: default)
    ([400, 260, 31], None, 4, 128, OURO_G32, 16, "anchor", None, 0),
    ([400, 260, 31], None, 4, 128, OURO_G32, 16, "anchor", None, 1),
    ([130, 47], None, 3, 96, OURO_G16, 16, "anchor", None, 0),
    ([130, 47], None, 3, 96, OURO_G16, 32, "anchor", None, 1),
    ([70, 33], None, 2, 128, ADJACENT, 16, "adjacent", 0, 0),
    ([300, 45], [8, 7], 2, 128, OURO_G32, 16, "anchor", None, 0),    # multi-row route
    ([210, 100], [9, 6], 2, 128, OURO_G16, 32, "anchor", None, 0),   # multi-row route, 32-token pages
]


def _ids(case):
    rows = case[1] or [1] * len(case[0])
    return f"{case[3]}d-{case[6]}-pt{case[5]}-rows{sum(rows)}-t{case[8]}"


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_stale_slots_do_not_reach_the_output(oracle, device, case):
    lengths, rows_per_request, heads, dim, records, pt, mode, anchor, target = case
    print(f"[case] stale slots {case}", flush=True)
    d = make_decode(lengths, heads, dim, records, seed=sum(lengths) + dim, page_tokens=pt, mode=mode,
                    anchor=anchor, rows_per_request=rows_per_request)
    g = d.group
    stale = np.full(g.cache_shape, 0xFF, dtype=np.uint8)
    cache_np = g.oracle_cache(oracle, stale)
    cache = torch.from_numpy(cache_np).to(device)
    kr, vr, km = g.device_args(device)
    q, k, v = d.query.to(device), d.key.to(device), d.value.to(device)
    qsl, sl, table = d.query_start_loc.to(device), d.seq_lens.to(device), d.table.to(device)
    multirow = rows_per_request is not None
    try:
        rq.ops.set_split_target(target)
        for loop in range(len(records)):
            calls = [("attention", rq.attention, oracle.attention)]
            if multirow:
                calls.append(("packed prefill", rq.packed_prefill_attention, oracle.attention_prefill))
            for name, op, reference in calls:
                expected = reference(_bits(d.query), _bits(d.key), _bits(d.value), cache_np,
                                     d.query_start_loc.numpy(), d.seq_lens.numpy(), d.table.numpy(),
                                     _bits(g.key_rotation), _bits(g.value_rotation),
                                     None if g.key_mean is None else g.key_mean.numpy(), g.records, g.mode,
                                     g.anchor, loop)
                out = torch.full_like(q, float("nan"))
                op(q, k, v, cache, out, qsl, sl, table, kr, vr, km, g.records, g.mode, g.anchor, loop)
                torch.cuda.synchronize()
                got = out.float().cpu().numpy()
                assert np.isfinite(got).all(), (name, loop)
                err = np.abs(got - (_bf16(expected) if multirow else expected))
                print(f"[case]   {name} loop {loop}: max {err.max():.3g} mean {err.mean():.3g}", flush=True)
                assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (name, loop, err.max(), err.mean())
    finally:
        rq.ops.set_split_target(0)
