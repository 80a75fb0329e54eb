"""Committed golden fixtures (tests/golden/*.npz, written by make_golden.py).

CPU: the oracle reproduces every stored output from the stored inputs
(regression pin of the oracle).  GPU: the HIP kernels reproduce the stored
packed cache and restored K/V bit for bit and the attention output within
2e-2 max-abs / 1e-3 mean-abs.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def _load(path):
    with np.load(path, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def _records(f):
    return tuple(tuple(int(v) for v in r) for r in f["records"])


def _bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _f16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.float16)


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_reproduces_fixture(oracle, path):
    f = _load(path)
    records = _records(f)
    cache = np.zeros_like(f["cache"])
    oracle.quantize(list(zip(f["keys"], f["values"])), cache, f["slots"], f.get("key_rotation"),
                    f.get("value_rotation"), f.get("key_mean"), records, "anchor", int(f["anchor"]), "ls")
    assert np.array_equal(cache, f["cache"])
    dim = f["keys"].shape[-1]
    for loop in range(len(records)):
        k, v = oracle.dequantize(cache, f["slots"], dim, f.get("key_mean"), records, "anchor", int(f["anchor"]), loop)
        assert np.array_equal(k, f[f"restored_k{loop}"]) and np.array_equal(v, f[f"restored_v{loop}"])
        out = oracle.attention(f["query"], f["key"], f["value"], cache, f["query_start_loc"], f["seq_lens"],
                               f["block_table"], f.get("key_rotation"), f.get("value_rotation"), f.get("key_mean"),
                               records, "anchor", int(f["anchor"]), loop)
        assert np.allclose(out, f[f"attention{loop}"], rtol=0, atol=1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_kernels_match_fixture(device, path):
    import residualquant_amd as rq

    print(f"[case] golden {os.path.basename(path)}", flush=True)
    f = _load(path)
    records = _records(f)
    anchor = int(f["anchor"])
    kr = _f16(f["key_rotation"]).to(device) if "key_rotation" in f else None
    vr = _f16(f["value_rotation"]).to(device) if "value_rotation" in f else None
    km = torch.from_numpy(f["key_mean"]).to(device) if "key_mean" in f else None
    cache = torch.zeros(f["cache"].shape, dtype=torch.uint8, device=device)
    slots = torch.from_numpy(f["slots"]).to(device)
    pairs = [(_bf16(k).to(device), _bf16(v).to(device)) for k, v in zip(f["keys"], f["values"])]
    rq.quantize(pairs, cache, slots, kr, vr, km, records, "anchor", anchor, "ls")
    assert np.array_equal(cache.cpu().numpy(), f["cache"])
    dim = f["keys"].shape[-1]
    q, k, v = (_bf16(f[n]).to(device) for n in ("query", "key", "value"))
    qsl = torch.from_numpy(f["query_start_loc"]).to(device)
    sl = torch.from_numpy(f["seq_lens"]).to(device)
    table = torch.from_numpy(f["block_table"]).to(device)
    for loop in range(len(records)):
        kk, vv = rq.dequantize(cache, slots, dim, km, records, "anchor", anchor, loop)
        assert np.array_equal(kk.cpu().view(torch.int16).numpy().view(np.uint16), f[f"restored_k{loop}"])
        assert np.array_equal(vv.cpu().view(torch.int16).numpy().view(np.uint16), f[f"restored_v{loop}"])
        out = torch.zeros_like(q)
        rq.attention(q, k, v, cache, out, qsl, sl, table, kr, vr, km, records, "anchor", anchor, loop)
        err = np.abs(out.float().cpu().numpy() - f[f"attention{loop}"])
        assert err.max() <= 2e-2 and err.mean() <= 1e-3, (loop, err.max(), err.mean())
