"""Write the committed golden fixtures (seeded inputs + CPU-oracle outputs).

    python tests/golden/make_golden.py

Each fixture holds one loop group quantized into a small paged cache and one
decode batch over it: BF16 inputs as uint16 bit patterns, FP16 rotations,
FP32 means, slot mapping, the expected packed cache bytes, the restored K/V
of every loop and the FP64 attention output of every loop.  The reference
implementation cannot run here (CUDA + vLLM), so the expected values come
from the CPU oracle; tests/test_golden.py checks that the oracle still
reproduces them and that the HIP kernels match them.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle  # noqa: E402
from residualquant_amd import workloads  # noqa: E402
from tests.cases import OURO_G16, OURO_G32, make_decode, oracle_attention  # noqa: E402

CASES = {
    # name: (lengths, heads, dim, records, page_tokens, rotation, mean, seed)
    "ouro_g32_pt16": ([29, 18, 1], 2, 128, OURO_G32, 16, True, True, 1001),
    "ouro_g16_pt32": ([40, 7], 2, 128, OURO_G16, 32, True, False, 1002),
    "huginn_d96_g16": ([21, 12], 3, 96, OURO_G16, 16, True, True, 1003),
}


def build(name):
    lengths, heads, dim, records, pt, rotation, mean, seed = CASES[name]
    d = make_decode(lengths, heads, dim, records, seed=seed, page_tokens=pt, rotation=rotation, mean=mean)
    g = d.group
    cache = g.oracle_cache(oracle)
    bits = workloads.bf16_bits
    out = {
        "records": np.array(records, dtype=np.int32),
        "page_tokens": np.int32(pt), "anchor": np.int32(g.anchor),
        "keys": np.stack([bits(k) for k, _ in g.pairs]), "values": np.stack([bits(v) for _, v in g.pairs]),
        "slots": g.slots.numpy(), "num_blocks": np.int32(g.num_blocks),
        "cache": cache,
        "query": bits(d.query), "key": bits(d.key), "value": bits(d.value),
        "query_start_loc": d.query_start_loc.numpy(), "seq_lens": d.seq_lens.numpy(), "block_table": d.table.numpy(),
    }
    if g.key_rotation is not None:
        out["key_rotation"] = bits(g.key_rotation)
        out["value_rotation"] = bits(g.value_rotation)
    if g.key_mean is not None:
        out["key_mean"] = g.key_mean.numpy()
    for loop in range(len(records)):
        k, v = oracle.dequantize(cache, g.slots.numpy(), dim, out.get("key_mean"), records, "anchor", g.anchor, loop)
        out[f"restored_k{loop}"], out[f"restored_v{loop}"] = k, v
        out[f"attention{loop}"] = oracle_attention(oracle, d, cache, loop)
    return out


def main():
    for name in CASES:
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **build(name))
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
