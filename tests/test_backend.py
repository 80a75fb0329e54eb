"""Batch slicing and call contract of the packed backend without vLLM
(residualquant_amd/backend.py; the reference's PackedBuilder.build and
PackedImpl.forward, src/residual_quantization/packed_backend.py:28-99,
:151-199, :221-223).  Host logic only: no kernel runs here."""

from __future__ import annotations

import pytest
import torch

from residualquant_amd import backend


def _meta(starts, seq_lens, pages=4):
    qsl = torch.tensor(starts, dtype=torch.int32)
    lens = torch.tensor(seq_lens, dtype=torch.int32)
    table = torch.arange(len(seq_lens) * pages, dtype=torch.int32).reshape(len(seq_lens), pages)
    slots = torch.arange(starts[-1] - starts[0], dtype=torch.int64) + 1000
    return backend.build_metadata(qsl, lens, table, slots)


def test_kv_cache_shape_and_name():
    assert backend.kv_cache_shape(7, 16, 4, 200) == (2, 7, 4, 16, 200)
    assert backend.BACKEND_NAME == "LOOP_PACKED_ACCELERATED"


def test_decode_batch_is_one_slice():
    meta = _meta([0, 1, 2, 3], [9, 30, 4])
    assert meta.max_query_len == 1
    assert len(meta.request_metadata) == 1
    begin, end, part = meta.request_metadata[0]
    assert (begin, end) == (0, 3)
    assert part.query_start_loc.tolist() == [0, 1, 2, 3]
    assert part.seq_lens.tolist() == [9, 30, 4]
    assert part.block_table.shape == (3, 4)
    assert part.slot_mapping.tolist() == [1000, 1001, 1002]


def test_mixed_batch_splits_decode_prefix_from_prompts():
    meta = _meta([0, 1, 2, 7, 10], [21, 38, 5, 3])
    assert meta.max_query_len == 5
    (b0, e0, decode), (b1, e1, prompts) = meta.request_metadata
    assert (b0, e0, b1, e1) == (0, 2, 2, 10)
    assert decode.max_query_len == 1 and prompts.max_query_len == 5
    assert decode.query_start_loc.tolist() == [0, 1, 2]
    assert prompts.query_start_loc.tolist() == [0, 5, 8]
    assert decode.seq_lens.tolist() == [21, 38] and prompts.seq_lens.tolist() == [5, 3]
    assert torch.equal(prompts.block_table, meta.block_table[2:4])
    assert prompts.slot_mapping.tolist() == list(range(1002, 1010))


def test_prompts_only_is_one_prompt_slice():
    meta = _meta([0, 4, 10], [4, 6])
    assert len(meta.request_metadata) == 1
    begin, end, part = meta.request_metadata[0]
    assert (begin, end, part.max_query_len) == (0, 10, 6)
    assert part.query_start_loc.tolist() == [0, 4, 10]


def test_chunked_prefill_is_rejected():
    with pytest.raises(ValueError, match="Chunked/recomputed partial prefill is unsupported"):
        _meta([0, 1, 6], [12, 9])


def test_one_token_request_after_a_prompt_is_rejected():
    with pytest.raises(ValueError, match="must precede"):
        _meta([0, 5, 6], [5, 40])


def test_forward_contract_without_kernels():
    meta = _meta([0, 1], [3])
    layer = backend.PackedLayer(group=None, loop_index=0)
    x = torch.zeros((1, 2, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="BF16 output required"):
        backend.forward(layer, x, x, x, None, meta, None)
    with pytest.raises(ValueError, match="BF16 output required"):
        backend.forward(layer, x, x, x, None, meta, x, output_scale=1.0)
    out = torch.ones_like(x)
    assert backend.forward(layer, x, x, x, None, None, out) is out
