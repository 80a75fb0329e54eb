"""Packed attention backend without vLLM: batch slicing and per-call routing.

Restates the vLLM-independent part of the reference backend
(src/residual_quantization/packed_backend.py):

- ``build_metadata`` is ``PackedBuilder.build`` (:151-199): a batch whose
  requests all have one query token is one decode slice; otherwise the
  one-token prefix and the full-prompt suffix become two slices, and a prompt
  whose query length differs from its sequence length (chunked or recomputed
  prefill) is rejected;
- ``forward`` is ``PackedImpl.forward`` (:28-99): the prompt slice runs the
  causal varlen attention over its raw K/V, the decode slice runs the packed
  ``attention`` over the cache with the current token passed live, and then
  ``_store_kv`` (:101-137) hands the layer's K/V to its loop group
  (``DeferredKVGroup.store``), with the offload lookahead prepared before the
  attention calls;
- ``kv_cache_shape`` is ``PackedBackend.get_kv_cache_shape`` (:221-223).

The metadata are plain tensors instead of vLLM's ``CommonAttentionMetadata``,
and the per-layer state (loop group, rotations, key means, loop index) is a
``PackedLayer`` instead of attributes on a vLLM ``Attention`` module
(install_model.py:154-196).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import torch

from . import ops
from .group import DeferredKVGroup

BACKEND_NAME = "LOOP_PACKED_ACCELERATED"  # PackedBackend.get_name (packed_backend.py:205-207)


def kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int) -> Tuple[int, ...]:
    """Cache tensor shape: [K/V, blocks, KV heads, block tokens, page width bytes] (packed_backend.py:221-223)."""
    return (2, num_blocks, num_kv_heads, block_size, head_size)


@dataclass
class PackedMetadata:
    """Attention metadata of one batch (or one slice of it).

    ``query_start_loc`` INT32 [requests + 1] and ``seq_lens`` INT32 [requests]
    (query plus history tokens, as vLLM counts them) and ``block_table`` INT32
    [requests, pages] on the device; ``slot_mapping`` INT64 [tokens];
    ``request_metadata`` the ``(token_begin, token_end, slice)`` list that
    ``forward`` walks."""

    query_start_loc: torch.Tensor
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    max_query_len: int
    request_metadata: List[Tuple[int, int, "PackedMetadata"]] = field(default_factory=list)


def _slice(metadata: PackedMetadata, requests: slice, tokens: slice, query_start_cpu: List[int]) -> PackedMetadata:
    begin = query_start_cpu[requests.start]
    starts = query_start_cpu[requests.start:requests.stop + 1]
    return PackedMetadata(
        query_start_loc=metadata.query_start_loc[requests.start:requests.stop + 1] - begin,
        seq_lens=metadata.seq_lens[requests],
        block_table=metadata.block_table[requests],
        slot_mapping=metadata.slot_mapping[tokens],
        max_query_len=max(b - a for a, b in zip(starts, starts[1:])))


def build_metadata(query_start_loc_cpu: torch.Tensor, seq_lens_cpu: torch.Tensor, block_table: torch.Tensor,
                   slot_mapping: torch.Tensor) -> PackedMetadata:
    """Batch metadata with its decode/prompt slices (``PackedBuilder.build``, packed_backend.py:151-199).

    ``query_start_loc_cpu``/``seq_lens_cpu`` are host INT32 tensors (the
    builder reads them on the host); the device copies go to the block
    table's device.  One-token requests must come first, as vLLM orders them
    (``reorder_batch_threshold = 1``, packed_backend.py:141-142)."""
    device = block_table.device
    starts = [int(v) for v in query_start_loc_cpu.tolist()]
    lengths = [b - a for a, b in zip(starts, starts[1:])]
    requests = len(lengths)
    if seq_lens_cpu.numel() != requests or block_table.size(0) < requests:
        raise ValueError("Query starts, sequence lengths and block table rows must describe the same requests")
    metadata = PackedMetadata(
        query_start_loc=query_start_loc_cpu.to(device=device, dtype=torch.int32),
        seq_lens=seq_lens_cpu.to(device=device, dtype=torch.int32),
        block_table=block_table,
        slot_mapping=slot_mapping,
        max_query_len=max(lengths, default=0))
    tokens = starts[-1] - starts[0] if requests else 0
    if metadata.max_query_len <= 1:
        # Decode: one slice over the whole batch (packed_backend.py:158-163).
        metadata.request_metadata = [(0, tokens, PackedMetadata(
            metadata.query_start_loc, metadata.seq_lens, metadata.block_table, metadata.slot_mapping,
            metadata.max_query_len))]
        return metadata
    seq_lens = [int(v) for v in seq_lens_cpu.tolist()]
    first_prompt = None
    for request, length in enumerate(lengths):
        if length > 1:
            if length != seq_lens[request]:
                raise ValueError("Chunked/recomputed partial prefill is unsupported")
            if first_prompt is None:
                first_prompt = request
        elif first_prompt is not None:
            raise ValueError("One-token requests must precede the full prompts of a batch")
    slices = []
    if first_prompt > 0:
        slices.append((slice(0, first_prompt), slice(0, starts[first_prompt] - starts[0])))
    slices.append((slice(first_prompt, requests), slice(starts[first_prompt] - starts[0], tokens)))
    metadata.request_metadata = [(token_slice.start, token_slice.stop,
                                  _slice(metadata, request_slice, token_slice, starts))
                                 for request_slice, token_slice in slices]
    return metadata


@dataclass
class PackedLayer:
    """What one attention layer passes to the ops: its loop group, its
    rotations and key means (``artifact.SlotTensors``) and its loop position
    within the group (``group_loop_index``, install_model.py:154-196)."""

    group: DeferredKVGroup
    loop_index: int
    key_rotation: Optional[torch.Tensor] = None
    value_rotation: Optional[torch.Tensor] = None
    key_mean: Optional[torch.Tensor] = None


def forward(layer: PackedLayer, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
            kv_cache: torch.Tensor, metadata: Optional[PackedMetadata], output: Optional[torch.Tensor],
            output_scale=None, output_block_scale=None) -> Optional[torch.Tensor]:
    """One layer call (``PackedImpl.forward``, packed_backend.py:28-99).

    query/key/value/output BF16 [tokens, heads, D]; the prompt slice attends
    over its own K/V (causal), the decode slice over the cache plus the
    current token; then the call's K/V are staged in the layer's group, which
    quantizes into ``kv_cache`` on its last loop."""
    if output is None or output_scale is not None or output_block_scale is not None:
        raise ValueError("BF16 output required")
    if metadata is None:
        return output
    group = layer.group
    tokens = metadata.slot_mapping.numel()
    prefill = metadata.max_query_len > 1
    lookahead = group.wants_lookahead(prefill)
    if lookahead:
        group.prefill_offload.prepare(group, tokens)

    for begin, end, part in metadata.request_metadata:
        request_query, request_key = query[begin:end], key[begin:end]
        request_value, request_output = value[begin:end], output[begin:end]
        if part.max_query_len > 1:
            ops.flash_attn_varlen_func(
                q=request_query, k=request_key, v=request_value, out=request_output,
                cu_seqlens_q=part.query_start_loc, cu_seqlens_k=part.query_start_loc,
                max_seqlen_q=part.max_query_len, max_seqlen_k=part.max_query_len,
                softmax_scale=query.shape[-1] ** -0.5, causal=True)
        else:
            ops.attention(request_query, request_key, request_value, kv_cache, request_output,
                          part.query_start_loc, part.seq_lens, part.block_table, layer.key_rotation,
                          layer.value_rotation, layer.key_mean, group.records, group.reference_mode,
                          group.anchor_index, layer.loop_index)

    group.store(key, value, kv_cache, metadata.slot_mapping, layer.key_rotation, layer.value_rotation,
                layer.key_mean, prefill=prefill, lookahead=lookahead)
    return output
