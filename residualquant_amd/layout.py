"""Packed page layout on the host (no device code).

A page of one (plane, block, head) holds ``page_tokens`` rows of
``page_width`` bytes; records follow loop order and each record region is
[codes | FP8 scales | FP8 offsets | BF16 alpha] (common/cache.cuh:10-106,
quantize/kernel.cuh:205-227).
"""

from __future__ import annotations

from typing import Sequence


def record_bytes(head_dim: int, bits: int, group: int) -> int:
    """Bytes per token of one record (QuantizationRecord::Bytes, common/cache.cuh:14-17)."""
    return head_dim * bits // 8 + 2 * head_dim // group + 2


def page_width(head_dim: int, records: Sequence[Sequence[int]]) -> int:
    """Bytes per token row of a page (DeferredKVGroup.page_width, install_model.py:34-38)."""
    if head_dim <= 0 or head_dim % 32:
        raise ValueError("Head dimension must be a positive multiple of 32")
    for bits, group in records:
        if bits not in (2, 4) or group <= 0 or head_dim % group:
            raise ValueError("Head dimension must be divisible by every quantization group size")
    return sum(record_bytes(head_dim, bits, group) for bits, group in records)


def record_offsets(head_dim: int, records: Sequence[Sequence[int]], page_tokens: int):
    """Byte offset of each record region from the page base (PT * StorageOffset)."""
    offsets, running = [], 0
    for bits, group in records:
        offsets.append(page_tokens * running)
        running += record_bytes(head_dim, bits, group)
    return offsets


def staged_bytes(head_dim: int, records: Sequence[Sequence[int]], page_tokens: int,
                 reference_mode: str, anchor_index: int, loop_index: int) -> int:
    """Bytes of one K or V page a decode call must read (async_copy.cuh:24-42).

    Anchor mode: the anchor record without its alpha, plus the current
    residual record when the loop is not the anchor.  Adjacent mode: every
    record up to and including the current loop.
    """
    if reference_mode == "adjacent" and len(records) > 1:
        return page_tokens * sum(record_bytes(head_dim, *records[r]) for r in range(loop_index + 1))
    anchor = page_tokens * (record_bytes(head_dim, *records[anchor_index]) - 2)
    if loop_index == anchor_index:
        return anchor
    return anchor + page_tokens * record_bytes(head_dim, *records[loop_index])
