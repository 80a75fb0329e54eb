"""Pinned-host storage of a loop group's pending prefill K/V.

During prefill a loop group keeps the raw K/V of its earlier loops until its
last loop quantizes the whole group.  For long prompts that raw K/V can move
to pinned host memory and come back just in time, as the reference's optional
offload does (src/residual_quantization/prefill_offload.py:10-200, driven by
packed_backend.py:47-55, :101-137 and install_model.py:55-91):

- ``store`` copies a loop's K/V into a device staging buffer on the caller's
  stream, then to a pinned host buffer on a side stream (D2H);
- the completing call gets the pending records back either in chunks of
  ``chunk_tokens`` through a two-slot device ring (H2D of chunk i + 1 runs
  while chunk i is quantized), or, with lookahead, whole from a ring of
  layer-sized device slots that ``preload``/``prepare`` fill while earlier
  layers compute.

All copies run on side streams of default priority; every hand-off between
the caller's stream and a side stream is an event, never a device-wide sync.
The D2H copies and the chunked H2D copies share one stream, so a pinned
buffer is never rewritten while a copy out of it is pending.  Pinned buffers
are allocated pinned (``pin_memory=True``).
"""

from __future__ import annotations

from typing import Dict, Iterator, List, Optional, Sequence, Tuple

import torch

Pair = Tuple[torch.Tensor, torch.Tensor]

# Lookahead ring: whole-layer slots, as many as fit in the target bytes,
# within [2, 8] (prefill_offload.py:5-7).
RING_MIN_LAYERS = 2
RING_MAX_LAYERS = 8
RING_TARGET_BYTES = 800 * 1024**2


class PrefillCPUOffload:
    """Pending-loop K/V on pinned host memory with overlapped transfers.

    ``chunk_tokens`` tokens per H2D chunk; ``pending_records`` the most raw
    loops any group keeps (records - 1); ``heads``/``head_dim`` the K/V shape."""

    def __init__(self, chunk_tokens: int, pending_records: int, heads: int, head_dim: int):
        if chunk_tokens <= 0:
            raise ValueError("prefill_offload_chunk_tokens must be a positive integer")
        self.chunk_tokens = chunk_tokens
        self.heads, self.head_dim = heads, head_dim
        self.lookahead_enabled = True
        self.copy_stream = torch.cuda.Stream()
        self.ring_stream = torch.cuda.Stream()
        # D2H: the device staging copy of the latest stored loop, and the
        # event after its copy to the host.
        self.staging: Optional[torch.Tensor] = None
        self._staged = torch.cuda.Event()
        self._stored = torch.cuda.Event()
        self._store_pending = False
        # Two chunk slots [slot, record, K/V, token, head, channel], allocated
        # up front so a memory profile taken before the KV pool sees them.
        self.chunk_ring = torch.empty((2, pending_records, 2, chunk_tokens, heads, head_dim), dtype=torch.bfloat16,
                                      device="cuda")
        # Lookahead ring of layer slots [slot, record, K/V, token, head, channel].
        self.ring: Optional[torch.Tensor] = None
        self.ring_slots = RING_MAX_LAYERS
        self.ring_ready = [torch.cuda.Event() for _ in range(RING_MAX_LAYERS)]
        self.ring_free = [torch.cuda.Event() for _ in range(RING_MAX_LAYERS)]
        self.ring_used = [False] * RING_MAX_LAYERS
        self.prefetched: Dict[object, int] = {}

    # ---------------------------------------------------------------- memory

    def reserve(self, tokens: int) -> None:
        """Allocate the staging buffer (and the lookahead ring) for up to ``tokens`` tokens."""
        pending = self.chunk_ring.size(1)
        self._grow_staging(tokens)
        if self.lookahead_enabled:
            self._allocate_ring(tokens, pending)

    def _grow_staging(self, tokens: int) -> None:
        if self.staging is None or self.staging.size(1) < tokens:
            self.staging = torch.empty((2, tokens, self.heads, self.head_dim), dtype=torch.bfloat16, device="cuda")
            self.staging.record_stream(self.copy_stream)

    def _allocate_ring(self, tokens: int, records: int) -> None:
        layer_bytes = records * 2 * tokens * self.heads * self.head_dim * 2
        self.ring_slots = max(RING_MIN_LAYERS, min(RING_MAX_LAYERS, RING_TARGET_BYTES // max(layer_bytes, 1)))
        self.ring = torch.empty((self.ring_slots, records, 2, tokens, self.heads, self.head_dim),
                                dtype=torch.bfloat16, device="cuda")
        self.ring.record_stream(self.ring_stream)
        self.ring_used = [False] * RING_MAX_LAYERS

    # ---------------------------------------------------------------- D2H

    def store(self, key: torch.Tensor, value: torch.Tensor, buffer: Optional[torch.Tensor]) -> torch.Tensor:
        """Copy one loop's K/V [tokens, heads, D] to pinned host memory.

        Reuses ``buffer`` (pinned [2, >= tokens, heads, D]) when large enough.
        Returns the buffer; its rows are complete once the copy stream has
        passed this call's D2H (later reads are ordered after it)."""
        tokens = key.size(0)
        if buffer is None or buffer.size(1) < tokens:
            buffer = torch.empty((2, tokens, self.heads, self.head_dim), dtype=key.dtype, device="cpu",
                                 pin_memory=True)
        current = torch.cuda.current_stream()
        if self._store_pending:
            current.wait_event(self._stored)  # the staging buffer is free again
        self._grow_staging(tokens)
        self.staging[0, :tokens].copy_(key)
        self.staging[1, :tokens].copy_(value)
        self._staged.record(current)
        with torch.cuda.stream(self.copy_stream):
            self.copy_stream.wait_event(self._staged)
            buffer[0, :tokens].copy_(self.staging[0, :tokens], non_blocking=True)
            buffer[1, :tokens].copy_(self.staging[1, :tokens], non_blocking=True)
            self._stored.record(self.copy_stream)
        self._store_pending = True
        return buffer

    # ---------------------------------------------------------------- lookahead

    def _ensure_ring(self, group, tokens: int) -> None:
        records = len(group.pending)
        if self.ring is None or self.ring.size(3) < tokens or self.ring.size(1) < records:
            self._allocate_ring(tokens, records)

    def _prefetch(self, group, tokens: int) -> None:
        if group in self.prefetched:
            return
        slot = group.offload_index % self.ring_slots
        self.ring_stream.wait_stream(torch.cuda.current_stream())
        if self._store_pending:
            self.ring_stream.wait_event(self._stored)  # the host rows are written
        with torch.cuda.stream(self.ring_stream):
            if self.ring_used[slot]:
                self.ring_stream.wait_event(self.ring_free[slot])
            for i, (key, value) in enumerate(group.pending):
                self.ring[slot, i, 0, :tokens].copy_(key[:tokens], non_blocking=True)
                self.ring[slot, i, 1, :tokens].copy_(value[:tokens], non_blocking=True)
            self.ring_ready[slot].record(self.ring_stream)
        self.prefetched[group] = slot

    def preload(self, group, tokens: int) -> None:
        """Start the H2D of the first ring layers during the loop before their completing call."""
        if group.offload_index == 0:
            self.prefetched.clear()
        self._ensure_ring(group, tokens)
        if group.offload_index < self.ring_slots:
            self._prefetch(group, tokens)

    def prepare(self, group, tokens: int) -> None:
        """Before ``group``'s completing call: fill the ring for it and the next layers."""
        if group.offload_index == 0 and group not in self.prefetched:
            self.prefetched.clear()
        self._ensure_ring(group, tokens)
        count = len(group.pending)
        start = group.offload_index
        for future in group.offload_chain[start:start + self.ring_slots]:
            if len(future.pending) == count:
                self._prefetch(future, tokens)

    # ---------------------------------------------------------------- H2D

    def chunks(self, records: Sequence[Pair], slot_mapping: torch.Tensor,
               group=None) -> Iterator[Tuple[List[Pair], torch.Tensor]]:
        """Yield ``(records, slots)`` pieces of a completing call with the pending
        (host) records on the device.  The caller enqueues its quantize of a
        piece before asking for the next one."""
        current = torch.cuda.current_stream()
        if group is not None and group in self.prefetched:
            slot = self.prefetched.pop(group)
            current.wait_event(self.ring_ready[slot])
            tokens = slot_mapping.numel()
            staged = [(self.ring[slot, i, 0, :tokens], self.ring[slot, i, 1, :tokens])
                      for i in range(len(records) - 1)]
            staged.append(records[-1])
            yield staged, slot_mapping
            self.ring_free[slot].record(current)
            self.ring_used[slot] = True
            return

        # Two chunk slots: the H2D of the next chunk overlaps the caller's work
        # on this one.  The copy stream first waits for the caller's stream, so
        # a previous group's use of the slots has finished.
        self.copy_stream.wait_stream(current)
        total = slot_mapping.numel()
        ready = [torch.cuda.Event(), torch.cuda.Event()]
        free = [torch.cuda.Event(), torch.cuda.Event()]
        used = [False, False]

        def fill(begin: int, slot: int) -> None:
            end = min(begin + self.chunk_tokens, total)
            with torch.cuda.stream(self.copy_stream):
                if used[slot]:
                    self.copy_stream.wait_event(free[slot])
                for i, (key, value) in enumerate(records[:-1]):
                    self.chunk_ring[slot, i, 0, :end - begin].copy_(key[begin:end], non_blocking=True)
                    self.chunk_ring[slot, i, 1, :end - begin].copy_(value[begin:end], non_blocking=True)
                ready[slot].record(self.copy_stream)

        if total:
            fill(0, 0)
        for step, begin in enumerate(range(0, total, self.chunk_tokens)):
            slot = step & 1
            end = min(begin + self.chunk_tokens, total)
            current.wait_event(ready[slot])
            if end < total:
                fill(end, slot ^ 1)
            staged = [(self.chunk_ring[slot, i, 0, :end - begin], self.chunk_ring[slot, i, 1, :end - begin])
                      for i in range(len(records) - 1)]
            key, value = records[-1]
            staged.append((key[begin:end], value[begin:end]))
            yield staged, slot_mapping[begin:end]
            free[slot].record(current)
            used[slot] = True
