"""Pinned-host spill of a loop group's pending prefill K/V.

A loop group keeps the raw K/V of its earlier loops until its last loop
quantizes every record.  For long prompts those pending loops can wait in
pinned host memory instead of HBM.  The contract with the write path is the
one of the reference's optional offload (used from packed_backend.py:47-55,
:101-137 and install_model.py:40-91): ``store`` one loop's K/V,
``reserve`` device buffers before the KV pool is sized, ``preload`` and
``prepare`` a lookahead ring of 2-8 whole-layer slots within 800 MiB
(prefill_offload.py:5-7), and ``chunks`` hands the completing call its
records on the device.  The buffering below is this module's own:

- Two copy streams of default priority: ``spill_stream`` carries every
  device-to-host copy and ``recall_stream`` every host-to-device copy, so a
  spill of one layer and a recall of another use both directions of the host
  link at once.
- Every copy moves one contiguous row range of one plane (a strided pinned
  source would make torch stage it through pageable memory).
- Every pinned block is a ``HostSpill`` that carries its own two fences:
  ``written`` (its spill has landed) and ``read`` (the last recall out of it
  has finished).  A recall waits on ``written``; a new spill into the block
  waits on ``read``.  Nothing else orders the two streams.
- Device buffers are ``_SlotRing`` objects: slots handed out from a free
  list, each with a ``filled`` event for its consumer and a release fence
  that the next producer waits on.  The same ring type serves the two-slot
  spill staging (a store never waits for the previous store's spill), the
  two recall windows of chunked completion, and the lookahead ring of
  layer slots.
- Lookahead recalls groups strictly in their chain order (a group's
  position among the groups of one loop position across layers), into
  whichever layer slot is free, never waiting for one; a group that finds no
  slot completes through the recall windows instead.
"""

from __future__ import annotations

from typing import Dict, Iterator, List, Optional, Sequence, Tuple

import torch

Pair = Tuple[torch.Tensor, torch.Tensor]

# Lookahead ring: as many whole-layer slots as fit in the byte budget,
# within [2, 8] (the reference's budget, prefill_offload.py:5-7).
RING_MIN_LAYERS = 2
RING_MAX_LAYERS = 8
RING_TARGET_BYTES = 800 * 1024**2

STAGING_SLOTS = 2
RECALL_WINDOWS = 2


class HostSpill:
    """Pinned [2, capacity, heads, D] block for one pending loop's K and V."""

    def __init__(self, capacity: int, heads: int, head_dim: int, dtype: torch.dtype):
        self.block = torch.empty((2, capacity, heads, head_dim), dtype=dtype, device="cpu", pin_memory=True)
        self.written = torch.cuda.Event()
        self.read: Optional[torch.cuda.Event] = None
        self.rows = 0

    @property
    def capacity(self) -> int:
        return self.block.size(1)

    def views(self) -> Pair:
        return self.block[0, :self.rows], self.block[1, :self.rows]


class _SlotRing:
    """Device slots of one shape, handed out in FIFO order from a free list."""

    def __init__(self, slots: int, shape: Tuple[int, ...], dtype: torch.dtype, streams: Sequence):
        self.buffer = torch.empty((slots, *shape), dtype=dtype, device="cuda")
        for stream in streams:
            self.buffer.record_stream(stream)
        self.filled = [torch.cuda.Event() for _ in range(slots)]
        self.released: List[Optional[torch.cuda.Event]] = [None] * slots
        self.free = list(range(slots))

    @property
    def slots(self) -> int:
        return self.buffer.size(0)

    def fits(self, shape: Tuple[int, ...]) -> bool:
        return all(have >= want for have, want in zip(self.buffer.shape[1:], shape))

    def acquire(self, producer) -> int:
        """Take the oldest free slot; ``producer`` waits until its last consumer released it."""
        slot = self.free.pop(0)
        if self.released[slot] is not None:
            producer.wait_event(self.released[slot])
        return slot

    def give_back(self, slot: int, consumer) -> None:
        """Return ``slot`` once the work ``consumer`` has enqueued on it is done."""
        fence = torch.cuda.Event()
        fence.record(consumer)
        self.released[slot] = fence
        self.free.append(slot)


class PrefillCPUOffload:
    """Pending-loop K/V in pinned host memory, recalled in windows or ahead by layer.

    ``chunk_tokens``: tokens per recall window; ``pending_records``: the most
    pending loops a group keeps (records - 1); ``heads``/``head_dim``: the
    K/V row shape."""

    def __init__(self, chunk_tokens: int, pending_records: int, heads: int, head_dim: int):
        if chunk_tokens <= 0:
            raise ValueError("prefill_offload_chunk_tokens must be a positive integer")
        self.chunk_tokens = chunk_tokens
        self.pending_records = pending_records
        self.heads, self.head_dim = heads, head_dim
        self.dtype = torch.bfloat16
        self.lookahead_enabled = True
        self.spill_stream = torch.cuda.Stream()
        self.recall_stream = torch.cuda.Stream()
        streams = (self.spill_stream, self.recall_stream)
        # Recall windows exist from the start, so a memory profile taken
        # before the KV pool is sized sees them.
        self.windows = _SlotRing(RECALL_WINDOWS, (pending_records, 2, chunk_tokens, heads, head_dim), self.dtype,
                                 streams)
        self.staging: Optional[_SlotRing] = None
        self.layers: Optional[_SlotRing] = None
        # Groups whose pending records are in a layer slot (or on their way).
        self.prefetched: Dict[object, int] = {}
        self._spills: Dict[int, HostSpill] = {}

    # ---------------------------------------------------------------- buffers

    def _ring(self, slots: int, shape: Tuple[int, ...]) -> _SlotRing:
        return _SlotRing(slots, shape, self.dtype, (self.spill_stream, self.recall_stream))

    def _layer_slots(self, tokens: int, records: int) -> int:
        layer_bytes = max(1, records * 2 * tokens * self.heads * self.head_dim * 2)
        return max(RING_MIN_LAYERS, min(RING_MAX_LAYERS, RING_TARGET_BYTES // layer_bytes))

    def _ensure_staging(self, tokens: int) -> None:
        shape = (2, tokens, self.heads, self.head_dim)
        if self.staging is None or not self.staging.fits(shape):
            self.staging = self._ring(STAGING_SLOTS, shape)

    def _ensure_layers(self, tokens: int, records: int) -> bool:
        """Layer ring for ``records`` x ``tokens``; replaced only while no group holds a slot."""
        shape = (max(records, 1), 2, tokens, self.heads, self.head_dim)
        if self.layers is not None and self.layers.fits(shape):
            return True
        if self.prefetched:
            return False
        self.layers = self._ring(self._layer_slots(tokens, max(records, 1)), shape)
        return True

    def reserve(self, tokens: int) -> None:
        """Allocate the spill staging (and the lookahead ring) for prompts of up to ``tokens`` tokens."""
        self._ensure_staging(tokens)
        if self.lookahead_enabled:
            self._ensure_layers(tokens, self.pending_records)

    # ---------------------------------------------------------------- spill (D2H)

    def store(self, key: torch.Tensor, value: torch.Tensor, spill: Optional[HostSpill]) -> HostSpill:
        """Spill one loop's K/V [tokens, heads, D] to pinned host memory.

        ``spill`` is the block this pending position used before (reused when
        large enough).  The caller may overwrite ``key``/``value`` as soon as
        this returns: they are copied to a staging slot on its stream first."""
        tokens = key.size(0)
        if spill is None or spill.capacity < tokens:
            if spill is not None:
                self._spills.pop(spill.block.untyped_storage().data_ptr(), None)
            spill = HostSpill(tokens, self.heads, self.head_dim, key.dtype)
            self._spills[spill.block.untyped_storage().data_ptr()] = spill
        current = torch.cuda.current_stream()
        self._ensure_staging(tokens)
        staging = self.staging
        slot = staging.acquire(current)
        staged = staging.buffer[slot]
        staged[0, :tokens].copy_(key)
        staged[1, :tokens].copy_(value)
        staging.filled[slot].record(current)
        with torch.cuda.stream(self.spill_stream):
            self.spill_stream.wait_event(staging.filled[slot])
            if spill.read is not None:
                self.spill_stream.wait_event(spill.read)
            for plane in range(2):  # contiguous rows of each plane
                spill.block[plane, :tokens].copy_(staged[plane, :tokens], non_blocking=True)
            spill.written.record(self.spill_stream)
        staging.give_back(slot, self.spill_stream)
        spill.rows = tokens
        return spill

    def _spill_of(self, tensor: torch.Tensor) -> HostSpill:
        return self._spills[tensor.untyped_storage().data_ptr()]

    # ---------------------------------------------------------------- recall (H2D)

    def _recall_group(self, group, tokens: int) -> bool:
        """Start the recall of ``group``'s pending records into a free layer slot."""
        if group in self.prefetched:
            return True
        if self.layers is None or not self.layers.free or any(key.is_cuda for key, _ in group.pending):
            return False
        ring = self.layers
        stream = self.recall_stream
        slot = ring.acquire(stream)
        spills = [self._spill_of(key) for key, _ in group.pending]
        with torch.cuda.stream(stream):
            for i, spill in enumerate(spills):
                stream.wait_event(spill.written)
                for plane in range(2):
                    ring.buffer[slot, i, plane, :tokens].copy_(spill.block[plane, :tokens], non_blocking=True)
            ring.filled[slot].record(stream)
        self._mark_read(spills, stream)
        self.prefetched[group] = slot
        return True

    @staticmethod
    def _mark_read(spills: Sequence[HostSpill], stream) -> None:
        fence = torch.cuda.Event()
        fence.record(stream)
        for spill in spills:
            spill.read = fence

    def _recall_in_order(self, chain: Sequence, start: int, tokens: int, pending: int) -> None:
        """Recall the groups of ``chain`` from ``start`` on whose pending loops are all spilled,
        in chain order, while layer slots are free."""
        for group in chain[start:]:
            if len(group.pending) != pending or not self._recall_group(group, tokens):
                return

    def preload(self, group, tokens: int) -> None:
        """After ``group`` spilled its last pending loop: recall it now if a layer slot is free."""
        if not self._ensure_layers(tokens, len(group.pending)):
            return
        chain = group.offload_chain or [group]
        position = group.offload_index if group.offload_chain else 0
        earlier = chain[:position]
        if all(g in self.prefetched or len(g.pending) != len(group.pending) for g in earlier):
            self._recall_group(group, tokens)

    def prepare(self, group, tokens: int) -> None:
        """Before ``group``'s completing call: recall it and the groups after it in its chain."""
        if not self._ensure_layers(tokens, len(group.pending)):
            return
        if group.offload_chain:
            self._recall_in_order(group.offload_chain, group.offload_index, tokens, len(group.pending))
        else:
            self._recall_group(group, tokens)

    def chunks(self, records: Sequence[Pair], slot_mapping: torch.Tensor,
               group=None) -> Iterator[Tuple[List[Pair], torch.Tensor]]:
        """Yield ``(records, slots)`` pieces of a completing call with the pending
        (host) records on the device.  The caller enqueues its quantize of a
        piece before asking for the next one."""
        current = torch.cuda.current_stream()
        total = slot_mapping.numel()
        pending = len(records) - 1
        if group is not None and group in self.prefetched:
            slot = self.prefetched.pop(group)
            ring = self.layers
            current.wait_event(ring.filled[slot])
            recalled = [(ring.buffer[slot, i, 0, :total], ring.buffer[slot, i, 1, :total]) for i in range(pending)]
            yield recalled + [records[-1]], slot_mapping
            ring.give_back(slot, current)
            return

        spills = [self._spill_of(key) for key, _ in records[:-1]]
        windows = self.windows
        stream = self.recall_stream
        starts = list(range(0, total, self.chunk_tokens))

        def fill(begin: int) -> int:
            end = min(begin + self.chunk_tokens, total)
            slot = windows.acquire(stream)
            with torch.cuda.stream(stream):
                for i, spill in enumerate(spills):
                    stream.wait_event(spill.written)
                    for plane in range(2):
                        windows.buffer[slot, i, plane, :end - begin].copy_(spill.block[plane, begin:end],
                                                                          non_blocking=True)
                windows.filled[slot].record(stream)
            if end == total:
                self._mark_read(spills, stream)
            return slot

        in_flight = [fill(starts[0])] if starts else []
        try:
            for n, begin in enumerate(starts):
                end = min(begin + self.chunk_tokens, total)
                slot = in_flight[0]
                if n + 1 < len(starts):
                    in_flight.append(fill(starts[n + 1]))
                current.wait_event(windows.filled[slot])
                piece = [(windows.buffer[slot, i, 0, :end - begin], windows.buffer[slot, i, 1, :end - begin])
                         for i in range(pending)]
                key, value = records[-1]
                yield piece + [(key[begin:end], value[begin:end])], slot_mapping[begin:end]
                windows.give_back(in_flight.pop(0), current)
        finally:
            # A consumer that stops early still returns the windows it holds.
            for slot in in_flight:
                windows.give_back(slot, current)
