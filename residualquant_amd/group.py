"""Quantize-on-write of one loop group.

A loop group is the set of loops whose K/V share one packed record set in
the cache.  Its earlier loops cannot be quantized alone (their residuals and
coefficients depend on the anchor loop), so each earlier loop's K/V is held
back until the group's last loop arrives, and that call quantizes every
record in one launch.  The write path's order is the reference's
(``DeferredKVGroup``, src/residual_quantization/install_model.py:17-52;
``PackedImpl._store_kv``, src/residual_quantization/packed_backend.py:101-137).
During prefill the held-back loops may wait in pinned host memory through a
``PrefillCPUOffload`` (prefill_offload.py) and come back in pieces or ahead
of time.
"""

from __future__ import annotations

from typing import Iterable, List, Optional, Sequence, Tuple

import torch

from . import ops
from .layout import page_width as _page_width

Pair = Tuple[torch.Tensor, torch.Tensor]

_MODES = ("anchor", "adjacent")
_COEFFICIENTS = ("unit", "norm", "ls")


class DeferredKVGroup:
    """Packed record schedule of one loop group plus the K/V held back for it.

    ``config`` holds ``reference_mode``, ``anchor_index`` and
    ``coefficient_method``; ``records`` is the (bits, group) schedule in loop
    order.  ``pending`` holds one (K, V) pair per loop seen since the group
    last completed (device copies, or pinned host views when spilled)."""

    def __init__(self, config: dict, records: Sequence[Sequence[int]], page_tokens: int, prefill_offload=None):
        self.records = tuple(tuple(int(v) for v in record) for record in records)
        if not self.records:
            raise ValueError("Every packed group must contain at least one record")
        self.reference_mode = config["reference_mode"]
        self.anchor_index = config["anchor_index"]
        self.coefficient_method = config["coefficient_method"]
        if self.reference_mode not in _MODES:
            raise ValueError("Unsupported reference")
        if self.reference_mode == "adjacent" and self.anchor_index != 0:
            raise ValueError("Adjacent reference currently requires anchor_index=0")
        if self.coefficient_method not in _COEFFICIENTS:
            raise ValueError("Unsupported coefficient method")
        self.page_tokens = page_tokens
        self.prefill_offload = prefill_offload
        self.pending: List[Pair] = []
        # One pinned spill block per held-back position, reused across prompts.
        self.host_spills: list = [None] * (len(self.records) - 1)
        # Lookahead order: the groups of this loop position across layers
        # and this group's index in that list (install_model.py:174-178).
        self.offload_chain: list = []
        self.offload_index = 0

    def page_width(self, head_dim: int) -> int:
        return _page_width(head_dim, self.records)

    @property
    def completes_next(self) -> bool:
        """Whether the next loop to arrive is the group's last."""
        return len(self.pending) == len(self.records) - 1

    def _hold(self, key: torch.Tensor, value: torch.Tensor, spill: bool) -> Pair:
        if not spill:
            return key.clone(), value.clone()
        position = len(self.pending)
        block = self.prefill_offload.store(key, value, self.host_spills[position])
        self.host_spills[position] = block
        return block.views()

    def stage(self, key: torch.Tensor, value: torch.Tensor, offload: bool = False) -> Optional[List[Pair]]:
        """Take one loop's K/V.  Returns every record of the group (loop order)
        when this loop completes it, the last one being the caller's own
        tensors; otherwise holds a copy (in pinned host memory with
        ``offload``) and returns None."""
        if not self.completes_next:
            self.pending.append(self._hold(key, value, offload))
            return None
        complete, self.pending = self.pending + [(key, value)], []
        return complete

    def wants_lookahead(self, prefill: bool) -> bool:
        """Whether this call completes the group from the lookahead ring
        (the ``lookahead`` flag of packed_backend.py:47-54)."""
        offload = self.prefill_offload
        return (offload is not None and offload.lookahead_enabled and prefill and len(self.records) > 1
                and self.completes_next)

    def _pieces(self, records: List[Pair], slot_mapping: torch.Tensor, spilled: bool,
                lookahead: bool) -> Iterable[Tuple[List[Pair], torch.Tensor]]:
        """The (records, slots) pieces to quantize for a completing call."""
        if not spilled or len(records) == 1:
            return ((records, slot_mapping),)
        return self.prefill_offload.chunks(records, slot_mapping, group=self if lookahead else None)

    def store(self, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
              slot_mapping: torch.Tensor, key_rotation: Optional[torch.Tensor],
              value_rotation: Optional[torch.Tensor], key_mean: Optional[torch.Tensor],
              prefill: bool = False, lookahead: Optional[bool] = None) -> bool:
        """Write one loop's K/V; on the group's last loop quantize every record
        into ``kv_cache``.  Returns whether this call completed the group.

        ``prefill`` marks a call with more than one query token per request,
        the only calls that spill (packed_backend.py:47).  A caller that
        already asked ``wants_lookahead`` and called the offload's ``prepare``
        before its attention passes that answer as ``lookahead``."""
        tokens = slot_mapping.numel()
        spill = self.prefill_offload is not None and prefill
        if lookahead is None:
            lookahead = self.wants_lookahead(prefill)
            if lookahead:
                self.prefill_offload.prepare(self, tokens)
        records = self.stage(key[:tokens], value[:tokens], offload=spill)
        if records is None:
            # The last held-back loop just went to the host: its recall can
            # start while the remaining layers of this loop run.
            if spill and self.completes_next and self.prefill_offload.lookahead_enabled:
                self.prefill_offload.preload(self, tokens)
            return False
        spilled = spill and all(not k.is_cuda for k, _ in records[:-1])
        for piece, piece_slots in self._pieces(records, slot_mapping, spilled, lookahead):
            ops.quantize(piece, kv_cache, piece_slots, key_rotation, value_rotation, key_mean, self.records,
                         self.reference_mode, self.anchor_index, self.coefficient_method)
        return True
