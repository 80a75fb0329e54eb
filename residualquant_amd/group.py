"""Write-path orchestration of one loop group (quantize-on-write).

Restates ``DeferredKVGroup`` (src/residual_quantization/install_model.py:17-52)
and the ``_store_kv`` call order of ``PackedImpl``
(src/residual_quantization/packed_backend.py:101-137): raw K/V of the group's
earlier loops is kept (cloned) until its last loop runs, and that call hands
every record to ``quantize`` at once.  With a ``PrefillCPUOffload``
(prefill_offload.py) the earlier loops of a prefill call can wait in pinned
host memory instead (install_model.py:40-52, packed_backend.py:47-55,
:101-137).
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from . import ops
from .layout import page_width as _page_width


class DeferredKVGroup:
    """Own the packed format and keep raw KV until every group loop completes."""

    def __init__(self, config: dict, records: Sequence[Sequence[int]], page_tokens: int, prefill_offload=None):
        self.pending: List[Tuple[torch.Tensor, torch.Tensor]] = []
        self.records = tuple(tuple(int(v) for v in record) for record in records)
        self.page_tokens = page_tokens
        self.prefill_offload = prefill_offload
        self.host_buffers: List[Optional[torch.Tensor]] = [None] * (len(self.records) - 1)
        # Lookahead order: this group's position among the groups of its loop
        # position across layers, and that list (install_model.py:174-178).
        self.offload_chain: list = []
        self.offload_index = 0
        self.reference_mode = config["reference_mode"]
        self.anchor_index = config["anchor_index"]
        self.coefficient_method = config["coefficient_method"]
        if self.reference_mode not in ("adjacent", "anchor"):
            raise ValueError("Unsupported reference")
        if self.reference_mode == "adjacent" and self.anchor_index != 0:
            raise ValueError("Adjacent reference currently requires anchor_index=0")
        if self.coefficient_method not in ("unit", "norm", "ls"):
            raise ValueError("Unsupported coefficient method")
        if not self.records:
            raise ValueError("Every packed group must contain at least one record")

    def page_width(self, head_dim: int) -> int:
        return _page_width(head_dim, self.records)

    def stage(self, key: torch.Tensor, value: torch.Tensor, offload: bool = False):
        """Return all records when this call completes the group, else keep a
        copy (on the device, or with ``offload`` in pinned host memory)."""
        if len(self.pending) + 1 == len(self.records):
            records = self.pending + [(key, value)]
            self.pending = []
            return records
        if offload:
            index = len(self.pending)
            buffer = self.prefill_offload.store(key, value, self.host_buffers[index])
            self.host_buffers[index] = buffer
            self.pending.append((buffer[0, :key.size(0)], buffer[1, :value.size(0)]))
        else:
            self.pending.append((key.clone(), value.clone()))
        return None

    def wants_lookahead(self, prefill: bool) -> bool:
        """Whether this call completes the group from the lookahead ring
        (the ``lookahead`` flag of packed_backend.py:47-54)."""
        return (self.prefill_offload is not None and prefill and len(self.records) > 1
                and len(self.pending) + 1 == len(self.records) and self.prefill_offload.lookahead_enabled)

    def store(self, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
              slot_mapping: torch.Tensor, key_rotation: Optional[torch.Tensor],
              value_rotation: Optional[torch.Tensor], key_mean: Optional[torch.Tensor],
              prefill: bool = False, lookahead: Optional[bool] = None) -> bool:
        """One loop's write: stage, and quantize the whole group on its last loop.

        ``prefill`` marks a call with more than one query token per request
        (the only calls that use the offload, packed_backend.py:47).  A caller
        that has already taken ``wants_lookahead`` and called the offload's
        ``prepare`` before its attention (as ``PackedImpl.forward`` does,
        packed_backend.py:47-55) passes that flag as ``lookahead``."""
        tokens = slot_mapping.numel()
        offload = self.prefill_offload is not None and prefill
        if lookahead is None:
            lookahead = self.wants_lookahead(prefill)
            if lookahead:
                self.prefill_offload.prepare(self, tokens)
        records = self.stage(key[:tokens], value[:tokens], offload=offload)
        if (offload and records is None and len(self.pending) + 1 == len(self.records)
                and self.prefill_offload.lookahead_enabled):
            self.prefill_offload.preload(self, tokens)
        if records is None:
            return False
        if lookahead:
            chunks = self.prefill_offload.chunks(records, slot_mapping, group=self)
        elif offload and len(records) > 1:
            chunks = self.prefill_offload.chunks(records, slot_mapping)
        else:
            chunks = ((records, slot_mapping),)
        for chunk_records, chunk_slots in chunks:
            ops.quantize(chunk_records, kv_cache, chunk_slots, key_rotation, value_rotation, key_mean,
                         self.records, self.reference_mode, self.anchor_index, self.coefficient_method)
        return True
