"""Write-path orchestration of one loop group (quantize-on-write).

Restates ``DeferredKVGroup`` (src/residual_quantization/install_model.py:17-52)
and the ``_store_kv`` call order of ``PackedImpl``
(src/residual_quantization/packed_backend.py:101-137): raw K/V of the group's
earlier loops is kept (cloned) until its last loop runs, and that call hands
every record to ``quantize`` at once.  The optional pinned-host prefill
offload of the reference is not part of this path.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from . import ops
from .layout import page_width as _page_width


class DeferredKVGroup:
    """Own the packed format and keep raw KV until every group loop completes."""

    def __init__(self, config: dict, records: Sequence[Sequence[int]], page_tokens: int):
        self.pending: List[Tuple[torch.Tensor, torch.Tensor]] = []
        self.records = tuple(tuple(int(v) for v in record) for record in records)
        self.page_tokens = page_tokens
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

    def stage(self, key: torch.Tensor, value: torch.Tensor):
        """Return all records when this call completes the group, else keep a copy."""
        if len(self.pending) + 1 == len(self.records):
            records = self.pending + [(key, value)]
            self.pending = []
            return records
        self.pending.append((key.clone(), value.clone()))
        return None

    def store(self, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
              slot_mapping: torch.Tensor, key_rotation: Optional[torch.Tensor],
              value_rotation: Optional[torch.Tensor], key_mean: Optional[torch.Tensor]) -> bool:
        """One loop's write: stage, and quantize the whole group on its last loop."""
        tokens = slot_mapping.numel()
        records = self.stage(key[:tokens], value[:tokens])
        if records is None:
            return False
        ops.quantize(records, kv_cache, slot_mapping, key_rotation, value_rotation, key_mean,
                     self.records, self.reference_mode, self.anchor_index, self.coefficient_method)
        return True
