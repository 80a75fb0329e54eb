"""The packed-cache signatures the reference compiles, and the start-up warm-up.

The reference registers one attention and three quantize launchers per
(heads, head_dim, records, anchor, reference mode, has_mean, page_tokens)
in csrc/dispatch/decode_{ouro,huginn}_{anchor,adjacent}_{0,3}_g{16,32}.cu
(each a list of record schedules, expanded over page tokens 16/32 and
mean on/off by dispatch/schedules.cuh:9-77).  This library takes any head
count and a superset of those schedules; ``REFERENCE_SIGNATURES`` lists the
reference's set so that callers and tests can sweep exactly what a
reference build would accept.

``warmup`` is the plugin's start-up pass (install_cache.py:187-256): one
quantize of a single zero token and one attention call per loop with no
history, for every distinct layer signature, so that the kernels' code is
loaded before the KV pool is sized.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from . import ops
from .layout import page_width

Schedule = Tuple[Tuple[int, int], ...]

_G16 = ((2, 16), (2, 16), (2, 16), (2, 16))
_G16_ANCHOR_FIRST = ((4, 32), (2, 16), (2, 16), (2, 16))
_G16_ANCHOR_LAST = ((2, 16), (2, 16), (2, 16), (4, 32))
_G32 = ((2, 32), (2, 32), (2, 32), (2, 32))
_G32_INT4 = ((4, 32), (4, 32), (4, 32), (4, 32))
_G32_ANCHOR_FIRST = ((4, 32), (2, 32), (2, 32), (2, 32))
_G32_ANCHOR_LAST = ((2, 32), (2, 32), (2, 32), (4, 32))

# (mode, anchor) -> schedules, the same for both geometries
# (dispatch/decode_*_{adjacent_0,anchor_0,anchor_3}_g{16,32}.cu).
_SCHEDULES = {
    ("adjacent", 0): (_G16, _G16_ANCHOR_FIRST, _G16_ANCHOR_LAST, ((2, 16),),
                      _G32, _G32_INT4, _G32_ANCHOR_FIRST, _G32_ANCHOR_LAST, ((2, 32),), ((4, 32),)),
    ("anchor", 0): (_G16, _G16_ANCHOR_FIRST, _G16_ANCHOR_LAST, ((2, 16),),
                    _G32, _G32_INT4, _G32_ANCHOR_FIRST, _G32_ANCHOR_LAST, ((2, 32),), ((4, 32),)),
    ("anchor", 3): (_G16, _G16_ANCHOR_FIRST, _G16_ANCHOR_LAST,
                    _G32, _G32_INT4, _G32_ANCHOR_FIRST, _G32_ANCHOR_LAST),
}
# (heads, head_dim) of the two model families (Ouro, Huginn).
_GEOMETRIES = ((16, 128), (55, 96))


@dataclass(frozen=True)
class Signature:
    heads: int
    head_dim: int
    records: Schedule
    page_tokens: int
    reference_mode: str
    anchor_index: int
    has_mean: bool


def reference_signatures() -> List[Signature]:
    """Every (geometry, schedule, mode, anchor, page tokens, mean) the reference registers."""
    out = []
    for heads, dim in _GEOMETRIES:
        for (mode, anchor), schedules in _SCHEDULES.items():
            for records in schedules:
                for page_tokens in (16, 32):
                    for has_mean in (False, True):
                        out.append(Signature(heads, dim, records, page_tokens, mode, anchor, has_mean))
    return out


REFERENCE_SIGNATURES = tuple(reference_signatures())


@dataclass
class WarmupLayer:
    """What ``warmup`` needs from one attention layer (the fields the
    reference reads from the layer and its packed group)."""

    heads: int
    head_dim: int
    records: Schedule
    page_tokens: int
    reference_mode: str
    anchor_index: int
    coefficient_method: str
    key_rotation: Optional[torch.Tensor] = None
    value_rotation: Optional[torch.Tensor] = None
    key_mean: Optional[torch.Tensor] = None

    def signature(self) -> tuple:
        """The fields that select compiled kernels and argument shapes: two
        layers with equal signatures exercise the same code."""
        present = tuple(t is not None for t in (self.key_mean, self.key_rotation, self.value_rotation))
        return (self.heads, self.head_dim, tuple(self.records), self.page_tokens, self.reference_mode,
                self.anchor_index, self.coefficient_method) + present


@dataclass
class _EmptyCall:
    """Device buffers of a one-token request with no history: the token, its
    output, a one-block cache, slot 0, and the batch metadata."""

    token: torch.Tensor
    output: torch.Tensor
    cache: torch.Tensor
    slot: torch.Tensor
    query_start_loc: torch.Tensor
    seq_lens: torch.Tensor
    block_table: torch.Tensor

    @classmethod
    def for_layer(cls, layer: WarmupLayer, device: torch.device) -> "_EmptyCall":
        token = torch.zeros((1, layer.heads, layer.head_dim), dtype=torch.bfloat16, device=device)
        shape = (2, 1, layer.heads, layer.page_tokens, page_width(layer.head_dim, layer.records))
        return cls(token=token, output=torch.empty_like(token),
                   cache=torch.zeros(shape, dtype=torch.uint8, device=device),
                   slot=torch.zeros(1, dtype=torch.int64, device=device),
                   query_start_loc=torch.arange(2, dtype=torch.int32, device=device),
                   seq_lens=torch.ones(1, dtype=torch.int32, device=device),
                   block_table=torch.zeros((1, 1), dtype=torch.int32, device=device))


def warmup(layers: Sequence[WarmupLayer], device: torch.device) -> int:
    """Run each distinct layer signature once: quantize one zero token into a
    fresh one-block cache, then one attention call per loop over it (no
    history).  Returns the number of signatures run, and synchronizes the
    device when any ran (the reference's start-up pass,
    install_cache.py:187-256, before the KV pool is sized)."""
    done = set()
    for layer in layers:
        key = layer.signature()
        if key in done:
            continue
        done.add(key)
        call = _EmptyCall.for_layer(layer, device)
        rotations = (layer.key_rotation, layer.value_rotation, layer.key_mean)
        schedule = (layer.records, layer.reference_mode, layer.anchor_index)
        pairs = [(call.token, call.token) for _ in layer.records]
        ops.quantize(pairs, call.cache, call.slot, *rotations, *schedule, layer.coefficient_method)
        for loop in range(len(layer.records)):
            ops.attention(call.token, call.token, call.token, call.cache, call.output, call.query_start_loc,
                          call.seq_lens, call.block_table, *rotations, *schedule, loop)
    if done:
        torch.cuda.synchronize(device)
    return len(done)
