"""Seeded test scenarios shared by the CPU and GPU tests."""

from __future__ import annotations

import dataclasses
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from residualquant_amd import workloads
from residualquant_amd.layout import page_width

OURO_G32 = ((2, 32), (2, 32), (2, 32), (4, 32))
OURO_G16 = ((2, 16), (2, 16), (2, 16), (4, 32))


@dataclasses.dataclass
class Group:
    dim: int
    heads: int
    page_tokens: int
    records: Tuple[Tuple[int, int], ...]
    mode: str
    anchor: int
    coefficient: str
    pairs: List[Tuple[torch.Tensor, torch.Tensor]]
    key_rotation: Optional[torch.Tensor]
    value_rotation: Optional[torch.Tensor]
    key_mean: Optional[torch.Tensor]
    slots: torch.Tensor
    num_blocks: int

    @property
    def width(self) -> int:
        return page_width(self.dim, self.records)

    @property
    def cache_shape(self):
        return (2, self.num_blocks, self.heads, self.page_tokens, self.width)

    def oracle_cache(self, oracle, cache: Optional[np.ndarray] = None) -> np.ndarray:
        if cache is None:
            cache = np.zeros(self.cache_shape, dtype=np.uint8)
        oracle.quantize(
            [(workloads.bf16_bits(k), workloads.bf16_bits(v)) for k, v in self.pairs], cache,
            self.slots.numpy(), _bits(self.key_rotation), _bits(self.value_rotation),
            None if self.key_mean is None else self.key_mean.numpy(), self.records, self.mode,
            self.anchor, self.coefficient)
        return cache

    def device_args(self, device):
        move = (lambda t: None if t is None else t.to(device))
        return (move(self.key_rotation), move(self.value_rotation), move(self.key_mean))


def _bits(tensor):
    return None if tensor is None else workloads.bf16_bits(tensor)


def make_group(tokens: int, heads: int, dim: int, records: Sequence[Tuple[int, int]], seed: int,
               page_tokens: int = 16, mode: str = "anchor", anchor: Optional[int] = None,
               coefficient: str = "ls", rotation: bool = True, mean: bool = True,
               skipped: int = 0, spare_blocks: int = 2) -> Group:
    records = tuple(tuple(r) for r in records)
    loops = len(records)
    anchor = loops - 1 if anchor is None else anchor
    pairs = workloads.loop_kv(tokens, heads, dim, loops, seed, anchor_index=anchor)
    key_rotation = workloads.random_sign_rotation(heads, dim, seed + 101) if rotation else None
    value_rotation = workloads.random_sign_rotation(heads, dim, seed + 102) if rotation else None
    key_mean = workloads.key_means(loops, heads, dim, seed + 103) if mean else None
    num_blocks = (tokens + page_tokens - 1) // page_tokens + spare_blocks
    generator = torch.Generator().manual_seed(seed + 104)
    slots = torch.randperm(num_blocks * page_tokens, generator=generator)[:tokens].to(torch.int64)
    if skipped:
        slots[torch.randperm(tokens, generator=generator)[:skipped]] = -1
    return Group(dim, heads, page_tokens, records, mode, anchor, coefficient, pairs, key_rotation,
                 value_rotation, key_mean, slots, num_blocks)


@dataclasses.dataclass
class Decode:
    group: Group
    lengths: List[int]            # seq_lens (history + current token) per request
    rows_per_request: List[int]
    table: torch.Tensor           # INT32 [requests, max_pages]
    query: torch.Tensor           # BF16 [rows, heads, D]
    key: torch.Tensor
    value: torch.Tensor

    @property
    def query_start_loc(self) -> torch.Tensor:
        starts = np.concatenate([[0], np.cumsum(self.rows_per_request)])
        return torch.tensor(starts, dtype=torch.int32)

    @property
    def seq_lens(self) -> torch.Tensor:
        return torch.tensor(self.lengths, dtype=torch.int32)


def make_decode(lengths: Sequence[int], heads: int, dim: int, records, seed: int, page_tokens: int = 16,
                mode: str = "anchor", anchor: Optional[int] = None, coefficient: str = "ls",
                rotation: bool = True, mean: bool = True, rows_per_request: Optional[Sequence[int]] = None,
                extra_pages: int = 1) -> Decode:
    """Requests whose histories (seq_len - 1 tokens) are quantized into a shared paged cache."""
    lengths = [int(x) for x in lengths]
    histories = [max(0, x - 1) for x in lengths]
    max_pages = max(1, max((h + page_tokens - 1) // page_tokens for h in histories)) + extra_pages
    table = workloads.block_tables(len(lengths), max_pages, seed + 201)
    total = sum(histories)
    group = make_group(max(total, 1), heads, dim, records, seed, page_tokens=page_tokens, mode=mode,
                       anchor=anchor, coefficient=coefficient, rotation=rotation, mean=mean)
    group.num_blocks = len(lengths) * max_pages
    slots = workloads.history_slots(table, histories, page_tokens)
    if total == 0:
        slots = torch.full((1,), -1, dtype=torch.int64)
    group.slots = slots
    rows_per_request = [1] * len(lengths) if rows_per_request is None else list(rows_per_request)
    rows = sum(rows_per_request)
    generator = torch.Generator().manual_seed(seed + 202)
    query = torch.randn((rows, heads, dim), generator=generator).to(torch.bfloat16)
    key = torch.randn((rows, heads, dim), generator=generator).to(torch.bfloat16)
    value = torch.randn((rows, heads, dim), generator=generator).to(torch.bfloat16)
    return Decode(group, lengths, rows_per_request, table, query, key, value)


def oracle_attention(oracle, decode: Decode, cache: np.ndarray, loop: int) -> np.ndarray:
    g = decode.group
    return oracle.attention(
        workloads.bf16_bits(decode.query), workloads.bf16_bits(decode.key),
        workloads.bf16_bits(decode.value), cache, decode.query_start_loc.numpy(),
        decode.seq_lens.numpy(), decode.table.numpy(), _bits(g.key_rotation), _bits(g.value_rotation),
        None if g.key_mean is None else g.key_mean.numpy(), g.records, g.mode, g.anchor, loop)


def bf16_from_bits(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)
