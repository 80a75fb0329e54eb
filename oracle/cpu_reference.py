"""Vectorised PyTorch-CPU restatement of the packed decode attention (the CPU
baseline of the benchmark; test infrastructure, never part of the product).

It follows the same reference semantics as the C oracle (rq_oracle.c):
records decoded from the page bytes (plugins/residual_quantization/csrc/
common/cache.cuh:10-106, quantize/kernel.cuh:205-227), values restored as
the reference's BF16 chain (attention/compute.cuh:28-107: V_A = bf16(c.s+o),
V_L = bf16(alpha_L * V_A + bf16(c.s+o)_L)), keys as the unrounded
decomposition the reference decode kernel scores (compute.cuh:397-505:
alpha_L * (c.s+o + bf16(mu_A))_A + (c.s+o)_L + mu_L), the live token scored
as q.k / sqrt(D) (prepare.cuh:13-54), float64 softmax, and the output
(sum p V) R_v^T + p_live v_live (merge.cuh:66-83, output.cuh:9-31).

Anchor mode only (the benchmark configurations).  Whole requests are
processed at once with torch tensor ops on every host thread torch uses.
tests/test_cpu_reference.py checks it against the C oracle: restored values
bit for bit, attention within 1e-9.
"""

from __future__ import annotations

from typing import Optional, Sequence, Tuple

import numpy as np
import torch

_FP8 = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).double()


def _rne_bf16(x: torch.Tensor) -> torch.Tensor:
    """Round exact float64 values to the nearest BF16, ties to even (as float64)."""
    _, e = torch.frexp(x)
    quantum = torch.ldexp(torch.ones_like(x), torch.clamp(e, min=-125) - 8)
    return torch.round(x / quantum) * quantum


def _bf16_of_float(x: torch.Tensor) -> torch.Tensor:
    return x.float().to(torch.bfloat16).double()


def _offsets(dim: int, records: Sequence[Tuple[int, int]], page_tokens: int):
    offsets, at = [], 0
    for bits, group in records:
        offsets.append(page_tokens * at)
        at += dim * bits // 8 + 2 * dim // group + 2
    return offsets


def decode_record(pages: torch.Tensor, dim: int, records, r: int, page_tokens: int):
    """Record r of pages [..., page_tokens, width] (uint8) -> (c*s + o exact float64 [..., T, D], alpha [..., T])."""
    bits, group = records[r]
    code_bytes, groups = dim * bits // 8, dim // group
    base = _offsets(dim, records, page_tokens)[r]
    flat = pages.reshape(*pages.shape[:-2], -1)
    region = flat[..., base:base + page_tokens * (code_bytes + 2 * groups + 2)]
    lead = region.shape[:-1]
    codes = region[..., :page_tokens * code_bytes].reshape(*lead, page_tokens, code_bytes).to(torch.int32)
    per_byte = 8 // bits
    shifts = torch.arange(per_byte, dtype=torch.int32) * bits
    values = ((codes[..., None] >> shifts) & ((1 << bits) - 1)).reshape(*lead, page_tokens, dim).double()
    params = region[..., page_tokens * code_bytes:page_tokens * (code_bytes + 2 * groups)].long()
    scale = _FP8[params[..., :page_tokens * groups]].reshape(*lead, page_tokens, groups, 1)
    offset = _FP8[params[..., page_tokens * groups:]].reshape(*lead, page_tokens, groups, 1)
    restored = (values.reshape(*lead, page_tokens, groups, group) * scale + offset).reshape(*lead, page_tokens, dim)
    a = region[..., page_tokens * (code_bytes + 2 * groups):].reshape(*lead, page_tokens, 2).to(torch.int32)
    alpha = ((a[..., 0] | (a[..., 1] << 8)).to(torch.int16)).view(torch.bfloat16).double()
    return restored, alpha


def request_keys_values(cache: torch.Tensor, blocks: torch.Tensor, history: int, dim: int, records, anchor: int,
                        loop: int, key_mean: Optional[torch.Tensor]):
    """Keys (exact decomposition) and BF16-restored values [heads, history, D] of one request."""
    page_tokens, heads = cache.size(3), cache.size(2)
    if history == 0:
        empty = torch.zeros((heads, 0, dim), dtype=torch.float64)
        return empty, empty
    pages = cache[:, blocks]                                  # [2, pages, heads, PT, width]
    key_a, _ = decode_record(pages[0], dim, records, anchor, page_tokens)
    value_a, _ = decode_record(pages[1], dim, records, anchor, page_tokens)
    value = _rne_bf16(value_a)
    if key_mean is not None:
        key_a = key_a + (_bf16_of_float(key_mean[anchor]) if loop != anchor else key_mean[anchor].double())[
            None, :, None, :]
    key = key_a
    if loop != anchor:
        key_l, alpha_k = decode_record(pages[0], dim, records, loop, page_tokens)
        value_l, alpha_v = decode_record(pages[1], dim, records, loop, page_tokens)
        key = alpha_k[..., None] * key_a + key_l
        if key_mean is not None:
            key = key + key_mean[loop].double()[None, :, None, :]
        value = _rne_bf16(alpha_v[..., None] * value + _rne_bf16(value_l))
    # [pages, heads, PT, D] -> [heads, pages * PT, D], first `history` tokens
    key = key.permute(1, 0, 2, 3).reshape(heads, -1, dim)[:, :history]
    value = value.permute(1, 0, 2, 3).reshape(heads, -1, dim)[:, :history]
    return key, value


def attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, cache: torch.Tensor,
              query_start_loc, seq_lens, block_table, key_rotation: Optional[torch.Tensor],
              value_rotation: Optional[torch.Tensor], key_mean: Optional[torch.Tensor], records, anchor: int,
              loop: int, requests: Optional[Sequence[int]] = None) -> torch.Tensor:
    """float64 [rows, heads, D] decode attention over a packed cache (CPU tensors).

    ``requests`` limits the work to those requests (their rows only are filled)."""
    rows, heads, dim = query.shape
    out = torch.zeros((rows, heads, dim), dtype=torch.float64)
    scale = 1.0 / np.sqrt(dim)
    kr = key_rotation.double() if key_rotation is not None else None
    vr = value_rotation.double() if value_rotation is not None else None
    chosen = range(len(seq_lens)) if requests is None else requests
    for b in chosen:
        history = max(0, int(seq_lens[b]) - 1)
        page_tokens = cache.size(3)
        pages = (history + page_tokens - 1) // page_tokens
        blocks = torch.as_tensor(block_table[b][:pages], dtype=torch.long)
        keys, values = request_keys_values(cache, blocks, history, dim, records, anchor, loop, key_mean)
        for i in range(int(query_start_loc[b]), int(query_start_loc[b + 1])):
            q = query[i].double()                                                 # [heads, D]
            rotated = (torch.einsum("hd,hde->he", q, kr) if kr is not None else q) * scale
            scores = torch.einsum("he,hte->ht", rotated, keys)                   # [heads, T]
            live = (q * key[i].double()).sum(-1) * scale                         # [heads]
            top = torch.maximum(scores.max(-1).values if history else live, live)
            weights = torch.exp(scores - top[:, None])
            live_weight = torch.exp(live - top)
            total = weights.sum(-1) + live_weight
            hist = torch.einsum("ht,htd->hd", weights, values)
            if vr is not None:
                hist = torch.einsum("hcd,hd->hc", vr, hist)
            out[i] = (hist + live_weight[:, None] * value[i].double()) / total[:, None]
    return out
