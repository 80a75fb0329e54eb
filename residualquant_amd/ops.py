"""Operator surface of the packed KV-cache path on MI355X.

``quantize`` and ``attention`` keep the reference ops' signatures, keyword
names, in-place semantics and error messages
(plugins/residual_quantization/csrc/dispatch/binding.cpp:19-38;
validation quantize/api.cpp:18-85, attention/api.cpp:23-104,
common/api.h:42-64, dispatch/kernel_registry.h:42-72).  Tensor checks that a
pointer interface cannot see (device, dtype, strides) run here and raise
``RuntimeError``; everything else is checked by ``librq_hip.so`` before any
device work.  Work is enqueued on the current HIP stream of the cache's
device; nothing synchronizes.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

_MODES = {"anchor": 0, "adjacent": 1}
_COEFFICIENTS = {"unit": 0, "norm": 1, "ls": 2}


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def _validate_bf16_token_tensor(tensor: torch.Tensor) -> None:
    # common/api.h:42-49
    _require(tensor.is_cuda and tensor.dtype == torch.bfloat16 and tensor.dim() == 3
             and tensor.stride(1) == tensor.size(2) and tensor.stride(2) == 1,
             "BF16 [tokens, heads, channels] with packed trailing strides required")


def _rotation_pointer(rotation: Optional[torch.Tensor], device, heads: int, head_dim: int):
    # common/api.h:51-64
    if rotation is None:
        return None
    _require(rotation.device == device and rotation.is_contiguous() and rotation.dtype == torch.float16
             and rotation.dim() == 3 and rotation.size(0) == heads and rotation.size(1) == head_dim
             and rotation.size(2) == head_dim,
             "Contiguous FP16 [heads, channels, channels] rotation required")
    return rotation.data_ptr()


def _schedule(records: Sequence[Sequence[int]]):
    bits = (ctypes.c_int * max(1, len(records)))(*[int(r[0]) for r in records])
    groups = (ctypes.c_int * max(1, len(records)))(*[int(r[1]) for r in records])
    return bits, groups


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def quantize(key_value_pairs: Sequence[Tuple[torch.Tensor, torch.Tensor]], kv_cache: torch.Tensor,
             slot_mapping: torch.Tensor, key_rotation: Optional[torch.Tensor],
             value_rotation: Optional[torch.Tensor], key_mean: Optional[torch.Tensor],
             records: Sequence[Sequence[int]], reference_mode: str, anchor_index: int,
             coefficient_method: str) -> None:
    """Quantize one completed loop group into the packed paged cache, in place.

    Mirrors quantize() (quantize/api.cpp:8-95): ``key_value_pairs[r]`` holds
    the BF16 [tokens, heads, D] K/V of record r in loop order; token i goes to
    cache slot ``slot_mapping[i]`` (negative = skipped).
    """
    _require(len(records) > 0 and len(key_value_pairs) == len(records),
             "A nonempty group with one K/V input per record required")
    _require(kv_cache.is_cuda and kv_cache.dtype == torch.uint8 and kv_cache.is_contiguous()
             and kv_cache.dim() == 5 and kv_cache.size(0) == 2,
             "Contiguous CUDA UINT8 [2, blocks, heads, page tokens, page width] cache required")
    heads = kv_cache.size(2)
    head_dim = key_value_pairs[0][0].size(-1)
    _require(slot_mapping.device == kv_cache.device and slot_mapping.dtype == torch.int64
             and slot_mapping.dim() == 1 and slot_mapping.is_contiguous(),
             "Contiguous INT64 slot mapping on the cache device required")
    for pair in key_value_pairs:
        for tensor in pair:
            _validate_bf16_token_tensor(tensor)
            _require(tensor.device == kv_cache.device and tensor.size(1) == heads
                     and tensor.size(2) == head_dim,
                     "K/V must match the cache device/head count and logical channel count")
            _require(tensor.size(0) >= slot_mapping.numel(), "Input has fewer rows than slot mapping")
    if key_mean is not None:
        _require(key_mean.device == kv_cache.device and key_mean.dtype == torch.float32
                 and key_mean.is_contiguous() and key_mean.dim() == 3
                 and key_mean.size(0) == len(records) and key_mean.size(1) == heads
                 and key_mean.size(2) == head_dim,
                 "Contiguous FP32 [records, heads, channels] key mean required")
    key_rotation_ptr = _rotation_pointer(key_rotation, kv_cache.device, heads, head_dim)
    value_rotation_ptr = _rotation_pointer(value_rotation, kv_cache.device, heads, head_dim)
    _require(coefficient_method in _COEFFICIENTS, "Unsupported coefficient")
    _require(reference_mode in _MODES, f"Unknown packed reference mode: {reference_mode}")

    count = len(records)
    keys = (ctypes.c_void_p * count)(*[pair[0].data_ptr() for pair in key_value_pairs])
    values = (ctypes.c_void_p * count)(*[pair[1].data_ptr() for pair in key_value_pairs])
    key_strides = (ctypes.c_int64 * count)(*[pair[0].stride(0) for pair in key_value_pairs])
    value_strides = (ctypes.c_int64 * count)(*[pair[1].stride(0) for pair in key_value_pairs])
    input_rows = min(min(pair[0].size(0), pair[1].size(0)) for pair in key_value_pairs)
    bits, groups = _schedule(records)
    with torch.cuda.device(kv_cache.device):
        status = _lib.lib().rq_quantize(
            count, ctypes.cast(keys, ctypes.c_void_p), ctypes.cast(key_strides, ctypes.c_void_p),
            ctypes.cast(values, ctypes.c_void_p), ctypes.cast(value_strides, ctypes.c_void_p),
            input_rows, kv_cache.data_ptr(), kv_cache.size(1), heads, kv_cache.size(3),
            kv_cache.size(4), slot_mapping.data_ptr(), slot_mapping.numel(), head_dim,
            key_rotation_ptr, value_rotation_ptr,
            key_mean.data_ptr() if key_mean is not None else None,
            ctypes.cast(bits, ctypes.c_void_p), ctypes.cast(groups, ctypes.c_void_p),
            _MODES[reference_mode], int(anchor_index), _COEFFICIENTS[coefficient_method],
            _stream(kv_cache.device))
    _lib.check(status)


def attention_workspace_bytes(rows: int, heads: int, head_dim: int, max_pages: int,
                              page_tokens: int) -> int:
    """Device workspace (bytes) that ``attention`` needs; depends on shapes only."""
    return int(_lib.lib().rq_attention_workspace_bytes(rows, heads, head_dim, max_pages, page_tokens))


def _workspace(workspace: Optional[torch.Tensor], needed: int, device) -> torch.Tensor:
    if workspace is None:
        return torch.empty(needed, dtype=torch.uint8, device=device)
    _require(workspace.is_cuda and workspace.device == device and workspace.is_contiguous()
             and workspace.numel() * workspace.element_size() >= needed,
             f"Attention workspace of {needed} bytes required")
    return workspace


def _validate_attention_inputs(query, key, value, output, query_start_loc, seq_lens, block_table):
    _validate_bf16_token_tensor(query)
    for tensor in (key, value, output):
        _validate_bf16_token_tensor(tensor)
        _require(tensor.device == query.device and tensor.shape == query.shape,
                 "Q/K/V/output must have matching shapes and devices")
    for tensor in (query, key):
        _require(tensor.data_ptr() % 8 == 0 and tensor.stride(0) % 4 == 0,
                 "Q/K addresses and token strides must be 8-byte aligned")
    _require(query_start_loc.device == query.device and query_start_loc.dtype == torch.int32
             and query_start_loc.dim() == 1 and query_start_loc.is_contiguous()
             and query_start_loc.numel() == seq_lens.numel() + 1,
             "Contiguous INT32 query starts with one final boundary required")
    _require(seq_lens.device == query.device and seq_lens.dtype == torch.int32
             and seq_lens.dim() == 1 and seq_lens.is_contiguous(),
             "Contiguous INT32 sequence lengths required")
    _require(block_table.device == query.device and block_table.dtype == torch.int32
             and block_table.dim() == 2 and block_table.stride(1) == 1
             and block_table.size(0) >= seq_lens.numel(),
             "INT32 page table with packed rows required")


def attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
              output: torch.Tensor, query_start_loc: torch.Tensor, seq_lens: torch.Tensor,
              block_table: torch.Tensor, key_rotation: Optional[torch.Tensor],
              value_rotation: Optional[torch.Tensor], key_mean: Optional[torch.Tensor],
              records: Sequence[Sequence[int]], reference_mode: str, anchor_index: int,
              loop_index: int, workspace: Optional[torch.Tensor] = None) -> None:
    """Paged decode attention of loop ``loop_index`` over the packed cache, writing ``output``.

    Mirrors attention() (attention/api.cpp:8-115).  ``key``/``value`` are the
    current token's K/V (not yet in the cache).  ``workspace`` (optional, not
    in the reference) lets a caller reuse one device buffer of
    ``attention_workspace_bytes(...)`` bytes, e.g. across graph replays.
    """
    key_rotation_ptr, value_rotation_ptr = _validate_packed_inputs(
        query, key, value, kv_cache, output, query_start_loc, seq_lens, block_table, key_rotation, value_rotation,
        key_mean, records, reference_mode, loop_index)
    _call_packed_attention(_lib.lib().rq_attention, query, key, value, kv_cache, output, query_start_loc,
                           seq_lens, block_table, key_rotation_ptr, value_rotation_ptr, key_mean, records,
                           reference_mode, anchor_index, loop_index, workspace)


def _validate_packed_inputs(query, key, value, kv_cache, output, query_start_loc, seq_lens, block_table,
                            key_rotation, value_rotation, key_mean, records, reference_mode, loop_index):
    _validate_attention_inputs(query, key, value, output, query_start_loc, seq_lens, block_table)
    heads, head_dim = query.size(1), query.size(2)
    _require(kv_cache.device == query.device and kv_cache.dtype == torch.uint8
             and kv_cache.is_contiguous() and kv_cache.dim() == 5 and kv_cache.size(0) == 2
             and kv_cache.size(2) == heads,
             "Contiguous UINT8 KV cache on the query device required")
    if key_mean is not None:
        _require(key_mean.device == query.device and key_mean.dtype == torch.float32
                 and key_mean.is_contiguous() and key_mean.data_ptr() % 16 == 0
                 and key_mean.numel() == len(records) * heads * head_dim,
                 "16-byte aligned contiguous FP32 key mean with matching dimensions required")
    value_rotation_ptr = _rotation_pointer(value_rotation, query.device, heads, head_dim)
    key_rotation_ptr = _rotation_pointer(key_rotation, query.device, heads, head_dim)
    _require(key_rotation_ptr is None or key_rotation_ptr % 16 == 0,
             "16-byte aligned key rotation required for asynchronous copies")
    _require(0 <= loop_index < len(records), "Invalid loop index")
    _require(reference_mode in _MODES, f"Unknown packed reference mode: {reference_mode}")
    return key_rotation_ptr, value_rotation_ptr


def packed_prefill_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                             kv_cache: torch.Tensor, output: torch.Tensor, query_start_loc: torch.Tensor,
                             seq_lens: torch.Tensor, block_table: torch.Tensor,
                             key_rotation: Optional[torch.Tensor], value_rotation: Optional[torch.Tensor],
                             key_mean: Optional[torch.Tensor], records: Sequence[Sequence[int]],
                             reference_mode: str, anchor_index: int, loop_index: int,
                             workspace: Optional[torch.Tensor] = None) -> None:
    """Attention of each request's last n tokens (its query rows) over its packed history.

    Request b's rows ``query_start_loc[b]..query_start_loc[b+1]`` are the
    last n of its ``seq_lens[b]`` tokens: they attend to the first
    ``seq_lens[b] - n`` tokens from the cache and, causally, to the request's
    own new ``key``/``value`` rows (row r sees new rows 0..r).  This is the
    prefill of a prompt chunk over a packed prefix, which the reference
    cannot run (its scheduler forbids partial prefill, rq/scheduler.py:11-18);
    arguments and validation are those of ``attention`` (head_dim 96 or
    128, anchor or adjacent mode); a request may have no new rows.
    """
    key_rotation_ptr, value_rotation_ptr = _validate_packed_inputs(
        query, key, value, kv_cache, output, query_start_loc, seq_lens, block_table, key_rotation, value_rotation,
        key_mean, records, reference_mode, loop_index)
    _call_packed_attention(_lib.lib().rq_packed_prefill_attention, query, key, value, kv_cache, output,
                           query_start_loc, seq_lens, block_table, key_rotation_ptr, value_rotation_ptr, key_mean,
                           records, reference_mode, anchor_index, loop_index, workspace)


def _call_packed_attention(function, query, key, value, kv_cache, output, query_start_loc, seq_lens, block_table,
                           key_rotation_ptr, value_rotation_ptr, key_mean, records, reference_mode, anchor_index,
                           loop_index, workspace):
    heads, head_dim = query.size(1), query.size(2)
    rows = query.size(0)
    max_pages = block_table.size(1)
    needed = attention_workspace_bytes(rows, heads, head_dim, max_pages, kv_cache.size(3))
    ws = _workspace(workspace, needed, query.device)
    bits, groups = _schedule(records)
    with torch.cuda.device(query.device):
        status = function(
            query.data_ptr(), query.stride(0), key.data_ptr(), key.stride(0), value.data_ptr(),
            value.stride(0), output.data_ptr(), output.stride(0), rows, heads, head_dim,
            kv_cache.data_ptr(), kv_cache.size(1), kv_cache.size(3), kv_cache.size(4),
            query_start_loc.data_ptr(), seq_lens.data_ptr(), seq_lens.numel(),
            block_table.data_ptr(), block_table.stride(0), max_pages, key_rotation_ptr,
            value_rotation_ptr, key_mean.data_ptr() if key_mean is not None else None,
            len(records), ctypes.cast(bits, ctypes.c_void_p), ctypes.cast(groups, ctypes.c_void_p),
            _MODES[reference_mode], int(anchor_index), int(loop_index), ws.data_ptr(),
            ws.numel() * ws.element_size(), _stream(query.device))
    _lib.check(status)


def dequantize(kv_cache: torch.Tensor, slots: torch.Tensor, head_dim: int,
               key_mean: Optional[torch.Tensor], records: Sequence[Sequence[int]],
               reference_mode: str, anchor_index: int, loop_index: int):
    """Restored BF16 K and V [tokens, heads, D] of ``loop_index`` at ``slots`` (rotated space).

    The record value both reference kernels reconstruct internally
    (quantize/kernel.cuh:160-203, attention/compute.cuh:28-197).
    """
    _require(kv_cache.is_cuda and kv_cache.dtype == torch.uint8 and kv_cache.is_contiguous()
             and kv_cache.dim() == 5 and kv_cache.size(0) == 2,
             "Contiguous CUDA UINT8 [2, blocks, heads, page tokens, page width] cache required")
    _require(slots.device == kv_cache.device and slots.dtype == torch.int64 and slots.dim() == 1
             and slots.is_contiguous(), "Contiguous INT64 slot mapping on the cache device required")
    heads = kv_cache.size(2)
    if key_mean is not None:
        _require(key_mean.device == kv_cache.device and key_mean.dtype == torch.float32
                 and key_mean.is_contiguous() and key_mean.numel() == len(records) * heads * head_dim,
                 "Contiguous FP32 [records, heads, channels] key mean required")
    _require(reference_mode in _MODES, f"Unknown packed reference mode: {reference_mode}")
    key_out = torch.empty((slots.numel(), heads, head_dim), dtype=torch.bfloat16, device=kv_cache.device)
    value_out = torch.empty_like(key_out)
    bits, groups = _schedule(records)
    with torch.cuda.device(kv_cache.device):
        status = _lib.lib().rq_dequantize(
            kv_cache.data_ptr(), kv_cache.size(1), heads, kv_cache.size(3), kv_cache.size(4),
            slots.data_ptr(), slots.numel(), head_dim,
            key_mean.data_ptr() if key_mean is not None else None, len(records),
            ctypes.cast(bits, ctypes.c_void_p), ctypes.cast(groups, ctypes.c_void_p),
            _MODES[reference_mode], int(anchor_index), int(loop_index), key_out.data_ptr(),
            value_out.data_ptr(), _stream(kv_cache.device))
    _lib.check(status)
    return key_out, value_out


def paged_attention_bf16(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                         cache: torch.Tensor, output: torch.Tensor, query_start_loc: torch.Tensor,
                         seq_lens: torch.Tensor, block_table: torch.Tensor,
                         workspace: Optional[torch.Tensor] = None) -> None:
    """BF16 paged decode attention over ``cache`` [2, blocks, heads, PT, D] (the baseline)."""
    _validate_attention_inputs(query, key, value, output, query_start_loc, seq_lens, block_table)
    heads, head_dim = query.size(1), query.size(2)
    _require(cache.device == query.device and cache.dtype == torch.bfloat16 and cache.is_contiguous()
             and cache.dim() == 5 and cache.size(0) == 2 and cache.size(2) == heads
             and cache.size(4) == head_dim,
             "Contiguous BF16 [2, blocks, heads, page tokens, channels] cache required")
    rows = query.size(0)
    max_pages = block_table.size(1)
    needed = attention_workspace_bytes(rows, heads, head_dim, max_pages, cache.size(3))
    ws = _workspace(workspace, needed, query.device)
    with torch.cuda.device(query.device):
        status = _lib.lib().rq_paged_attention_bf16(
            query.data_ptr(), query.stride(0), key.data_ptr(), key.stride(0), value.data_ptr(),
            value.stride(0), output.data_ptr(), output.stride(0), rows, heads, head_dim,
            cache.data_ptr(), cache.size(1), cache.size(3), query_start_loc.data_ptr(),
            seq_lens.data_ptr(), seq_lens.numel(), block_table.data_ptr(), block_table.stride(0),
            max_pages, ws.data_ptr(), ws.numel() * ws.element_size(), _stream(query.device))
    _lib.check(status)


def flash_attn_varlen_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, max_seqlen_q: int,
                           cu_seqlens_q: torch.Tensor, max_seqlen_k: int,
                           cu_seqlens_k: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                           softmax_scale: Optional[float] = None, causal: bool = False,
                           window_size=None, softcap: float = 0.0, alibi_slopes=None,
                           deterministic: bool = False, return_attn_probs: bool = False,
                           block_table=None, return_softmax_lse: bool = False,
                           out: Optional[torch.Tensor] = None, fa_version=None) -> torch.Tensor:
    """Varlen (causal) attention over raw BF16 Q/K/V, the full-prompt branch.

    Drop-in for the ``flash_attn_varlen_func`` call of the reference backend
    (src/residual_quantization/packed_backend.py:63-77, vLLM 0.10.2): q
    [tokens_q, heads_q, D], k/v [tokens_k, heads_k, D] BF16, sequence s spans
    cu_seqlens[s]..cu_seqlens[s+1]; with ``causal`` query i of a sequence sees
    keys j <= i + len_k - len_q.  The features that call does not use
    (dropout, windows, softcap, ALiBi, paged K/V, returned LSE or
    probabilities) raise.  ``fa_version`` is accepted and ignored.
    """
    _require(dropout_p == 0.0 and softcap == 0.0 and alibi_slopes is None and block_table is None
             and not return_attn_probs and not return_softmax_lse
             and (window_size is None or tuple(window_size) == (-1, -1)),
             "Only dropout-free, unwindowed attention without ALiBi, softcap, paged K/V or returned "
             "LSE is supported")
    cu_seqlens_k = cu_seqlens_q if cu_seqlens_k is None else cu_seqlens_k
    for tensor in (q, k, v):
        _validate_bf16_token_tensor(tensor)
    _require(k.device == q.device and v.device == q.device and k.shape == v.shape
             and k.size(2) == q.size(2), "Q/K/V must share device and head_dim; K and V must match")
    if out is None:
        out = torch.empty_like(q)
    _validate_bf16_token_tensor(out)
    _require(out.device == q.device and out.shape == q.shape, "out must match q")
    for seqlens in (cu_seqlens_q, cu_seqlens_k):
        _require(seqlens.device == q.device and seqlens.dtype == torch.int32 and seqlens.dim() == 1
                 and seqlens.is_contiguous(), "Contiguous INT32 cu_seqlens on the Q device required")
    _require(cu_seqlens_q.numel() == cu_seqlens_k.numel() and cu_seqlens_q.numel() >= 1,
             "cu_seqlens_q and cu_seqlens_k must describe the same sequences")
    head_dim = q.size(2)
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    batch = cu_seqlens_q.numel() - 1
    same = cu_seqlens_q.data_ptr() == cu_seqlens_k.data_ptr()
    needed = _lib.lib().rq_prefill_workspace_bytes(batch, q.size(1), head_dim, int(max_seqlen_q),
                                                   int(max_seqlen_k), 1 if causal else 0, 1 if same else 0)
    workspace = torch.empty(max(needed, 1), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        status = _lib.lib().rq_prefill_attention(
            q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), out.data_ptr(),
            out.stride(0), q.size(1), k.size(1), head_dim, cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(),
            batch, int(max_seqlen_q), int(max_seqlen_k), scale, 1 if causal else 0, workspace.data_ptr(),
            workspace.numel(), _stream(q.device))
    _lib.check(status)
    return out


prefill_attention = flash_attn_varlen_func


def timing_enable(enabled: bool) -> None:
    """Record HIP events around every split-K decode launch (for measurement)."""
    _lib.lib().rq_timing_enable(1 if enabled else 0)


def timing_read():
    """(milliseconds, launches) summed over the recorded split-K launches, then cleared."""
    ms = ctypes.c_double()
    launches = ctypes.c_int64()
    _lib.check(_lib.lib().rq_timing_read(ctypes.byref(ms), ctypes.byref(launches)))
    return ms.value, launches.value


def set_split_target(workgroups: int) -> None:
    """Target number of split-K workgroups per decode launch (0 restores the default)."""
    _lib.lib().rq_set_split_target(int(workgroups))
