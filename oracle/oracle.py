"""ctypes front end of the CPU oracle (``oracle/rq_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the checker.  The product
package (``residualquant_amd``) never imports it.

Arrays are numpy: BF16 and FP16 tensors travel as ``uint16`` bit patterns,
the packed cache as ``uint8`` [2, blocks, heads, page_tokens, page_width].
Argument meaning follows the reference ops ``quantize(...)`` /
``attention(...)`` (plugins/residual_quantization/csrc/dispatch/binding.cpp:19-38).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "librq_oracle.so")
_lib = None

MODES = {"anchor": 0, "adjacent": 1}
COEFFICIENTS = {"unit": 0, "norm": 1, "ls": 2}


def build() -> str:
    """Compile the oracle with its Makefile (gcc), every time; returns the library path."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(l):
    c_int, c_i64, c_f, c_vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
    l.rq_oracle_bf16_rn.restype = ctypes.c_uint16
    l.rq_oracle_bf16_rn.argtypes = [c_f]
    l.rq_oracle_bf16_to_f32.restype = c_f
    l.rq_oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
    l.rq_oracle_f16_to_f32.restype = c_f
    l.rq_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    for name in ("rq_oracle_bf16_fma_rn",):
        getattr(l, name).restype = ctypes.c_uint16
        getattr(l, name).argtypes = [ctypes.c_uint16] * 3
    l.rq_oracle_bf16_add_rn.restype = ctypes.c_uint16
    l.rq_oracle_bf16_add_rn.argtypes = [ctypes.c_uint16] * 2
    l.rq_oracle_e4m3_to_f32.restype = c_f
    l.rq_oracle_e4m3_to_f32.argtypes = [ctypes.c_uint8]
    l.rq_oracle_e4m3_from_f32.restype = ctypes.c_uint8
    l.rq_oracle_e4m3_from_f32.argtypes = [c_f]
    l.rq_oracle_record_bytes.restype = c_int
    l.rq_oracle_record_bytes.argtypes = [c_int, c_int, c_int]
    l.rq_oracle_page_width.restype = c_int
    l.rq_oracle_page_width.argtypes = [c_int, c_int, c_vp, c_vp]
    l.rq_oracle_rotate.restype = None
    l.rq_oracle_rotate.argtypes = [c_vp, c_vp, c_int, c_vp]
    l.rq_oracle_quantize.restype = c_int
    l.rq_oracle_quantize.argtypes = [
        c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_int, c_int, c_int, c_vp, c_i64, c_int,
        c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int]
    l.rq_oracle_dequantize.restype = c_int
    l.rq_oracle_dequantize.argtypes = [
        c_vp, c_i64, c_int, c_int, c_int, c_vp, c_i64, c_int, c_vp, c_int, c_vp, c_vp,
        c_int, c_int, c_int, c_vp, c_vp]
    l.rq_oracle_attention.restype = c_int
    l.rq_oracle_attention.argtypes = [
        c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_int, c_int, c_vp, c_i64, c_int,
        c_int, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_int, c_vp, c_vp, c_int,
        c_int, c_int]
    l.rq_oracle_attention_prefill.restype = c_int
    l.rq_oracle_attention_prefill.argtypes = l.rq_oracle_attention.argtypes
    l.rq_oracle_paged_attention_bf16.restype = c_int
    l.rq_oracle_paged_attention_bf16.argtypes = [
        c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_int, c_int, c_vp, c_i64, c_int,
        c_vp, c_vp, c_i64, c_vp, c_i64]
    l.rq_oracle_prefill_attention.restype = c_int
    l.rq_oracle_prefill_attention.argtypes = [
        c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_int, c_int, c_int, c_vp, c_vp, c_i64,
        ctypes.c_double, c_int]


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _records(records):
    bits = np.ascontiguousarray([int(b) for b, _ in records], dtype=np.int32)
    groups = np.ascontiguousarray([int(g) for _, g in records], dtype=np.int32)
    return bits, groups


# ---------------------------------------------------------------- scalars

def bf16_rn(x: float) -> int:
    return int(lib().rq_oracle_bf16_rn(float(x)))


def bf16_to_f32(h: int) -> float:
    return float(lib().rq_oracle_bf16_to_f32(int(h)))


def f16_to_f32(h: int) -> float:
    return float(lib().rq_oracle_f16_to_f32(int(h)))


def bf16_fma_rn(a: int, b: int, c: int) -> int:
    return int(lib().rq_oracle_bf16_fma_rn(int(a), int(b), int(c)))


def bf16_add_rn(a: int, b: int) -> int:
    return int(lib().rq_oracle_bf16_add_rn(int(a), int(b)))


def e4m3_to_f32(v: int) -> float:
    return float(lib().rq_oracle_e4m3_to_f32(int(v)))


def e4m3_from_f32(x: float) -> int:
    return int(lib().rq_oracle_e4m3_from_f32(float(x)))


def record_bytes(head_dim: int, bits: int, group: int) -> int:
    return int(lib().rq_oracle_record_bytes(head_dim, bits, group))


def page_width(head_dim: int, records) -> int:
    bits, groups = _records(records)
    return int(lib().rq_oracle_page_width(head_dim, len(records), _ptr(bits), _ptr(groups)))


def rotate(x_bf16: np.ndarray, rotation_f16: np.ndarray) -> np.ndarray:
    """Canonical FP32 rotation of one BF16 row by an FP16 [D, D] matrix."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m = np.ascontiguousarray(rotation_f16, dtype=np.uint16)
    y = np.zeros(x.shape[-1], dtype=np.float32)
    lib().rq_oracle_rotate(_ptr(x), _ptr(m), x.shape[-1], _ptr(y))
    return y


# ---------------------------------------------------------------- ops

def quantize(key_value_pairs, kv_cache, slot_mapping, key_rotation, value_rotation, key_mean,
             records, reference_mode, anchor_index, coefficient_method):
    """In-place quantize-on-write into ``kv_cache`` (uint8, 5-D)."""
    keys = [np.ascontiguousarray(k, dtype=np.uint16) for k, _ in key_value_pairs]
    values = [np.ascontiguousarray(v, dtype=np.uint16) for _, v in key_value_pairs]
    count = len(records)
    kp = (ctypes.c_void_p * count)(*[k.ctypes.data for k in keys])
    vp = (ctypes.c_void_p * count)(*[v.ctypes.data for v in values])
    ks = np.ascontiguousarray([k.shape[1] * k.shape[2] for k in keys], dtype=np.int64)
    vs = np.ascontiguousarray([v.shape[1] * v.shape[2] for v in values], dtype=np.int64)
    slots = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    bits, groups = _records(records)
    assert kv_cache.dtype == np.uint8 and kv_cache.flags["C_CONTIGUOUS"]
    _, blocks, heads, page_tokens, width = kv_cache.shape
    kr = None if key_rotation is None else np.ascontiguousarray(key_rotation, dtype=np.uint16)
    vr = None if value_rotation is None else np.ascontiguousarray(value_rotation, dtype=np.uint16)
    km = None if key_mean is None else np.ascontiguousarray(key_mean, dtype=np.float32)
    rc = lib().rq_oracle_quantize(
        count, ctypes.cast(kp, ctypes.c_void_p), _ptr(ks), ctypes.cast(vp, ctypes.c_void_p),
        _ptr(vs), _ptr(kv_cache), blocks, heads, page_tokens, width, _ptr(slots), slots.size,
        keys[0].shape[2], _ptr(kr), _ptr(vr), _ptr(km), _ptr(bits), _ptr(groups),
        MODES[reference_mode], anchor_index, COEFFICIENTS[coefficient_method])
    if rc != 0:
        raise RuntimeError("oracle quantize rejected its arguments")


def dequantize(kv_cache, slots, head_dim, key_mean, records, reference_mode, anchor_index, loop):
    """Restored BF16 (uint16) K and V [tokens, heads, D] of ``loop`` at ``slots``."""
    _, blocks, heads, page_tokens, width = kv_cache.shape
    slots = np.ascontiguousarray(slots, dtype=np.int64)
    bits, groups = _records(records)
    km = None if key_mean is None else np.ascontiguousarray(key_mean, dtype=np.float32)
    k = np.zeros((slots.size, heads, head_dim), dtype=np.uint16)
    v = np.zeros_like(k)
    rc = lib().rq_oracle_dequantize(
        _ptr(kv_cache), blocks, heads, page_tokens, width, _ptr(slots), slots.size, head_dim,
        _ptr(km), len(records), _ptr(bits), _ptr(groups), MODES[reference_mode], anchor_index,
        loop, _ptr(k), _ptr(v))
    if rc != 0:
        raise RuntimeError("oracle dequantize rejected its arguments")
    return k, v


def attention(query, key, value, kv_cache, query_start_loc, seq_lens, block_table, key_rotation,
              value_rotation, key_mean, records, reference_mode, anchor_index, loop_index):
    """FP64 decode attention [rows, heads, D] over the restored packed history."""
    return _attention(lib().rq_oracle_attention, query, key, value, kv_cache, query_start_loc, seq_lens,
                      block_table, key_rotation, value_rotation, key_mean, records, reference_mode, anchor_index,
                      loop_index)


def _attention(function, query, key, value, kv_cache, query_start_loc, seq_lens, block_table, key_rotation,
               value_rotation, key_mean, records, reference_mode, anchor_index, loop_index):
    q = np.ascontiguousarray(query, dtype=np.uint16)
    k = np.ascontiguousarray(key, dtype=np.uint16)
    v = np.ascontiguousarray(value, dtype=np.uint16)
    rows, heads, head_dim = q.shape
    _, blocks, cache_heads, page_tokens, width = kv_cache.shape
    assert cache_heads == heads
    qsl = np.ascontiguousarray(query_start_loc, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    bits, groups = _records(records)
    kr = None if key_rotation is None else np.ascontiguousarray(key_rotation, dtype=np.uint16)
    vr = None if value_rotation is None else np.ascontiguousarray(value_rotation, dtype=np.uint16)
    km = None if key_mean is None else np.ascontiguousarray(key_mean, dtype=np.float32)
    out = np.zeros((rows, heads, head_dim), dtype=np.float64)
    rc = function(
        _ptr(q), heads * head_dim, _ptr(k), heads * head_dim, _ptr(v), heads * head_dim,
        _ptr(out), rows, heads, head_dim, _ptr(kv_cache), blocks, page_tokens, width,
        _ptr(qsl), _ptr(sl), sl.size, _ptr(bt), bt.shape[1], _ptr(kr), _ptr(vr), _ptr(km),
        len(records), _ptr(bits), _ptr(groups), MODES[reference_mode], anchor_index, loop_index)
    if rc != 0:
        raise RuntimeError("oracle attention rejected its arguments")
    return out


def attention_prefill(query, key, value, kv_cache, query_start_loc, seq_lens, block_table, key_rotation,
                      value_rotation, key_mean, records, reference_mode, anchor_index, loop_index):
    """FP64 attention of each request's last n tokens (its query rows) over the packed history
    (seq_len - n tokens) and, causally, over the request's new keys/values."""
    return _attention(lib().rq_oracle_attention_prefill, query, key, value, kv_cache, query_start_loc, seq_lens,
                      block_table, key_rotation, value_rotation, key_mean, records, reference_mode, anchor_index,
                      loop_index)


def paged_attention_bf16(query, key, value, cache, query_start_loc, seq_lens, block_table):
    """FP64 decode attention over a BF16 paged cache [2, blocks, heads, PT, D]."""
    q = np.ascontiguousarray(query, dtype=np.uint16)
    k = np.ascontiguousarray(key, dtype=np.uint16)
    v = np.ascontiguousarray(value, dtype=np.uint16)
    rows, heads, head_dim = q.shape
    cache = np.ascontiguousarray(cache, dtype=np.uint16)
    _, blocks, _, page_tokens, _ = cache.shape
    qsl = np.ascontiguousarray(query_start_loc, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    out = np.zeros((rows, heads, head_dim), dtype=np.float64)
    rc = lib().rq_oracle_paged_attention_bf16(
        _ptr(q), heads * head_dim, _ptr(k), heads * head_dim, _ptr(v), heads * head_dim,
        _ptr(out), rows, heads, head_dim, _ptr(cache), blocks, page_tokens, _ptr(qsl), _ptr(sl),
        sl.size, _ptr(bt), bt.shape[1])
    if rc != 0:
        raise RuntimeError("oracle bf16 attention rejected its arguments")
    return out


def prefill_attention(query, key, value, cu_seqlens_q, cu_seqlens_k, scale, causal=True):
    """FP64 varlen attention: query [Nq, Hq, D], key/value [Nk, Hk, D] as BF16 bits (uint16)."""
    q = np.ascontiguousarray(query, dtype=np.uint16)
    k = np.ascontiguousarray(key, dtype=np.uint16)
    v = np.ascontiguousarray(value, dtype=np.uint16)
    tokens_q, heads_q, head_dim = q.shape
    heads_k = k.shape[1]
    cq = np.ascontiguousarray(cu_seqlens_q, dtype=np.int32)
    ck = np.ascontiguousarray(cu_seqlens_k, dtype=np.int32)
    out = np.zeros((tokens_q, heads_q, head_dim), dtype=np.float64)
    rc = lib().rq_oracle_prefill_attention(
        _ptr(q), heads_q * head_dim, _ptr(k), heads_k * head_dim, _ptr(v), heads_k * head_dim, _ptr(out),
        heads_q, heads_k, head_dim, _ptr(cq), _ptr(ck), cq.size - 1, ctypes.c_double(scale), 1 if causal else 0)
    if rc != 0:
        raise RuntimeError("oracle prefill attention rejected its arguments")
    return out

