"""Pins of the oracle's prefill attention (CPU): the flash_attn_varlen_func
call of the full-prompt branch (src/residual_quantization/packed_backend.py:63-77).

- Against torch's float64 scaled_dot_product_attention with an explicit
  bottom-right-aligned causal mask, grouped heads and unequal query/key
  lengths (a library routine, not the oracle's formula).
- Closed forms: one-token sequences return v; q = 0 gives the causal prefix
  means of V; a query that sees no key (len_k < len_q) gets a zero row.
"""

from __future__ import annotations

import numpy as np
import torch


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _random(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(shape, generator=g)).to(torch.bfloat16)


def _torch_reference(q, k, v, cu_q, cu_k, scale, causal):
    heads_q, heads_k = q.size(1), k.size(1)
    out = torch.zeros(q.shape, dtype=torch.float64)
    for s in range(len(cu_q) - 1):
        qs, ks = q[cu_q[s]:cu_q[s + 1]].double(), k[cu_k[s]:cu_k[s + 1]].double()
        vs = v[cu_k[s]:cu_k[s + 1]].double()
        lq, lk = qs.size(0), ks.size(0)
        ks = ks.repeat_interleave(heads_q // heads_k, dim=1)
        vs = vs.repeat_interleave(heads_q // heads_k, dim=1)
        mask = None
        if causal:
            mask = torch.arange(lk)[None, :] <= torch.arange(lq)[:, None] + (lk - lq)
        res = torch.nn.functional.scaled_dot_product_attention(
            qs.transpose(0, 1), ks.transpose(0, 1), vs.transpose(0, 1), attn_mask=mask, scale=scale)
        out[cu_q[s]:cu_q[s + 1]] = res.transpose(0, 1)
    return out.numpy()


def test_matches_torch_float64_sdpa(oracle):
    for (q_lens, k_lens, heads_q, heads_k, dim, causal) in (
            ([1, 7, 33], [1, 7, 33], 2, 2, 128, True),
            ([5, 20], [9, 31], 4, 2, 96, True),
            ([12, 3], [12, 8], 3, 1, 128, False)):
        cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
        cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
        q = _random((cu_q[-1], heads_q, dim), 1)
        k = _random((cu_k[-1], heads_k, dim), 2)
        v = _random((cu_k[-1], heads_k, dim), 3)
        scale = dim ** -0.5
        got = oracle.prefill_attention(_bits(q), _bits(k), _bits(v), cu_q, cu_k, scale, causal)
        ref = _torch_reference(q, k, v, cu_q, cu_k, scale, causal)
        assert np.abs(got - ref).max() < 1e-12


def test_single_token_sequences_return_v(oracle):
    cu = np.arange(5, dtype=np.int32)
    q, k, v = (_random((4, 2, 128), s) for s in (4, 5, 6))
    out = oracle.prefill_attention(_bits(q), _bits(k), _bits(v), cu, cu, 128 ** -0.5, True)
    assert np.array_equal(out, v.double().numpy())


def test_zero_query_gives_causal_prefix_means(oracle):
    n = 23
    cu = np.array([0, n], dtype=np.int32)
    q = torch.zeros((n, 1, 128), dtype=torch.bfloat16)
    k, v = _random((n, 1, 128), 7), _random((n, 1, 128), 8)
    out = oracle.prefill_attention(_bits(q), _bits(k), _bits(v), cu, cu, 128 ** -0.5, True)
    prefix = np.cumsum(v.double().numpy(), axis=0) / np.arange(1, n + 1)[:, None, None]
    assert np.abs(out - prefix).max() < 1e-14


def test_query_without_keys_is_zero(oracle):
    cu_q, cu_k = np.array([0, 6], dtype=np.int32), np.array([0, 4], dtype=np.int32)
    q, k, v = _random((6, 1, 96), 9), _random((4, 1, 96), 10), _random((4, 1, 96), 11)
    out = oracle.prefill_attention(_bits(q), _bits(k), _bits(v), cu_q, cu_k, 96 ** -0.5, True)
    assert np.all(out[:2] == 0) and np.all(np.abs(out[2:]).sum(axis=-1) > 0)
