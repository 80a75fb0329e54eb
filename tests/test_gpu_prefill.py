"""Prefill attention on the GPU (csrc/prefill.hip) against the FP64 oracle:
the flash_attn_varlen_func call of the full-prompt branch
(src/residual_quantization/packed_backend.py:63-77).  Tolerance on the BF16
output: 2e-2 max-abs and 1e-3 mean-abs (BF16 Q/K/V, FP32 accumulation,
BF16 probabilities in the P.V product)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import residualquant_amd as rq

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 1e-3


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _random(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def _check(got, expected, label):
    err = np.abs(got.float().cpu().numpy().astype(np.float64) - expected)
    print(f"{label}: max {err.max():.2e} mean {err.mean():.2e}", flush=True)
    assert err.max() < MAX_ABS and err.mean() < MEAN_ABS, label


CASES = [
    # (query lengths, key lengths, heads_q, heads_k, head_dim, causal)
    ([1, 37, 128, 300], None, 4, 4, 128, True),
    ([200, 65, 1], None, 3, 3, 96, True),
    ([129, 64], None, 8, 2, 128, True),
    ([40, 90], [100, 90], 2, 2, 128, True),
    ([77, 5], [33, 140], 2, 1, 96, False),
    # long enough for many block pairs, the merge of a heavy block's halves and the lone middle block
    ([1500, 700], None, 2, 2, 128, True),
    ([300, 200], [1300, 1250], 2, 1, 96, False),
    ([640, 130], [700, 200], 2, 2, 128, True),   # keys beyond the queries (bottom-right alignment)
    ([3, 260], [1, 70], 2, 2, 96, True),         # first rows that see no key
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[4]}d-{c[2]}x{c[3]}h-{'causal' if c[5] else 'full'}"
                                                      f"-{len(c[0])}seq")
def test_prefill_matches_oracle(oracle, device, case):
    q_lens, k_lens, heads_q, heads_k, dim, causal = case
    k_lens = q_lens if k_lens is None else k_lens
    print(f"prefill case q={q_lens} k={k_lens} heads={heads_q}/{heads_k} D={dim} causal={causal}", flush=True)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    q = _random((cu_q[-1], heads_q, dim), sum(q_lens))
    k = _random((cu_k[-1], heads_k, dim), sum(k_lens) + 1)
    v = _random((cu_k[-1], heads_k, dim), sum(k_lens) + 2)
    expected = oracle.prefill_attention(_bits(q), _bits(k), _bits(v), cu_q, cu_k, dim ** -0.5, causal)
    out = rq.flash_attn_varlen_func(
        q=q.to(device), k=k.to(device), v=v.to(device), out=torch.empty_like(q, device=device),
        cu_seqlens_q=torch.from_numpy(cu_q).to(device), cu_seqlens_k=torch.from_numpy(cu_k).to(device),
        max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), softmax_scale=dim ** -0.5, causal=causal)
    _check(out, expected, "prefill")


def test_prefill_separate_equal_seqlens(oracle, device):
    """cu_seqlens_k a separate tensor with the same lengths: the general split plan."""
    lens, heads, dim = [1200, 33], 2, 128
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v = (_random((cu[-1], heads, dim), s) for s in (21, 22, 23))
    expected = oracle.prefill_attention(_bits(q), _bits(k), _bits(v), cu, cu, dim ** -0.5, True)
    out = rq.flash_attn_varlen_func(q.to(device), k.to(device), v.to(device), max(lens),
                                    torch.from_numpy(cu).to(device), max(lens),
                                    cu_seqlens_k=torch.from_numpy(cu.copy()).to(device), softmax_scale=dim ** -0.5,
                                    causal=True)
    _check(out, expected, "separate seqlens")


def test_prefill_fused_qkv_views(oracle, device):
    """Q, K and V as views into one [tokens, 3 * heads, D] projection output."""
    lens, heads, dim = [50, 19], 2, 128
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    qkv = _random((cu[-1], 3 * heads, dim), 99)
    q, k, v = qkv[:, :heads], qkv[:, heads:2 * heads], qkv[:, 2 * heads:]
    expected = oracle.prefill_attention(_bits(q), _bits(k), _bits(v), cu, cu, dim ** -0.5, True)
    dev = qkv.to(device)
    out = rq.flash_attn_varlen_func(dev[:, :heads], dev[:, heads:2 * heads], dev[:, 2 * heads:], max(lens),
                                    torch.from_numpy(cu).to(device), max(lens), softmax_scale=dim ** -0.5,
                                    causal=True)
    _check(out, expected, "fused qkv")


def test_prefill_long_prompt_edges(oracle, device):
    """A 4096-token prompt x 16 heads: its first and last 64 queries against the
    oracle (the last rows as a 64-query problem over all 4096 keys, whose
    bottom-right causal alignment is the same attention)."""
    n, heads, dim, edge = 4096, 16, 128, 64
    q, k, v = (_random((n, heads, dim), s) for s in (5, 6, 7))
    cu = torch.tensor([0, n], dtype=torch.int32)
    out = rq.flash_attn_varlen_func(q.to(device), k.to(device), v.to(device), n, cu.to(device), n,
                                    softmax_scale=dim ** -0.5, causal=True).cpu()
    head_cu = np.array([0, edge], dtype=np.int32)
    first = oracle.prefill_attention(_bits(q[:edge]), _bits(k[:edge]), _bits(v[:edge]), head_cu, head_cu,
                                     dim ** -0.5, True)
    _check(out[:edge], first, "first rows")
    last = oracle.prefill_attention(_bits(q[-edge:]), _bits(k), _bits(v), head_cu,
                                    np.array([0, n], dtype=np.int32), dim ** -0.5, True)
    _check(out[-edge:], last, "last rows")


def test_prefill_split_merge_repeats_exactly(device):
    """Heavy blocks whose keys are split over the two wave groups of a
    workgroup are merged in LDS; repeated calls, and calls of other shapes in
    between, give bit-identical outputs."""
    n, heads, dim = 3000, 4, 128
    q, k, v = (_random((n, heads, dim), s).to(device) for s in (11, 12, 13))
    cu = torch.tensor([0, n], dtype=torch.int32, device=device)
    first = rq.flash_attn_varlen_func(q, k, v, n, cu, n, causal=True)
    for _ in range(3):
        again = rq.flash_attn_varlen_func(q, k, v, n, cu, n, causal=True)
        assert torch.equal(first, again)
    # A different shape in between, then the first again.
    rq.flash_attn_varlen_func(q[:1500], k[:2500], v[:2500], 1500, cu.new_tensor([0, 1500]), 2500,
                              cu_seqlens_k=cu.new_tensor([0, 2500]), causal=True)
    assert torch.equal(first, rq.flash_attn_varlen_func(q, k, v, n, cu, n, causal=True))


def test_prefill_rejects_unsupported(device):
    q = torch.zeros((4, 2, 64), dtype=torch.bfloat16, device=device)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=device)
    with pytest.raises(RuntimeError, match="No compiled prefill attention kernel for head_dim=64"):
        rq.flash_attn_varlen_func(q, q, q, 4, cu, 4, causal=True)
    q = torch.zeros((4, 2, 128), dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError, match="Only dropout-free"):
        rq.flash_attn_varlen_func(q, q, q, 4, cu, 4, causal=True, dropout_p=0.1)
