"""Pins of the oracle's quantize-on-write (CPU).

Each test fixes something the mathematics or the reference's byte layout
determines independently of the oracle's code: grid values quantize to their
grid index, constant groups have zero scale, ties round down
(quantize/kernel.cuh:150-155), the INT2 radius is clipped by 0.9 (:135-139),
alpha is 1 for the anchor and for x == reference and 0 for a zero reference
(:87-101), LS alpha is the least-squares optimum, the rotation is x.R,
negative slots are skipped (:259), tokens are independent.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from residualquant_amd import workloads
from residualquant_amd.layout import page_width, record_offsets

from .cases import OURO_G32, make_group

E4M3_QUARTER = 0x28  # 0.25
BF16_ONE = 0x3F80


def _bf16(values) -> np.ndarray:
    return torch.tensor(np.asarray(values, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _quantize_one(oracle, records, key_rows, value_rows=None, *, slot=5, page_tokens=16, mode="anchor",
                  anchor=None, coefficient="ls", key_mean=None):
    """Quantize one token (one head) whose per-record K rows are given (no rotation)."""
    records = tuple(tuple(r) for r in records)
    dim = len(key_rows[0])
    anchor = len(records) - 1 if anchor is None else anchor
    value_rows = key_rows if value_rows is None else value_rows
    pairs = [(_bf16(k).reshape(1, 1, dim), _bf16(v).reshape(1, 1, dim)) for k, v in zip(key_rows, value_rows)]
    cache = np.zeros((2, 1, 1, page_tokens, page_width(dim, records)), dtype=np.uint8)
    oracle.quantize(pairs, cache, np.array([slot], np.int64), None, None, key_mean, records, mode, anchor,
                    coefficient)
    return cache


def _record(cache, plane, records, r, page_tokens=16, dim=128):
    bits, group = records[r]
    offset = record_offsets(dim, records, page_tokens)[r]
    code_bytes, groups = dim * bits // 8, dim // group
    page = cache[plane, 0, 0].reshape(-1)
    region = page[offset:]
    codes = region[: page_tokens * code_bytes].reshape(page_tokens, code_bytes)
    scales = region[page_tokens * code_bytes: page_tokens * (code_bytes + groups)].reshape(page_tokens, groups)
    offsets = region[page_tokens * (code_bytes + groups): page_tokens * (code_bytes + 2 * groups)].reshape(
        page_tokens, groups)
    alpha = region[page_tokens * (code_bytes + 2 * groups): page_tokens * (code_bytes + 2 * groups + 2)]
    alpha = alpha.reshape(page_tokens, 2)
    return codes, scales, offsets, alpha[:, 0].astype(np.uint16) | (alpha[:, 1].astype(np.uint16) << 8)


def _unpack(codes_row: np.ndarray, bits: int) -> np.ndarray:
    """Little-endian bitstream: channel c at bit c*bits (np.unpackbits, LSB first)."""
    stream = np.unpackbits(codes_row, bitorder="little")
    return stream.reshape(-1, bits) @ (1 << np.arange(bits))


def test_int4_grid_values_pack_to_their_index(oracle):
    dim = 128
    levels = np.array([(c + c // 32) % 16 for c in range(dim)], dtype=np.float32)
    row = levels * 0.25  # every 32-group spans 0 .. 3.75 exactly
    records = ((4, 32),)
    cache = _quantize_one(oracle, records, [row], anchor=0)
    codes, scales, offsets, alpha = _record(cache, 0, records, 0)
    token = 5
    assert np.array_equal(_unpack(codes[token], 4), levels.astype(int))
    # channel 0 in the low nibble of byte 0 (kernel.cuh:145-158, :205-209)
    assert codes[token, 0] == (int(levels[0]) | (int(levels[1]) << 4))
    assert np.all(scales[token] == E4M3_QUARTER) and np.all(offsets[token] == 0)
    assert alpha[token] == BF16_ONE
    untouched = np.ones(16, bool)
    untouched[token] = False
    assert not codes[untouched].any() and not scales[untouched].any() and not alpha[untouched].any()


def test_int2_grid_values_and_clip(oracle):
    """INT2 radius is (hi-lo)*0.9/2: a group spanning [0, 3] gets offset e4m3(0.15), scale e4m3(0.9)."""
    dim = 128
    row = np.tile(np.array([0.0, 1.0, 2.0, 3.0], np.float32), dim // 4)
    records = ((2, 32),)
    cache = _quantize_one(oracle, records, [row], anchor=0)
    codes, scales, offsets, _ = _record(cache, 0, records, 0)
    expected_offset = torch.tensor([0.15], dtype=torch.float32).to(torch.float8_e4m3fn).view(torch.uint8).item()
    expected_scale = torch.tensor([0.9], dtype=torch.float32).to(torch.float8_e4m3fn).view(torch.uint8).item()
    assert np.all(offsets[5] == expected_offset) and np.all(scales[5] == expected_scale)
    s = torch.tensor([expected_scale], dtype=torch.uint8).view(torch.float8_e4m3fn).float().item()
    o = torch.tensor([expected_offset], dtype=torch.uint8).view(torch.float8_e4m3fn).float().item()
    expected = np.clip(np.floor((row - o) / s) + ((row - o) / s - np.floor((row - o) / s) > 0.5), 0, 3)
    assert np.array_equal(_unpack(codes[5], 2), expected.astype(int))
    # INT4 uses no clip: the same span gives offset 0 and scale e4m3(3/15)
    cache4 = _quantize_one(oracle, ((4, 32),), [row], anchor=0)
    _, scales4, offsets4, _ = _record(cache4, 0, ((4, 32),), 0)
    assert np.all(offsets4[5] == 0)
    assert np.all(scales4[5] == torch.tensor([0.2]).to(torch.float8_e4m3fn).view(torch.uint8).item())


def test_ties_round_down(oracle):
    dim = 128
    row = np.zeros(dim, np.float32)
    row[0::32] = 3.75  # every group spans [0, 3.75] -> scale 0.25, offset 0
    row[1] = 1.125     # normalized 4.5 exactly -> code 4
    row[2] = 1.1875    # normalized 4.75 -> code 5
    row[3] = 1.0625    # normalized 4.25 -> code 4
    cache = _quantize_one(oracle, ((4, 32),), [row], anchor=0)
    codes, _, _, _ = _record(cache, 0, ((4, 32),), 0)
    got = _unpack(codes[5], 4)
    assert got[1] == 4 and got[2] == 5 and got[3] == 4 and got[0] == 15


def test_constant_group_has_zero_scale(oracle):
    row = np.full(128, 1.5, np.float32)
    cache = _quantize_one(oracle, ((4, 32),), [row], anchor=0)
    codes, scales, offsets, _ = _record(cache, 0, ((4, 32),), 0)
    assert np.all(scales[5] == 0) and np.all(codes[5] == 0)
    assert np.all(offsets[5] == 0x3C)  # e4m3(1.5)


def test_residual_equal_to_reference_gives_alpha_one(oracle):
    levels = np.array([(c * 7) % 16 for c in range(128)], np.float32)
    levels[0::32] = 15
    levels[1::32] = 0
    anchor_row = levels * 0.25  # exactly on the INT4 grid -> restored anchor == input
    records = ((2, 32), (4, 32))
    cache = _quantize_one(oracle, records, [anchor_row, anchor_row], anchor=1)
    codes, scales, offsets, alpha = _record(cache, 0, records, 0)
    assert alpha[5] == BF16_ONE
    assert not codes[5].any() and not scales[5].any() and not offsets[5].any()


def test_zero_reference_gives_alpha_zero(oracle):
    rng = np.random.default_rng(3)
    residual = rng.standard_normal(128).astype(np.float32)
    records = ((2, 32), (4, 32))
    cache = _quantize_one(oracle, records, [residual, np.zeros(128, np.float32)], anchor=1)
    _, _, _, alpha = _record(cache, 0, records, 0)
    assert alpha[5] == 0x0000


def test_unit_and_norm_alpha(oracle):
    levels = np.array([(c * 5) % 16 for c in range(128)], np.float32)
    levels[0::32] = 15
    levels[1::32] = 0
    anchor_row = levels * 0.25
    records = ((2, 32), (4, 32))
    unit = _quantize_one(oracle, records, [2 * anchor_row, anchor_row], anchor=1, coefficient="unit")
    assert _record(unit, 0, records, 0)[3][5] == BF16_ONE
    norm = _quantize_one(oracle, records, [2 * anchor_row, anchor_row], anchor=1, coefficient="norm")
    assert _record(norm, 0, records, 0)[3][5] == 0x4000  # ||2x|| / ||x|| = 2
    ls = _quantize_one(oracle, records, [2 * anchor_row, anchor_row], anchor=1, coefficient="ls")
    assert _record(ls, 0, records, 0)[3][5] == 0x4000


def test_ls_alpha_is_least_squares_optimum(oracle):
    """Stored alpha = bf16(<x, ref> / <ref, ref>) with ref the restored anchor (to FP32 sum error)."""
    g = make_group(40, 3, 128, OURO_G32, seed=17, rotation=False, mean=False)
    cache = g.oracle_cache(oracle)
    anchor_k, _ = oracle.dequantize(cache, g.slots.numpy(), 128, None, g.records, "anchor", 3, 3)
    ref = torch.from_numpy(anchor_k.view(np.int16)).view(torch.bfloat16).double()
    checked = 0
    for loop in range(3):
        x = g.pairs[loop][0].double()
        optimum = (x * ref).sum(-1) / (ref * ref).sum(-1)
        offset = record_offsets(128, g.records, 16)[loop]
        for n, slot in enumerate(g.slots.tolist()):
            block, token = divmod(slot, 16)
            for h in range(3):
                page = cache[0, block, h].reshape(-1)
                a = page[offset + 16 * (32 + 8) + 2 * token: offset + 16 * (32 + 8) + 2 * token + 2]
                stored = torch.tensor([int(a[0]) | (int(a[1]) << 8)], dtype=torch.int32).to(torch.int16)
                value = stored.view(torch.bfloat16).double().item()
                target = optimum[n, h].item()
                assert abs(value - target) <= abs(target) * 2.0 ** -8 + 1e-6
                checked += 1
    assert checked == 3 * 40 * 3


def test_rotation_is_x_times_r(oracle):
    rng = np.random.default_rng(4)
    dim = 128
    x = _bf16(rng.standard_normal(dim))
    rotation = workloads.random_sign_rotation(1, dim, 9)[0]
    got = oracle.rotate(x, workloads.bf16_bits(rotation))
    xd = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).double()
    expected = (xd @ rotation.double()).numpy()
    bound = dim * 2.0 ** -24 * (np.abs(xd.numpy()) @ np.abs(rotation.double().numpy()))
    assert np.all(np.abs(got - expected) <= bound + 1e-12)
    # a transposed operand is far off
    wrong = (rotation.double() @ xd).numpy()
    assert np.abs(got - wrong).max() > 1e-2


def test_identity_rotation_equals_no_rotation(oracle):
    g = make_group(23, 2, 128, OURO_G32, seed=8, rotation=False)
    plain = g.oracle_cache(oracle)
    eye = torch.eye(128, dtype=torch.float16).expand(2, 128, 128).contiguous()
    g.key_rotation, g.value_rotation = eye, eye
    assert np.array_equal(g.oracle_cache(oracle), plain)


def test_negative_slots_leave_cache_untouched(oracle):
    g = make_group(30, 2, 128, OURO_G32, seed=10, skipped=30)
    sentinel = np.full(g.cache_shape, 0xA5, np.uint8)
    assert np.array_equal(g.oracle_cache(oracle, sentinel.copy()), sentinel)


def test_token_order_invariance(oracle):
    g = make_group(29, 2, 96, ((2, 16),) * 3 + ((4, 32),), seed=12)
    baseline = g.oracle_cache(oracle)
    perm = torch.randperm(29, generator=torch.Generator().manual_seed(1))
    g.pairs = [(k[perm], v[perm]) for k, v in g.pairs]
    g.slots = g.slots[perm]
    assert np.array_equal(g.oracle_cache(oracle), baseline)


def test_anchor_restore_matches_independent_decode(oracle):
    """Restored anchor = bf16(code*scale + offset) [+ bf16(mean)], decoded here with numpy/torch."""
    g = make_group(12, 2, 128, OURO_G32, seed=14, rotation=True, mean=True)
    cache = g.oracle_cache(oracle)
    k, v = oracle.dequantize(cache, g.slots.numpy(), 128, g.key_mean.numpy(), g.records, "anchor", 3, 3)
    offset = record_offsets(128, g.records, 16)[3]
    fp8 = lambda b: torch.from_numpy(np.ascontiguousarray(b)).view(torch.float8_e4m3fn).float().numpy()
    for n, slot in enumerate(g.slots.tolist()):
        block, token = divmod(slot, 16)
        for plane, got in ((0, k), (1, v)):
            for h in range(2):
                region = cache[plane, block, h].reshape(-1)[offset:]
                codes = _unpack(region[64 * token: 64 * token + 64], 4)
                scales = fp8(region[16 * 64 + 4 * token: 16 * 64 + 4 * token + 4])
                offsets = fp8(region[16 * 68 + 4 * token: 16 * 68 + 4 * token + 4])
                deq = torch.from_numpy((codes * np.repeat(scales, 32) + np.repeat(offsets, 32)).astype(np.float32))
                deq = deq.to(torch.bfloat16)
                if plane == 0:
                    deq = (deq.float() + g.key_mean[3, h].to(torch.bfloat16).float()).to(torch.bfloat16)
                assert np.array_equal(got[n, h], deq.view(torch.int16).numpy().view(np.uint16))


def test_adjacent_chain_restores_from_previous_loop(oracle):
    g = make_group(16, 2, 128, ((4, 32), (2, 32), (2, 32)), seed=15, mode="adjacent", anchor=0,
                   rotation=False, mean=False)
    cache = g.oracle_cache(oracle)
    k0, _ = oracle.dequantize(cache, g.slots.numpy(), 128, None, g.records, "adjacent", 0, 0)
    k1, _ = oracle.dequantize(cache, g.slots.numpy(), 128, None, g.records, "adjacent", 0, 1)
    k2, _ = oracle.dequantize(cache, g.slots.numpy(), 128, None, g.records, "adjacent", 0, 2)
    to = lambda b: torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).double().numpy()
    # each loop's restored key tracks its own input better than the previous loop's restore does
    for loop, restored, previous in ((1, k1, k0), (2, k2, k1)):
        x = g.pairs[loop][0].double().numpy()
        assert np.abs(to(restored) - x).mean() < np.abs(to(previous) - x).mean()
        assert np.abs(to(restored) - x).mean() < 0.08
