"""Pins of the oracle's scalar formats and page layout (CPU).

FP8 E4M3 against torch.float8_e4m3fn (an independent OCP implementation),
BF16 rounding against torch and exact rationals, page widths against the
known answers the reference states three times (common/cache.cuh:14-17,
src/residual_quantization/install_model.py:34-38,
experiments/kv_memory_latency/capacity.py:48-51).
"""

from __future__ import annotations

import math
import struct
from fractions import Fraction

import numpy as np
import pytest
import torch

from residualquant_amd import layout


def _f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def test_e4m3_decode_table_matches_torch(oracle):
    codes = torch.arange(256, dtype=torch.int64).to(torch.uint8)
    expected = codes.view(torch.float8_e4m3fn).float().numpy()
    got = np.array([oracle.e4m3_to_f32(c) for c in range(256)], dtype=np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(np.isnan(got), nan)
    assert nan.sum() == 2  # S.1111.111 only
    assert np.array_equal(got[~nan], expected[~nan])
    assert oracle.e4m3_to_f32(0x7E) == 448.0 and oracle.e4m3_to_f32(0x01) == 2.0 ** -9


def _torch_e4m3(values: np.ndarray) -> np.ndarray:
    clamped = torch.from_numpy(values.astype(np.float32)).clamp(-448, 448)
    return clamped.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_encode_matches_torch_on_random_and_midpoints(oracle):
    rng = np.random.default_rng(0)
    randoms = np.concatenate([
        rng.standard_normal(4000) * 10.0 ** rng.integers(-4, 3, 4000),
        rng.uniform(-600, 600, 2000),
    ]).astype(np.float32)
    finite = np.array([oracle.e4m3_to_f32(c) for c in range(256) if (c & 0x7F) != 0x7F], np.float32)
    finite = np.unique(finite)
    midpoints = ((finite[1:].astype(np.float64) + finite[:-1]) / 2).astype(np.float32)
    nudged = np.concatenate([np.nextafter(midpoints, np.float32(np.inf)),
                             np.nextafter(midpoints, np.float32(-np.inf))])
    values = np.concatenate([randoms, midpoints, nudged, finite, [0.0, -0.0, 448.0, 449.0, 1e6, -1e6]])
    values = values.astype(np.float32)
    got = np.array([oracle.e4m3_from_f32(float(v)) for v in values], dtype=np.uint8)
    assert np.array_equal(got, _torch_e4m3(values))


def test_e4m3_ties_go_to_even(oracle):
    # 1.0625 lies halfway between 1.0 (even mantissa) and 1.125.
    assert oracle.e4m3_from_f32(1.0625) == 0x38
    # 1.1875 lies halfway between 1.125 (odd) and 1.25 (even).
    assert oracle.e4m3_from_f32(1.1875) == 0x3A
    # Subnormal tie: 1.5 * 2^-9 -> 2 * 2^-9.
    assert oracle.e4m3_from_f32(1.5 * 2.0 ** -9) == 0x02
    assert oracle.e4m3_from_f32(-0.0) == 0x80 and oracle.e4m3_from_f32(0.0) == 0x00


def test_bf16_rn_matches_torch(oracle):
    rng = np.random.default_rng(1)
    values = (rng.standard_normal(20000) * 10.0 ** rng.integers(-20, 20, 20000)).astype(np.float32)
    bits = values.view(np.uint32)
    ties = ((bits & 0xFFFF0000) | 0x8000).view(np.float32)  # exact BF16 midpoints
    values = np.concatenate([values, ties])
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle.bf16_rn(float(v)) for v in values], dtype=np.uint16)
    assert np.array_equal(got, expected)


def _bf16_value(bits: int) -> Fraction:
    return Fraction(struct.unpack("<f", struct.pack("<I", bits << 16))[0])


def _exact_bf16_rne(x: Fraction) -> int:
    """RNE to BF16 of an exact rational by bracketing between BF16 neighbours."""
    if x == 0:
        return 0
    sign = 0x8000 if x < 0 else 0
    a = abs(x)
    exponent = math.floor(math.log2(a))
    while Fraction(2) ** exponent > a:
        exponent -= 1
    while Fraction(2) ** (exponent + 1) <= a:
        exponent += 1
    ulp = Fraction(2) ** (exponent - 7)
    low = (a // ulp) * ulp
    high = low + ulp
    rem = a - low
    if rem * 2 < ulp:
        chosen = low
    elif rem * 2 > ulp:
        chosen = high
    else:
        chosen = low if int(low / ulp) % 2 == 0 else high
    bits = struct.unpack("<I", struct.pack("<f", float(chosen)))[0] >> 16
    return sign | bits


def test_bf16_fma_single_rounding_against_rationals(oracle):
    rng = np.random.default_rng(2)
    checked = 0
    for _ in range(3000):
        a, b, c = (int(v) for v in rng.integers(0x3C00, 0x4400, 3))
        if rng.random() < 0.5:
            c |= 0x8000
        exact = _bf16_value(a) * _bf16_value(b) + _bf16_value(c)
        assert oracle.bf16_fma_rn(a, b, c) == _exact_bf16_rne(exact)
        checked += 1
    # Adversarial: a*b lands half an ulp away from a BF16 value with a tiny c.
    for _ in range(2000):
        a = int(rng.integers(0x3F80, 0x4000))
        b = int(rng.integers(0x3F80, 0x4000))
        p = _bf16_value(a) * _bf16_value(b)
        exponent = math.floor(math.log2(p))
        tiny = Fraction(2) ** (exponent - 30)
        c_bits = struct.unpack("<I", struct.pack("<f", float(tiny)))[0] >> 16
        for c in (c_bits, c_bits | 0x8000):
            exact = p + _bf16_value(c)
            assert oracle.bf16_fma_rn(a, b, c) == _exact_bf16_rne(exact)
    assert checked == 3000


def test_bf16_fma_double_rounding_case(oracle):
    """FP32 rounding lands exactly on a BF16 midpoint: the dropped term must decide."""
    a = 0x3F88  # 1.0625; a*a = 1.12890625, the midpoint of 1.125 and 1.1328125
    assert oracle.bf16_fma_rn(a, a, 0x0000) == 0x3F90  # tie to even
    assert oracle.bf16_fma_rn(a, a, 0x3080) == 0x3F91  # + 2^-30: just above the midpoint
    assert oracle.bf16_fma_rn(a, a, 0xB080) == 0x3F90  # - 2^-30: just below
    # FP32 alone would round 1.12890625 + 2^-30 back onto the midpoint.
    assert _f32(1.12890625 + 2.0 ** -30) == 1.12890625


def test_f16_decode_matches_numpy(oracle):
    bits = np.arange(0, 65536, 7, dtype=np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(expected)
    assert np.array_equal(got[finite], expected[finite])


@pytest.mark.parametrize("dim, records, width", [
    (128, ((2, 32), (2, 32), (2, 32), (4, 32)), 200),
    (128, ((2, 16), (2, 16), (2, 16), (4, 32)), 224),
    (96, ((2, 16), (2, 16), (2, 16), (4, 32)), 170),
    (96, ((2, 32), (2, 32), (2, 32), (4, 32)), 152),
    (128, ((4, 32),) * 4, 4 * 74),
    (128, ((2, 32),), 42),
])
def test_page_width_known_answers(oracle, dim, records, width):
    assert oracle.page_width(dim, records) == width
    assert layout.page_width(dim, records) == width


def test_footprint_ratio_matches_reference_statement():
    """Packed [2,32]x3+[4,32] is 6400 B per token-layer vs 32768 B BF16 (5.12x)."""
    heads, dim, loops = 16, 128, 4
    packed = 2 * heads * layout.page_width(dim, ((2, 32),) * 3 + ((4, 32),))
    bf16 = 2 * loops * heads * dim * 2
    assert packed == 6400 and bf16 == 32768
    assert abs(bf16 / packed - 5.12) < 1e-9


def test_staged_bytes_known_answers():
    g32 = ((2, 32),) * 3 + ((4, 32),)
    # anchor region without alpha (72 B/token) + residual record (42 B/token)
    assert layout.staged_bytes(128, g32, 16, "anchor", 3, 0) == 16 * (72 + 42)
    assert layout.staged_bytes(128, g32, 16, "anchor", 3, 3) == 16 * 72
    g16 = ((2, 16),) * 3 + ((4, 32),)
    assert layout.staged_bytes(128, g16, 16, "anchor", 3, 1) == 16 * (72 + 50)
    assert layout.staged_bytes(96, g16, 16, "anchor", 3, 1) == 16 * (54 + 38)
