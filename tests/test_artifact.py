"""Rotation artifact loader, slot binding and V-rotation absorption
(residualquant_amd/artifact.py), after the reference's
plugins/residual_quantization/src/residual_quantization/plugin.py:25-64,
install_model.py:154-196 and weights.py:8-62.

The artifacts are written here with torch.save (no reference files exist
for this format); the absorption is checked against the identity it must
keep, (x W_v^T) R = x (R^T W_v)^T per head and a W_o^T = (a R)(W_o R)^T for
an orthogonal R, in FP64."""

from __future__ import annotations

import hashlib

import pytest
import torch

from residualquant_amd import artifact as art
from residualquant_amd import workloads

GROUPS = [[(2, 32), (4, 32)], [(2, 16), (2, 32), (4, 32)]]
GEOMETRY = art.ModelGeometry(heads=2, head_dim=32, layers=3, recurrence=5, model="ouro-test")


def _artifact(rotation_dims=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    shape = (3, 2, 32, 32) if rotation_dims == 4 else (2, 3, 2, 32, 32)
    records = [r for group in GROUPS for r in group]
    return {
        "format_version": 2,
        "model": "ouro-test",
        "schedule": [b for b, _ in records],
        "groups": [s for _, s in records],
        "key_rotations": torch.randn(shape, generator=g).to(torch.float16),
        "value_rotations": torch.randn(shape, generator=g).to(torch.float16),
        "key_means": torch.randn((5, 3, 2, 32), generator=g),
    }


def _save(tmp_path, data, name="rotations.pt"):
    path = tmp_path / name
    torch.save(data, path)
    return path, hashlib.sha256(path.read_bytes()).hexdigest()


@pytest.mark.parametrize("dims", [4, 5])
def test_load_round_trip(tmp_path, dims):
    data = _artifact(dims)
    path, digest = _save(tmp_path, data)
    loaded = art.load_rotation_artifact(path, digest, GROUPS, GEOMETRY)
    for name in ("key_rotations", "value_rotations", "key_means"):
        assert torch.equal(loaded[name], data[name])


def _expect(tmp_path, data, error, match, geometry=GEOMETRY, groups=GROUPS, digest=None):
    path, good = _save(tmp_path, data)
    with pytest.raises(error, match=match):
        art.load_rotation_artifact(path, digest or good, groups, geometry)


def test_load_rejects(tmp_path):
    _expect(tmp_path, _artifact(), ValueError, "hash mismatch", digest="0" * 64)
    bad = _artifact()
    bad["schedule"][0] = 4
    _expect(tmp_path, bad, AssertionError, "schedule")
    bad = _artifact()
    bad["format_version"] = 1
    _expect(tmp_path, bad, AssertionError, "format_version")
    _expect(tmp_path, _artifact(), AssertionError, "model",
            geometry=art.ModelGeometry(2, 32, 3, 5, model="other"))
    _expect(tmp_path, _artifact(), ValueError, "every model recurrence",
            geometry=art.ModelGeometry(2, 32, 3, 6))
    bad = _artifact()
    bad["key_rotations"] = bad["key_rotations"][0]
    _expect(tmp_path, bad, ValueError, "four or five dimensions")
    bad = _artifact()
    bad["value_rotations"] = bad["value_rotations"][:, :, :, :16]
    _expect(tmp_path, bad, ValueError, r"value_rotations shape \(3, 2, 32, 16\) != model shape \(3, 2, 32, 32\)")
    bad = _artifact()
    bad["key_rotations"] = bad["key_rotations"].float()
    _expect(tmp_path, bad, AssertionError, "FP16")
    bad = _artifact()
    bad["value_rotations"][1, 0, 3, 4] = float("inf")
    _expect(tmp_path, bad, AssertionError, "finite")
    bad = _artifact()
    bad["key_means"] = bad["key_means"].double()
    _expect(tmp_path, bad, AssertionError, "FP32")


def test_prepare_value_rotation_splits_four_dimensional():
    data = _artifact(4)
    prepared, rotations = art.prepare_value_rotation(data)
    assert prepared["value_rotations"] is None and torch.equal(rotations, data["value_rotations"])
    assert data["value_rotations"] is not None  # the input is not modified
    data5 = _artifact(5)
    prepared, rotations = art.prepare_value_rotation(data5)
    assert rotations is None and prepared is data5
    assert art.prepare_value_rotation(None) == (None, None)


@pytest.mark.parametrize("dims", [4, 5])
def test_bind_slots(dims):
    data, _ = art.prepare_value_rotation(_artifact(dims))
    slots = art.bind_slots(data, GROUPS, 3, torch.device("cpu"))
    assert [len(row) for row in slots] == [3, 3]
    starts = [0, 2]
    for group, row in enumerate(slots):
        for layer, slot in enumerate(row):
            keys = data["key_rotations"]
            expected_key = keys[layer] if dims == 4 else keys[group][layer]
            assert torch.equal(slot.key_rotation, expected_key)
            if dims == 4:
                assert slot.value_rotation is None
            else:
                assert torch.equal(slot.value_rotation, data["value_rotations"][group][layer])
            size = len(GROUPS[group])
            expected_mean = data["key_means"][starts[group]:starts[group] + size, layer]
            assert slot.key_mean.shape == (size, 2, 32) and torch.equal(slot.key_mean, expected_mean)
    empty = art.bind_slots(None, GROUPS, 3, torch.device("cpu"))
    assert all(s.key_rotation is None and s.value_rotation is None and s.key_mean is None
               for row in empty for s in row)


def test_absorb_value_rotation_keeps_the_layer_function():
    heads, dim, hidden = 2, 32, 48
    q_size = kv_size = heads * dim
    g = torch.Generator().manual_seed(4)
    qkv = (torch.randn((q_size + 2 * kv_size, hidden), generator=g) * 0.1).to(torch.bfloat16)
    o = (torch.randn((hidden, heads * dim), generator=g) * 0.1).to(torch.bfloat16)
    rotation = workloads.random_sign_rotation(heads, dim, 5)
    qkv0, o0 = qkv.clone(), o.clone()
    art.absorb_value_rotation(qkv, o, rotation, heads, dim, q_size, kv_size)
    assert torch.equal(qkv[:q_size + kv_size], qkv0[:q_size + kv_size])  # Q and K rows untouched
    r = rotation.double()
    x = torch.randn((5, hidden), generator=g, dtype=torch.float64)
    v_rotated = torch.einsum("nhd,hde->nhe", (x @ qkv0[q_size + kv_size:].double().t()).view(5, heads, dim), r)
    v_absorbed = (x @ qkv[q_size + kv_size:].double().t()).view(5, heads, dim)
    assert torch.allclose(v_absorbed, v_rotated, rtol=2e-2, atol=2e-2)
    a = torch.randn((5, heads, dim), generator=g, dtype=torch.float64)
    a_rotated = torch.einsum("nhd,hde->nhe", a, r).reshape(5, -1)
    assert torch.allclose(a_rotated @ o.double().t(), a.reshape(5, -1) @ o0.double().t(), rtol=2e-2, atol=2e-2)


def test_absorb_rejects():
    qkv = torch.zeros((6 * 32, 16), dtype=torch.bfloat16)
    o = torch.zeros((16, 64), dtype=torch.bfloat16)
    rotation = torch.zeros((2, 32, 32), dtype=torch.float16)
    with pytest.raises(ValueError, match="geometry"):
        art.absorb_value_rotation(qkv, o, rotation[:1], 2, 32, 64, 64)
    with pytest.raises(ValueError, match="BF16 weights"):
        art.absorb_value_rotation(qkv.float(), o, rotation, 2, 32, 64, 64)
    with pytest.raises(ValueError, match="tensor parallel size 1"):
        art.absorb_value_rotation(qkv[:-32], o, rotation, 2, 32, 64, 64)
