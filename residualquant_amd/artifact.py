"""Rotation artifact: loading, validation, per-slot binding and V-rotation absorption.

The calibrated rotations and key means reach the packed path through an
artifact file (format_version 2), as in the reference's loader
(plugins/residual_quantization/src/residual_quantization/plugin.py:25-64),
its slot binding (install_model.py:154-196) and its weight transform
(weights.py:8-62).  This module keeps those semantics without vLLM: the
geometry comes from a ``ModelGeometry`` instead of the HF config, the binding
returns tensors per (group, physical layer) instead of setting attributes on
vLLM ``Attention`` objects, and the absorption takes the two projection
weights instead of a model.  The checks raise the reference's exception types
(``ValueError`` where it raises, ``AssertionError`` where it asserts).

Artifact dictionary (``torch.load(..., weights_only=True)``):
  format_version   2
  model            the looped model's name (``model_config.loop_model``)
  schedule, groups bits and group sizes of every record, group-major
  key_rotations    FP16 [layers, H, D, D] (shared by every group) or
                   [groups, layers, H, D, D]
  value_rotations  the same shapes; 4-D matrices are folded into the
                   projection weights, 5-D ones are applied in the kernels
  key_means        FP32 [recurrence, layers, H, D]
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass
from pathlib import Path
from typing import List, Optional, Sequence, Tuple

import torch

Records = Sequence[Tuple[int, int]]


@dataclass(frozen=True)
class ModelGeometry:
    """The model fields the artifact is checked against (plugin.py:38-42)."""

    heads: int
    head_dim: int
    layers: int  # n_layers_in_recurrent_block (physical recurrent layers)
    recurrence: int  # mean_recurrence (loops)
    model: Optional[str] = None  # loop_model; None skips the name check


def _require(condition: bool, message: str) -> None:
    # The reference asserts these (plugin.py:35-37, :44-45, :61-63).
    if not condition:
        raise AssertionError(message)


def load_rotation_artifact(path, sha256: str, packed_groups: Sequence[Records],
                           geometry: ModelGeometry) -> dict:
    """Read and validate a rotation artifact (plugin.py:25-64).

    ``packed_groups`` is the ``packed_groups`` configuration: one list of
    ``(bits, group)`` records per loop group.  Returns the loaded dictionary
    (CPU tensors)."""
    path = Path(path)
    if hashlib.sha256(path.read_bytes()).hexdigest() != sha256:
        raise ValueError("Rotation artifact hash mismatch")
    data = torch.load(path, map_location="cpu", weights_only=True)
    records = [tuple(record) for schedule in packed_groups for record in schedule]
    _require(list(data["schedule"]) == [bits for bits, _ in records], "artifact schedule differs from packed_groups")
    _require(list(data["groups"]) == [group for _, group in records], "artifact groups differ from packed_groups")
    h, d, layers = geometry.heads, geometry.head_dim, geometry.layers
    _require(data["format_version"] == 2, "artifact format_version must be 2")
    if geometry.model is not None:
        _require(data["model"] == geometry.model, "artifact model differs from the loop model")
    if sum(map(len, packed_groups)) != geometry.recurrence:
        raise ValueError("Packed groups must describe every model recurrence exactly once")
    group_count = len(packed_groups)
    matrix_shape = (layers, h, d, d)
    for name in ("key_rotations", "value_rotations"):
        rotation = data[name]
        if rotation.ndim not in (4, 5):
            raise ValueError(f"{name} must have four or five dimensions")
        expected = (group_count, *matrix_shape) if rotation.ndim == 5 else matrix_shape
        if tuple(rotation.shape) != expected:
            raise ValueError(f"{name} shape {tuple(rotation.shape)} != model shape {expected}")
        _require(rotation.dtype == torch.float16, f"{name} must be FP16")
        _require(bool(torch.isfinite(rotation).all()), f"{name} must be finite")
    _require(tuple(data["key_means"].shape) == (geometry.recurrence, layers, h, d), "key_means shape")
    _require(data["key_means"].dtype == torch.float32, "key_means must be FP32")
    _require(bool(torch.isfinite(data["key_means"]).all()), "key_means must be finite")
    return data


def prepare_value_rotation(artifact: Optional[dict]):
    """Split off 4-D value rotations for weight folding (weights.py:40-49).

    Returns ``(artifact, rotations)``: 5-D value rotations stay in the
    artifact (the kernels apply them) and ``rotations`` is None; 4-D ones are
    returned for ``absorb_value_rotation`` and removed from the artifact."""
    if artifact is None:
        return None, None
    rotation = artifact["value_rotations"]
    if rotation.ndim == 5:
        return artifact, None
    if rotation.ndim != 4:
        raise ValueError("Value rotations must have four or five dimensions")
    return dict(artifact, value_rotations=None), rotation


@dataclass
class SlotTensors:
    """What one (group, physical layer) attention slot passes to the ops:
    K rotation FP16 [H, D, D] (or None), V rotation FP16 [H, D, D] (or None,
    also when folded into the weights), key means FP32 [records, H, D] (or None)."""

    key_rotation: Optional[torch.Tensor]
    value_rotation: Optional[torch.Tensor]
    key_mean: Optional[torch.Tensor]


def bind_slots(artifact: Optional[dict], packed_groups: Sequence[Records], layers: int,
               device: torch.device) -> List[List[SlotTensors]]:
    """Per-group, per-layer tensors of the slot binding (install_model.py:154-196).

    ``artifact`` is the result of ``prepare_value_rotation`` (4-D value
    rotations already split off).  Returns ``slots[group][layer]``; the loops
    of a group share their layer's tensors, each loop passing its own
    ``loop_index`` to the ops."""
    shared_key_rotations = None
    if artifact is not None and artifact["key_rotations"].ndim == 4:
        shared_key_rotations = artifact["key_rotations"].contiguous().to(device)
    slots: List[List[SlotTensors]] = []
    group_start = 0
    for group_index, schedule in enumerate(packed_groups):
        size = len(schedule)
        group_key_rotations = shared_key_rotations
        group_value_rotations = group_key_means = None
        if artifact is not None:
            group_key_means = artifact["key_means"][group_start:group_start + size]
            if artifact["key_rotations"].ndim == 5:
                group_key_rotations = artifact["key_rotations"][group_index].contiguous().to(device)
            if artifact["value_rotations"] is not None:
                group_value_rotations = artifact["value_rotations"][group_index].contiguous().to(device)
        row = []
        for layer in range(layers):
            row.append(SlotTensors(
                key_rotation=None if group_key_rotations is None else group_key_rotations[layer],
                value_rotation=None if group_value_rotations is None else group_value_rotations[layer],
                key_mean=None if group_key_means is None else group_key_means[:, layer].contiguous().to(device)))
        slots.append(row)
        group_start += size
    return slots


@torch.no_grad()
def absorb_value_rotation(qkv_weight: torch.Tensor, o_weight: torch.Tensor, rotation: torch.Tensor,
                          heads: int, head_dim: int, q_size: int, kv_size: int) -> None:
    """Fold row-vector ``V @ R`` and ``output @ R.T`` into BF16 projections (weights.py:8-37).

    ``qkv_weight`` BF16 [q_size + 2 kv_size, hidden] (Q, K, V rows, as vLLM's
    fused QKV holds them), ``o_weight`` BF16 [hidden, heads * head_dim],
    ``rotation`` [heads, head_dim, head_dim].  In place, FP32 arithmetic: the
    V rows of head h become R_h^T W_v,h and the O columns of head h become
    W_o,h R_h, so an orthogonal R leaves the layer's function unchanged while
    the values the cache stores are rotated."""
    if tuple(rotation.shape) != (heads, head_dim, head_dim):
        raise ValueError("Value rotation does not match attention geometry")
    if qkv_weight.dtype != torch.bfloat16 or o_weight.dtype != torch.bfloat16:
        raise ValueError("Value rotation absorption requires BF16 weights")
    value = qkv_weight[q_size + kv_size:]
    hidden = value.shape[1]
    if value.shape[0] != heads * head_dim or o_weight.shape[1] != heads * head_dim:
        raise ValueError("Value rotation absorption requires tensor parallel size 1")
    r = rotation.to(device=qkv_weight.device, dtype=torch.float32)
    allow_tf32 = torch.backends.cuda.matmul.allow_tf32
    try:
        # Full FP32 products (no reduced-precision inner products), with
        # contiguous operands (batched BF16 products with a transposed operand
        # are avoided on this platform).
        torch.backends.cuda.matmul.allow_tf32 = False
        transformed = torch.bmm(r.transpose(1, 2).contiguous(), value.float().reshape(heads, head_dim, hidden))
        value.copy_(transformed.reshape_as(value))
        columns = o_weight.float().reshape(-1, heads, head_dim).permute(1, 0, 2).contiguous()
        transformed = torch.bmm(columns, r)
        o_weight.copy_(transformed.permute(1, 0, 2).reshape_as(o_weight))
    finally:
        torch.backends.cuda.matmul.allow_tf32 = allow_tf32
