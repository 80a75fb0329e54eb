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


def _check_finite(tensor: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    _require(tensor.dtype == dtype, f"{name} must be {'FP16' if dtype == torch.float16 else 'FP32'}")
    _require(bool(torch.isfinite(tensor).all()), f"{name} must be finite")


@dataclass(frozen=True)
class _Expected:
    """What a valid artifact holds for one model and packed_groups."""

    bits: Tuple[int, ...]
    group_sizes: Tuple[int, ...]
    groups: int  # loop groups
    matrices: Tuple[int, int, int, int]  # [layers, H, D, D] of one group's rotations
    key_means: Tuple[int, int, int, int]  # [recurrence, layers, H, D]

    @classmethod
    def of(cls, packed_groups: Sequence[Records], geometry: ModelGeometry) -> "_Expected":
        flat = [tuple(record) for schedule in packed_groups for record in schedule]
        h, d, layers = geometry.heads, geometry.head_dim, geometry.layers
        return cls(bits=tuple(b for b, _ in flat), group_sizes=tuple(g for _, g in flat),
                   groups=len(packed_groups), matrices=(layers, h, d, d),
                   key_means=(geometry.recurrence, layers, h, d))

    def rotation_shape(self, ndim: int) -> Tuple[int, ...]:
        # Shared by every group (4-D) or one set per group (5-D).
        return self.matrices if ndim == 4 else (self.groups, *self.matrices)


def load_rotation_artifact(path, sha256: str, packed_groups: Sequence[Records],
                           geometry: ModelGeometry) -> dict:
    """Read and validate a rotation artifact (plugin.py:25-64).

    ``packed_groups`` is the ``packed_groups`` configuration: one list of
    ``(bits, group)`` records per loop group.  The file must match ``sha256``;
    its schedule must be ``packed_groups`` flattened; the groups together must
    cover the model's recurrence; each rotation set must be FP16, finite and
    shaped for the model (shared or per group), and the key means FP32 and
    finite.  Returns the loaded dictionary (CPU tensors)."""
    raw = Path(path).read_bytes()
    if hashlib.sha256(raw).hexdigest() != sha256:
        raise ValueError("Rotation artifact hash mismatch")
    data = torch.load(path, map_location="cpu", weights_only=True)
    want = _Expected.of(packed_groups, geometry)
    _require(tuple(data["schedule"]) == want.bits, "artifact schedule differs from packed_groups")
    _require(tuple(data["groups"]) == want.group_sizes, "artifact groups differ from packed_groups")
    _require(data["format_version"] == 2, "artifact format_version must be 2")
    _require(geometry.model is None or data["model"] == geometry.model, "artifact model differs from the loop model")
    if len(want.bits) != geometry.recurrence:
        raise ValueError("Packed groups must describe every model recurrence exactly once")
    for name in ("key_rotations", "value_rotations"):
        tensor = data[name]
        if tensor.ndim not in (4, 5):
            raise ValueError(f"{name} must have four or five dimensions")
        shape = want.rotation_shape(tensor.ndim)
        if tuple(tensor.shape) != shape:
            raise ValueError(f"{name} shape {tuple(tensor.shape)} != model shape {shape}")
        _check_finite(tensor, name, torch.float16)
    _require(tuple(data["key_means"].shape) == want.key_means, "key_means shape")
    _check_finite(data["key_means"], "key_means", torch.float32)
    return data


def prepare_value_rotation(artifact: Optional[dict]):
    """Split off 4-D value rotations for weight folding (weights.py:40-49).

    Returns ``(artifact, rotations)``: 5-D value rotations are applied by the
    kernels and stay in the artifact (``rotations`` None); a 4-D set is
    returned for ``absorb_value_rotation`` and cleared in a copy of the
    artifact."""
    if artifact is None:
        return None, None
    rotation = artifact["value_rotations"]
    if rotation.ndim not in (4, 5):
        raise ValueError("Value rotations must have four or five dimensions")
    if rotation.ndim == 5:
        return artifact, None
    kept = dict(artifact)
    kept["value_rotations"] = None
    return kept, rotation


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
