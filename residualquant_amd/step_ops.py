"""Fused elementwise ops around the packed attention in one looped-decoder layer.

One Ouro layer (plugins/looped_transformers/src/looped_transformers/ouro.py:101-157)
brackets its attention with vLLM's fused add + RMSNorm, the rotary embedding
of Q and K, and Qwen2MLP's SiLU(gate) * up.  Each op here is one HIP launch
through ``librq_hip.so`` (rq_rms_norm, rq_rope_qkv, rq_silu_mul); there is no
CPU or torch fallback.  Work is enqueued on the current HIP stream of the
input's device.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _rows(tensor: torch.Tensor, name: str) -> None:
    _require(tensor.is_cuda and tensor.dtype == torch.bfloat16 and tensor.dim() == 2 and tensor.stride(1) == 1,
             f"{name} must be BF16 [rows, channels] on a HIP device with unit channel stride")


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: Optional[torch.Tensor] = None,
             out: Optional[torch.Tensor] = None, pre_weight: Optional[torch.Tensor] = None):
    """RMSNorm of ``x`` (vLLM RMSNorm.forward); with ``residual``, the fused form.

    Without a residual returns ``y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight)``.
    With one, ``residual`` is updated in place to ``bf16(x + residual)`` and
    ``(y, residual)`` is returned, y normalizing the updated residual
    (vLLM's fused_add_rms_norm contract).  With ``pre_weight``, ``x`` is
    first replaced by ``rms_norm(x, pre_weight, eps)`` in the same launch.
    """
    _rows(x, "x")
    rows, hidden = x.shape
    for w in (weight, pre_weight):
        if w is not None:
            _require(w.is_cuda and w.dtype == torch.bfloat16 and w.shape == (hidden,) and w.is_contiguous(),
                     "RMSNorm weight must be a contiguous BF16 [hidden] vector")
    if residual is not None:
        _rows(residual, "residual")
        _require(residual.shape == x.shape and residual.device == x.device, "residual must match x")
    if out is None:
        out = torch.empty_like(x, memory_format=torch.contiguous_format)
    _rows(out, "out")
    _require(out.shape == x.shape and out.device == x.device, "out must match x")
    with torch.cuda.device(x.device):
        status = _lib.lib().rq_rms_norm(
            x.data_ptr(), x.stride(0), pre_weight.data_ptr() if pre_weight is not None else None,
            residual.data_ptr() if residual is not None else None,
            residual.stride(0) if residual is not None else 0,
            residual.data_ptr() if residual is not None else None,
            residual.stride(0) if residual is not None else 0, weight.data_ptr(), out.data_ptr(), out.stride(0),
            rows, hidden, float(eps), _stream(x.device))
    _lib.check(status)
    return out if residual is None else (out, residual)


def rope_qkv(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int,
             head_dim: int, key_stage: Optional[torch.Tensor] = None,
             value_stage: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rotate-half rotary embedding of the Q and K parts of fused ``[q | k | v]`` rows.

    ``cos``/``sin`` are FP32 ``[max_position, head_dim / 2]`` tables
    (get_rope with rotary_dim = head_dim); positions int64 ``[rows]`` (clamped
    to the tables).  Returns rotated ``(q, k)`` as ``[rows, heads, head_dim]``;
    when ``key_stage``/``value_stage`` are given (``[rows, heads, head_dim]``,
    sharing one row stride) the rotated K and the raw V are also copied there.
    """
    _rows(qkv, "qkv")
    rows = qkv.size(0)
    _require(qkv.size(1) == 3 * heads * head_dim, "qkv rows must hold [q | k | v] of heads * head_dim each")
    _require(positions.is_cuda and positions.dtype == torch.int64 and positions.is_contiguous()
             and positions.numel() == rows, "Contiguous INT64 positions, one per row, required")
    for table in (cos, sin):
        _require(table.is_cuda and table.dtype == torch.float32 and table.is_contiguous() and table.dim() == 2
                 and table.size(1) == head_dim // 2 and table.shape == cos.shape,
                 "Contiguous FP32 [positions, head_dim / 2] cos/sin tables required")
    query = torch.empty((rows, heads, head_dim), dtype=qkv.dtype, device=qkv.device)
    key = torch.empty_like(query)
    stage_stride = 0
    for stage in (key_stage, value_stage):
        if stage is not None:
            _require(stage.is_cuda and stage.dtype == torch.bfloat16 and stage.shape == (rows, heads, head_dim)
                     and stage.stride(2) == 1 and stage.stride(1) == head_dim,
                     "K/V staging must be BF16 [rows, heads, head_dim] with packed trailing strides")
            _require(stage_stride in (0, stage.stride(0)), "K and V staging must share one row stride")
            stage_stride = stage.stride(0)
    with torch.cuda.device(qkv.device):
        status = _lib.lib().rq_rope_qkv(
            qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.size(0), heads,
            head_dim, rows, query.data_ptr(), query.stride(0), key.data_ptr(), key.stride(0),
            key_stage.data_ptr() if key_stage is not None else None,
            value_stage.data_ptr() if value_stage is not None else None, stage_stride, _stream(qkv.device))
    _lib.check(status)
    return query, key


def silu_mul(gate_up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``bf16(silu(gate) * up)`` of ``[rows, 2 * width]`` rows (vLLM SiluAndMul)."""
    _rows(gate_up, "gate_up")
    rows, double = gate_up.shape
    _require(double % 4 == 0, "gate_up rows must hold two halves of an even width")
    width = double // 2
    if out is None:
        out = torch.empty((rows, width), dtype=gate_up.dtype, device=gate_up.device)
    _rows(out, "out")
    _require(out.shape == (rows, width) and out.device == gate_up.device, "out must be [rows, width]")
    with torch.cuda.device(gate_up.device):
        status = _lib.lib().rq_silu_mul(gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(), out.stride(0), rows,
                                        width, _stream(gate_up.device))
    _lib.check(status)
    return out


LINEAR_MAX_ROWS = 8


def linear_rows(x: torch.Tensor, weight: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``bf16(x @ weight.T)`` for 1-8 BF16 rows (rq_linear_rows), FP32 accumulation.

    ``weight`` is a contiguous BF16 ``[out_features, in_features]`` linear
    weight; ``in_features`` a multiple of 8 up to 6144.  The projections of a
    decode step at small batch, streamed as matrix-vector products."""
    _rows(x, "x")
    rows, in_features = x.shape
    _require(weight.is_cuda and weight.dtype == torch.bfloat16 and weight.dim() == 2 and weight.is_contiguous()
             and weight.size(1) == in_features and weight.device == x.device,
             "weight must be a contiguous BF16 [out_features, in_features] tensor on x's device")
    if out is None:
        out = torch.empty((rows, weight.size(0)), dtype=torch.bfloat16, device=x.device)
    _rows(out, "out")
    _require(out.shape == (rows, weight.size(0)) and out.device == x.device, "out must be [rows, out_features]")
    with torch.cuda.device(x.device):
        status = _lib.lib().rq_linear_rows(x.data_ptr(), x.stride(0), weight.data_ptr(), out.data_ptr(), out.stride(0),
                                          rows, weight.size(0), in_features, _stream(x.device))
    _lib.check(status)
    return out
