"""Fused elementwise ops of the looped decoder step (residualquant_amd/step_ops.py)
against plain PyTorch FP32 references of the same ops.

The references restate vLLM's RMSNorm (fused add + norm), rotate-half
rotary embedding and SiluAndMul as the Ouro layer calls them
(plugins/looped_transformers/src/looped_transformers/ouro.py:93-157).  The
tolerance is two BF16 units in the last place of the reference,
|got - want| <= 2^-7 |want| (the kernels reduce the mean square in another
order and use the hardware exp); residual sums and copies are bit-exact."""

from __future__ import annotations

import pytest
import torch

from residualquant_amd import step_ops

pytestmark = pytest.mark.gpu


def _close(got: torch.Tensor, want: torch.Tensor) -> None:
    g, w = got.float(), want.float()
    bad = (g - w).abs() > w.abs() * 2.0 ** -7 + 1e-30
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside 2 ulps; max diff {(g - w).abs().max()}"


def _rms_reference(x, weight, eps, residual=None):
    total = x.float() if residual is None else (x.float() + residual.float()).to(torch.bfloat16).float()
    scale = torch.rsqrt(total.pow(2).mean(-1, keepdim=True) + eps)
    y = ((total * scale).to(torch.bfloat16).float() * weight.float()).to(torch.bfloat16)
    return y, total.to(torch.bfloat16)


@pytest.mark.parametrize("rows,hidden", [(1, 8), (5, 256), (33, 2048), (3, 1000)])
def test_rms_norm(device, rows, hidden):
    print(f"rms_norm rows={rows} hidden={hidden}", flush=True)
    g = torch.Generator(device=device).manual_seed(rows * 7 + hidden)
    x = (torch.randn((rows, hidden), generator=g, device=device) * 3).to(torch.bfloat16)
    weight = (torch.rand(hidden, generator=g, device=device) + 0.5).to(torch.bfloat16)
    y = step_ops.rms_norm(x, weight, 1e-6)
    want, _ = _rms_reference(x, weight, 1e-6)
    _close(y, want)


@pytest.mark.parametrize("rows,hidden", [(4, 2048), (17, 512)])
def test_fused_add_rms_norm(device, rows, hidden):
    print(f"fused add rms_norm rows={rows} hidden={hidden}", flush=True)
    g = torch.Generator(device=device).manual_seed(rows + hidden)
    x = torch.randn((rows, hidden), generator=g, device=device).to(torch.bfloat16)
    residual = (torch.randn((rows, hidden), generator=g, device=device) * 4).to(torch.bfloat16)
    weight = torch.randn(hidden, generator=g, device=device).to(torch.bfloat16)
    want, want_total = _rms_reference(x, weight, 1e-5, residual)
    y, updated = step_ops.rms_norm(x, weight, 1e-5, residual=residual)
    assert updated.data_ptr() == residual.data_ptr()
    assert torch.equal(residual, want_total)
    _close(y, want)


@pytest.mark.parametrize("rows,hidden", [(3, 2048), (32, 256)])
def test_two_norms_fused(device, rows, hidden):
    """rms_norm(x, w2, residual, pre_weight=w1) == fused_add(rms_norm(x, w1), residual) then norm with w2."""
    print(f"two fused norms rows={rows} hidden={hidden}", flush=True)
    g = torch.Generator(device=device).manual_seed(3 * rows + hidden)
    x = (torch.randn((rows, hidden), generator=g, device=device) * 5).to(torch.bfloat16)
    residual = torch.randn((rows, hidden), generator=g, device=device).to(torch.bfloat16)
    w1 = (torch.rand(hidden, generator=g, device=device) + 0.5).to(torch.bfloat16)
    w2 = (torch.rand(hidden, generator=g, device=device) + 0.5).to(torch.bfloat16)
    first, _ = _rms_reference(x, w1, 1e-6)
    want, want_total = _rms_reference(first, w2, 1e-6, residual)
    staged = residual.clone()
    y, _ = step_ops.rms_norm(x, w2, 1e-6, residual=staged, pre_weight=w1)
    chained = residual.clone()
    y2, _ = step_ops.rms_norm(step_ops.rms_norm(x, w1, 1e-6), w2, 1e-6, residual=chained)
    assert torch.equal(staged, chained) and torch.equal(y, y2)
    _close(y, want)
    _close(staged, want_total)


def test_rms_norm_strided_rows(device):
    base = torch.randn((6, 3 * 256), device=device).to(torch.bfloat16)
    x = base[:, 256:512]
    weight = torch.ones(256, dtype=torch.bfloat16, device=device)
    _close(step_ops.rms_norm(x, weight, 1e-6), _rms_reference(x, weight, 1e-6)[0])


def _rope_tables(positions, half, theta, device):
    inv = 1.0 / (theta ** (torch.arange(0, 2 * half, 2, device=device, dtype=torch.float32) / (2 * half)))
    angles = torch.arange(positions, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    return angles.cos(), angles.sin()


def _rope_reference(x, cos, sin, positions):
    c, s = cos[positions][:, None, :], sin[positions][:, None, :]
    x1, x2 = x.float().chunk(2, dim=-1)
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1).to(torch.bfloat16)


@pytest.mark.parametrize("rows,heads,head_dim", [(3, 2, 128), (32, 16, 128), (5, 4, 96)])
def test_rope_qkv_and_staging(device, rows, heads, head_dim):
    print(f"rope rows={rows} heads={heads} head_dim={head_dim}", flush=True)
    g = torch.Generator(device=device).manual_seed(rows * heads)
    cos, sin = _rope_tables(4096, head_dim // 2, 1e6, device)
    qkv = torch.randn((rows, 3 * heads * head_dim), generator=g, device=device).to(torch.bfloat16)
    positions = torch.randint(0, 4096, (rows,), generator=g, device=device)
    stage = torch.zeros((2, rows, heads, head_dim), dtype=torch.bfloat16, device=device)
    q, k = step_ops.rope_qkv(qkv, positions, cos, sin, heads, head_dim, key_stage=stage[0], value_stage=stage[1])
    size = heads * head_dim
    view = qkv.view(rows, 3, heads, head_dim)
    _close(q, _rope_reference(view[:, 0], cos, sin, positions))
    _close(k, _rope_reference(view[:, 1], cos, sin, positions))
    assert torch.equal(stage[0], k)
    assert torch.equal(stage[1], qkv[:, 2 * size:].view(rows, heads, head_dim))


def test_rope_clamps_positions_to_the_table(device):
    cos, sin = _rope_tables(64, 64, 1e4, device)
    qkv = torch.randn((2, 3 * 128), device=device).to(torch.bfloat16)
    q, k = step_ops.rope_qkv(qkv, torch.tensor([63, 500], device=device), cos, sin, 1, 128)
    last = torch.tensor([63, 63], device=device)
    _close(q, _rope_reference(qkv[:, :128].view(2, 1, 128), cos, sin, last))


@pytest.mark.parametrize("rows,width", [(1, 2), (7, 5632), (32, 1000)])
def test_silu_mul(device, rows, width):
    print(f"silu_mul rows={rows} width={width}", flush=True)
    g = torch.Generator(device=device).manual_seed(rows + width)
    gate_up = (torch.randn((rows, 2 * width), generator=g, device=device) * 4).to(torch.bfloat16)
    out = step_ops.silu_mul(gate_up)
    gate, up = gate_up.float().chunk(2, dim=-1)
    _close(out, (torch.nn.functional.silu(gate) * up).to(torch.bfloat16))


def test_rejects_unsupported_shapes(device):
    with pytest.raises(RuntimeError, match="multiple of 8 up to 2048"):
        step_ops.rms_norm(torch.zeros((2, 4096), dtype=torch.bfloat16, device=device),
                          torch.ones(4096, dtype=torch.bfloat16, device=device), 1e-6)
    with pytest.raises(RuntimeError, match="even width"):
        step_ops.silu_mul(torch.zeros((2, 6), dtype=torch.bfloat16, device=device))


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("out_features,in_features", [(6144, 2048), (2048, 5632), (100, 2048), (20, 8)])
def test_linear_rows_matches_fp32_product(device, rows, out_features, in_features):
    """bf16(x @ w^T) with FP32 accumulation: within one BF16 rounding of the
    FP32 product (the summation order differs from torch's)."""
    g = torch.Generator(device=device).manual_seed(rows * 7919 + out_features + in_features)
    weight = (torch.randn((out_features, in_features), generator=g, device=device) * 0.02).to(torch.bfloat16)
    x = torch.randn((rows, in_features), generator=g, device=device).to(torch.bfloat16)
    got = step_ops.linear_rows(x, weight)
    want = x.float() @ weight.float().t()
    assert got.shape == (rows, out_features)
    err = (got.float() - want).abs()
    assert bool((err <= want.abs() * 2.0 ** -8 + 1e-4).all()), float(err.max())


def test_linear_rows_strided_rows_and_rejections(device):
    g = torch.Generator(device=device).manual_seed(3)
    weight = (torch.randn((64, 256), generator=g, device=device) * 0.05).to(torch.bfloat16)
    wide = torch.randn((3, 512), generator=g, device=device).to(torch.bfloat16)
    x = wide[:, 128:384]  # row stride 512, 16-byte aligned
    out = torch.empty((3, 96), dtype=torch.bfloat16, device=device)[:, 16:80]
    step_ops.linear_rows(x, weight, out=out)
    want = x.float() @ weight.float().t()
    assert bool(((out.float() - want).abs() <= want.abs() * 2.0 ** -8 + 1e-4).all())
    with pytest.raises(RuntimeError, match="No compiled row-projection kernel"):
        step_ops.linear_rows(torch.zeros((9, 256), dtype=torch.bfloat16, device=device), weight)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        step_ops.linear_rows(torch.zeros((1, 12), dtype=torch.bfloat16, device=device),
                             torch.zeros((4, 12), dtype=torch.bfloat16, device=device))
