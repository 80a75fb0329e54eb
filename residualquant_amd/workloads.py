"""Seeded synthetic inputs for the packed KV-cache path.

The distributions follow the benchmark configurations of this build: the
anchor (last loop of a group) K/V is N(0, 1) with a few seeded K channels
scaled as outliers, earlier loops are anchor + N(0, 0.15^2), rotations are
random-sign Hadamard matrices (the constructions of the reference's
scripts/calibration/rotation_math.py:6-32: Sylvester for powers of two,
Paley-12 x Sylvester-8 for 96), stored FP16 [heads, D, D].
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch


def _sylvester(dim: int) -> np.ndarray:
    matrix = np.ones((1, 1))
    while matrix.shape[0] < dim:
        matrix = np.block([[matrix, matrix], [matrix, -matrix]])
    return matrix


def hadamard(dim: int) -> np.ndarray:
    """An unnormalized +-1 Hadamard matrix of order ``dim`` (power of two or 96)."""
    if dim == 96:
        residues = {(i * i) % 11 for i in range(1, 11)}
        paley = np.ones((12, 12))
        for i in range(11):
            for j in range(11):
                paley[i + 1, j + 1] = -1 if i == j else (1 if (i - j) % 11 in residues else -1)
        return np.kron(paley, _sylvester(8))
    if dim <= 0 or dim & (dim - 1):
        raise ValueError("Hadamard dimension must be a power of two or 96")
    return _sylvester(dim)


def random_sign_rotation(heads: int, dim: int, seed: int, device="cpu") -> torch.Tensor:
    """FP16 [heads, D, D]: diag(random signs) . H / sqrt(D), orthogonal up to FP16 rounding."""
    generator = torch.Generator().manual_seed(seed)
    base = torch.from_numpy(hadamard(dim) / np.sqrt(dim))
    signs = torch.randint(0, 2, (heads, dim, 1), generator=generator, dtype=torch.int64) * 2 - 1
    return (signs.double() * base.unsqueeze(0)).to(torch.float16).to(device)


def loop_kv(tokens: int, heads: int, dim: int, loops: int, seed: int, device="cpu",
            outlier_channels: int = 4, outlier_scale: float = 8.0, residual_std: float = 0.15,
            anchor_index: Optional[int] = None) -> List[Tuple[torch.Tensor, torch.Tensor]]:
    """Per-loop BF16 (K, V) [tokens, heads, D]; the anchor loop is the group's last by default."""
    anchor_index = loops - 1 if anchor_index is None else anchor_index
    generator = torch.Generator(device=device).manual_seed(seed)
    channel_generator = torch.Generator().manual_seed(seed + 1)
    outliers = torch.randperm(dim, generator=channel_generator)[:outlier_channels].to(device)
    anchor_k = torch.randn((tokens, heads, dim), generator=generator, device=device)
    anchor_v = torch.randn((tokens, heads, dim), generator=generator, device=device)
    anchor_k[:, :, outliers] *= outlier_scale
    pairs = []
    for loop in range(loops):
        if loop == anchor_index:
            k, v = anchor_k, anchor_v
        else:
            k = anchor_k + residual_std * torch.randn(anchor_k.shape, generator=generator, device=device)
            v = anchor_v + residual_std * torch.randn(anchor_v.shape, generator=generator, device=device)
        pairs.append((k.to(torch.bfloat16), v.to(torch.bfloat16)))
    return pairs


def key_means(loops: int, heads: int, dim: int, seed: int, device="cpu", std: float = 0.5) -> torch.Tensor:
    """FP32 [loops, heads, D] per-loop K channel means (rotated space)."""
    generator = torch.Generator().manual_seed(seed)
    return (std * torch.randn((loops, heads, dim), generator=generator)).float().to(device)


def block_tables(batch: int, pages: int, seed: int, device="cpu", extra_blocks: int = 0) -> torch.Tensor:
    """INT32 [batch, pages]: a random permutation of ``batch*pages + extra`` block ids."""
    generator = torch.Generator().manual_seed(seed)
    ids = torch.randperm(batch * pages + extra_blocks, generator=generator)[: batch * pages]
    return ids.view(batch, pages).to(torch.int32).to(device)


def history_slots(table: torch.Tensor, lengths: Sequence[int], page_tokens: int) -> torch.Tensor:
    """INT64 slots of tokens 0..lengths[b]-1 of every request, request-major."""
    table_cpu = table.cpu().long()
    parts = []
    for b, length in enumerate(lengths):
        positions = torch.arange(length, dtype=torch.int64)
        parts.append(table_cpu[b, positions // page_tokens] * page_tokens + positions % page_tokens)
    if not parts:
        return torch.empty(0, dtype=torch.int64, device=table.device)
    return torch.cat(parts).to(table.device)


def bf16_bits(tensor: torch.Tensor) -> np.ndarray:
    """uint16 bit patterns of a BF16 / FP16 tensor (for the CPU oracle)."""
    return tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
