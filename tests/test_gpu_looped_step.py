"""The graph-captured decode step of the Ouro-shaped looped model
(residualquant_amd/looped_decode.py; model loop of
plugins/looped_transformers/src/looped_transformers/ouro.py:102-242).

Replaying the captured step must give the same logits, next tokens and
cache bytes as running the step eagerly, on every replay, with unrelated
eager work between replays."""

from __future__ import annotations

import pytest
import torch

from residualquant_amd.looped_decode import LoopedConfig, LoopedDecoder

pytestmark = pytest.mark.gpu

TINY = LoopedConfig(layers=2, loops=4, hidden=256, heads=2, head_dim=128, intermediate=512, vocab=1000)


def _model(device, batch=3):
    model = LoopedDecoder(TINY, batch=batch, context=37, max_new_tokens=8, device=device, seed=3)
    model.build_history(seed=5)
    return model


@pytest.mark.parametrize("batch", [3, 1])
def test_graph_replay_matches_eager_steps(device, batch):
    """Batch 1 takes the matrix-vector form of the projections."""
    eager, graphed = _model(device, batch), _model(device, batch)
    for a, b in zip(eager.caches, graphed.caches):
        assert torch.equal(a, b)
    graphed.capture()
    for step in range(4):
        print(f"looped step {step} batch {batch}", flush=True)
        logits = eager.step()
        graphed.graph.replay()
        torch.cuda.synchronize()
        torch.randn(1 << 20, device=device).sum()  # unrelated eager work between replays
        assert torch.equal(logits, graphed.logits), step
        assert torch.equal(eager.tokens, graphed.tokens)
        assert torch.equal(eager.positions, graphed.positions) and int(eager.positions[0]) == 37 + step + 1
        for a, b in zip(eager.caches, graphed.caches):
            assert torch.equal(a, b), step


def test_step_writes_the_new_token_of_every_layer(device):
    model = _model(device)
    before = [cache.clone() for cache in model.caches]
    slots = model.slots.clone()
    logits = model.step()
    torch.cuda.synchronize()
    assert torch.isfinite(logits.float()).all()
    pt = TINY.page_tokens
    for layer, (old, new) in enumerate(zip(before, model.caches)):
        changed = (old != new).nonzero()
        assert changed.numel() > 0, layer
        # Only the pages holding this step's slots change (a page keeps each
        # record's codes, scales, offsets and alpha in separate regions, so a
        # token's bytes are spread over the page).
        touched = {int(b) for b in changed[:, 1]}
        assert touched <= {int(s) // pt for s in slots}, layer


def test_single_row_projection_matches_linear(device):
    from residualquant_amd.looped_decode import _project

    g = torch.Generator(device=device).manual_seed(11)
    weight = (torch.randn((3072, 2048), generator=g, device=device) * 0.02).to(torch.bfloat16)
    x = torch.randn((1, 2048), generator=g, device=device).to(torch.bfloat16)
    got = _project(x, weight)
    assert got.shape == (1, 3072) and got.is_contiguous()
    want = x.float() @ weight.float().t()
    assert ((got.float() - want).abs() <= want.abs() * 2.0 ** -7 + 1e-3).all()
