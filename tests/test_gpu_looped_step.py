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
    """Batch 1 takes the row-projection kernel (rq_linear_rows), batch 3 hipBLASLt."""
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


def _tiny_artifact(value_dims, seed=21):
    import torch as t
    from residualquant_amd import workloads
    c = TINY
    key = t.stack([workloads.random_sign_rotation(c.heads, c.head_dim, seed + l) for l in range(c.layers)])
    value = t.stack([workloads.random_sign_rotation(c.heads, c.head_dim, seed + 50 + l) for l in range(c.layers)])
    if value_dims == 5:
        value = value[None]
    g = t.Generator().manual_seed(seed)
    return {"format_version": 2, "model": "tiny", "schedule": [b for b, _ in c.schedule],
            "groups": [s for _, s in c.schedule], "key_rotations": key, "value_rotations": value,
            "key_means": t.randn((c.loops, c.layers, c.heads, c.head_dim), generator=g) * 0.5}


def test_artifact_folded_value_rotation_matches_kernel_rotation(device):
    """With the V rotation folded into the QKV/O weights (4-D artifact,
    weights.py:8-37) the step computes what the kernels' own V rotation (5-D
    artifact) computes: the same logits up to BF16 and quantization rounding.
    Key means and K rotations come from the artifact in both."""
    kernel_side = LoopedDecoder(TINY, batch=2, context=40, max_new_tokens=4, device=device, seed=7)
    folded = LoopedDecoder(TINY, batch=2, context=40, max_new_tokens=4, device=device, seed=7)
    kernel_side.use_artifact(_tiny_artifact(5))
    folded.use_artifact(_tiny_artifact(4))
    assert all(v is None for v in folded.value_rotation) and all(m is not None for m in folded.key_mean)
    for model in (kernel_side, folded):
        model.build_history(seed=5)
    a = kernel_side.step().float()
    b = folded.step().float()
    torch.cuda.synchronize()
    cosine = torch.nn.functional.cosine_similarity(a, b, dim=-1)
    print(f"artifact folded vs kernel rotation: cosine {cosine.tolist()}", flush=True)
    assert bool((cosine > 0.995).all())


def test_graph_replay_with_artifact_means(device):
    eager = _model(device)
    graphed = _model(device)
    for model in (eager, graphed):
        model.use_artifact(_tiny_artifact(5))
    # Rebuild the history with the artifact's rotations and means.
    for model in (eager, graphed):
        for cache in model.caches:
            cache.zero_()
        model.build_history(seed=5)
    graphed.capture()
    for step in range(2):
        logits = eager.step()
        graphed.graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, graphed.logits), step
