"""The graph-captured decode step of the Ouro-shaped looped model
(residualquant_amd/looped_decode.py; model loop of
plugins/looped_transformers/src/looped_transformers/ouro.py:102-242).

- The step's logits match an independent float64 forward of the same
  weights (torch RMSNorm / RoPE / linear / SiLU and the CPU oracle's packed
  attention, tests/looped_reference.py).
- Replaying the captured step gives the same logits, next tokens and cache
  bytes as running the step eagerly, on every replay, with unrelated eager
  work between replays.
- Steps past the cache's capacity are refused on the host, and the slot of a
  position past the block table is -1 on the device."""

from __future__ import annotations

import pytest
import torch

from residualquant_amd.looped_decode import LoopedConfig, LoopedDecoder

from .looped_reference import check_layers, compare_logits, reference_step

pytestmark = pytest.mark.gpu

TINY = LoopedConfig(layers=2, loops=4, hidden=256, heads=2, head_dim=128, intermediate=512, vocab=1000)


def _model(device, batch=3):
    model = LoopedDecoder(TINY, batch=batch, context=37, max_new_tokens=8, device=device, seed=3)
    model.build_history(seed=5)
    return model


def _random_norms(model, seed):
    g = torch.Generator(device=model.device).manual_seed(seed)
    hidden = model.config.hidden
    near_one = lambda: (1 + 0.2 * torch.randn(hidden, generator=g, device=model.device)).to(torch.bfloat16)
    model.norms = [[near_one() for _ in range(4)] for _ in range(model.config.layers)]
    model.final_norm = near_one()


# The free-running float64 forward drifts from the step as BF16 rounding
# differences are amplified through the random-weight layers (measured:
# cosine >= 0.998, max |logit error| ~0.2 at logits of ~4); a wrong layer
# order, a missing residual or a misplaced norm gives cosine far below 0.99.
FREE_COSINE = 0.99
FREE_TOKEN_MARGIN = 0.5


@pytest.mark.parametrize("batch", [3, 1])
def test_step_logits_match_independent_forward(oracle, device, batch):
    """Batch 1 takes the row-projection kernel (rq_linear_rows), batch 3 hipBLASLt."""
    model = _model(device, batch)
    _random_norms(model, 17)
    for step in range(2):  # the second step reads the token the first one quantized
        want = reference_step(model, oracle)
        got = model.step()
        torch.cuda.synchronize()
        err, cosine, margin = compare_logits(got, want)
        print(f"[case] looped step {step} batch {batch}: logits max {err.max():.3g} mean {err.mean():.3g} "
              f"cosine {cosine.min():.6f} scale {want.abs().max():.3g}", flush=True)
        assert bool((cosine >= FREE_COSINE).all()), step
        clear = margin > FREE_TOKEN_MARGIN
        assert torch.equal(model.tokens.cpu()[clear], want.argmax(-1)[clear]), step


def assert_layers(stats: dict) -> None:
    """Bars of check_layers: q/k/v (one product and RoPE from the layer input)
    within 2**-7 of the largest reference value (max: one to two BF16 ulps of
    that value, by where it sits in its binade) and 2**-10 relative on average
    (they are equal but for rare rounding flips); attention within the parity
    bar of the oracle; logits within 2**-7 of their scale.  A layer output,
    residual or loop input follows three products (o_proj, then the MLP's
    two) whose FP32 accumulation order differs from the float64 recompute,
    each rounded to BF16, then the residual adds and the norms: flips there
    reach the output as two ulps (0.03125 at values below 3.92 measured, just
    over 2**-7 of 3.92), so their max bar is 2**-6 of the largest reference
    value, with the same 2**-10 mean bar."""
    for name, (err_max, err_mean, ref_max, ref_mean) in stats.items():
        if name.startswith("attention"):
            assert err_max <= 2e-2 and err_mean <= 1e-3, (name, err_max, err_mean)
        elif name == "logits":
            assert err_max <= 2.0 ** -7 * ref_max and err_mean <= 2.0 ** -8 * ref_mean, (name, err_max, err_mean)
        elif name.startswith(("output", "residual", "loop_input")):
            assert err_max <= 2.0 ** -6 * ref_max and err_mean <= 2.0 ** -10 * ref_mean, (name, err_max, err_mean)
        else:
            assert err_max <= 2.0 ** -7 * ref_max and err_mean <= 2.0 ** -10 * ref_mean, (name, err_max, err_mean)


@pytest.mark.parametrize("batch", [3, 1])
def test_step_layers_match_reference_from_their_inputs(oracle, device, batch):
    """Every (loop, layer) of the step recomputed in float64 from the step's
    own layer inputs: q/k/v, the packed attention against the oracle, the
    layer output and residual, the loop boundaries and the logits."""
    model = _model(device, batch)
    _random_norms(model, 19)
    c = model.config
    for step in range(2):
        before = {layer: cache.cpu().numpy() for layer, cache in enumerate(model.caches)}
        model.taps = {(loop, layer) for loop in range(c.loops) for layer in range(c.layers)}
        logits = model.step()
        torch.cuda.synchronize()
        stats = check_layers(model, oracle, model.tapped, before, logits)
        assert len(stats) == c.loops * c.layers * 5 + c.loops * (c.layers - 1) + 2 * (c.loops - 1) + 1
        worst = max(stats.items(), key=lambda kv: kv[1][0] / max(kv[1][2], 1e-30))
        print(f"[case] looped layers step {step} batch {batch}: worst {worst[0]} {worst[1]}", flush=True)
        assert_layers(stats)


def test_replay_refuses_steps_past_the_cache(device):
    model = LoopedDecoder(TINY, batch=2, context=30, max_new_tokens=2, device=device, seed=3)
    model.build_history(seed=5)
    model.capture()
    model.replay()
    model.replay()
    torch.cuda.synchronize()
    # positions now equal max_tokens = 32 = 2 pages of 16: no page left
    assert int(model.positions[0]) == 32 and bool((model.slots == -1).all())
    with pytest.raises(RuntimeError, match="max_new_tokens"):
        model.replay()
    with pytest.raises(RuntimeError, match="max_new_tokens"):
        model.step()


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
        graphed.replay()
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


def test_artifact_folded_value_rotation_matches_kernel_rotation(oracle, device):
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
    expected = [reference_step(model, oracle) for model in (kernel_side, folded)]
    a = kernel_side.step().float()
    b = folded.step().float()
    torch.cuda.synchronize()
    # Each against the float64 forward of its own weights and cache.
    for name, got, want in (("kernel rotation", a, expected[0]), ("folded", b, expected[1])):
        err, cos, _ = compare_logits(got, want)
        print(f"[case] artifact {name}: logits max {err.max():.3g} mean {err.mean():.3g}", flush=True)
        assert bool((cos >= FREE_COSINE).all()), name
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
        graphed.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, graphed.logits), step
