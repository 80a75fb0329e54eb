"""The C3 shape on the GPU: the Ouro-2.6B-shaped decode step (48 layers,
hidden 2048, 16 heads x 128, 4 loops, vocab 49152) over packed history, at
batch x context points of the benchmark's sweep (B1 x 2048, B8 x 2048,
B32 x 8192).

- Sampled (loop, layer) slots of an eager step are recomputed in float64
  from the step's own layer inputs (tests/looped_reference.py:
  check_layers): q/k/v, the packed attention against the CPU oracle (within
  2e-2 max-abs / 1e-3 mean-abs; at B32 on three sampled rows, whose pages
  alone the oracle reads), the layer output and residual; and the logits
  from the last loop's output.
- The loop-3 quantize of the new token writes, in every one of the 48
  layers, the oracle's bytes for the staged K/V of all four loops
  (check_new_tokens), after the eager step and after a graph replay.
- At B1 and B8 a twin decoder replays the captured step to the same logits,
  tokens and cache bytes as the eager step, for two steps.  (At B32 x 8192
  the packed caches take 82 GB, so there is one decoder: its replayed step
  is checked through its cache writes.)"""

from __future__ import annotations

import pytest
import torch

from residualquant_amd.looped_decode import LoopedConfig, LoopedDecoder

from .looped_reference import check_layers, check_new_tokens, new_token_pages, row_blocks
from .test_gpu_looped_step import assert_layers

pytestmark = pytest.mark.gpu

TAPS = {(0, 0), (0, 1), (1, 17), (1, 18), (3, 46), (3, 47)}


def _check_eager_step(model, oracle, rows, label):
    tap_layers = sorted({layer for _, layer in TAPS})
    if rows is None:
        before = {layer: model.caches[layer].cpu().numpy() for layer in tap_layers}
    else:
        blocks = row_blocks(model, rows)
        before = {layer: model.caches[layer][:, blocks].cpu().numpy() for layer in tap_layers}
    slots, blocks_new, pages_new = new_token_pages(model)
    model.taps = TAPS
    logits = model.step()
    torch.cuda.synchronize()
    model.taps = set()
    stats = check_layers(model, oracle, model.tapped, before, logits, rows=rows)
    for name, values in sorted(stats.items()):
        print(f"[case] {label} {name}: max {values[0]:.3g} mean {values[1]:.3g} ref max {values[2]:.3g}",
              flush=True)
    assert len(stats) == 6 * 4 + 7 + 1
    assert_layers(stats)
    checked = check_new_tokens(model, oracle, slots, blocks_new, pages_new)
    print(f"[case] {label} eager step: new-token pages of {checked} layers equal the oracle's", flush=True)
    return logits


@pytest.mark.parametrize("batch,context", [(8, 2048), (1, 2048)], ids=["b8-2k", "b1-2k"])
def test_c3_step(oracle, device, batch, context):
    config = LoopedConfig()
    label = f"C3 B{batch} x {context}"
    print(f"[case] {label}, 48 layers", flush=True)
    eager = LoopedDecoder(config, batch=batch, context=context, max_new_tokens=4, device=device, seed=31)
    graphed = LoopedDecoder(config, batch=batch, context=context, max_new_tokens=4, device=device, seed=31,
                            weights_from=eager)
    for model in (eager, graphed):
        model.build_history(seed=7)
    torch.cuda.synchronize()
    assert torch.equal(eager.tokens, graphed.tokens)
    for a, b in zip(eager.caches, graphed.caches):
        assert torch.equal(a, b)
    # Taken before the capture: its warm-up step already writes the first
    # step's new-token bytes (the same bytes the replay writes again).
    slots, blocks, pages = new_token_pages(graphed)
    graphed.capture()
    for step in range(2):
        print(f"[case] {label} step {step}", flush=True)
        if step == 0:
            logits = _check_eager_step(eager, oracle, None, label)
        else:
            logits = eager.step()
        graphed.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, graphed.logits), step
        assert torch.equal(eager.tokens, graphed.tokens), step
        for layer, (a, b) in enumerate(zip(eager.caches, graphed.caches)):
            assert torch.equal(a, b), (step, layer)
        if step == 0:
            check_new_tokens(graphed, oracle, slots, blocks, pages)


def test_c3_step_b32_8k(oracle, device):
    config = LoopedConfig()
    label = "C3 B32 x 8192"
    print(f"[case] {label}, 48 layers, rows 0, 13 and 31", flush=True)
    model = LoopedDecoder(config, batch=32, context=8192, max_new_tokens=4, device=device, seed=41)
    model.build_history(seed=9)
    torch.cuda.synchronize()
    _check_eager_step(model, oracle, (0, 13, 31), label)
    slots, blocks, pages = new_token_pages(model)  # before the capture's warm-up step writes them
    model.capture()
    print(f"[case] {label} replayed step", flush=True)
    model.replay()
    torch.cuda.synchronize()
    assert bool(torch.isfinite(model.logits.float()).all())
    checked = check_new_tokens(model, oracle, slots, blocks, pages)
    print(f"[case] {label} replayed step: new-token pages of {checked} layers equal the oracle's", flush=True)
