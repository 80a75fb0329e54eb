"""The C3 shape on the GPU: the Ouro-2.6B-shaped decode step (48 layers,
hidden 2048, 16 heads x 128, 4 loops, vocab 49152) at batch 8 x 2048 tokens
of packed history.

- The captured step replays to the same logits, tokens and cache bytes as
  the eager step, for two steps.
- Sampled (loop, layer) slots of the eager step are recomputed in float64
  from the step's own layer inputs (tests/looped_reference.py:
  check_layers): q/k/v, the packed attention against the CPU oracle (within
  2e-2 max-abs / 1e-3 mean-abs), the layer output and residual; and the
  logits from the last loop's output."""

from __future__ import annotations

import pytest
import torch

from residualquant_amd.looped_decode import LoopedConfig, LoopedDecoder

from .looped_reference import check_layers
from .test_gpu_looped_step import assert_layers

pytestmark = pytest.mark.gpu

TAPS = {(0, 0), (0, 1), (1, 17), (1, 18), (3, 46), (3, 47)}


def test_c3_step_b8_2k(oracle, device):
    config = LoopedConfig()
    print("[case] C3 step B8 x 2048, 48 layers", flush=True)
    eager = LoopedDecoder(config, batch=8, context=2048, max_new_tokens=4, device=device, seed=31)
    graphed = LoopedDecoder(config, batch=8, context=2048, max_new_tokens=4, device=device, seed=31,
                            weights_from=eager)
    for model in (eager, graphed):
        model.build_history(seed=7)
    torch.cuda.synchronize()
    assert torch.equal(eager.tokens, graphed.tokens)
    for a, b in zip(eager.caches, graphed.caches):
        assert torch.equal(a, b)
    before = {layer: eager.caches[layer].cpu().numpy() for layer in sorted({layer for _, layer in TAPS})}
    graphed.capture()
    for step in range(2):
        print(f"[case] C3 step {step}", flush=True)
        eager.taps = TAPS if step == 0 else set()
        logits = eager.step()
        graphed.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, graphed.logits), step
        assert torch.equal(eager.tokens, graphed.tokens), step
        for layer, (a, b) in enumerate(zip(eager.caches, graphed.caches)):
            assert torch.equal(a, b), (step, layer)
        if step == 0:
            stats = check_layers(eager, oracle, eager.tapped, before, logits)
            for name, values in sorted(stats.items()):
                print(f"[case] C3 {name}: max {values[0]:.3g} mean {values[1]:.3g} ref max {values[2]:.3g}",
                      flush=True)
            assert len(stats) == 6 * 4 + 7 + 1
            assert_layers(stats)
