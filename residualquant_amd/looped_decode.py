"""A graph-captured decode step of an Ouro-shaped looped model over the packed cache.

The model loop follows the reference's Ouro implementation
(plugins/looped_transformers/src/looped_transformers/ouro.py:38-242): the
physical layers are shared by every recurrent step ("loop"); each
(loop, layer) pair owns an attention slot (``virtual_index = loop * layers +
layer``, :48-52), and a layer is

    x, residual = input_layernorm(h, residual)     (fused add + RMSNorm)
    a = o_proj(attention(rope(q), rope(k), v))     (:102-110)
    x, residual = post_attention_layernorm(input_layernorm_2(a), residual)
    h = post_attention_layernorm_2(mlp(x))         (Qwen2MLP: SiLU(gate) * up)

with the final ``norm(h, residual)`` after each loop (:240).  The packed
backend stages the K/V of loops 0..2 of every layer and quantizes the whole
loop group at the anchor loop (install_model.py:17-52,
packed_backend.py:101-137), so one decode step runs 48 x 4 attention calls
over the packed history plus 48 quantize calls.

Weights are random BF16 (there are no checkpoints here), stored
``[out, in]`` as vLLM's linear layers hold them.  Plain GEMMs go to torch
(hipBLASLt); attention, quantize, the fused add + RMSNorm, the rotary
embedding (which also writes the loop-group staging copies) and SiLU * up are
this package's HIP kernels.  The whole step, including advancing positions,
slots and the greedy next token, is captured once in a HIP graph and replayed
per token.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

import torch.nn.functional as F

from . import artifact as artifact_module
from . import ops, step_ops, workloads
from .layout import page_width


# Rows up to which the projections run on rq_linear_rows (measured per layer
# at hidden 2048, graph replay over 48 layers' weights, against hipBLASLt:
# 25.6 vs 37.7 us at one row, 26.0 vs 48.0 at two, 31.3 vs 48.1 at four,
# 42.8 vs 48.0 at eight).
LINEAR_ROWS_MAX = 8


def _project(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``x @ weight.T`` for a linear weight held ``[out, in]``.

    At up to eight rows the product is a weight stream: ``step_ops.linear_rows``
    reads every weight row once with 16-byte loads and FP32 accumulation.
    Larger batches take hipBLASLt through ``F.linear``."""
    rows, in_features = x.shape
    if (rows <= LINEAR_ROWS_MAX and in_features % 8 == 0 and in_features <= 6144 and x.stride(1) == 1
            and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 and weight.is_contiguous()
            and weight.data_ptr() % 16 == 0):
        return step_ops.linear_rows(x, weight)
    return F.linear(x, weight)


@dataclass
class LoopedConfig:
    """Ouro-2.6B-shaped decoder.

    ``intermediate`` is not given by the benchmark configuration; 5632 (the
    Ouro-1.4B MLP width at the same hidden size) is an assumption, as are
    ``rope_theta`` and ``rms_eps``.
    """

    layers: int = 48
    loops: int = 4
    hidden: int = 2048
    heads: int = 16
    head_dim: int = 128
    intermediate: int = 5632
    vocab: int = 49152
    rms_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    schedule: Tuple[Tuple[int, int], ...] = ((2, 32), (2, 32), (2, 32), (4, 32))
    anchor: int = 3
    coefficient: str = "ls"
    page_tokens: int = 16


class LoopedDecoder:
    """Synthetic Ouro-shaped model with a packed paged cache for ``batch`` requests."""

    def __init__(self, config: LoopedConfig, batch: int, context: int, max_new_tokens: int,
                 device: torch.device, seed: int = 0, weights_from: Optional["LoopedDecoder"] = None):
        if config.loops != len(config.schedule):
            raise ValueError("one packed record per loop is required")
        self.config = c = config
        self.batch, self.context, self.device = batch, context, device
        self.max_tokens = context + max_new_tokens
        generator = torch.Generator(device=device).manual_seed(seed)

        def weight(fan_out, fan_in):
            scale = 1.0 / math.sqrt(fan_in)
            return (torch.randn((fan_out, fan_in), generator=generator, device=device) * scale).to(torch.bfloat16)

        q_size = c.heads * c.head_dim
        if weights_from is not None:
            if weights_from.config != c:
                raise ValueError("shared weights need the same model configuration")
            for name in ("embed", "qkv", "o", "gate_up", "down", "norms", "final_norm", "lm_head", "key_rotation",
                         "value_rotation"):
                setattr(self, name, getattr(weights_from, name))
        else:
            self.embed = (torch.randn((c.vocab, c.hidden), generator=generator, device=device) * 0.02).to(
                torch.bfloat16)
            self.qkv = [weight(3 * q_size, c.hidden) for _ in range(c.layers)]
            self.o = [weight(c.hidden, q_size) for _ in range(c.layers)]
            self.gate_up = [weight(2 * c.intermediate, c.hidden) for _ in range(c.layers)]
            self.down = [weight(c.hidden, c.intermediate) for _ in range(c.layers)]
            ones = torch.ones(c.hidden, dtype=torch.bfloat16, device=device)
            self.norms = [[ones.clone() for _ in range(4)] for _ in range(c.layers)]
            self.final_norm = ones.clone()
            self.lm_head = weight(c.vocab, c.hidden)
            self.key_rotation = [workloads.random_sign_rotation(c.heads, c.head_dim, seed + 11 + 2 * l, device=device)
                                 for l in range(c.layers)]
            self.value_rotation = [
                workloads.random_sign_rotation(c.heads, c.head_dim, seed + 12 + 2 * l, device=device)
                for l in range(c.layers)]
        self.key_mean: list = [None] * c.layers
        # V rotations folded into the projection weights (use_artifact), used
        # only to rotate the synthetic history the way those weights would.
        self.folded_value_rotation: list = [None] * c.layers

        # Paged cache: every request owns ceil(max_tokens / PT) blocks, shuffled.
        pages = (self.max_tokens + c.page_tokens - 1) // c.page_tokens
        self.block_table = workloads.block_tables(batch, pages, seed + 5, device=device)
        blocks = batch * pages
        self.width = page_width(c.head_dim, c.schedule)
        self.caches = [torch.zeros((2, blocks, c.heads, c.page_tokens, self.width), dtype=torch.uint8, device=device)
                       for _ in range(c.layers)]

        inv = 1.0 / (c.rope_theta ** (torch.arange(0, c.head_dim, 2, device=device, dtype=torch.float32) / c.head_dim))
        angles = torch.arange(self.max_tokens, device=device, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos, self.sin = angles.cos(), angles.sin()

        # Step state (static tensors for graph capture).
        # Own generator: the first tokens do not depend on whether the weights were drawn or shared.
        token_generator = torch.Generator(device=device).manual_seed(seed + 3)
        self.tokens = torch.randint(0, c.vocab, (batch,), generator=token_generator, device=device)
        self.positions = torch.full((batch,), context, dtype=torch.int64, device=device)
        self.seq_lens = torch.full((batch,), context + 1, dtype=torch.int32, device=device)
        self.query_start_loc = torch.arange(batch + 1, dtype=torch.int32, device=device)
        self.slots = torch.empty(batch, dtype=torch.int64, device=device)
        self._update_slots()
        self.attn_out = torch.empty((batch, c.heads, c.head_dim), dtype=torch.bfloat16, device=device)
        self.residual = torch.empty((batch, c.hidden), dtype=torch.bfloat16, device=device)
        self.staged = torch.empty((c.layers, c.loops, 2, batch, c.heads, c.head_dim), dtype=torch.bfloat16,
                                  device=device)
        self.workspace = torch.empty(ops.attention_workspace_bytes(batch, c.heads, c.head_dim, pages, c.page_tokens),
                                     dtype=torch.uint8, device=device)
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        # Host mirror of the next position (the same for every request).
        self.next_position = context
        # (loop, layer) pairs whose inputs and attention an eager step()
        # keeps in ``tapped`` (for tests; never inside a capture): the layer
        # input x and residual, the roped q and k, v, the attention output;
        # and ("h", loop) the loop's final hidden state.
        self.taps: set = set()
        self.tapped: dict = {}

    # ------------------------------------------------------------ artifact

    def use_artifact(self, artifact: dict) -> None:
        """Take the K/V rotations and key means of a rotation artifact
        (``artifact.load_rotation_artifact``), one packed group covering the
        model's loops, as the reference binds them (install_model.py:154-196).
        4-D value rotations are folded into this decoder's QKV and O weights
        (weights.py:8-37), in place: call before building the history, and
        before sharing the weights with another decoder."""
        c = self.config
        q_size = c.heads * c.head_dim
        prepared, folded = artifact_module.prepare_value_rotation(artifact)
        slots = artifact_module.bind_slots(prepared, [c.schedule], c.layers, self.device)[0]
        # Own lists (a decoder built with weights_from shares the originals).
        self.key_rotation, self.value_rotation = list(self.key_rotation), list(self.value_rotation)
        for layer, slot in enumerate(slots):
            self.key_rotation[layer] = slot.key_rotation
            self.value_rotation[layer] = slot.value_rotation
            self.key_mean[layer] = slot.key_mean
            if folded is not None:
                rotation = folded[layer].to(self.device)
                artifact_module.absorb_value_rotation(self.qkv[layer], self.o[layer], rotation, c.heads, c.head_dim,
                                                      q_size, q_size)
                self.folded_value_rotation[layer] = rotation

    # ------------------------------------------------------------ history

    def build_history(self, seed: int = 0, chunk: int = 16384) -> None:
        """Quantize synthetic K/V of tokens 0..context-1 into every layer's cache (the prefill stand-in)."""
        c = self.config
        if self.context == 0:
            return
        slots = workloads.history_slots(self.block_table, [self.context] * self.batch, c.page_tokens).to(self.device)
        for layer in range(c.layers):
            for start in range(0, slots.numel(), chunk):
                part = slots[start:start + chunk]
                pairs = workloads.loop_kv(part.numel(), c.heads, c.head_dim, c.loops, seed + 97 * layer + start,
                                          device=self.device, anchor_index=c.anchor)
                value_rotation = self.value_rotation[layer]
                if value_rotation is None:
                    value_rotation = self.folded_value_rotation[layer]
                ops.quantize(pairs, self.caches[layer], part, self.key_rotation[layer], value_rotation,
                             self.key_mean[layer], c.schedule, "anchor", c.anchor, c.coefficient)

    # ------------------------------------------------------------ the step

    def _update_slots(self) -> None:
        """Slot of each request's next position; -1 (quantize skips it) past
        the block table, so a step beyond ``max_tokens`` writes no page."""
        pt = self.config.page_tokens
        pages = self.block_table.size(1)
        page = torch.div(self.positions, pt, rounding_mode="floor").clamp(0, pages - 1)
        block = self.block_table.long().gather(1, page[:, None])[:, 0]
        slots = torch.where(self.positions < pages * pt, block * pt + self.positions % pt,
                            torch.full_like(self.positions, -1))
        self.slots.copy_(slots)

    def _check_room(self) -> None:
        if self.next_position >= self.max_tokens:
            raise RuntimeError(f"decode step at position {self.next_position} is past the cache's "
                               f"{self.max_tokens} tokens (max_new_tokens reached)")

    def step(self) -> torch.Tensor:
        """One decode step for every request; returns the logits and advances the state in place."""
        capturing = torch.cuda.is_current_stream_capturing()
        if not capturing:
            self._check_room()
        c = self.config
        q_size = c.heads * c.head_dim
        eps = c.rms_eps
        h = self.embed[self.tokens]
        for loop in range(c.loops):
            # input_layernorm of layer 0, ouro.py:148-150 (the residual starts as the loop input).
            self.residual.copy_(h)
            x = step_ops.rms_norm(h, self.norms[0][0], eps)
            for layer in range(c.layers):
                norms = self.norms[layer]
                tap = (loop, layer) in self.taps and not capturing
                if tap:
                    layer_input = (x.clone(), self.residual.clone())
                qkv = _project(x, self.qkv[layer])
                key_stage, value_stage = self.staged[layer, loop, 0], self.staged[layer, loop, 1]
                q, k = step_ops.rope_qkv(qkv, self.positions, self.cos, self.sin, c.heads, c.head_dim,
                                         key_stage=key_stage, value_stage=value_stage)
                ops.attention(q, k, value_stage, self.caches[layer], self.attn_out, self.query_start_loc,
                              self.seq_lens, self.block_table, self.key_rotation[layer], self.value_rotation[layer],
                              self.key_mean[layer], c.schedule, "anchor", c.anchor, loop, workspace=self.workspace)
                if tap:
                    self.tapped[(loop, layer)] = dict(x=layer_input[0], residual=layer_input[1], q=q.clone(),
                                                      k=k.clone(), v=value_stage.clone(), out=self.attn_out.clone())
                # Loop group quantize at the anchor loop (install_model.py:40-52).
                if loop == c.anchor:
                    pairs = [(self.staged[layer, r, 0], self.staged[layer, r, 1]) for r in range(c.loops)]
                    ops.quantize(pairs, self.caches[layer], self.slots, self.key_rotation[layer],
                                 self.value_rotation[layer], self.key_mean[layer], c.schedule, "anchor", c.anchor,
                                 c.coefficient)
                a = _project(self.attn_out.view(self.batch, q_size), self.o[layer])
                # input_layernorm_2 then post_attention_layernorm with the fused add (ouro.py:154-155), one launch.
                x, _ = step_ops.rms_norm(a, norms[2], eps, residual=self.residual, pre_weight=norms[1])
                m = _project(step_ops.silu_mul(_project(x, self.gate_up[layer])), self.down[layer])
                # post_attention_layernorm_2 (ouro.py:157), then the next layer's input_layernorm
                # with the fused add (:151-152) or the loop's final norm (:240), one launch.
                following = self.norms[layer + 1][0] if layer + 1 < c.layers else self.final_norm
                x, _ = step_ops.rms_norm(m, following, eps, residual=self.residual, pre_weight=norms[3])
            h = x
            if self.taps and not capturing:
                self.tapped[("h", loop)] = h.clone()
        logits = _project(h, self.lm_head)
        # Greedy next token and the next position, slot and sequence length.
        self.tokens.copy_(logits.argmax(dim=-1))
        self.positions.add_(1)
        self.seq_lens.add_(1)
        self._update_slots()
        if not capturing:
            self.next_position += 1
        return logits

    def capture(self) -> torch.cuda.CUDAGraph:
        """Capture one step as a HIP graph (the state tensors advance on every replay)."""
        snapshot = (self.tokens.clone(), self.positions.clone(), self.seq_lens.clone(), self.slots.clone())
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            self.step()  # warm-up outside capture (allocator pools, library handles)
        torch.cuda.current_stream(self.device).wait_stream(stream)
        self._restore(snapshot)
        self.next_position -= 1  # the warm-up step is undone
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.logits = self.step()
        self._restore(snapshot)
        self.graph = graph
        return graph

    def replay(self) -> torch.Tensor:
        """Run the captured step once; refuses a step past ``max_tokens``."""
        if self.graph is None:
            raise RuntimeError("capture() the step first")
        self._check_room()
        self.graph.replay()
        self.next_position += 1
        return self.logits

    def _restore(self, snapshot) -> None:
        for tensor, saved in zip((self.tokens, self.positions, self.seq_lens, self.slots), snapshot):
            tensor.copy_(saved)
