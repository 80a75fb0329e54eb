"""An independent float64 forward of one decode step of the Ouro-shaped looped
model (plugins/looped_transformers/src/looped_transformers/ouro.py:101-158,
:217-242), for checking residualquant_amd.looped_decode.LoopedDecoder.

It takes the decoder's weights, state and packed cache, and computes the
step with torch on the CPU (RMSNorm, rotate-half RoPE, linear layers, SiLU)
plus the CPU oracle's packed attention over each (loop, layer) slot's pages.
Tensors are rounded to BF16 where the decoder stores BF16 tensors.

- ``reference_step`` runs the whole step on its own.  Its logits drift from
  the decoder's as BF16 rounding differences (one ulp here and there, and
  the attention kernel's own error) are amplified through the random-weight
  layers, so only a loose comparison is meaningful.
- ``check_layers`` is the sharp check: from the decoder's own tapped layer
  inputs it recomputes each tapped layer (q, k, v; the attention over the
  cache with the oracle; the layer output from the decoder's attention
  output) and the logits, so that every comparison covers one layer's
  arithmetic only.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from residualquant_amd import workloads


def _bf(t: torch.Tensor) -> torch.Tensor:
    return t.float().to(torch.bfloat16).double()


def _f64(t: torch.Tensor) -> torch.Tensor:
    return t.detach().cpu().double()


def reference_step(model, oracle, record: dict = None) -> torch.Tensor:
    """float64 logits [batch, vocab] of the decoder's next step (its state is not advanced).

    With ``record``, keeps (q, k, v, attention output) of every (loop, layer)."""
    c = model.config
    batch = model.batch
    eps = c.rms_eps

    def rms(x, weight):
        inv = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
        return _bf(_bf(x * inv) * _f64(weight))

    def add_rms(x, residual, weight, pre):
        # RMSNorm with a fused residual add, after a norm of x itself
        # (input_layernorm_2 -> post_attention_layernorm, ouro.py:154-155;
        # post_attention_layernorm_2 -> next input_layernorm / final norm).
        total = _bf(rms(x, pre) + residual)
        return rms(total, weight), total

    positions = model.positions.cpu()
    cos, sin = _f64(model.cos)[positions], _f64(model.sin)[positions]   # [batch, D/2]

    def rope(x):  # [batch, heads, D], rotate-half
        half = x.size(-1) // 2
        a, b = x[..., :half], x[..., half:]
        cs, sn = cos[:, None, :], sin[:, None, :]
        return _bf(torch.cat([a * cs - b * sn, b * cs + a * sn], -1))

    query_start_loc = model.query_start_loc.cpu().numpy()
    seq_lens = model.seq_lens.cpu().numpy()
    table = model.block_table.cpu().numpy()
    caches = [cache.cpu().numpy() for cache in model.caches]
    bits = lambda t: None if t is None else workloads.bf16_bits(t)
    q_size = c.heads * c.head_dim

    h = _f64(model.embed)[model.tokens.cpu()]
    for loop in range(c.loops):
        residual = h.clone()
        x = rms(h, model.norms[0][0])
        for layer in range(c.layers):
            norms = model.norms[layer]
            qkv = _bf(x @ _f64(model.qkv[layer]).t())
            q = rope(qkv[:, :q_size].reshape(batch, c.heads, c.head_dim))
            k = rope(qkv[:, q_size:2 * q_size].reshape(batch, c.heads, c.head_dim))
            v = qkv[:, 2 * q_size:].reshape(batch, c.heads, c.head_dim)
            to_bf16 = lambda t: t.float().to(torch.bfloat16)
            mean = model.key_mean[layer]
            attention = oracle.attention(
                bits(to_bf16(q)), bits(to_bf16(k)), bits(to_bf16(v)), caches[layer], query_start_loc, seq_lens,
                table, bits(model.key_rotation[layer]), bits(model.value_rotation[layer]),
                None if mean is None else mean.cpu().numpy(), c.schedule, "anchor", c.anchor, loop)
            if record is not None:
                record[(loop, layer)] = (q, k, v, torch.from_numpy(attention))
            a = _bf(_bf(torch.from_numpy(attention)).reshape(batch, q_size) @ _f64(model.o[layer]).t())
            x, residual = add_rms(a, residual, norms[2], norms[1])
            gate_up = _bf(x @ _f64(model.gate_up[layer]).t())
            gate, up = gate_up[:, :c.intermediate], gate_up[:, c.intermediate:]
            m = _bf(_bf(F.silu(gate) * up) @ _f64(model.down[layer]).t())
            following = model.norms[layer + 1][0] if layer + 1 < c.layers else model.final_norm
            x, residual = add_rms(m, residual, following, norms[3])
        h = x
    return h @ _f64(model.lm_head).t()


def compare_logits(got: torch.Tensor, want: torch.Tensor):
    """Error statistics of the decoder's logits against the reference's."""
    got = got.detach().cpu().double()
    err = (got - want).abs()
    cosine = F.cosine_similarity(got, want, dim=-1)
    top2 = want.topk(2, dim=-1).values
    margin = top2[:, 0] - top2[:, 1]
    return err, cosine, margin


def _stats(got: torch.Tensor, want: torch.Tensor):
    got = got.detach().cpu().double()
    err = (got - want).abs()
    return float(err.max()), float(err.mean()), float(want.abs().max()), float(want.abs().mean())


def row_blocks(model, rows) -> torch.Tensor:
    """Block ids (device, int64) of the pages of ``rows``, row-major: the
    layout of the sub-caches ``check_layers`` takes when given ``rows``."""
    return model.block_table[list(rows)].flatten().long()


def check_layers(model, oracle, tapped: dict, caches_before: dict, logits: torch.Tensor, rows=None) -> dict:
    """Recompute every tapped layer of one eager step from the decoder's own
    inputs; returns {name: (max err, mean err, max |ref|, mean |ref|)}.

    ``tapped`` is the decoder's ``tapped`` after the step, ``caches_before``
    the layer caches (numpy) as the step's attention saw them, ``logits``
    the step's logits.  With ``rows``, the packed attention is checked on
    those rows only and ``caches_before[layer]`` holds just their pages
    (``cache[:, row_blocks(model, rows)]``); a row's attention reads its own
    pages only, so the renumbered sub-cache gives the same result."""
    c = model.config
    batch, eps = model.batch, c.rms_eps
    q_size = c.heads * c.head_dim
    f = lambda t: t.detach().cpu().double()

    def rms(x, weight):
        inv = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
        return _bf(_bf(x * inv) * _f64(weight))

    def add_rms(x, residual, weight, pre):
        total = _bf(rms(x, pre) + residual)
        return rms(total, weight), total

    positions = model.positions.cpu() - 1  # the step has advanced them
    cos, sin = _f64(model.cos)[positions][:, None, :], _f64(model.sin)[positions][:, None, :]

    def rope(x):
        half = x.size(-1) // 2
        a, b = x[..., :half], x[..., half:]
        return _bf(torch.cat([a * cos - b * sin, b * cos + a * sin], -1))

    seq_lens = model.seq_lens.cpu().numpy() - 1
    table = model.block_table.cpu().numpy()
    query_start_loc = model.query_start_loc.cpu().numpy()
    picked = slice(None)
    if rows is not None:
        picked = list(rows)
        seq_lens = seq_lens[picked]
        table = np.arange(len(picked) * table.shape[1], dtype=np.int32).reshape(len(picked), table.shape[1])
        query_start_loc = np.arange(len(picked) + 1, dtype=np.int32)
    bits = lambda t: None if t is None else workloads.bf16_bits(t)
    out = {}
    for key in sorted(k for k in tapped if isinstance(k[0], int)):
        loop, layer = key
        t = tapped[key]
        x, residual = f(t["x"]), f(t["residual"])
        qkv = _bf(x @ _f64(model.qkv[layer]).t())
        out[f"q{key}"] = _stats(t["q"], rope(qkv[:, :q_size].reshape(batch, c.heads, c.head_dim)))
        out[f"k{key}"] = _stats(t["k"], rope(qkv[:, q_size:2 * q_size].reshape(batch, c.heads, c.head_dim)))
        out[f"v{key}"] = _stats(t["v"], qkv[:, 2 * q_size:].reshape(batch, c.heads, c.head_dim))
        mean = model.key_mean[layer]
        attention = oracle.attention(
            bits(t["q"][picked]), bits(t["k"][picked]), bits(t["v"][picked]), caches_before[layer],
            query_start_loc, seq_lens, table, bits(model.key_rotation[layer]), bits(model.value_rotation[layer]),
            None if mean is None else mean.cpu().numpy(), c.schedule, "anchor", c.anchor, loop)
        # Both sides in BF16 (the parity bar is on BF16 outputs): rounding the
        # oracle keeps the BF16 quantum of outputs of magnitude ~1 (half of
        # the 1e-3 mean bar at short histories) out of the kernel's error.
        out[f"attention{key}"] = _stats(t["out"][picked], _bf(torch.from_numpy(attention)))
        norms = model.norms[layer]
        a = _bf(f(t["out"]).reshape(batch, q_size) @ _f64(model.o[layer]).t())
        x1, residual1 = add_rms(a, residual, norms[2], norms[1])
        gate_up = _bf(x1 @ _f64(model.gate_up[layer]).t())
        m = _bf(_bf(F.silu(gate_up[:, :c.intermediate]) * gate_up[:, c.intermediate:]) @ _f64(model.down[layer]).t())
        last = layer + 1 == c.layers
        following = model.final_norm if last else model.norms[layer + 1][0]
        x2, residual2 = add_rms(m, residual1, following, norms[3])
        if last and ("h", loop) in tapped:
            out[f"output{key}"] = _stats(tapped[("h", loop)], x2)
        elif not last and (loop, layer + 1) in tapped:
            nxt = tapped[(loop, layer + 1)]
            out[f"output{key}"] = _stats(nxt["x"], x2)
            out[f"residual{key}"] = _stats(nxt["residual"], residual2)
    for loop in range(c.loops - 1):
        if ("h", loop) in tapped and (loop + 1, 0) in tapped:
            h = f(tapped[("h", loop)])
            out[f"loop_input{loop + 1}"] = _stats(tapped[(loop + 1, 0)]["x"], rms(h, model.norms[0][0]))
            out[f"loop_residual{loop + 1}"] = _stats(tapped[(loop + 1, 0)]["residual"], h)
    if ("h", c.loops - 1) in tapped:
        out["logits"] = _stats(logits, f(tapped[("h", c.loops - 1)]) @ _f64(model.lm_head).t())
    return out


def new_token_pages(model):
    """Before a step: (slots, blocks, {layer: numpy pages}) of the pages the
    step's loop-group quantize writes (the blocks of the requests' next
    slots; slot -1 writes nothing)."""
    slots = model.slots.clone()
    live = slots[slots >= 0]
    blocks = torch.unique(torch.div(live, model.config.page_tokens, rounding_mode="floor"))
    pages = {layer: cache[:, blocks].cpu().numpy() for layer, cache in enumerate(model.caches)}
    return slots, blocks, pages


def check_new_tokens(model, oracle, slots, blocks, pages_before: dict) -> int:
    """After a step (eager or replayed): every layer's pages written by the
    step's quantize equal the oracle's quantize of the staged K/V of all
    loops (the decoder's ``staged`` buffer, as the step left it) into the
    pages as they were before the step, bit for bit.  Returns the layers
    checked."""
    c = model.config
    pt = c.page_tokens
    bits = lambda t: None if t is None else workloads.bf16_bits(t)
    index = {int(b): i for i, b in enumerate(blocks.cpu().tolist())}
    sub_slots = np.array([-1 if s < 0 else index[s // pt] * pt + s % pt for s in slots.cpu().tolist()],
                         dtype=np.int64)
    for layer, cache in enumerate(model.caches):
        got = cache[:, blocks].cpu().numpy()
        expected = pages_before[layer].copy()
        pairs = [(bits(model.staged[layer, r, 0]), bits(model.staged[layer, r, 1])) for r in range(c.loops)]
        value_rotation = model.value_rotation[layer]
        mean = model.key_mean[layer]
        oracle.quantize(pairs, expected, sub_slots, bits(model.key_rotation[layer]), bits(value_rotation),
                        None if mean is None else mean.cpu().numpy(), c.schedule, "anchor", c.anchor,
                        c.coefficient)
        assert np.array_equal(got, expected), f"new-token pages of layer {layer}"
        assert not np.array_equal(got, pages_before[layer]), f"layer {layer}: the step wrote nothing"
    return len(model.caches)
