"""Paged decode-attention benchmark of the packed INT2/INT4 KV cache on one MI355X.

Workload: an Ouro-1.4B-shaped layer, 16 query/KV heads,
head_dim 128, 4 loops, batch 32, 8192 history tokens per sequence, one
query token per sequence, page size 16, schedule [2,32]x3+[4,32] with the
INT4 anchor at loop 3, least-squares coefficients, seeded random-sign
Hadamard rotations on K and V.  One step = one decode step of the layer:
the three residual-loop calls and the anchor-loop call.  The BF16 paged
baseline runs the same four calls over a BF16 cache of the same shape.

``--workload quantize`` instead times quantize-on-write at BASELINE config 1
(C1): 4096 new tokens x 16 KV heads x D128 x 4 loops with the INT4 g32
anchor and INT2 residuals at g32 ([2,32]x3+[4,32], the headline) and at g16
([2,16]x3+[4,32]), plus the mixed [2,16]x2+[2,32]+[4,32]; least-squares
coefficients, seeded random-sign Hadamard rotations, scattered to random
slots of a paged cache of 16-token blocks.

Prints ONE JSON line on stdout; everything else goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0
PEAK_FP32_TFLOPS = 157.3
PEAK_BF16_TFLOPS = 2500.0
SCHEDULE = ((2, 32), (2, 32), (2, 32), (4, 32))
QUANTIZE_SCHEDULE = ((2, 16), (2, 16), (2, 32), (4, 32))
HUGINN_SCHEDULE = ((2, 16), (2, 16), (2, 16), (4, 32))
ADJACENT_SCHEDULE = ((4, 32), (2, 32), (2, 32), (2, 32))
ANCHOR = 3


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def staged_call_bytes(batch, history, heads, dim, page_tokens, loop, schedule=SCHEDULE, mode="anchor",
                      anchor=ANCHOR):
    """Algorithmic HBM bytes of one decode call (packed pages + Q/K/V/out + page table)."""
    from residualquant_amd.layout import staged_bytes

    pages = (history + page_tokens - 1) // page_tokens
    per_page = staged_bytes(dim, schedule, page_tokens, mode, anchor, loop)
    cache = batch * pages * heads * 2 * per_page
    live = 4 * batch * heads * dim * 2
    table = batch * pages * 4
    return cache + live + table


def bf16_call_bytes(batch, history, heads, dim):
    return batch * history * heads * dim * 2 * 2 + 4 * batch * heads * dim * 2 + batch * (history // 16) * 4


def build_packed_cache(torch, rq, workloads, batch, history, heads, dim, page_tokens, device, seed,
                       schedule=SCHEDULE, mode="anchor", anchor=ANCHOR):
    """Quantize synthetic K/V for every history token into a packed paged cache (on the GPU)."""
    pages = (history + page_tokens - 1) // page_tokens
    table = workloads.block_tables(batch, pages, seed + 5, device=device)
    num_blocks = batch * pages
    width = rq.page_width(dim, schedule)
    cache = torch.zeros((2, num_blocks, heads, page_tokens, width), dtype=torch.uint8, device=device)
    key_rotation = workloads.random_sign_rotation(heads, dim, seed + 3, device=device)
    value_rotation = workloads.random_sign_rotation(heads, dim, seed + 4, device=device)
    slots = workloads.history_slots(table, [history] * batch, page_tokens)
    chunk = 16384
    for start in range(0, slots.numel(), chunk):
        part = slots[start:start + chunk]
        pairs = workloads.loop_kv(part.numel(), heads, dim, len(schedule), seed + start, device=device)
        rq.quantize(pairs, cache, part, key_rotation, value_rotation, None, schedule, mode, anchor, "ls")
        del pairs
    torch.cuda.synchronize()
    return cache, table, key_rotation, value_rotation


def timed(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - start) / steps


def capture(torch, fn):
    """Capture fn's launches into one HIP graph (torch.cuda.CUDAGraph is hipGraph on ROCm)."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    torch.cuda.synchronize()
    return graph


def measured_traffic(summary="decode_c2_counters.json", key="residual_loop_traffic_bytes"):
    """HBM bytes per launch of the dominant kernel (by default the residual-loop
    decode launch) from a committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary,
    with the commit it was measured on."""
    path = os.path.join(ROOT, "profiles", summary)
    if not os.path.exists(path):
        return {"bytes": None, "commit": None}
    with open(path) as handle:
        data = json.load(handle)
    return {"bytes": data.get(key), "commit": data.get("commit")}


def kernel_durations_ms(ops, calls, reps, warmup=10):
    """Per-launch split-K kernel durations (HIP events on the launch stream) of
    each call in ``calls``, launched in turn as a step launches them; the first
    ``warmup`` rounds are dropped.  Returns one list of ``reps`` durations per call."""
    out = [[] for _ in calls]
    for round_ in range(warmup + reps):
        for i, call in enumerate(calls):
            ops.timing_read()
            ops.timing_enable(True)
            call()
            ms, launches = ops.timing_read()
            ops.timing_enable(False)
            if round_ >= warmup and launches == 1:
                out[i].append(ms)
    return out


def settle(torch, fn, seconds):
    """Run ``fn`` untimed for ``seconds``: the GPU's clocks leave their idle state.

    Measured on MI355X: the first ~50 replays of the C2 step after an idle
    second run up to 20% slower (744 -> 610 us per step over the first 60 ms)."""
    torch.cuda.synchronize()
    end = time.perf_counter() + seconds
    while time.perf_counter() < end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def host_description(torch):
    # A virtual machine may report a generic model name ("AMD EPYC"), so the
    # family / model / stepping numbers of the first processor come with it.
    fields = {}
    try:
        with open("/proc/cpuinfo") as handle:
            for line in handle:
                if not line.strip():
                    break  # end of the first processor's block
                key, _, value = line.partition(":")
                fields.setdefault(key.strip(), value.strip())
    except OSError:
        pass
    model = fields.get("model name") or platform.processor() or "cpu"
    ids = [f"{name} {fields[key]}" for key, name in (("cpu family", "family"), ("model", "model"),
                                                      ("stepping", "stepping")) if key in fields]
    if ids:
        model = f"{model} ({', '.join(ids)})"
    return {"cpu_model": model, "host_cores": len(os.sched_getaffinity(0)), "torch": torch.__version__}


def cpu_baseline(torch, workloads, cache, table, key_rotation, value_rotation, query, key, value, history,
                 budget_s):
    """The vectorised torch-CPU restatement (oracle/cpu_reference.py) on the host.

    One C2 residual-loop call (loop 0) on a bounded sample of its requests,
    with every host thread torch is given and with one thread, plus the whole
    C0 call (B1 x 512 history tokens, 4 loops) at both thread counts; each
    timing the median of 5 runs after a warm-up.  Reported in GB/s of the
    same algorithmic bytes as the GPU figures."""
    import statistics

    import numpy as np
    from oracle import cpu_reference

    heads, dim, page_tokens = query.size(1), query.size(2), cache.size(3)
    cpu = dict(query=query.cpu(), key=key.cpu(), value=value.cpu(), kr=key_rotation.cpu(), vr=value_rotation.cpu())
    table_np = table.cpu().numpy()
    pages = (history + page_tokens - 1) // page_tokens
    threads_all = max(1, min(torch.get_num_threads(), len(os.sched_getaffinity(0))))
    saved_threads = torch.get_num_threads()

    def c2_request(b):
        blocks = torch.as_tensor(table_np[b][:pages], dtype=torch.long)
        sub = cache[:, blocks.to(cache.device)].cpu()
        local = np.arange(pages, dtype=np.int32).reshape(1, pages)
        start = time.perf_counter()
        cpu_reference.attention(cpu["query"][b:b + 1], cpu["key"][b:b + 1], cpu["value"][b:b + 1], sub, [0, 1],
                                [history + 1], local, cpu["kr"], cpu["vr"], None, SCHEDULE, ANCHOR, 0)
        return time.perf_counter() - start

    def c0_call(c0):
        start = time.perf_counter()
        for loop in range(4):
            cpu_reference.attention(c0["query"], c0["key"], c0["value"], c0["cache"], [0, 1], [513], c0["table"],
                                    c0["kr"], c0["vr"], None, SCHEDULE, ANCHOR, loop)
        return time.perf_counter() - start

    # C0: 16 heads x D128, B1, 512 history tokens, built on the GPU.
    import residualquant_amd as rq
    c0_cache, c0_table, c0_kr, c0_vr = build_packed_cache(torch, rq, workloads, 1, 512, heads, dim, page_tokens,
                                                          query.device, 7)
    g = torch.Generator().manual_seed(8)
    c0 = dict(cache=c0_cache.cpu(), table=c0_table.cpu().numpy(), kr=c0_kr.cpu(), vr=c0_vr.cpu(),
              query=torch.randn((1, heads, dim), generator=g).to(torch.bfloat16),
              key=torch.randn((1, heads, dim), generator=g).to(torch.bfloat16),
              value=torch.randn((1, heads, dim), generator=g).to(torch.bfloat16))
    c0_bytes = sum(staged_call_bytes(1, 512, heads, dim, page_tokens, loop) for loop in range(4))
    request_bytes = staged_call_bytes(1, history, heads, dim, page_tokens, 0)
    rows = {}
    for threads in (threads_all, 1):
        torch.set_num_threads(threads)
        c0_call(c0)
        c0_s = statistics.median(c0_call(c0) for _ in range(5))
        c2_request(0)
        times, spent, b = [], 0.0, 0
        while b < query.size(0) and (len(times) < 1 or spent < budget_s / 2):
            times.append(c2_request(b))
            spent += times[-1]
            b += 1
        rows[threads] = {"c2_GBps": request_bytes / statistics.median(times) / 1e9, "c2_requests": len(times),
                         "c2_s_per_request": statistics.median(times), "c0_GBps": c0_bytes / c0_s / 1e9,
                         "c0_us_per_4_loop_call": c0_s * 1e6}
        log(f"[bench] cpu {threads} threads: C2 residual call {rows[threads]['c2_GBps']:.4f} GB/s "
            f"({len(times)} requests), C0 {rows[threads]['c0_GBps']:.4f} GB/s")
    torch.set_num_threads(saved_threads)
    host = host_description(torch)
    return {
        "value": rows[threads_all]["c2_GBps"],
        "unit": "GB/s",
        "cores": threads_all,
        "kind": "port",
        "sample": f"vectorised torch-CPU restatement (oracle/cpu_reference.py, float64, checked against the C "
                  f"oracle) of one C2 residual-loop call, {rows[threads_all]['c2_requests']} of "
                  f"{query.size(0)} requests x {history} history tokens x {heads} heads, median time per "
                  f"request at {threads_all} threads; {host['cpu_model']}, torch {host['torch']}",
        "single_core": rows[1],
        "all_cores": rows[threads_all],
        **host,
    }


def quantize_cpu_baseline(torch, workloads, pairs, slots, key_rotation, value_rotation, cache_shape, schedule,
                          budget_s):
    """The CPU oracle (single thread) quantizing a bounded prefix of the same tokens."""
    import numpy as np
    from oracle import oracle

    oracle.lib()
    bits = workloads.bf16_bits
    keys = [bits(k) for k, _ in pairs]
    values = [bits(v) for _, v in pairs]
    kr, vr = bits(key_rotation), bits(value_rotation)
    cache = np.zeros(cache_shape, dtype=np.uint8)
    slot_array = slots.cpu().numpy()
    done, elapsed, chunk = 0, 0.0, 16
    while done < slot_array.size and elapsed < budget_s:
        part = slice(done, min(done + chunk, slot_array.size))
        start = time.perf_counter()
        oracle.quantize([(k[part], v[part]) for k, v in zip(keys, values)], cache, slot_array[part], kr, vr,
                        None, schedule, "anchor", ANCHOR, "ls")
        elapsed += time.perf_counter() - start
        done = part.stop
    host = host_description(torch)
    return {
        "value": done / elapsed,
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"first {done} of {slot_array.size} tokens (all heads, both planes) of the g32 schedule, "
                  f"oracle/rq_oracle.c single-threaded; {elapsed:.2f} s; {host['cpu_model']}",
        **host,
    }


def schedule_name(schedule):
    """'[2,32]x3+[4,32]'-style name of a record schedule."""
    parts, i = [], 0
    while i < len(schedule):
        n = 1
        while i + n < len(schedule) and schedule[i + n] == schedule[i]:
            n += 1
        parts.append(f"[{schedule[i][0]},{schedule[i][1]}]" + (f"x{n}" if n > 1 else ""))
        i += n
    return "+".join(parts)


def run_quantize(args):
    """C1: one quantize-on-write call per step for each record schedule.

    The two schedules of the configuration (INT2 residuals at g32 and at g16,
    INT4 g32 anchor) and a mixed one; each is timed with HIP events around
    every call on torch's current stream (the launch stream) after a settle
    phase, and reported as the median call.  ``value`` is the g32 schedule."""
    import statistics

    import torch

    import residualquant_amd as rq
    from residualquant_amd import workloads

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    tokens, heads, dim, page_tokens, seed = args.tokens, 16, 128, 16, 2026
    blocks = 2 * ((tokens + page_tokens - 1) // page_tokens)
    generator = torch.Generator().manual_seed(seed)
    slots = torch.randperm(blocks * page_tokens, generator=generator)[:tokens].to(device)
    pairs = workloads.loop_kv(tokens, heads, dim, 4, seed + 1, device=device)
    key_rotation = workloads.random_sign_rotation(heads, dim, seed + 3, device=device)
    value_rotation = workloads.random_sign_rotation(heads, dim, seed + 4, device=device)
    flop = 2.0 * tokens * heads * 2 * 4 * dim * dim
    input_bytes = tokens * heads * dim * 2 * 4 * 2

    results = {}
    wanted = args.schedules.split(",")
    for name, schedule in (("g32", SCHEDULE), ("g16", HUGINN_SCHEDULE), ("mixed", QUANTIZE_SCHEDULE)):
        if name not in wanted:
            continue
        width = rq.page_width(dim, schedule)
        cache = torch.zeros((2, blocks, heads, page_tokens, width), dtype=torch.uint8, device=device)

        def step(cache=cache, schedule=schedule):
            rq.quantize(pairs, cache, slots, key_rotation, value_rotation, None, schedule, "anchor", ANCHOR, "ls")

        settle(torch, step, 0.3)
        for _ in range(args.warmup):
            step()
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(args.steps)]
        torch.cuda.synchronize()
        start = time.perf_counter()
        for begin, end in events:
            begin.record()
            step()
            end.record()
        torch.cuda.synchronize()
        wall_s = (time.perf_counter() - start) / args.steps
        kernel_ms = statistics.median(b.elapsed_time(e) for b, e in events)  # one launch per call
        output_bytes = tokens * heads * 2 * width
        results[name] = {
            "schedule": schedule_name(schedule) + " anchor 3 ls",
            "us_per_call": kernel_ms * 1e3,
            "us_per_call_wall": wall_s * 1e6,
            "tokens_per_s": tokens / (kernel_ms * 1e-3),
            "rotation_TFLOPs": flop / (kernel_ms * 1e-3) / 1e12,
            "hbm_GBps": (input_bytes + output_bytes) / (kernel_ms * 1e-3) / 1e9,
            "bytes_per_call": input_bytes + output_bytes,
        }
        log(f"[bench] quantize {name}: {kernel_ms * 1e3:.1f} us/call "
            f"({results[name]['rotation_TFLOPs']:.1f} TFLOP/s rotation)")
        del cache

    head = results["g32"] if "g32" in results else next(iter(results.values()))
    cpu = None
    if args.cpu_budget > 0:
        log("[bench] cpu baseline (oracle quantize) ...")
        width = rq.page_width(dim, SCHEDULE)
        cpu = quantize_cpu_baseline(torch, workloads, pairs, slots, key_rotation, value_rotation,
                                    (2, blocks, heads, page_tokens, width), SCHEDULE, args.cpu_budget)
        log(f"[bench] cpu {cpu['value']:.1f} tokens/s")

    result = {
        "metric": "quantize-on-write tokens/s (C1), 1 GPU",
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["us_per_call"] * 1e-3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 rotation and fitting, int2/int4 codes, fp8 scales",
        "data": "synthetic (seeded anchor N(0,1) with 4 outlier channels x8 + loop residuals N(0,0.15^2), "
                "random-sign Hadamard rotations, random slots)",
        "config": {
            "workload": "C1 quantize-on-write micro-benchmark",
            "tokens": tokens, "heads": heads, "head_dim": dim, "loops": 4, "page_tokens": page_tokens,
            "schedule": head["schedule"], "cache_blocks": blocks,
        },
        "timing": "median of per-call HIP events after >= 0.3 s of untimed calls per schedule",
        "schedules": results,
        "roofline": {
            "bound": "mfma",
            "achieved": head["rotation_TFLOPs"],
            "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": head["rotation_TFLOPs"] / PEAK_FP32_TFLOPS,
            "traffic": measured_traffic("quantize_c1_counters.json", "traffic_bytes")["bytes"],
            "traffic_measured_at": measured_traffic("quantize_c1_counters.json", "traffic_bytes")["commit"],
            "kernel": "quantize_mfma_kernel<128,4,3,true>: FP32 rotation FMAs (K=1 v_mfma_f32_16x16x1_4b_f32 "
                      "chains) against the published FP32 peak; HBM traffic is 9% of peak at this rate; on gfx950 "
                      "the FP32 MFMAs and the commit's VALU do not overlap, so the call is their sum",
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def run_prefill(args):
    """A12: causal varlen prefill attention over one prompt; HIP events on torch's stream."""
    import torch

    import residualquant_amd as rq

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    tokens, heads, dim, seed = args.tokens, 16, 128, 2026
    generator = torch.Generator(device=device).manual_seed(seed)
    q, k, v = (torch.randn((tokens, heads, dim), generator=generator, device=device).to(torch.bfloat16)
               for _ in range(3))
    out = torch.empty_like(q)
    cu = torch.tensor([0, tokens], dtype=torch.int32, device=device)
    scale = dim ** -0.5

    def step():
        rq.flash_attn_varlen_func(q=q, k=k, v=v, out=out, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=tokens,
                                  max_seqlen_k=tokens, softmax_scale=scale, causal=True)

    def event_ms(fn, settle_s=0.3):
        """Median of per-call HIP events after a settle phase and the warm-up calls."""
        settle(torch, fn, settle_s)
        for _ in range(args.warmup):
            fn()
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(args.steps)]
        torch.cuda.synchronize()
        for begin, end in events:
            begin.record()
            fn()
            end.record()
        torch.cuda.synchronize()
        return statistics.median(b.elapsed_time(e) for b, e in events)

    kernel_ms = event_ms(step)  # one launch per call
    flop = 2.0 * 2.0 * heads * dim * tokens * (tokens + 1) / 2.0  # QK^T and PV over the causal half
    achieved = flop / (kernel_ms * 1e-3) / 1e12
    log(f"[bench] prefill {kernel_ms * 1e3:.1f} us/call ({achieved:.0f} TFLOP/s)")

    qt, kt, vt = (t.transpose(0, 1).contiguous() for t in (q, k, v))  # [heads, tokens, D]
    torch_ms = event_ms(lambda: torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True,
                                                                                   scale=scale), settle_s=0.0)
    log(f"[bench] torch scaled_dot_product_attention {torch_ms * 1e3:.1f} us/call")

    result = {
        "metric": "prefill attention TFLOP/s (causal, 1 GPU)",
        "value": achieved,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": kernel_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 in, fp32 accumulate",
        "data": "synthetic N(0,1) Q/K/V",
        "config": {"workload": "A12 causal prefill over one prompt", "tokens": tokens, "heads": heads,
                   "head_dim": dim, "softmax_scale": scale},
        "us_per_call": kernel_ms * 1e3,
        "tokens_per_s": tokens / (kernel_ms * 1e-3),
        "timing": "median of per-call HIP events after >= 0.3 s of untimed calls",
        "roofline": {
            "bound": "mfma",
            "achieved": achieved,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / PEAK_BF16_TFLOPS,
            "traffic": measured_traffic("prefill_a12_counters.json", "traffic_bytes")["bytes"],
            "traffic_measured_at": measured_traffic("prefill_a12_counters.json", "traffic_bytes")["commit"],
            "kernel": "prefill_kernel<128>: causal-half QK^T + PV FLOPs against the dense BF16 MFMA peak",
        },
        "torch_sdpa": {"us_per_call": torch_ms * 1e3, "TFLOPs": flop / (torch_ms * 1e-3) / 1e12},
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)




def run_multiquery(args):
    """Several query rows per request over a packed history (multi-row MFMA kernels).

    --geometry ouro (default): B requests x R rows (--rows-per-request) x 8192
    history tokens x 16 heads x D128, the C2 cache and schedule; --geometry
    huginn: 8 requests x 4096 tokens x 55 heads x D96, the C4 cache and
    schedule (--batch / --history override either).  --mode adjacent uses
    the adjacent-mode schedule [4,32]+[2,32]x3 (anchor 0), whose loops past 0
    rebuild the restore chain.  One step = the 4 loop calls.  Timed three ways
    on the same rows: rq.attention with R rows per request (the multi-row
    kernels, the reference's decode semantics: every row sees the history and
    its own key), the same rows as B*R one-row requests (the per-row decode
    kernel, which streams each request's pages R times), and
    rq.packed_prefill_attention (the rows as the requests' last R tokens,
    causal among themselves, over the same history)."""
    import torch

    import residualquant_amd as rq
    from residualquant_amd import ops, workloads

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    huginn = args.geometry == "huginn"
    heads, dim = (55, 96) if huginn else (16, 128)
    batch = args.batch if args.batch is not None else (8 if huginn else 32)
    history = args.history if args.history is not None else (4096 if huginn else 8192)
    rows_per, page_tokens = args.rows_per_request, 16
    adjacent = args.mode == "adjacent"
    if adjacent:
        schedule, mode, anchor = ADJACENT_SCHEDULE, "adjacent", 0
    else:
        schedule, mode, anchor = (HUGINN_SCHEDULE if huginn else SCHEDULE), "anchor", ANCHOR
    seed = 2026
    log(f"[bench] building packed cache B={batch} T={history} H={heads} D={dim} {mode}, {rows_per} rows per request")
    cache, table, key_rotation, value_rotation = build_packed_cache(
        torch, rq, workloads, batch, history, heads, dim, page_tokens, device, seed, schedule, mode, anchor)
    rows = batch * rows_per
    generator = torch.Generator(device=device).manual_seed(seed + 7)
    query, key, value = (torch.randn((rows, heads, dim), generator=generator, device=device).to(torch.bfloat16)
                         for _ in range(3))
    output = torch.empty_like(query)
    qsl = torch.arange(0, rows + 1, rows_per, dtype=torch.int32, device=device)
    seq_decode = torch.full((batch,), history + 1, dtype=torch.int32, device=device)
    seq_prefill = torch.full((batch,), history + rows_per, dtype=torch.int32, device=device)
    # Per-row baseline: every row its own request over its request's pages.
    qsl_rows = torch.arange(rows + 1, dtype=torch.int32, device=device)
    seq_rows = torch.full((rows,), history + 1, dtype=torch.int32, device=device)
    table_rows = table.repeat_interleave(rows_per, dim=0).contiguous()
    workspace = torch.empty(ops.attention_workspace_bytes(rows, heads, dim, table.size(1), page_tokens),
                            dtype=torch.uint8, device=device)

    def multi(loop):
        rq.attention(query, key, value, cache, output, qsl, seq_decode, table, key_rotation, value_rotation, None,
                     schedule, mode, anchor, loop, workspace=workspace)

    def per_row(loop):
        rq.attention(query, key, value, cache, output, qsl_rows, seq_rows, table_rows, key_rotation, value_rotation,
                     None, schedule, mode, anchor, loop, workspace=workspace)

    def prefill(loop):
        rq.packed_prefill_attention(query, key, value, cache, output, qsl, seq_prefill, table, key_rotation,
                                    value_rotation, None, schedule, mode, anchor, loop, workspace=workspace)

    loops = len(schedule)
    # The call the roofline is quoted on: the residual loops in anchor mode,
    # the longest chain (loop 3) in adjacent mode.
    measured = [loops - 1] if adjacent else [loop for loop in range(loops) if loop != anchor]
    results = {}
    for name, call in (("multirow", multi), ("per_row_decode", per_row), ("packed_prefill", prefill)):
        def step(call=call):
            for loop in range(loops):
                call(loop)
        settle(torch, step, 0.2)
        durations = kernel_durations_ms(ops, [lambda loop=loop, call=call: call(loop) for loop in range(loops)],
                                        max(50, args.steps))
        graph = capture(torch, step)
        settle(torch, graph.replay, 0.1)
        step_s = timed(torch, graph.replay, args.steps, args.warmup)
        measured_ms = statistics.median([d for loop in measured for d in durations[loop]])
        results[name] = {"us_per_step": step_s * 1e6, "measured_call_us": measured_ms * 1e3,
                         "per_loop_median_us": [statistics.median(d) * 1e3 for d in durations],
                         "launches_timed": len(durations[0]) * loops}
        log(f"[bench] {name}: step {step_s * 1e6:.1f} us, per loop "
            f"{' / '.join(f'{x:.1f}' for x in results[name]['per_loop_median_us'])} us")
        del graph
    # Algorithmic bytes: the pages once per (request, head) plus the rows' Q/K/V/out.
    extra_rows = 4 * (rows - batch) * heads * dim * 2

    def call_bytes(loop):
        return staged_call_bytes(batch, history, heads, dim, page_tokens, loop, schedule, mode, anchor) + extra_rows

    step_bytes = sum(call_bytes(loop) for loop in range(loops))
    measured_bytes = statistics.mean(call_bytes(loop) for loop in measured)
    m = results["multirow"]
    measured_gbps = measured_bytes / (m["measured_call_us"] * 1e-6) / 1e9
    # MFMA work of one call: per (request, head), 32-token tile and row tile,
    # S and P.V take 2 * 32 * tile_rows * D FLOP each; calls averaging 16 rows
    # per request or fewer run on 16-row tiles.
    tile_rows = 16 if rows_per <= 16 else 32
    tiles = batch * heads * ((history + 31) // 32) * ((rows_per + tile_rows - 1) // tile_rows)
    mfma_flop = tiles * 2 * 2 * 32 * tile_rows * dim
    kernel = (f"multirow_chain_kernel<{dim},16,{tile_rows},4>" if adjacent else
              f"multirow_stream_kernel<{dim},16,{tile_rows},true,...>") + " + multirow_finish_kernel"
    result = {
        "metric": "paged decode-attn µs/step + achieved HBM GB/s (% peak), INT2/INT4 vs bf16, 1 GPU",
        "value": step_bytes / (m["us_per_step"] * 1e-6) / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": m["us_per_step"] * 1e-3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int2/int4 packed codes, fp16/bf16 MFMA operands, fp32 accumulate",
        "data": "synthetic (seeded anchor N(0,1) + loop residuals N(0,0.15^2), random-sign Hadamard rotations)",
        "config": {"workload": "several query rows per request over the "
                               f"{'C4' if huginn else 'C2'} packed history ({mode} mode)",
                   "batch": batch, "rows_per_request": rows_per, "history_tokens": history, "heads": heads,
                   "head_dim": dim, "page_tokens": page_tokens, "schedule": str(schedule), "mode": mode,
                   "anchor": anchor},
        "us_per_step": m["us_per_step"],
        "timing": "one HIP-graph replay of the 4 loop calls per step after settle replays; per-call medians of "
                  ">= 50 launches (HIP events around the call's launches)",
        "bytes_per_step": step_bytes,
        "modes": results,
        "speedup_vs_per_row_decode": results["per_row_decode"]["us_per_step"] / m["us_per_step"],
        "roofline": {
            "bound": "hbm",
            "achieved": measured_gbps,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": measured_gbps / PEAK_HBM_GBPS,
            "traffic": None,
            "kernel": f"{kernel} (loops {measured}), median of {m['launches_timed'] * len(measured) // loops} calls",
            "mfma_TFLOPs": mfma_flop / (m["measured_call_us"] * 1e-6) / 1e12,
        },
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)


def run_adjacent(args):
    """Adjacent-mode decode at the C2 shape: every loop a residual of the
    previous one ([4,32]+[2,32]x3, anchor 0), so loop L reads and rebuilds the
    restore chain of records 0..L.  No BASELINE configuration uses this mode;
    it measures decode_chain_kernel (loops 1-3)."""
    import torch

    import residualquant_amd as rq
    from residualquant_amd import ops, workloads

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    batch, history, heads, dim, page_tokens = args.batch or 32, args.history or 8192, 16, 128, 16
    schedule = ADJACENT_SCHEDULE
    seed = 2027
    log(f"[bench] building adjacent-mode packed cache B={batch} T={history} H={heads} D={dim}")
    cache, table, key_rotation, value_rotation = build_packed_cache(
        torch, rq, workloads, batch, history, heads, dim, page_tokens, device, seed, schedule, "adjacent", 0)
    generator = torch.Generator(device=device).manual_seed(seed + 7)
    query = torch.randn((batch, heads, dim), generator=generator, device=device).to(torch.bfloat16)
    key = torch.randn((batch, heads, dim), generator=generator, device=device).to(torch.bfloat16)
    value = torch.randn((batch, heads, dim), generator=generator, device=device).to(torch.bfloat16)
    output = torch.empty_like(query)
    qsl = torch.arange(batch + 1, dtype=torch.int32, device=device)
    seq_lens = torch.full((batch,), history + 1, dtype=torch.int32, device=device)
    workspace = torch.empty(ops.attention_workspace_bytes(batch, heads, dim, table.size(1), page_tokens),
                            dtype=torch.uint8, device=device)

    def call(loop):
        rq.attention(query, key, value, cache, output, qsl, seq_lens, table, key_rotation, value_rotation,
                     None, schedule, "adjacent", 0, loop, workspace=workspace)

    def step():
        for loop in range(len(schedule)):
            call(loop)

    settle(torch, step, 0.3)
    reps = max(50, args.steps)
    durations = kernel_durations_ms(ops, [lambda loop=loop: call(loop) for loop in range(4)], reps)
    per_loop_ms = [statistics.median(d) for d in durations]
    loop_bytes = [staged_call_bytes(batch, history, heads, dim, page_tokens, loop, schedule, "adjacent", 0)
                  for loop in range(4)]
    for loop in range(4):
        log(f"[bench] adjacent loop {loop}: {per_loop_ms[loop] * 1e3:.1f} us "
            f"({loop_bytes[loop] / (per_loop_ms[loop] * 1e-3) / 1e9:.0f} GB/s on {loop_bytes[loop] / 1e6:.1f} MB)")
    step_ms = sum(per_loop_ms)
    last = loop_bytes[3] / (per_loop_ms[3] * 1e-3) / 1e9
    result = {
        "metric": "adjacent-mode paged decode GB/s (restore chain), 1 GPU",
        "value": sum(loop_bytes) / (step_ms * 1e-3) / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": reps,
        "warmup": 10,
        "ms_per_step": step_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int2/int4 packed codes, bf16 restore chain, fp32 accumulate",
        "data": "synthetic (seeded anchor N(0,1) + loop residuals N(0,0.15^2), random-sign Hadamard rotations)",
        "config": {"workload": "adjacent-mode decode at the C2 shape (no BASELINE configuration)",
                   "batch": batch, "history_tokens": history, "heads": heads, "head_dim": dim,
                   "page_tokens": page_tokens, "schedule": "[4,32]+[2,32]x3 adjacent anchor 0"},
        "timing": "per-loop median of HIP events around each launch (step order) after a settle phase",
        "per_loop_us": [ms * 1e3 for ms in per_loop_ms],
        "per_loop_bytes": loop_bytes,
        "roofline": {
            "bound": "hbm",
            "achieved": last,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": last / PEAK_HBM_GBPS,
            "traffic": None,
            "kernel": "decode_chain_kernel<128,16> at loop 3 (the chain of all 4 records)",
        },
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)


def run_huginn(args):
    """C4: Huginn-shaped deep-loop decode attention, 55 heads x D96, g16 residuals, B8 x T4096.

    One step is the 4 calls of one loop group (3 residual loops + the anchor);
    the recurrent core of 4 layers unrolled 32 loops runs 32 such groups per
    generated token.
    """
    import torch

    import residualquant_amd as rq
    from residualquant_amd import ops, workloads

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.split_target:
        ops.set_split_target(args.split_target)
    batch, history, heads, dim, page_tokens = 8, 4096, 55, 96, 16
    schedule = HUGINN_SCHEDULE
    seed = 4096
    log(f"[bench] building packed cache B={batch} T={history} H={heads} D={dim} {schedule}")
    cache, table, key_rotation, value_rotation = build_packed_cache(
        torch, rq, workloads, batch, history, heads, dim, page_tokens, device, seed, schedule)
    generator = torch.Generator(device=device).manual_seed(seed + 7)
    query = torch.randn((batch, heads, dim), generator=generator, device=device).to(torch.bfloat16)
    key = torch.randn((batch, heads, dim), generator=generator, device=device).to(torch.bfloat16)
    value = torch.randn((batch, heads, dim), generator=generator, device=device).to(torch.bfloat16)
    output = torch.empty_like(query)
    qsl = torch.arange(batch + 1, dtype=torch.int32, device=device)
    seq_lens = torch.full((batch,), history + 1, dtype=torch.int32, device=device)
    workspace = torch.empty(ops.attention_workspace_bytes(batch, heads, dim, table.size(1), page_tokens),
                            dtype=torch.uint8, device=device)

    def call(loop):
        rq.attention(query, key, value, cache, output, qsl, seq_lens, table, key_rotation, value_rotation,
                     None, schedule, "anchor", ANCHOR, loop, workspace=workspace)

    def step():
        for loop in range(len(schedule)):
            call(loop)

    settle(torch, step, 0.3)
    durations = kernel_durations_ms(ops, [lambda loop=loop: call(loop) for loop in range(4)], max(50, args.steps))
    residual_runs = durations[0] + durations[1] + durations[2]
    residual_ms, launches = statistics.median(residual_runs), len(residual_runs)
    anchor_ms = statistics.median(durations[ANCHOR])
    graph = capture(torch, step)
    settle(torch, graph.replay, 0.2)
    step_s = timed(torch, graph.replay, args.steps, args.warmup)
    step_bytes = sum(staged_call_bytes(batch, history, heads, dim, page_tokens, loop, schedule) for loop in range(4))
    residual_bytes = staged_call_bytes(batch, history, heads, dim, page_tokens, 0, schedule)
    anchor_bytes = staged_call_bytes(batch, history, heads, dim, page_tokens, ANCHOR, schedule)
    residual_gbps = residual_bytes / (residual_ms * 1e-3) / 1e9
    log(f"[bench] C4 step {step_s * 1e6:.1f} us; residual call {residual_ms * 1e3:.1f} us ({residual_gbps:.0f} GB/s), "
        f"anchor {anchor_ms * 1e3:.1f} us")

    del workspace
    bf16_cache = torch.randn((2, cache.size(1), heads, page_tokens, dim), device=device,
                             generator=generator).to(torch.bfloat16)
    bf16_ws = torch.empty(ops.attention_workspace_bytes(batch, heads, dim, table.size(1), page_tokens),
                          dtype=torch.uint8, device=device)

    def bf16_call():
        rq.paged_attention_bf16(query, key, value, bf16_cache, output, qsl, seq_lens, table, workspace=bf16_ws)

    settle(torch, bf16_call, 0.2)
    bf16_ms = statistics.median(kernel_durations_ms(ops, [bf16_call], max(50, args.steps))[0])
    bytes_bf16 = bf16_call_bytes(batch, history, heads, dim)
    log(f"[bench] C4 bf16 call {bf16_ms * 1e3:.1f} us ({bytes_bf16 / (bf16_ms * 1e-3) / 1e9:.0f} GB/s)")
    result = {
        "metric": "paged decode-attn µs/step + achieved HBM GB/s (% peak), INT2/INT4 vs bf16, 1 GPU",
        "value": step_bytes / step_s / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int2/int4 packed codes, fp32 accumulate",
        "data": "synthetic (seeded anchor N(0,1) + loop residuals N(0,0.15^2), random-sign Hadamard rotations, "
                "Paley-12 x Sylvester-8 at D96)",
        "config": {
            "workload": "C4 Huginn-shaped deep-loop decode attention",
            "batch": batch, "history_tokens": history, "heads": heads, "head_dim": dim, "loops": 4,
            "page_tokens": page_tokens, "schedule": "[2,16]x3+[4,32] anchor 3 ls",
            "step": "one loop group: 3 residual-loop calls + 1 anchor-loop call",
        },
        "us_per_step": step_s * 1e6,
        "timing": "one HIP-graph replay of the 4 calls per step, timed after >= 0.2 s of untimed replays; "
                  "per-call medians of HIP events after a settle phase",
        "pct_peak_step": 100.0 * step_bytes / step_s / 1e9 / PEAK_HBM_GBPS,
        "bytes_per_step": step_bytes,
        "decode_kernel": {
            "residual_loop_us": residual_ms * 1e3,
            "anchor_loop_us": anchor_ms * 1e3,
            "residual_loop_bytes": residual_bytes,
            "anchor_loop_bytes": anchor_bytes,
            "anchor_loop_GBps": anchor_bytes / (anchor_ms * 1e-3) / 1e9,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": residual_gbps,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": residual_gbps / PEAK_HBM_GBPS,
            "traffic": measured_traffic("decode_c4_counters.json")["bytes"],
            "traffic_measured_at": measured_traffic("decode_c4_counters.json")["commit"],
            "kernel": f"decode96_dma_kernel<16,4,32,2,16,true> (residual loops 0-2), median of {launches} launches "
                      "(HIP events on the launch stream, step order, after 10 warm-up rounds)",
        },
        "bf16_baseline": {
            "us_per_call_kernel": bf16_ms * 1e3,
            "kernel_GBps": bytes_bf16 / (bf16_ms * 1e-3) / 1e9,
            "bytes_per_call": bytes_bf16,
            "residual_call_speedup_packed_vs_bf16": bf16_ms / residual_ms,
        },
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)


def run_step(args):
    """C3: one graph replay = one decode step of all requests through 48 layers x 4 loops."""
    import torch

    from residualquant_amd import ops
    from residualquant_amd.looped_decode import LoopedConfig, LoopedDecoder

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    config = LoopedConfig()
    sweep = [(32, 8192)] if args.no_sweep else [(b, t) for t in (2048, 4096, 8192) for b in (1, 8, 32)]
    new_tokens = args.steps
    weights = None
    results = []
    for batch, context in sweep:
        t0 = time.perf_counter()
        model = LoopedDecoder(config, batch, context, new_tokens + args.warmup + 2, device, seed=2026,
                              weights_from=weights)
        weights = weights or model
        model.build_history(seed=7)
        torch.cuda.synchronize()
        build_s = time.perf_counter() - t0
        # Attention share: one eager step with the library's kernel timing.
        ops.timing_read()
        ops.timing_enable(True)
        model.step()
        torch.cuda.synchronize()
        ops.timing_enable(False)
        attention_ms, attention_calls = ops.timing_read()
        model.capture()
        for _ in range(args.warmup):
            model.replay()
        torch.cuda.synchronize()
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        for _ in range(new_tokens):
            model.replay()
        end.record()
        torch.cuda.synchronize()
        step_ms = begin.elapsed_time(end) / new_tokens
        entry = {"batch": batch, "context": context, "ms_per_step": step_ms, "tokens_per_s": batch / step_ms * 1e3,
                 "attention_kernel_ms_per_step": attention_ms, "attention_calls_per_step": attention_calls,
                 "history_build_s": build_s}
        log(f"[bench] step B={batch} ctx={context}: {step_ms:.2f} ms/step, {entry['tokens_per_s']:.0f} tokens/s, "
            f"split-K attention kernels {attention_ms:.2f} ms in {attention_calls} calls")
        results.append(entry)
        del model
        torch.cuda.empty_cache()
    head = next(r for r in results if (r["batch"], r["context"]) == (32, 8192)) if any(
        (r["batch"], r["context"]) == (32, 8192) for r in results) else results[-1]
    result = {
        "metric": "looped-model decode tokens/s (C3, graph-captured step, 1 GPU)",
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": new_tokens,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 weights/activations, int2/int4 packed KV",
        "data": "synthetic: random-init bf16 weights; history K/V quantized from seeded synthetic loops",
        "config": {"workload": "C3 Ouro-2.6B-shaped looped decode step", "layers": config.layers,
                   "loops": config.loops, "hidden": config.hidden, "heads": config.heads,
                   "head_dim": config.head_dim, "intermediate_assumed": config.intermediate, "vocab": config.vocab,
                   "batch": head["batch"], "context": head["context"], "generated_tokens": new_tokens,
                   "schedule": "[2,32]x3+[4,32] anchor 3 ls"},
        "sweep": results,
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--workload", choices=("decode", "quantize", "prefill", "step", "huginn", "multiquery",
                                               "adjacent"),
                        default="decode",
                        help="decode: C2 paged decode attention (the headline); quantize: C1 quantize-on-write; "
                             "prefill: causal prompt attention; step: C3 looped-model decode step; "
                             "huginn: C4 deep-loop decode attention (55 heads x D96, g16); "
                             "multiquery: several rows per request over the C2 history (multi-row MFMA kernels); "
                             "adjacent: adjacent-mode decode at the C2 shape (the restore-chain kernel)")
    parser.add_argument("--rows-per-request", type=int, default=4, help="multiquery: query rows per request")
    parser.add_argument("--geometry", choices=("ouro", "huginn"), default="ouro",
                        help="multiquery: the C2 (16 heads x D128) or C4 (55 heads x D96) cache")
    parser.add_argument("--mode", choices=("anchor", "adjacent"), default="anchor",
                        help="multiquery: anchor-mode schedule or the adjacent-mode one")
    parser.add_argument("--no-sweep", action="store_true", help="step workload: batch 32 x 8k only")
    parser.add_argument("--tokens", type=int, default=4096, help="tokens per quantize call or prompt")
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--batch", type=int, default=None, help="requests (default: the workload's configuration)")
    parser.add_argument("--history", type=int, default=None, help="history tokens per request (default: the "
                                                                  "workload's configuration)")
    parser.add_argument("--cpu-budget", type=float, default=10.0,
                        help="seconds of CPU oracle work for the cpu_baseline sample (0 = skip)")
    parser.add_argument("--no-bf16", action="store_true")
    parser.add_argument("--schedules", default="g32,g16,mixed",
                        help="quantize: the schedules to time (g32 first: the headline; for counter runs)")
    parser.add_argument("--split-target", type=int, default=0,
                        help="split-K workgroups per decode launch (0 = the library's default)")
    parser.add_argument("--eager", action="store_true",
                        help="time the step as eager launches instead of one HIP-graph replay")
    parser.add_argument("--copy-calibration-mib", type=int, default=0,
                        help="also run a plain FP32 copy kernel of this size (rocprofv3 counter calibration)")
    args = parser.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this path has no multi-GPU component "
              "(the reference forbids TP>1 and DCP>1); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.workload == "quantize":
        run_quantize(args)
        return
    if args.workload == "prefill":
        run_prefill(args)
        return
    if args.workload == "step":
        run_step(args)
        return
    if args.workload == "adjacent":
        run_adjacent(args)
        return
    if args.workload == "huginn":
        run_huginn(args)
        return
    if args.workload == "multiquery":
        run_multiquery(args)
        return
    run_decode(args)


def run_decode(args):
    """C2: one decode step = the 3 residual-loop calls + the anchor-loop call."""
    import torch

    import residualquant_amd as rq
    from residualquant_amd import ops, workloads

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.split_target:
        ops.set_split_target(args.split_target)
    batch, history, heads, dim, page_tokens = args.batch or 32, args.history or 8192, 16, 128, 16
    seed = 2026

    log(f"[bench] building packed cache B={batch} T={history} H={heads} D={dim}")
    t0 = time.perf_counter()
    cache, table, key_rotation, value_rotation = build_packed_cache(
        torch, rq, workloads, batch, history, heads, dim, page_tokens, device, seed)
    log(f"[bench] packed cache {tuple(cache.shape)} built in {time.perf_counter() - t0:.1f} s")

    generator = torch.Generator(device=device).manual_seed(seed + 7)
    query = torch.randn((batch, heads, dim), generator=generator, device=device).to(torch.bfloat16)
    key = torch.randn((batch, heads, dim), generator=generator, device=device).to(torch.bfloat16)
    value = torch.randn((batch, heads, dim), generator=generator, device=device).to(torch.bfloat16)
    output = torch.empty_like(query)
    qsl = torch.arange(batch + 1, dtype=torch.int32, device=device)
    seq_lens = torch.full((batch,), history + 1, dtype=torch.int32, device=device)
    workspace = torch.empty(ops.attention_workspace_bytes(batch, heads, dim, table.size(1), page_tokens),
                            dtype=torch.uint8, device=device)

    def call(loop):
        rq.attention(query, key, value, cache, output, qsl, seq_lens, table, key_rotation, value_rotation,
                     None, SCHEDULE, "anchor", ANCHOR, loop, workspace=workspace)

    def step():
        for loop in range(len(SCHEDULE)):
            call(loop)

    # Per-launch kernel durations in step order (median of >= 50 per loop after
    # 10 warm-up rounds), after the GPU's clocks have settled.
    settle(torch, step, 0.3)
    reps = max(50, args.steps)
    durations = kernel_durations_ms(ops, [lambda loop=loop: call(loop) for loop in range(4)], reps)
    residual_runs = durations[0] + durations[1] + durations[2]
    residual_ms = statistics.median(residual_runs)
    anchor_ms = statistics.median(durations[ANCHOR])
    residual_launches = len(residual_runs)

    eager_s = timed(torch, step, args.steps, args.warmup)
    graph_s = idle_s = None
    if not args.eager:
        graph = capture(torch, step)
        settle(torch, graph.replay, 0.2)
        graph_s = timed(torch, graph.replay, args.steps, args.warmup)
        # The same replays right after an idle second (clocks ramping up), for reference.
        time.sleep(1.0)
        idle_s = timed(torch, graph.replay, args.steps, 0)
    step_s = eager_s if graph_s is None else graph_s
    step_bytes = sum(staged_call_bytes(batch, history, heads, dim, page_tokens, loop) for loop in range(4))
    log(f"[bench] packed step {step_s * 1e6:.1f} us ({'eager' if graph_s is None else 'graph'}), "
        f"eager {eager_s * 1e6:.1f} us" + (f", from idle {idle_s * 1e6:.1f} us" if idle_s else ""))
    residual_bytes = staged_call_bytes(batch, history, heads, dim, page_tokens, 0)
    anchor_bytes = staged_call_bytes(batch, history, heads, dim, page_tokens, ANCHOR)
    residual_gbps = residual_bytes / (residual_ms * 1e-3) / 1e9
    log(f"[bench] residual decode kernel {residual_ms * 1e3:.1f} us ({residual_gbps:.0f} GB/s), "
        f"anchor {anchor_ms * 1e3:.1f} us")

    bf16 = None
    if not args.no_bf16:
        del workspace
        bf16_cache = torch.randn((2, cache.size(1), heads, page_tokens, dim), device=device,
                                 generator=generator).to(torch.bfloat16)
        bf16_ws = torch.empty(ops.attention_workspace_bytes(batch, heads, dim, table.size(1), page_tokens),
                              dtype=torch.uint8, device=device)

        def bf16_call():
            rq.paged_attention_bf16(query, key, value, bf16_cache, output, qsl, seq_lens, table,
                                    workspace=bf16_ws)

        def bf16_step():
            for _ in range(4):
                bf16_call()

        settle(torch, bf16_step, 0.2)
        bf16_ms = statistics.median(kernel_durations_ms(ops, [bf16_call], reps)[0])
        bf16_step_s = timed(torch, bf16_step, args.steps, args.warmup)
        if not args.eager:
            bf16_graph = capture(torch, bf16_step)
            settle(torch, bf16_graph.replay, 0.2)
            bf16_step_s = timed(torch, bf16_graph.replay, args.steps, args.warmup)
            del bf16_graph
        bytes_bf16 = bf16_call_bytes(batch, history, heads, dim)
        bf16 = {
            "us_per_step": bf16_step_s * 1e6,
            "us_per_call_kernel": bf16_ms * 1e3,
            "kernel_GBps": bytes_bf16 / (bf16_ms * 1e-3) / 1e9,
            "bytes_per_call": bytes_bf16,
            "step_speedup_packed_vs_bf16": bf16_step_s / step_s,
        }
        log(f"[bench] bf16 step {bf16_step_s * 1e6:.1f} us, kernel {bf16_ms * 1e3:.1f} us "
            f"({bf16['kernel_GBps']:.0f} GB/s)")
        del bf16_cache, bf16_ws

    if args.copy_calibration_mib:
        n = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: {args.copy_calibration_mib} MiB read + written per launch")
        del src, dst

    cpu = None
    if args.cpu_budget > 0:
        log("[bench] cpu baseline (torch-CPU restatement) ...")
        cpu = cpu_baseline(torch, workloads, cache, table, key_rotation, value_rotation, query, key, value,
                           history, args.cpu_budget)
        log(f"[bench] cpu {cpu['value']:.4f} GB/s at {cpu['cores']} threads")

    traffic = measured_traffic()
    result = {
        "metric": "paged decode-attn µs/step + achieved HBM GB/s (% peak), INT2/INT4 vs bf16, 1 GPU",
        "value": step_bytes / step_s / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int2/int4 packed codes, fp32 accumulate",
        "data": "synthetic (seeded anchor N(0,1) + loop residuals N(0,0.15^2), random-sign Hadamard rotations)",
        "config": {
            "workload": "C2 paged decode attention, Ouro-1.4B-shaped layer",
            "batch": batch, "history_tokens": history, "heads": heads, "head_dim": dim, "loops": 4,
            "page_tokens": page_tokens, "schedule": "[2,32]x3+[4,32] anchor 3 ls",
            "step": "3 residual-loop calls + 1 anchor-loop call (one split-K decode launch each: query preparation, page streaming, live-token merge, V inverse rotation)",
        },
        "us_per_step": step_s * 1e6,
        "us_per_step_eager": eager_s * 1e6,
        "us_per_step_from_idle": None if idle_s is None else idle_s * 1e6,
        "timing": ("one HIP-graph replay of the 4 calls per step, timed after >= 0.2 s of untimed replays "
                   "(the GPU's clocks ramp up over the first ~50 replays after idle; us_per_step_from_idle "
                   "times the same replays right after an idle second)") if graph_s is not None
                  else "eager launches",
        "pct_peak_step": 100.0 * step_bytes / step_s / 1e9 / PEAK_HBM_GBPS,
        "bytes_per_step": step_bytes,
        "tokens_per_s": batch / step_s,
        "decode_kernel": {
            "residual_loop_us": residual_ms * 1e3,
            "anchor_loop_us": anchor_ms * 1e3,
            "per_loop_median_us": [statistics.median(d) * 1e3 for d in durations],
            "residual_loop_bytes": residual_bytes,
            "anchor_loop_bytes": anchor_bytes,
            "anchor_loop_GBps": anchor_bytes / (anchor_ms * 1e-3) / 1e9,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": residual_gbps,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": residual_gbps / PEAK_HBM_GBPS,
            "traffic": traffic["bytes"],
            "traffic_measured_at": traffic["commit"],
            "kernel": "decode_kernel<128,16,4,32,2,32,true> (residual loops 0-2), median of "
                      f"{residual_launches} launches (HIP events on the launch stream, step order, "
                      "after 10 warm-up rounds)",
        },
        "bf16_baseline": bf16,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
