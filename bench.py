#!/usr/bin/env python3
"""End-to-end speculative-decoding step on one MI355X (benchmark config 5).

Workload: a random-init Gemma-4-31B-shaped FP8 target (60 layers, 5 sliding(1024) : 1 global,
hidden 5376, intermediate 21504, 32 query / 16 KV heads x 128, vocab 262144) and a random-init
4-layer assistant (hidden 1024 on the 5376 backbone, the reference's assistant dims), 24 slots with
~8.1k-token contexts, prefilled (untimed) from seeded random token ids through the runner's own
prefill_slots_chunks. One step = the reference scheduler's speculative cycle
(native_runtime_main.cpp:583-678, run in C++ by carat_hip_bench_speculative_cycle): draft_four
(forced + 4 drafts) -> acceptance caps -> verify_greedy_proposals -> commit_speculation. Drafts are overwritten, before verification, with
the target's own greedy chain (computed untimed by dry verifies that commit nothing) so that each
draft matches with probability 0.7 (geometric acceptance), as config 5 specifies.

Prints ONE JSON line. `value` = accepted tokens (sum of the reference's accepted_tokens, which
counts the forced token, = emitted tokens per step) / timed seconds. `roofline` times the step's
dominant kernel by total time, the global verify attention, after the timed steps: every global
layer's attention over its own cache runs back to back on the runner's stream between one pair of
HIP events (two passes), so the per-launch figure is kernel time as a profiler sees it, not
event-marker overhead. `roofline_gate_up` (the largest GEMM), `roofline_attention_sliding` and
`gemms` (every per-layer FP8 GEMM) are timed the same way; each `gemms` entry also carries the
vendor library's time (torch._scaled_mm, i.e. hipBLASLt, with cold weights) at the same shape.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

SLOTS = 24
DRAFTS = 4
DEPTH = DRAFTS + 1  # reference depth counts the forced token (native_runtime_main.cpp:604-610)
MAX_CONTEXT = 8192
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
ACCEPT_P = 0.7


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def prefill_contexts(runner, rng, vocab, length):
    """Config 5's contexts: `length` seeded random token ids per slot, made resident with
    prefill_slots_chunks (forced verify steps sharing the 1024-row step budget). Returns the
    target's greedy next token per slot (the first forced token) and each prompt's last token."""
    slots = list(range(SLOTS))
    prompts = [rng.integers(0, vocab, length).astype(np.int32).tolist() for _ in slots]
    for s in slots:
        runner.reset_slot(s)
    # each call packs at most the context's worth of chunk tokens (batch_model_runner.cu:1262);
    # a multiple of the 42 rows per slot that a 1024-row step gives 24 slots
    per_step = 1024 // SLOTS
    quantum = MAX_CONTEXT // SLOTS // per_step * per_step
    out = [None]
    while any(v is None for v in out):
        out = runner.prefill_slots_chunks(slots, prompts, quantum)
    return np.array(out, np.int32), np.array([p[-1] for p in prompts], np.int32)


def planted_proposals(runner, forced, slots, rng, vocab):
    """Greedy chain of the target from dry verifies (caps 0: nothing is committed), then drafts that
    follow it with probability ACCEPT_P per position, a random other token at the first miss."""
    chain = np.zeros((len(slots), DEPTH), np.int32)
    chain[:, 0] = forced
    for t in range(DRAFTS):
        props = np.zeros((len(slots), DEPTH), np.int32)
        props[:, : t + 1] = chain[:, : t + 1]
        runner.verify_greedy_proposals(props.tolist(), list(forced), slots, [0] * len(slots))
        pred = np.asarray(runner.last_predictions, np.int32).reshape(len(slots), DEPTH)
        chain[:, t + 1] = pred[:, t]
    proposals = chain.copy()
    for r in range(len(slots)):
        for j in range(1, DEPTH):
            if rng.random() >= ACCEPT_P:
                other = int(rng.integers(0, vocab - 1))
                proposals[r, j] = other if other < chain[r, j] else other + 1
                proposals[r, j + 1:] = rng.integers(0, vocab, DEPTH - j - 1)
                break
    return proposals


COPY_CALIBRATION_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "gemm_gate_up_config5_traffic.json")
ATTENTION_TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                      "attention_global_config5_traffic.json")


def measured_traffic():
    """HBM bytes per gate/up launch from the committed rocprofv3 FETCH_SIZE + WRITE_SIZE passes
    (scaled by the same counters on a plain copy of known size), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            return int(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def measured_attention_traffic():
    """HBM bytes per global verify attention launch from the same committed counter passes, or
    None."""
    try:
        with open(ATTENTION_TRAFFIC_FILE) as f:
            return int(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def global_attention_bytes(positions, tokens, kv_heads, head_dim, query_heads):
    # algorithmic bytes of one global verify attention launch: every visible cached K and V row
    # (positions p .. p + T - 1 see keys 0 .. p + T - 1, the last T from this step's rows), bf16,
    # plus the bf16 queries and outputs
    keys = sum(int(p) + tokens for p in positions)
    return keys * kv_heads * head_dim * 2 * 2 + 2 * len(positions) * tokens * query_heads * head_dim * 2


def gate_up_bytes(hidden, intermediate, rows):
    # algorithmic bytes of one gate/up launch: e4m3 weights + e4m3 activations + bf16 GELU output
    return 2 * intermediate * hidden + rows * hidden + rows * intermediate * 2


def gemm_plan(n, k, gate_up):
    import ctypes
    from carat_amd import _lib
    f, w, sp = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _lib.check(_lib.lib().carat_hip_gemm_plan(n, k, 1, int(gate_up), ctypes.byref(f), ctypes.byref(w),
                                              ctypes.byref(sp)))
    return f.value, w.value, sp.value


def library_gemm_us(m, n, k, cycle_bytes=1200 << 20):
    """The vendor library's time for the same fp8 GEMM shape, as a comparison: torch._scaled_mm
    (hipBLASLt on ROCm) with per-tensor scales and a bf16 output, cycling through enough weight
    copies (> the 256 MB memory-side cache) that every launch reads its weights from HBM, as each
    layer's GEMM does in the step. It has no split-K partials and no GELU epilogue."""
    import torch
    copies = max(2, -(-cycle_bytes // (n * k)))
    gen = torch.Generator(device="cuda").manual_seed(11)
    a = (torch.randn(m, k, device="cuda", generator=gen) * 0.5).to(torch.float8_e4m3fn)
    ws = [(torch.randn(n, k, device="cuda", generator=gen) * 0.5).to(torch.float8_e4m3fn).t()
          for _ in range(copies)]
    one = torch.ones((), device="cuda")
    run = lambda w: torch._scaled_mm(a, w, scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
    for w in ws:
        run(w)
    reps = max(20, 2 * copies)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(reps):
        run(ws[i % copies])
    stop.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(stop) * 1e3 / reps
    del ws
    torch.cuda.empty_cache()
    return us


def gemm_table(runner, desc, rows, library=True):
    """Every per-layer fp8 GEMM of the verify step timed back to back over all 60 layers' weights
    (stream_gemm_probe, two passes): HBM fraction of 8 TB/s over the algorithmic bytes (e4m3
    weights + e4m3 activations + outputs: fp32 split-K partials or the bf16 GELU output), raw fp8
    MFMA use (2*M*N*K flops per launch / 5 PFLOP/s), and the attainable MFMA use at that
    arithmetic intensity (min(1, AI * 8 TB/s / 5 PFLOP/s)). With `library`, each entry also
    carries the vendor library's time for the same shape (library_gemm_us) and the speedup over it."""
    H, I = desc.hidden, desc.intermediate
    g = next(l for l in desc.layers if not l.sliding)
    qkv_n = (g.query_heads + 2 * g.kv_heads) * g.head_dimension
    shapes = {"qkv_gemm": (qkv_n, H, False), "o_gemm": (H, g.query_heads * g.head_dimension, False),
              "gate_up_gemm": (2 * I, H, True), "down_gemm": (H, I, False)}
    out = {}
    for kind, (n, k, gate_up) in shapes.items():
        f, w, splits = gemm_plan(n, k, gate_up)
        avg_ms, launches = runner.stream_gemm_probe(kind, passes=2)
        out_bytes = rows * (n // 2) * 2 if gate_up else splits * rows * n * 4
        nbytes = n * k + rows * k + out_bytes
        flops = 2.0 * rows * n * k
        us = avg_ms * 1e3
        gbs = nbytes / us / 1e3
        util = flops / (us * 1e-6) / (FP8_PEAK_TFLOPS * 1e12)
        attainable = min(1.0, flops / nbytes * HBM_PEAK_GBS * 1e9 / (FP8_PEAK_TFLOPS * 1e12))
        out[kind.replace("_gemm", "")] = {
            "n": n, "k": k, "layout": f"F{f}/W{w}", "splits": splits, "avg_launch_us": round(us, 2),
            "bytes_per_launch": nbytes, "GB_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "mfma_util": round(util, 4), "mfma_attainable": round(attainable, 4),
            "frac_of_attainable": round(util / attainable, 4)}
    if library:
        add_library_times(out, rows)
    return out


def add_library_times(table, rows):
    """Adds the vendor library's time at each gemm_table entry's shape. Run it after every timing
    of this library's kernels: the kernels measured right after a burst of library GEMMs run
    slower (gate/up 45 -> 55 us, global attention 281 -> 296 us)."""
    for entry in table.values():
        lib_us = library_gemm_us(rows, entry["n"], entry["k"])
        entry["hipblaslt_us"] = round(lib_us, 2)
        entry["speedup_vs_hipblaslt"] = round(lib_us / entry["avg_launch_us"], 3)


def cpu_baseline(mean_accepted_per_step):
    """Plain OpenMP C evaluation (the oracle, a restatement of the reference's verify layer) timed
    on this host over a bounded sample: two sliding layers (averaged) and one global layer at the
    full config-5 shape, the whole lm_head with its argmax, and the argmax + greedy acceptance over
    24x5 rows, and one assistant draft step (x5 for the draft's depth).
    Extrapolated to 50 sliding + 10 global layers."""
    from oracle import oracle

    rng = np.random.default_rng(0)
    R, T, H, I, hq, hkv, D = SLOTS, DEPTH, 5376, 21504, 32, 16, 128
    M = R * T
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    bf = lambda shape, s=1.0: oracle.f32_to_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(s))
    fp8 = lambda shape: rng.integers(0, 0x7E, shape, dtype=np.uint8)
    x = bf((M, H))
    w_qkv, w_o, w_gu, w_down = fp8((8192, H)), fp8((H, 4096)), fp8((2 * I, H)), fp8((H, I))
    norm_w = bf((H,), 0.05)
    qn = bf((D,), 0.05)
    cos, sin = oracle.rope_table(D, False, MAX_CONTEXT)

    caches = {sliding: (bf((R, hkv, 1024 if sliding else MAX_CONTEXT, D), 1 / math.sqrt(D)),
                        bf((R, hkv, 1024 if sliding else MAX_CONTEXT, D), 1 / math.sqrt(D)))
              for sliding in (True, False)}

    def layer(sliding):
        C = 1024 if sliding else MAX_CONTEXT
        positions = np.full(R, MAX_CONTEXT - 64, np.int32)
        kc, vc = caches[sliding]
        t0 = time.perf_counter()
        n, _ = oracle.rms_norm(x, norm_w)
        qx, sx = oracle.quantize_e4m3(n)
        packed = oracle.fp8_linear(qx, sx, w_qkv, 0.001)
        rowpos = np.repeat(positions, T) + np.tile(np.arange(T, dtype=np.int32), R)
        q, k, v = oracle.qkv_post(packed, qn, qn, cos, sin, rowpos, hq, hkv, D)
        att = oracle.verify_attention(q.reshape(R, T, hq, D), kc, vc, k.reshape(R, T, hkv, D),
                                      v.reshape(R, T, hkv, D), np.arange(R, dtype=np.int32),
                                      positions, C, C if sliding else 0)
        qa, sa = oracle.quantize_e4m3(att.reshape(M, hq * D))
        proj = oracle.fp8_linear(qa, sa, w_o, 0.001)
        r1, pre, _ = oracle.rms_norm_add_and_norm(proj, norm_w, x, norm_w)
        qp, sp = oracle.quantize_e4m3(pre)
        gu = oracle.fp8_linear(qp, sp, w_gu, 0.001)
        act, _ = oracle.gelu_tanh_gate_rows(gu)
        qd, sd = oracle.quantize_e4m3(act)
        down = oracle.fp8_linear(qd, sd, w_down, 0.001)
        oracle.rms_norm_add_scale(down, norm_w, r1, 0x3F80)
        return time.perf_counter() - t0

    t_sliding = (layer(True) + layer(True)) / 2
    t_global = layer(False)
    emb = fp8((262144, H))  # the whole tied lm_head
    t0 = time.perf_counter()
    oracle.fp8_lm_head_argmax(x, emb, 0.001)
    t_lm = time.perf_counter() - t0
    del emb

    # One assistant draft step (assistant_runner.cu:218-338, bf16 weights; the dims of
    # ModelDesc's assistant): embedding | previous hidden -> pre-projection, three layers over the
    # sliding cache and one over the global one, final norm, lm_head + argmax, post-projection.
    AH, AI, AQ = 1024, 8192, 32
    a_layers = [dict(q=bf((AQ * D, AH), 0.03), o=bf((AH, AQ * D), 0.03),
                     gate_up=bf((2 * AI, AH), 0.03), down=bf((AH, AI), 0.03)) for _ in range(4)]
    a_norm = bf((AH,), 0.05)
    pre_w, post_w = bf((AH, 2 * H), 0.02), bf((H, AH), 0.03)
    a_head = bf((262144, AH), 0.03)
    token_table = bf((4096, H))  # a slice of the target embedding: the gather is not the cost
    context = np.full(R, MAX_CONTEXT - 64, np.int32)
    slot_ids = np.arange(R, dtype=np.int32)
    previous = bf((R, H))

    def draft_step():
        t0 = time.perf_counter()
        tokens = rng.integers(0, 4096, R).astype(np.int32)
        h = oracle.bf16_linear(np.concatenate([oracle.embedding(token_table, tokens, math.sqrt(H)),
                                               previous], axis=1), pre_w)
        for li, w in enumerate(a_layers):
            sliding = li < 3
            kc, vc = caches[sliding]
            n, _ = oracle.rms_norm(h, a_norm)
            q, _, _ = oracle.qkv_post(oracle.bf16_linear(n, w["q"]), qn, qn, cos, sin, context, AQ, 0, D)
            attn = oracle.decode_attention(q, kc, vc, slot_ids, context, hkv, 1024 if sliding else MAX_CONTEXT)
            o = oracle.bf16_linear(attn.reshape(R, AQ * D), w["o"])
            r1, pre_mlp, _ = oracle.rms_norm_add_and_norm(o, a_norm, h, a_norm)
            act, _ = oracle.gelu_tanh_gate_rows(oracle.bf16_linear(pre_mlp, w["gate_up"]))
            h = oracle.rms_norm_add_scale(oracle.bf16_linear(act, w["down"]), a_norm, r1, 0x3F80)
        fh, _ = oracle.rms_norm(h, a_norm)
        t_body = time.perf_counter() - t0
        t1 = time.perf_counter()
        oracle.argmax_bf16_rows(oracle.bf16_linear(fh, a_head))
        t_head = time.perf_counter() - t1
        t2 = time.perf_counter()
        oracle.bf16_linear(fh, post_w)
        return t_body + time.perf_counter() - t2, t_head

    t_draft_body, t_draft_head = draft_step()
    # depth 5: five steps, the first one forced (no lm_head)
    t_draft = DEPTH * t_draft_body + (DEPTH - 1) * t_draft_head
    logits = rng.standard_normal((M, 262144), dtype=np.float32)
    t0 = time.perf_counter()
    pred = oracle.argmax_f32_rows_as_bf16(logits).reshape(R, T)
    oracle.greedy_accept(pred, pred[:, 0], pred)
    for r in range(R):  # the reference's own host helpers (speculation.cpp), when built
        if oracle.ref() is not None:
            oracle.ref_acceptance_cap(DEPTH, 100, pred[r].tolist(), [1])
            oracle.ref_commit_speculation(int(pred[r, 0]), pred[r, 1:3].tolist(), int(pred[r, 3]), [1])
    t_accept = time.perf_counter() - t0
    step = 50 * t_sliding + 10 * t_global + t_lm + t_accept + t_draft
    return {
        "value": round(mean_accepted_per_step / step, 3),
        "unit": "accepted tok/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"2 sliding + 1 global verify layer at config-5 shape ({t_sliding:.2f}s each, "
                   f"{t_global:.2f}s), the whole 262144-row lm_head with argmax ({t_lm:.2f}s), "
                   f"argmax+acceptance over 24x5x262144 ({t_accept:.2f}s), one assistant draft "
                   f"step ({t_draft_body:.2f}s + lm_head {t_draft_head:.2f}s, x5 with 4 heads -> "
                   f"{t_draft:.2f}s); extrapolated to 50+10 layers = {step:.1f}s/step at "
                   f"{mean_accepted_per_step:.1f} accepted tokens/step"),
    }


# Attention shapes timed by --attention-shapes: (name, mode, kv heads, head_dim, capacity,
# position, tokens, e4m3 KV). 24 slots, 32 query heads. The native rows are Gemma-4 31B's own
# geometry (gemma4_config.cpp:174-203); the benchmark rows are config 5's, and config 3's e4m3
# KV variant of the global layer.
ATTENTION_SHAPES = [
    ("benchmark sliding verify D128", 0, 16, 128, 1024, 8000, 5, False),
    ("benchmark global verify D128", 1, 16, 128, 8192, 8124, 5, False),
    ("benchmark global verify D128, e4m3 KV (config 3)", 1, 16, 128, 8192, 8124, 5, True),
    ("native sliding verify D256", 0, 16, 256, 1024, 8000, 5, False),
    ("native global verify D512 (40 query rows per kv head)", 1, 4, 512, 8192, 8124, 5, False),
    ("native assistant sliding decode D256", 2, 16, 256, 1024, 8000, 1, False),
    ("native assistant global decode D512", 2, 4, 512, 8192, 8124, 1, False),
]


def attention_shapes(reps: int = 10) -> dict:
    """Times each ATTENTION_SHAPES case through the op-level C ABI: `reps` back-to-back launches
    (attention + merge when split) between two HIP events on torch's stream, after 2 warm-ups.
    The launches rotate over enough K/V copies (>= 1.6 GB) that every launch reads cold HBM, as a
    layer of the verify step does, rather than the 256 MB MALL. No output amax is requested (the
    runner's is striped; the op ABI's single float would serialise the merge's updates).
    Bytes = the visible K and V rows read (bf16, or e4m3 for the e4m3-KV row)."""
    import ctypes
    import torch
    from carat_amd import _lib
    out = []
    R, hq = 24, 32
    stream = torch.cuda.current_stream()
    for name, mode, hkv, d, cap, pos, tokens, fp8 in ATTENTION_SHAPES:
        g = torch.Generator(device="cuda").manual_seed(5)
        mk = lambda *shape: (torch.randn(*shape, device="cuda", generator=g) * 0.1).to(torch.bfloat16)
        # e4m3 K/V: the same values scaled into range and converted by torch (scale 1/448 of max)
        kv = (lambda *shape: (torch.randn(*shape, device="cuda", generator=g) * 64).clamp(-448, 448)
              .to(torch.float8_e4m3fn).view(torch.uint8)) if fp8 else mk
        copy_bytes = 2 * R * hkv * cap * d * (1 if fp8 else 2)
        copies = max(2, -(-(1600 << 20) // copy_bytes))
        caches = [(kv(R, hkv, cap, d), kv(R, hkv, cap, d)) for _ in range(copies)]
        kn, vn = kv(R, tokens, hkv, d), kv(R, tokens, hkv, d)
        q = mk(R, tokens, hq, d)
        o = torch.zeros_like(q)
        slots = torch.arange(R, dtype=torch.int32, device="cuda")
        positions = torch.full((R,), pos, dtype=torch.int32, device="cuda")
        window = cap if mode == 0 else 0
        max_keys = cap + tokens - 1 if mode == 0 else (pos + tokens if mode == 1 else min(pos + 1, cap))
        keys = {0: min(cap + tokens - 1, pos + tokens), 1: pos + tokens, 2: min(pos + 1, cap)}[mode]
        p = lambda t: ctypes.c_void_p(t.data_ptr())

        def launch(i):
            kc, vc = caches[i % copies]
            _lib.check(_lib.lib().carat_hip_verify_attention(
                mode, p(q), p(kc), p(vc), p(kn), p(vn), int(fp8), ctypes.c_float(1 / 448 if fp8 else 1.0),
                ctypes.c_float(1 / 448 if fp8 else 1.0),
                p(slots), p(positions), R, tokens, hq, hkv, d, cap, window, max_keys, p(o), None,
                0, ctypes.c_void_p(stream.cuda_stream)))
        for i in range(2):
            launch(i)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(reps):
            launch(i)
        stop.record(stream)
        torch.cuda.synchronize()
        us = start.elapsed_time(stop) * 1e3 / reps
        bytes_read = R * hkv * keys * d * 2 * (1 if fp8 else 2)
        out.append({"shape": name, "us": round(us, 2), "bytes": bytes_read,
                    "GB_s": round(bytes_read / us / 1e3, 1),
                    "frac": round(bytes_read / us / 1e3 / HBM_PEAK_GBS, 4)})
        del caches, kn, vn, q, o
    return {"metric": "attention kernel time per launch (cold HBM)", "unit": "us", "cases": out}


def prefill_throughput(tokens: int, seed: int, library: bool = True) -> dict:
    """Prefill of the config-5 model from empty slots: prefill_slots_chunks over all 24 slots
    (forced steps sharing the 1024-row step budget: 42 rows per slot), then prefill_slot on one
    slot (forced steps of up to 1024 rows, the sliding ring). Prompt tokens made resident per
    second; `gemms` times the per-layer GEMMs at the 1008-row step shape (gemm_table)."""
    from carat_amd import lib
    from carat_amd.runner import BatchModelRunner, ModelDesc
    rng = np.random.default_rng(seed)
    desc = ModelDesc.gemma4_benchmark(with_assistant=False)
    runner = BatchModelRunner(desc, SLOTS, MAX_CONTEXT)
    prompts = [rng.integers(0, desc.vocabulary, tokens).astype(np.int32).tolist() for _ in range(SLOTS)]
    slots = list(range(SLOTS))
    warm = [p[:8] for p in prompts]
    for s in slots:
        runner.reset_slot(s)
    runner.prefill_slots_chunks(slots, warm, 8)  # warm-up: one step
    runner.prefill_slot(0, prompts[0][:1024], 1024)  # warm-up: one deep step
    for s in slots:
        runner.reset_slot(s)
    lib().carat_hip_synchronize()
    t0 = time.perf_counter()
    # each call packs at most the context's worth of chunk tokens (batch_model_runner.cu:1262);
    # a multiple of the 42 rows per slot that a 1024-row step gives 24 slots
    per_step = 1024 // SLOTS
    quantum = MAX_CONTEXT // SLOTS // per_step * per_step
    calls = 0
    out = [None]
    while any(v is None for v in out):
        out = runner.prefill_slots_chunks(slots, prompts, quantum)
        calls += 1
    lib().carat_hip_synchronize()
    seconds = time.perf_counter() - t0
    runner.reset_slot(0)
    lib().carat_hip_synchronize()
    t0 = time.perf_counter()
    runner.prefill_slot(0, prompts[0], tokens)
    lib().carat_hip_synchronize()
    single = time.perf_counter() - t0
    # the per-layer GEMMs at the 1008-row step shape (one more 42-row-per-slot step sets it)
    for s in slots:
        runner.reset_slot(s)
    runner.prefill_slots_chunks(slots, prompts, per_step)
    gemms = gemm_table(runner, desc, SLOTS * per_step, library=library)
    return {"metric": "prefill tokens/s (24 slots, config-5 model, forced steps of 42 rows per slot)",
            "value": round(SLOTS * tokens / seconds, 1), "unit": "tokens/s",
            "prompt_tokens": tokens, "slots": SLOTS, "seconds": round(seconds, 3),
            "calls": calls, "chunk_tokens": quantum,
            "single_slot": {"value": round(tokens / single, 1), "unit": "tokens/s",
                            "seconds": round(single, 4), "steps": (tokens + 1023) // 1024},
            "gemms": gemms}


def acceptance_config1(seed: int, reps: int = 20, cpu_baseline: bool = True) -> dict:
    """Config 1 on the GPU: argmax over 24 x 5 x 262144 fp32 logits N(0,1) + greedy acceptance
    with drafts planted as the row argmax at p = 0.7 per position (carat_hip_argmax_accept, the
    op-level entry point). `reps` back-to-back calls between two HIP events on torch's stream."""
    import ctypes
    import torch
    from carat_amd import _lib
    R, T, V = SLOTS, DEPTH, 262144
    g = torch.Generator(device="cuda").manual_seed(seed)
    logits = torch.randn(R * T, V, device="cuda", generator=g, dtype=torch.float32)
    arg = logits.bfloat16().argmax(dim=1).view(R, T).cpu().numpy()  # the kernel ranks rows as bf16
    rng = np.random.default_rng(seed)
    proposals = np.zeros((R, T), np.int32)
    first = rng.integers(0, V, R).astype(np.int32)
    proposals[:, 0] = first
    for r in range(R):
        matching = True
        for j in range(T - 1):
            if matching and rng.random() < ACCEPT_P:
                proposals[r, j + 1] = arg[r, j]
            else:
                matching = False
                other = int(rng.integers(0, V - 1))
                proposals[r, j + 1] = other if other < arg[r, j] else other + 1
    d_prop = torch.from_numpy(proposals).cuda()
    d_first = torch.from_numpy(first).cuda()
    pred = torch.zeros(R * T, dtype=torch.int32, device="cuda")
    acc = torch.zeros(R, dtype=torch.int32, device="cuda")
    nxt = torch.zeros(R, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    p = lambda t: ctypes.c_void_p(t.data_ptr())

    def launch():
        _lib.check(_lib.lib().carat_hip_argmax_accept(
            p(logits), None, R, T, V, p(d_prop), p(d_first), None, p(pred), p(acc), p(nxt),
            ctypes.c_void_p(stream.cuda_stream)))
    for _ in range(3):
        launch()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        launch()
    stop.record(stream)
    torch.cuda.synchronize()
    us = start.elapsed_time(stop) * 1e3 / reps
    nbytes = R * T * V * 4
    out = {"metric": "config 1 argmax + greedy acceptance (24 x 5 x 262144 fp32 logits)",
           "us": round(us, 2), "unit": "us per call", "bytes": nbytes,
           "GB_s": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
           "mean_accepted": round(float(acc.float().mean()), 3)}
    if cpu_baseline:
        out["cpu_baseline"] = acceptance_cpu_baseline(
            logits.cpu().numpy(), proposals, first,
            (pred.cpu().numpy(), acc.cpu().numpy(), nxt.cpu().numpy()))
    return out


def acceptance_cpu_baseline(logits, proposals, first, gpu, seconds=3.0):
    """Config 1 on the host: the oracle's OpenMP row argmax over the same fp32 logits (ranked as
    bf16), its greedy acceptance (batch_model_runner.cu:1738-1759), and per slot the reference's
    own acceptance_cap and commit_speculation (speculation.cpp, compiled into oracle/_ref when
    the reference tree was present at build time; the oracle's restatement otherwise), repeated
    for about `seconds`. Also reports whether the host results equal the GPU's."""
    from oracle import oracle
    R, T = proposals.shape
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    use_ref = oracle.ref() is not None
    cap = oracle.ref_acceptance_cap if use_ref else oracle.acceptance_cap
    commit = oracle.ref_commit_speculation if use_ref else oracle.commit_speculation
    calls = 0
    t0 = time.perf_counter()
    while True:
        pred = oracle.argmax_f32_rows_as_bf16(logits)
        caps = np.array([cap(T, 1 << 20, proposals[r], []) for r in range(R)], np.int32)
        acc, nxt = oracle.greedy_accept(proposals, first, pred.reshape(R, T), caps)
        for r in range(R):
            commit(int(first[r]), proposals[r, 1:max(int(acc[r]), 1)].tolist(), int(nxt[r]), [])
        calls += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    matches = (np.array_equal(pred, gpu[0]) and np.array_equal(acc, gpu[1]) and
               np.array_equal(nxt, gpu[2]))
    return {"value": round(1e6 * elapsed / calls, 1), "unit": "us per call", "cores": threads,
            "kind": "reference" if use_ref else "port", "calls": calls, "matches_gpu": bool(matches),
            "sample": "the whole config-1 workload per call: OpenMP argmax over 120 x 262144 fp32, "
                      "greedy acceptance, 24 acceptance_cap + commit_speculation calls "
                      f"({'reference speculation.cpp' if use_ref else 'restated speculation'})"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--graphs", action="store_true", help="replay the verify step as a HIP graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-library-compare", action="store_true",
                    help="skip timing the vendor library (hipBLASLt) at the per-layer GEMM shapes")
    ap.add_argument("--assistant-fp8", choices=["off", "lm_head", "all"], default=None,
                    help="the assistant's AssistantFp8Mode (default: CARAT_ASSISTANT_FP8_MODE, "
                         "as the reference reads it; unset = off)")
    ap.add_argument("--fp8-scaling", choices=["tensor", "channel", "block_128"], default="tensor",
                    help="Fp8Scaling of the target's e4m3 weights (the reference serves per tensor)")
    ap.add_argument("--no-breakdown", action="store_true",
                    help="skip the per-kernel-family probe of one verify step (kernels_ms_per_verify)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one 256 MiB device-to-device copy (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--attention-shapes", action="store_true",
                    help="time the benchmark and native Gemma-4 attention shapes instead of the step")
    ap.add_argument("--acceptance", action="store_true",
                    help="time config 1 (argmax + greedy acceptance over 24x5x262144 fp32 logits)")
    ap.add_argument("--native", action="store_true",
                    help="the same step at the native Gemma-4 31B attention geometry (sliding D 256, "
                         "global D 512 with 4 kv heads and K = V) instead of config 5's D 128")
    ap.add_argument("--seeded-cache", action="store_true",
                    help="fill the KV caches with seeded N(0, 1/D) values instead of prefilling "
                         "the contexts from seeded random token ids (same bytes, faster set-up)")
    ap.add_argument("--prefill", type=int, default=0, metavar="TOKENS",
                    help="time prefill_slots_chunks of TOKENS-token prompts on all 24 slots of the "
                         "config-5 model instead of the step")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}); the verify step would shard by slot, one rank per GPU",
              file=sys.stderr)
        return 2
    if not args.no_library_compare:
        # torch's HIP runtime must be initialised before this library's first HIP call, or
        # torch finds no device later (the library-comparison timings use torch)
        import torch
        torch.cuda.init()
    if args.attention_shapes:
        print(json.dumps(attention_shapes()))
        return 0
    if args.acceptance:
        print(json.dumps(acceptance_config1(args.seed, cpu_baseline=not args.no_cpu_baseline)))
        return 0
    if args.prefill:
        print(json.dumps(prefill_throughput(args.prefill, args.seed, not args.no_library_compare)))
        return 0
    from carat_amd import lib
    from carat_amd.runner import BatchModelRunner, ModelDesc

    if args.calibrate_copy:
        import torch
        src = torch.zeros(COPY_CALIBRATION_BYTES, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    desc = (ModelDesc.gemma4_31b(with_assistant=True) if args.native
            else ModelDesc.gemma4_benchmark(with_assistant=True))
    desc.assistant_fp8_mode = args.assistant_fp8
    desc.fp8_scaling = args.fp8_scaling
    assistant_fp8 = args.assistant_fp8 or os.environ.get("CARAT_ASSISTANT_FP8_MODE") or "off"
    total = args.warmup + args.steps
    # config 5's 8192-token contexts; the cache holds the rows the warmup, timed and probe steps
    # add on top of them, rounded up to a multiple of 256 rows past 8192: a global cache row
    # stride of 8192 + 64 or + 68 rows (2 MiB + 16 / 17 KiB per (slot, kv head)) measured 10%
    # slower on the global attention than + 0, + 128, + 256 .. + 448 rows
    start_position = MAX_CONTEXT
    needed = MAX_CONTEXT + DEPTH * (total + 2) + 8
    runner_context = MAX_CONTEXT + max(256, (needed - MAX_CONTEXT + 255) // 256 * 256)
    rng = np.random.default_rng(args.seed)
    t0 = time.perf_counter()
    runner = BatchModelRunner(desc, SLOTS, runner_context)
    log(f"runner ready in {time.perf_counter() - t0:.1f}s; contexts start at {start_position}")
    slots = list(range(SLOTS))
    if args.seeded_cache:
        runner.seed_random_cache(start_position, seed=args.seed,
                                 stddev=1 / math.sqrt(256 if args.native else 128))
        forced = rng.integers(0, desc.vocabulary, SLOTS).astype(np.int32)
        last = rng.integers(0, desc.vocabulary, SLOTS).astype(np.int32)
    else:
        t0 = time.perf_counter()
        forced, last = prefill_contexts(runner, rng, desc.vocabulary, start_position)
        log(f"prefilled {SLOTS} x {start_position} tokens in {time.perf_counter() - t0:.1f}s")
    runner.set_graphs(args.graphs)
    remaining = 1 << 20

    timed_s = 0.0
    accepted_total = 0
    draft_ms = verify_ms = 0.0
    for step in range(total):
        proposals = planted_proposals(runner, forced, slots, rng, desc.vocabulary)
        timed = step >= args.warmup
        # one scheduler cycle in C++ (draft_four -> acceptance_cap -> verify_greedy_proposals ->
        # commit_speculation), timed on the host clock from a synchronised device
        acc, forced, last, seconds = runner.bench_speculative_cycle(last, slots, forced, proposals,
                                                                    remaining)
        if timed:
            timed_s += seconds
            accepted_total += int(acc.sum())
            v_ms, d_ms = runner.timing()
            verify_ms += v_ms
            draft_ms += d_ms
        log(f"step {step}: accepted={acc[:8].tolist()}... sum={int(acc.sum())} "
            f"wall={1e3 * seconds:.2f}ms draft={runner.timing()[1]:.2f}ms "
            f"verify={runner.timing()[0]:.2f}ms{' (timed)' if timed else ''}")
    avg_launch_ms, probe_launches = runner.stream_gemm_probe("gate_up_gemm", passes=2)
    gemms = gemm_table(runner, desc, SLOTS * DEPTH, library=False)
    # the verify attention kernels, the way the gate/up GEMM is timed: after one planted dry
    # verify, every global (sliding) layer's attention over its own cache back to back, two
    # passes, between one pair of HIP events on the runner's stream
    props = planted_proposals(runner, forced, slots, rng, desc.vocabulary)
    attn_positions = [runner.slot_position(s) for s in slots]
    sliding_positions = attn_positions
    runner.verify_greedy_proposals(props.tolist(), forced.tolist(), slots, [0] * SLOTS)
    attn_avg_ms, attn_launches = runner.stream_gemm_probe("global_attention", passes=2)
    sliding_avg_ms, sliding_launches = runner.stream_gemm_probe("sliding_attention", passes=2)

    breakdown = {}
    if not args.no_breakdown:
        for kind in BatchModelRunner.PROBES:
            props = planted_proposals(runner, forced, slots, rng, desc.vocabulary)
            runner.set_probe(kind)
            runner.read_probe()
            runner.verify_greedy_proposals(props.tolist(), forced.tolist(), slots, [0] * SLOTS)
            ms, n = runner.read_probe()
            breakdown[kind] = {"ms": round(ms, 3), "launches": n}
        runner.set_probe(None)
        log("per-verify kernel time:", json.dumps(breakdown))

    steps = args.steps
    ms_per_step = 1e3 * timed_s / steps
    value = accepted_total / timed_s
    rows = SLOTS * DEPTH
    bytes_per_launch = gate_up_bytes(desc.hidden, desc.intermediate, rows)
    achieved = bytes_per_launch / (avg_launch_ms * 1e-3) / 1e9
    result = {
        "metric": "accepted tok/s at 24 slots, draft=4, FP8 verify" +
                  (" (native Gemma-4 31B attention geometry)" if args.native else ""),
        "value": round(value, 2),
        "unit": "accepted tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8",
        "data": ("synthetic (seeded random weights and tokens; KV caches "
                 + ("seeded N(0,1/D) values" if args.seeded_cache else
                    "prefilled from seeded random token ids") + "; no checkpoint)"),
        "config": {
            "workload": ("native-geometry" if args.native else "config5") +
                        " end-to-end speculative step: 4-layer assistant draft + 60-layer "
                        "FP8 verify + fused lm_head argmax/acceptance/commit",
            "attention": ("sliding D256 32/16 heads, global D512 32/4 heads K=V" if args.native
                          else "D128 32/16 heads"),
            "slots": SLOTS, "draft": DRAFTS, "verify_rows": rows, "layers": 60,
            "context_start": start_position,
            "context_capacity": runner_context, "accept_p": ACCEPT_P,
            "contexts": ("seeded KV values" if args.seeded_cache
                         else "prefilled from seeded random token ids"),
            "graphs": bool(args.graphs), "assistant_fp8_mode": assistant_fp8,
            "fp8_scaling": args.fp8_scaling,
            "mean_accepted_per_step": round(accepted_total / steps, 2),
            "draft_ms": round(draft_ms / steps, 3), "verify_ms": round(verify_ms / steps, 3),
        },
        "roofline_gate_up": {
            "kernel": "gate_up fp8 GEMM (5376 -> 2x21504, M=120) + GELU gate epilogue",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None if args.native else measured_traffic(),
            "avg_launch_us": round(avg_launch_ms * 1e3, 2),
            "launches": probe_launches,
            "bytes_per_launch": bytes_per_launch,
        },
    }
    g = next(l for l in desc.layers if not l.sliding)
    attn_bytes = global_attention_bytes(attn_positions, DEPTH, g.kv_heads, g.head_dimension,
                                        g.query_heads)
    attn_us = 1e3 * attn_avg_ms
    attn_achieved = attn_bytes / (attn_us * 1e-6) / 1e9
    # the dominant kernel of the verify step by total time (10 launches of ~281 us against 60
    # gate/up launches of ~45 us): the global verify attention
    result["roofline"] = {
        "kernel": f"global verify attention (24 slots x {g.kv_heads} kv heads, D {g.head_dimension}, "
                  f"~{attn_positions[0] + DEPTH} keys)",
        "bound": "hbm",
        "achieved": round(attn_achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(attn_achieved / HBM_PEAK_GBS, 4),
        "traffic": None if args.native else measured_attention_traffic(),
        "avg_launch_us": round(attn_us, 2),
        "launches": attn_launches,
        "bytes_per_launch": attn_bytes,
        "timing": "every global layer's attention back to back, two passes, one pair of HIP events",
    }
    result["gemms"] = gemms
    sl = next(l for l in desc.layers if l.sliding)
    window = desc.sliding_window
    sliding_keys = sum(min(int(p), window - 1) + DEPTH for p in sliding_positions)
    sliding_bytes = (sliding_keys * sl.kv_heads * sl.head_dimension * 2 * 2 +
                     2 * SLOTS * DEPTH * sl.query_heads * sl.head_dimension * 2)
    sliding_us = 1e3 * sliding_avg_ms
    result["roofline_attention_sliding"] = {
        "kernel": f"sliding verify attention (24 slots x {sl.kv_heads} kv heads, D {sl.head_dimension}, "
                  f"{window}-key window + {DEPTH} rows)",
        "bound": "hbm",
        "achieved": round(sliding_bytes / (sliding_us * 1e-6) / 1e9, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(sliding_bytes / (sliding_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "avg_launch_us": round(sliding_us, 2),
        "launches": sliding_launches,
        "bytes_per_launch": sliding_bytes,
        "timing": "every sliding layer's attention back to back, two passes, one pair of HIP events",
    }
    if not args.no_library_compare:
        add_library_times(gemms, SLOTS * DEPTH)  # last: it slows the kernels timed after it
    if breakdown:
        # one eager verify step per kernel family, hip events around every launch (the marker
        # packets add a few us per launch)
        result["kernels_ms_per_verify"] = dict(breakdown, rest={
            "ms": round(verify_ms / steps - sum(v["ms"] for v in breakdown.values()), 3),
            "what": "verify_ms minus the probed kernels: the row, quantisation, QKV and "
                    "acceptance kernels and the kernel boundaries"})
        gl = breakdown.get("global_attention")
        if gl and gl["launches"]:
            step_us = 1e3 * gl["ms"] / gl["launches"]
            result["roofline"]["in_step"] = {
                "avg_launch_us": round(step_us, 2),
                "frac": round(attn_bytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "timing": "inside one verify step, hip events around each launch"}
    if not args.no_cpu_baseline and not args.native:
        log("cpu baseline (OpenMP oracle) ...")
        result["cpu_baseline"] = cpu_baseline(accepted_total / steps)
    print(json.dumps(result), flush=True)
    runner.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
