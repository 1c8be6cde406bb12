"""Parity at the benchmark shapes (benchmark configs 4 and 5) on the GPU.

- Config 4: the fp8 GEMMs at exactly the runner's dispatch (weight layout and split-K factor from
  carat_hip_gemm_plan): qkv 5376->8192, o 4096->5376, gate/up 5376->2x21504 with the GELU
  epilogue, down 21504->5376, and the tied lm_head 5376->262144 with its fused argmax, all at
  M = 120 against the oracle's fp32-accumulated GEMM over the same e4m3 bytes
  (linear.cu:780-803, batch_model_runner.cu:840-853).
- Config 5: a verify step of a two-layer (one sliding, one global) model at full Gemma-4-31B
  benchmark dimensions (hidden 5376, intermediate 21504, vocabulary 262144, 32/16 heads x 128,
  window 1024) with 24 slots at contexts U[1024, 8187] against tests/runner_oracle.verify_step,
  and one draft step of the full-size assistant against tests/runner_oracle.draft_steps; one
  1008-row batched prefill step; a verify step at Gemma-4 31B's own attention geometry
  (sliding D 256, global D 512 with K = V).

Bars: acceptance, bonus tokens, cache commit and hidden hand-off bit-exact given the GPU's own
predictions; K/V rows and activations within 3e-2 of the row maximum; every argmax mismatch
against the oracle a near-tie (gap <= 2 bf16 ulps of the row maximum), mismatch rate printed and
bounded.
"""
import math
import sys

import numpy as np
import pytest
from scipy.special import ndtri

from carat_amd import _lib
from carat_amd.runner import BatchModelRunner, LayerSpec, ModelDesc
from oracle import oracle
from tests.runner_oracle import draft_steps, verify_step

pytestmark = pytest.mark.gpu

H, INTER, VOCAB = 5376, 21504, 262144
M = 120
T = 5
SLOTS = 24
MAX_CONTEXT = 8192


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def e4m3_normal_codes(rng, shape, std=0.02):
    """e4m3 codes of N(0, std) values under the per-tensor scale std*6/448 (amax ~ 6 std), drawn
    through a 65536-entry inverse-CDF table so a 1.4 GB lm_head is quick to make."""
    table = oracle.f32_to_e4m3((ndtri((np.arange(65536) + 0.5) / 65536) * (448 / 6)).astype(np.float32))
    out = np.empty(shape, np.uint8)
    flat = out.reshape(-1)
    step = 1 << 26
    for start in range(0, flat.size, step):
        n = min(step, flat.size - start)
        flat[start:start + n] = table[rng.integers(0, 65536, n, dtype=np.uint16)]
    return out, std * 6 / 448


def plan(n, k, gate_up):
    f, w, s = (_lib.ctypes.c_int() for _ in range(3))
    _lib.check(_lib.lib().carat_hip_gemm_plan(n, k, 1, int(gate_up), _lib.ctypes.byref(f),
                                              _lib.ctypes.byref(w), _lib.ctypes.byref(s)))
    return f.value, w.value, s.value


# name, n, k, gate_up, the runner's (tiles per wave, waves, splits) for that weight
CONFIG4 = [("qkv", (32 + 2 * 16) * 128, H, False, (1, 4, 2)),
           ("o", H, 32 * 128, False, (1, 3, 2)),
           ("gate_up", 2 * INTER, H, True, (4, 3, 1)),
           ("down", H, INTER, False, (1, 4, 3)),
           ("lm_head", VOCAB, H, False, (4, 4, 1))]


@pytest.mark.parametrize("name,n,k,gate_up,expect_plan", CONFIG4, ids=[c[0] for c in CONFIG4])
def test_config4_fp8_gemm_at_runner_dispatch(torch_cuda, name, n, k, gate_up, expect_plan):
    torch = torch_cuda
    rng = np.random.default_rng(400 + n % 97)
    assert plan(n, k, gate_up) == expect_plan
    splits = expect_plan[2]
    say(f"case: config-4 {name} m={M} k={k} n={n} plan={expect_plan}")
    x = oracle.f32_to_bf16(rng.standard_normal((M, k)))
    amax = float(np.abs(oracle.bf16_to_f32(x)).max())
    qw, sw = e4m3_normal_codes(rng, (n, k))
    qx, sx = oracle.quantize_e4m3(x)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    d_x, d_w = dev(x.view(np.int16)), dev(qw)
    d_amax, d_sw = dev(np.array([amax], np.float32)), dev(np.array([sw], np.float32))
    stream = _lib.ptr(torch.cuda.current_stream().cuda_stream)
    lib = _lib.lib()

    def run(epilogue, s=1):
        width = n // 2 if epilogue == 3 else n
        y = torch.zeros((M, width), dtype=torch.int16, device="cuda")
        y_amax = torch.zeros(1, dtype=torch.float32, device="cuda")
        part = torch.zeros((s, M, n) if epilogue == 1 else (1,), dtype=torch.float32, device="cuda")
        pred = torch.zeros(M, dtype=torch.int32, device="cuda")
        _lib.check(lib.carat_hip_fp8_linear(_lib.ptr(d_x), M, k, _lib.ptr(d_amax), _lib.ptr(d_w), n,
                                            _lib.ptr(d_sw), epilogue, s, _lib.ptr(y), _lib.ptr(y_amax),
                                            _lib.ptr(part), _lib.ptr(pred), stream))
        torch.cuda.synchronize()
        return (y.cpu().numpy().view(np.uint16), float(y_amax.cpu()[0]), part.cpu().numpy(),
                pred.cpu().numpy())

    ref32 = oracle.fp8_linear_f32(qx, sx, qw, sw).astype(np.float64)
    tol = lambda r: np.abs(r) * 2 ** -7 + 1e-3 * np.abs(r).max()
    if gate_up:
        y, y_amax, _, _ = run(3)
        ref, _ = oracle.gelu_tanh_gate_rows(oracle.f32_to_bf16(ref32))
        g = oracle.bf16_to_f32(y).astype(np.float64)
        r = oracle.bf16_to_f32(ref).astype(np.float64)
        # gate and up each carry one bf16 rounding: 2e-2 of the row maximum (the stated bound for bf16 activations)
        err = np.abs(g - r).max() / np.abs(r).max()
        say(f"  gelu gate max rel err {err:.2e}")
        assert err <= 2e-2
        assert y_amax == np.abs(g).max()
        return
    y, y_amax, _, _ = run(0)
    g = oracle.bf16_to_f32(y).astype(np.float64)
    assert np.all(np.abs(g - ref32) <= tol(ref32))
    assert y_amax == np.abs(g).max()
    if name == "lm_head":
        _, _, _, pred = run(2)
        # bit-exact given identical logits, and a near-tie of the oracle's own argmax
        assert np.array_equal(pred, oracle.argmax_bf16_rows(y))
        ref_logits = oracle.bf16_to_f32(oracle.f32_to_bf16(ref32)).astype(np.float64)
        ref_pred = oracle.argmax_bf16_rows(oracle.f32_to_bf16(ref32))
        gap = ref_logits.max(1) - ref_logits[np.arange(M), pred]
        say(f"  lm_head argmax mismatches vs oracle {int(np.sum(pred != ref_pred))}/{M}")
        assert np.all(gap <= 2 * 2 ** -7 * np.abs(ref_logits).max(1))
        return
    # the runner's split-K partials, summed by its consumers in fp32
    _, _, part, _ = run(1, splits)
    summed = part.sum(0).astype(np.float64) * np.float32(sx * sw)
    assert np.allclose(summed, ref32, rtol=1e-3, atol=1e-4 * np.abs(ref32).max())


# ------------------------------------------------------------------ config 5 at full dimensions
def full_desc():
    return ModelDesc(hidden=H, intermediate=INTER, vocabulary=VOCAB, sliding_window=1024,
                     layers=[LayerSpec(True), LayerSpec(False)], assistant=True, seed=5,
                     weight_std=0.02)


def capacity_of(desc):
    return lambda li: min(MAX_CONTEXT, desc.sliding_window) if desc.layers[li].sliding else MAX_CONTEXT


@pytest.fixture(scope="module")
def full_model(torch_cuda):
    desc = full_desc()
    say("case: full-dimension two-layer runner create (24 slots, context 8192)")
    runner = BatchModelRunner(desc, SLOTS, MAX_CONTEXT)
    rng = np.random.default_rng(55)
    positions = rng.integers(1024, MAX_CONTEXT - T + 1, SLOTS).astype(np.int32)
    runner.seed_random_cache(int(positions.max()), seed=7, stddev=1 / math.sqrt(128))
    for slot, p in enumerate(positions):
        runner.set_slot_position(slot, int(p))
    yield desc, runner, positions
    runner.close()


def full_verify_case(runner, desc, slots, positions, first, depth, caps, rng, tag):
    """One verify step of `depth` rows per slot at full dimensions against the oracle: plants the
    target's greedy chain (dry verifies), rejects it at a seeded index in most slots, then checks
    acceptance (with `caps`), predictions (near-ties only), this step's K/V rows, the final
    hidden rows, the cache commit, the hidden hand-off and the positions."""
    T = depth
    M = SLOTS * T
    say(f"case: {tag} greedy chain ({T} dry verifies)")
    chain = np.zeros((SLOTS, T + 1), np.int32)
    chain[:, 0] = first
    for t in range(T):
        props = np.zeros((SLOTS, T), np.int32)
        props[:, : t + 1] = chain[:, : t + 1]
        res = runner.verify_greedy_proposals(props.tolist(), first.tolist(), slots.tolist(), [0] * SLOTS)
        assert res.accepted_tokens == [0] * SLOTS
        chain[:, t + 1] = np.array(runner.last_predictions, np.int32).reshape(SLOTS, T)[:, t]
    # proposals: the greedy chain, rejected at a seeded position in most slots
    proposals = chain[:, :T].copy()
    reject = rng.integers(0, T + 2, SLOTS)
    for r in range(SLOTS):
        if reject[r] < T:
            proposals[r, reject[r]] = (proposals[r, reject[r]] + 1) % VOCAB
    li_s, li_g = 0, 1
    before = {li: (runner.read(f"cache.{li}.k", np.uint16), runner.read(f"cache.{li}.v", np.uint16))
              for li in (li_s, li_g)}
    hidden_before = runner.read("target_hidden", np.uint16).reshape(SLOTS, H).copy()
    say(f"case: {tag} oracle verify step (CPU)")
    expect = verify_step(runner, desc, SLOTS, capacity_of(desc), proposals, slots, positions)
    say(f"case: {tag} runner verify")
    if caps is None:
        res = runner.verify_greedy_proposals(proposals.tolist(), first.tolist(), slots.tolist())
    else:
        res = runner.verify_greedy_proposals(proposals.tolist(), first.tolist(), slots.tolist(), caps.tolist())
    pred = np.array(runner.last_predictions, np.int32).reshape(SLOTS, T)
    acc, nxt = oracle.greedy_accept(proposals, first, pred, caps)
    assert res.accepted_tokens == acc.tolist() and res.next_tokens == nxt.tolist()
    for r in range(SLOTS):  # the planted pattern: accepted = first mismatching index, capped
        want = reject[r] if reject[r] < T else T
        assert res.accepted_tokens[r] == (want if caps is None else min(want, int(caps[r])))
    # predictions: near-ties only, mismatch rate reported
    logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(M, -1)
    flat = pred.reshape(-1)
    gap = logits.max(1) - logits[np.arange(M), flat]
    mism = int(np.sum(flat != expect["predictions"]))
    say(f"  {tag} argmax mismatches vs oracle {mism}/{M}, max gap {gap.max():.3e}")
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    assert mism <= M // 10
    # this step's K/V rows and the final hidden rows
    for li, spec in enumerate(desc.layers):
        kv_width = spec.kv_heads * spec.head_dimension
        for kind in ("k", "v"):
            got = oracle.bf16_to_f32(runner.read(f"new.{li}.{kind}", np.uint16)[: M * kv_width])
            want = oracle.bf16_to_f32(expect[f"{kind}_new"][li]).reshape(-1)
            err = np.abs(got - want).max() / np.abs(want).max()
            say(f"  layer {li} {kind} rows max rel err {err:.2e}")
            assert err <= 3e-2, (li, kind, err)
    fh = oracle.bf16_to_f32(runner.read("final_hidden", np.uint16)[: M * H]).astype(np.float64)
    efh = oracle.bf16_to_f32(expect["final_hidden"]).reshape(-1).astype(np.float64)
    err = np.abs(fh - efh).max() / np.abs(efh).max()
    say(f"  final hidden max rel err {err:.2e}")
    assert err <= 3e-2
    # commit: exact cache bytes, hidden hand-off and positions
    for li in (li_s, li_g):
        C = capacity_of(desc)(li)
        hkv, D = desc.layers[li].kv_heads, desc.layers[li].head_dimension
        k_exp = before[li][0].reshape(SLOTS, hkv, C, D)
        v_exp = before[li][1].reshape(SLOTS, hkv, C, D)
        k_new = runner.read(f"new.{li}.k", np.uint16)[: M * hkv * D].reshape(SLOTS, T, hkv, D)
        v_new = runner.read(f"new.{li}.v", np.uint16)[: M * hkv * D].reshape(SLOTS, T, hkv, D)
        kept = res.accepted_tokens if desc.layers[li].sliding else [T] * SLOTS
        oracle.commit_kv(k_exp, v_exp, k_new, v_new, slots, positions, kept, C)
        assert np.array_equal(runner.read(f"cache.{li}.k", np.uint16), k_exp.reshape(-1)), li
        assert np.array_equal(runner.read(f"cache.{li}.v", np.uint16), v_exp.reshape(-1)), li
    final_hidden = runner.read("final_hidden", np.uint16)[: M * H].reshape(M, H)
    hidden_after = runner.read("target_hidden", np.uint16).reshape(SLOTS, H)
    for r, slot in enumerate(slots):
        a = res.accepted_tokens[r]
        want = final_hidden[r * T + a - 1] if a > 0 else hidden_before[slot]
        assert np.array_equal(hidden_after[slot], want)
        assert runner.slot_position(int(slot)) == positions[r] + a


@pytest.fixture(scope="module")
def native_model(torch_cuda):
    """Gemma-4 31B's own attention geometry (gemma4_config.cpp:174-203) at full hidden,
    intermediate and vocabulary: a sliding layer with 32/16 heads x 256 and a global layer with
    32/4 heads x 512 and K = V, and the full-size assistant over those caches."""
    desc = ModelDesc(hidden=H, intermediate=INTER, vocabulary=VOCAB, sliding_window=1024,
                     layers=[LayerSpec(True, 32, 16, 256),
                             LayerSpec(False, 32, 4, 512, key_equals_value=True)],
                     assistant=True, seed=6, weight_std=0.02)
    say("case: native-geometry two-layer runner create (24 slots, context 8192)")
    runner = BatchModelRunner(desc, SLOTS, MAX_CONTEXT)
    rng = np.random.default_rng(65)
    positions = rng.integers(1024, MAX_CONTEXT - T + 1, SLOTS).astype(np.int32)
    runner.seed_random_cache(int(positions.max()), seed=8, stddev=1 / math.sqrt(256))
    for slot, p in enumerate(positions):
        runner.set_slot_position(slot, int(p))
    yield desc, runner, positions
    runner.close()


def test_native_geometry_verify_step_full_dimensions(native_model):
    """One verify step at the native geometry: qkv 5376 -> 16384 (sliding) and 18432 (global,
    K = V), o 8192 / 16384 -> 5376, the D 256 sliding and D 512 global verify attention kernels
    (40 query rows per kv head), against the oracle composition with the same bars as config 5."""
    desc, runner, positions_by_slot = native_model
    rng = np.random.default_rng(66)
    slots = rng.permutation(SLOTS).astype(np.int32)
    positions = positions_by_slot[slots]
    first = rng.integers(0, VOCAB, SLOTS).astype(np.int32)
    full_verify_case(runner, desc, slots, positions, first, T, None, rng, "native")


def test_native_geometry_draft_step_full_dimensions(native_model):
    """A forced step and one free step of the assistant whose attention reads the native caches
    (decode attention at D 256 over the sliding ring and D 512 over the K = V global cache)."""
    desc, runner, _ = native_model
    rng = np.random.default_rng(67)
    slots = rng.permutation(SLOTS).astype(np.int32).tolist()
    last = rng.integers(0, VOCAB, SLOTS).astype(np.int32).tolist()
    forced = rng.integers(0, VOCAB, SLOTS).astype(np.int32).tolist()
    say("case: native-geometry draft (depth 2, forced first token)")
    got = np.array(runner.draft_four(last, slots, forced, 2), np.int32)
    assert got[:, 0].tolist() == forced
    exp = draft_steps(runner, desc, SLOTS, capacity_of(desc), last, slots, forced, 2, feed=got)
    logits = oracle.bf16_to_f32(exp["logits"][1]).astype(np.float64)
    gap = logits.max(1) - logits[np.arange(SLOTS), got[:, 1]]
    mism = int(np.sum(got[:, 1] != exp["tokens"][:, 1]))
    say(f"  native draft argmax mismatches vs oracle {mism}/{SLOTS}, max gap {gap.max():.3e}")
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    assert mism <= 2
    hidden = runner.read("assistant.previous_hidden", np.uint16).reshape(SLOTS, H)
    g = oracle.bf16_to_f32(hidden).astype(np.float64)
    e = oracle.bf16_to_f32(exp["hidden"][-1]).astype(np.float64)
    err = np.abs(g - e).max() / np.abs(e).max()
    say(f"  native draft hidden hand-off max rel err {err:.2e}")
    assert err <= 2e-2


def test_config5_verify_step_full_dimensions(full_model):
    desc, runner, positions_by_slot = full_model
    rng = np.random.default_rng(56)
    slots = rng.permutation(SLOTS).astype(np.int32)
    positions = positions_by_slot[slots]
    first = rng.integers(0, VOCAB, SLOTS).astype(np.int32)
    full_verify_case(runner, desc, slots, positions, first, T, None, rng, "config-5")


def test_config5_depth8_verify_with_caps_full_dimensions(full_model):
    """The deepest verify step (8 rows per slot, 192 rows) with per-slot caps
    (batch_model_runner.h:56-60's maximum_accepted_tokens) at config-5 dimensions."""
    desc, runner, _ = full_model
    rng = np.random.default_rng(58)
    depth = 8
    positions = rng.integers(1024, MAX_CONTEXT - depth - 8, SLOTS).astype(np.int32)
    for slot, p in enumerate(positions):
        runner.set_slot_position(slot, int(p))
    slots = rng.permutation(SLOTS).astype(np.int32)
    positions = positions[slots]
    first = rng.integers(0, VOCAB, SLOTS).astype(np.int32)
    caps = rng.integers(0, depth + 1, SLOTS).astype(np.int32)
    full_verify_case(runner, desc, slots, positions, first, depth, caps, rng, "depth-8 capped")


def test_config5_fused_quantization_equals_the_separate_kernel(full_model):
    """At config-5 dimensions (120 rows: the 120 layer-end workgroups agree on the activation
    amax before quantising the next GEMM's operand), the fused step equals the one with the
    separate quantisation kernel bit for bit."""
    desc, runner, positions_by_slot = full_model
    rng = np.random.default_rng(57)
    slots = rng.permutation(SLOTS).astype(np.int32)
    props = rng.integers(0, VOCAB, (SLOTS, T)).astype(np.int32)
    first = props[:, 0].copy()
    names = ["final_hidden"] + [f"new.{li}.{kind}" for li in range(len(desc.layers)) for kind in ("k", "v")]
    out = []
    for fused in (True, False):
        say(f"case: config-5 dry verify, fused quantisation {fused}")
        runner.set_fused_quantization(fused)
        try:
            res = runner.verify_greedy_proposals(props.tolist(), first.tolist(), slots.tolist(), [0] * SLOTS)
            assert res.accepted_tokens == [0] * SLOTS
            out.append((list(runner.last_predictions), [runner.read(n, np.uint16).copy() for n in names]))
        finally:
            runner.set_fused_quantization(0)
    assert out[0][0] == out[1][0]
    for name, a, b in zip(names, out[0][1], out[1][1]):
        assert np.array_equal(a, b), name


def test_config5_qkv_fusion_equals_the_separate_kernel(full_model):
    """At config-5 dimensions (two split-K partials, 24 x 16 attention workgroups, each
    post-processing its own rows) the fused step equals the separate QKV kernel's bit for bit:
    predictions, final hidden rows, this step's K/V rows and the global layer's cache."""
    desc, runner, positions_by_slot = full_model
    rng = np.random.default_rng(59)
    slots = rng.permutation(SLOTS).astype(np.int32)
    props = rng.integers(0, VOCAB, (SLOTS, T)).astype(np.int32)
    first = props[:, 0].copy()
    names = ["final_hidden"] + [f"new.{li}.{kind}" for li in range(len(desc.layers)) for kind in ("k", "v")]
    names += [f"cache.{li}.{kind}" for li, l in enumerate(desc.layers) if not l.sliding for kind in ("k", "v")]
    out = []
    for fused in (True, False):
        say(f"case: config-5 dry verify, QKV fusion {fused}")
        runner.set_qkv_fusion(fused)
        try:
            res = runner.verify_greedy_proposals(props.tolist(), first.tolist(), slots.tolist(), [0] * SLOTS)
            assert res.accepted_tokens == [0] * SLOTS
            out.append((list(runner.last_predictions), [runner.read(n, np.uint16).copy() for n in names]))
        finally:
            runner.set_qkv_fusion(True)
    assert out[0][0] == out[1][0]
    for name, a, b in zip(names, out[0][1], out[1][1]):
        assert np.array_equal(a, b), name


def test_config5_draft_step_full_dimensions(full_model):
    """A forced step and one free step of the full-size assistant (hidden 1024, 4 layers, bf16)
    over the 24 slots' caches, against the oracle chain teacher-forced on the GPU's tokens."""
    desc, runner, _ = full_model
    rng = np.random.default_rng(57)
    slots = rng.permutation(SLOTS).astype(np.int32).tolist()
    last = rng.integers(0, VOCAB, SLOTS).astype(np.int32).tolist()
    forced = rng.integers(0, VOCAB, SLOTS).astype(np.int32).tolist()
    say("case: config-5 draft (depth 2, forced first token)")
    got = np.array(runner.draft_four(last, slots, forced, 2), np.int32)
    assert got[:, 0].tolist() == forced
    exp = draft_steps(runner, desc, SLOTS, capacity_of(desc), last, slots, forced, 2, feed=got)
    logits = oracle.bf16_to_f32(exp["logits"][1]).astype(np.float64)
    gap = logits.max(1) - logits[np.arange(SLOTS), got[:, 1]]
    mism = int(np.sum(got[:, 1] != exp["tokens"][:, 1]))
    say(f"  draft argmax mismatches vs oracle {mism}/{SLOTS}, max gap {gap.max():.3e}")
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    assert mism <= 2
    hidden = runner.read("assistant.previous_hidden", np.uint16).reshape(SLOTS, H)
    g = oracle.bf16_to_f32(hidden).astype(np.float64)
    e = oracle.bf16_to_f32(exp["hidden"][-1]).astype(np.float64)
    err = np.abs(g - e).max() / np.abs(e).max()
    say(f"  draft hidden hand-off max rel err {err:.2e}")
    assert err <= 2e-2


@pytest.mark.parametrize("mode", ["lm_head", "all"])
def test_config5_draft_fp8_modes_full_dimensions(torch_cuda, mode):
    """The full-size assistant in AssistantFp8Mode lm_head / all (assistant_runner.cu:29-43,
    147-160) over the 24 slots' caches: a forced step and one free step against the oracle chain
    of the same mode, teacher-forced on the GPU's tokens."""
    desc = full_desc()
    desc.assistant_fp8_mode = mode
    say(f"case: full-dimension runner create, assistant fp8 mode {mode}")
    runner = BatchModelRunner(desc, SLOTS, MAX_CONTEXT)
    try:
        rng = np.random.default_rng(58)
        positions = rng.integers(1024, MAX_CONTEXT - T + 1, SLOTS).astype(np.int32)
        runner.seed_random_cache(int(positions.max()), seed=8, stddev=1 / math.sqrt(128))
        for slot, p in enumerate(positions):
            runner.set_slot_position(slot, int(p))
        slots = rng.permutation(SLOTS).astype(np.int32).tolist()
        last = rng.integers(0, VOCAB, SLOTS).astype(np.int32).tolist()
        forced = rng.integers(0, VOCAB, SLOTS).astype(np.int32).tolist()
        say(f"case: config-5 draft {mode} (depth 2, forced first token)")
        got = np.array(runner.draft_four(last, slots, forced, 2), np.int32)
        assert got[:, 0].tolist() == forced
        exp = draft_steps(runner, desc, SLOTS, capacity_of(desc), last, slots, forced, 2, feed=got,
                          fp8_mode=mode)
        logits = oracle.bf16_to_f32(exp["logits"][1]).astype(np.float64)
        gap = logits.max(1) - logits[np.arange(SLOTS), got[:, 1]]
        mism = int(np.sum(got[:, 1] != exp["tokens"][:, 1]))
        say(f"  draft {mode} argmax mismatches vs oracle {mism}/{SLOTS}, max gap {gap.max():.3e}")
        assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
        assert mism <= 2
        hidden = runner.read("assistant.previous_hidden", np.uint16).reshape(SLOTS, H)
        g = oracle.bf16_to_f32(hidden).astype(np.float64)
        e = oracle.bf16_to_f32(exp["hidden"][-1]).astype(np.float64)
        err = np.abs(g - e).max() / np.abs(e).max()
        mean_err = np.abs(g - e).mean() / np.abs(e).max()
        say(f"  draft {mode} hidden hand-off max rel err {err:.2e}, mean {mean_err:.2e}")
        # lm_head mode keeps bf16 projections (2e-2); in `all` an element whose bf16 input
        # differs by an ulp can take the neighbouring e4m3 code in each projection, which the
        # following projections spread (6e-2; test_gpu_runner.py holds each e4m3 stage to two
        # bf16 ulps given its GPU inputs)
        tolerance = 6e-2 if mode == "all" else 2e-2
        assert err <= tolerance and mean_err <= tolerance / 5
    finally:
        runner.close()


def test_config5_append_ragged_full_dimensions(full_model):
    """append_ragged (batch_model_runner.cu:1544-1615) over all 24 slots at config-5 dimensions:
    a depth-1 step of 24 rows, which takes the GEMMs' small-M kernels (two 16-token tiles) at the
    runner's qkv, o, gate/up, down and lm_head shapes. Next tokens against the oracle (near-ties
    only), this step's K/V rows, their commit at each slot's position, positions + 1."""
    desc, runner, _ = full_model
    rng = np.random.default_rng(60)
    positions = rng.integers(1024, MAX_CONTEXT - 8, SLOTS).astype(np.int32)
    for slot, p in enumerate(positions):
        runner.set_slot_position(slot, int(p))
    slots = rng.permutation(SLOTS).astype(np.int32)
    positions = positions[slots]
    tokens = rng.integers(0, VOCAB, SLOTS).astype(np.int32)
    say("case: config-5 append_ragged oracle (CPU, 24 rows)")
    expect = verify_step(runner, desc, SLOTS, capacity_of(desc), tokens[:, None], slots, positions)
    say("case: config-5 append_ragged")
    nxt = np.array(runner.append_ragged(tokens.tolist(), slots.tolist()), np.int32)
    logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64)
    gap = logits.max(1) - logits[np.arange(SLOTS), nxt]
    mism = int(np.sum(nxt != expect["predictions"]))
    say(f"  append_ragged argmax mismatches vs oracle {mism}/{SLOTS}, max gap {gap.max():.3e}")
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    assert mism <= 2
    for li, spec in enumerate(desc.layers):
        C = capacity_of(desc)(li)
        hkv, D = spec.kv_heads, spec.head_dimension
        for kind in ("k", "v"):
            new = runner.read(f"new.{li}.{kind}", np.uint16)[: SLOTS * hkv * D].reshape(SLOTS, hkv, D)
            want = oracle.bf16_to_f32(expect[f"{kind}_new"][li][:, 0])
            err = np.abs(oracle.bf16_to_f32(new) - want).max() / np.abs(want).max()
            say(f"  layer {li} {kind} row max rel err {err:.2e}")
            assert err <= 3e-2, (li, kind)
            cache = runner.read(f"cache.{li}.{kind}", np.uint16).reshape(SLOTS, hkv, C, D)
            for r, slot in enumerate(slots):
                assert np.array_equal(cache[slot, :, positions[r] % C], new[r]), (li, kind, r)
    for r, slot in enumerate(slots):
        assert runner.slot_position(int(slot)) == positions[r] + 1


def test_config5_prefill_step_full_dimensions(full_model):
    """One batched prefill step at the benchmark's prefill shape (prefill_slots_chunks,
    batch_model_runner.h:40-43: 24 slots x 42 rows = 1008 rows in one forced step, the GEMMs'
    four-tile layout) over resident contexts of U[1024, 8100] tokens that complete in this step:
    K/V rows of both layers against tests/runner_oracle.verify_step, each slot's returned token
    (its last row's argmax) a near-tie of the oracle's, positions advanced, and the hidden
    hand-off equal to the step's last row of each slot."""
    desc, runner, _ = full_model
    rng = np.random.default_rng(59)
    rows = 42
    positions = rng.integers(1024, MAX_CONTEXT - rows - 8, SLOTS).astype(np.int32)
    for slot, p in enumerate(positions):
        runner.set_slot_position(slot, int(p))
    slots = rng.permutation(SLOTS).astype(np.int32)
    positions = positions[slots]
    prompts = [rng.integers(0, VOCAB, int(p) + rows).astype(np.int32) for p in positions]
    chunk = np.stack([pr[p:] for pr, p in zip(prompts, positions)])
    last_rows = np.arange(SLOTS) * rows + rows - 1
    say("case: config-5 prefill step oracle (CPU, 1008 rows)")
    expect = verify_step(runner, desc, SLOTS, capacity_of(desc), chunk, slots, positions,
                         head_rows=last_rows)
    say("case: config-5 prefill_slots_chunks (24 slots x 42 rows)")
    tokens = runner.prefill_slots_chunks(slots.tolist(), [pr.tolist() for pr in prompts], rows)
    pred = np.array(runner.last_predictions, np.int32)
    assert len(pred) == SLOTS * rows
    assert tokens == pred[last_rows].tolist()
    logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64)
    gap = logits.max(1) - logits[np.arange(SLOTS), pred[last_rows]]
    mism = int(np.sum(pred[last_rows] != expect["predictions"]))
    say(f"  prefill argmax mismatches vs oracle {mism}/{SLOTS}, max gap {gap.max():.3e}")
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    for li in range(len(desc.layers)):
        C = capacity_of(desc)(li)
        for kind in ("k", "v"):
            cache = runner.read(f"cache.{li}.{kind}", np.uint16).reshape(SLOTS, 16, C, 128)
            got = oracle.bf16_to_f32(np.stack([cache[s][:, (p + np.arange(rows)) % C].transpose(1, 0, 2)
                                               for s, p in zip(slots, positions)]))
            want = oracle.bf16_to_f32(expect[f"{kind}_new"][li])
            err = np.abs(got - want).max() / np.abs(want).max()
            rms = np.sqrt(np.mean((got - want) ** 2)) / np.abs(want).max()
            say(f"  layer {li} {kind} rows max rel err {err:.2e}, rms {rms:.2e}")
            assert err <= 3e-2 and rms <= 1e-2, (li, kind)
    final_hidden = runner.read("final_hidden", np.uint16)[: SLOTS * rows * H].reshape(SLOTS * rows, H)
    efh = oracle.bf16_to_f32(expect["final_hidden"]).astype(np.float64)
    err = np.abs(oracle.bf16_to_f32(final_hidden).astype(np.float64) - efh).max() / np.abs(efh).max()
    say(f"  final hidden max rel err {err:.2e}")
    assert err <= 3e-2
    hidden_after = runner.read("target_hidden", np.uint16).reshape(SLOTS, H)
    for r, slot in enumerate(slots):
        assert np.array_equal(hidden_after[slot], final_hidden[last_rows[r]])
        assert runner.slot_position(int(slot)) == positions[r] + rows


def test_config5_deep_prefill_step_full_dimensions(full_model):
    """One slot's 1024-row prefill step (prefill_slot_chunk, batch_model_runner.h:38-39) over a
    resident context of 3000 tokens at config-5 dimensions: the whole sliding ring is rewritten
    in one step, the attention runs its 32-row query tiles over the causal triangle and the
    sliding band, and the GEMMs run eight token blocks per weight block for one request. K/V rows
    of both layers against the oracle, the returned token a near-tie of the oracle's, the position
    advanced."""
    desc, runner, _ = full_model
    rng = np.random.default_rng(61)
    rows, slot, p = 1024, 7, 3000
    runner.set_slot_position(slot, p)
    prompt = rng.integers(0, VOCAB, p + rows).astype(np.int32)
    say("case: config-5 deep prefill step oracle (CPU, 1024 rows)")
    expect = verify_step(runner, desc, SLOTS, capacity_of(desc), prompt[None, p:], [slot],
                         np.array([p], np.int32), head_rows=[rows - 1])
    say("case: config-5 prefill_slot_chunk (one slot, 1024 rows)")
    token = runner.prefill_slot_chunk(slot, prompt.tolist(), rows)
    pred = np.array(runner.last_predictions, np.int32)
    assert token == int(pred[rows - 1])
    logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64)
    gap = logits.max(1) - logits[0, token]
    say(f"  deep prefill token {token} vs oracle {int(expect['predictions'][0])}, gap {gap[0]:.3e}")
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    for li, spec in enumerate(desc.layers):
        C = capacity_of(desc)(li)
        hkv, D = spec.kv_heads, spec.head_dimension
        for kind in ("k", "v"):
            cache = runner.read(f"cache.{li}.{kind}", np.uint16).reshape(SLOTS, hkv, C, D)
            got = oracle.bf16_to_f32(cache[slot][:, (p + np.arange(rows)) % C].transpose(1, 0, 2))
            want = oracle.bf16_to_f32(expect[f"{kind}_new"][li][0])
            err = np.abs(got - want).max() / np.abs(want).max()
            rms = np.sqrt(np.mean((got - want) ** 2)) / np.abs(want).max()
            say(f"  layer {li} {kind} rows max rel err {err:.2e}, rms {rms:.2e}")
            assert err <= 3e-2 and rms <= 1e-2, (li, kind)
    assert runner.slot_position(slot) == p + rows



@pytest.mark.parametrize("scaling", ["channel", "block_128"])
def test_config5_scaled_fp8_verify_step_full_dimensions(torch_cuda, scaling):
    """The verify step over channel / block_128-scaled weights (Fp8Scaling, linear.h:27) at
    config-5 dimensions: every projection and the lm_head quantise their activations per row /
    per 1 x 128 block and scale inside the GEMM (run_decode_linear, layer_runner.cu:220-238);
    same bars as the per-tensor step."""
    desc = ModelDesc(hidden=H, intermediate=INTER, vocabulary=VOCAB, sliding_window=1024,
                     layers=[LayerSpec(True), LayerSpec(False)], seed=8, weight_std=0.02,
                     fp8_scaling=scaling)
    say(f"case: full-dimension {scaling} runner create")
    runner = BatchModelRunner(desc, SLOTS, MAX_CONTEXT)
    try:
        rng = np.random.default_rng(59)
        positions_by_slot = rng.integers(1024, MAX_CONTEXT - T + 1, SLOTS).astype(np.int32)
        runner.seed_random_cache(int(positions_by_slot.max()), seed=9, stddev=1 / math.sqrt(128))
        for slot, p in enumerate(positions_by_slot):
            runner.set_slot_position(slot, int(p))
        slots = rng.permutation(SLOTS).astype(np.int32)
        first = rng.integers(0, VOCAB, SLOTS).astype(np.int32)
        full_verify_case(runner, desc, slots, positions_by_slot[slots], first, T, None, rng,
                         f"config-5 {scaling}")
    finally:
        runner.close()
