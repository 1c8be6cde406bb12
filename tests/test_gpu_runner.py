"""The MI355X runner behind the reference's runner interface (batch_model_runner.h:22-77): one
verify step of a small seeded model against the oracle composition of the same step, the exact
acceptance / commit / rollback bookkeeping, HIP-graph replay and the reference's error messages."""
import math
import sys

import numpy as np
import pytest

from carat_amd import CaratError
from carat_amd.runner import BatchModelRunner, LayerSpec, ModelDesc
from oracle import oracle
from tests.runner_oracle import draft_steps, verify_step

pytestmark = pytest.mark.gpu

BATCH = 4
MAX_CONTEXT = 128


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def tiny_desc(seed=3):
    layers = [LayerSpec(True, 4, 2, 128), LayerSpec(True, 4, 2, 128), LayerSpec(False, 4, 2, 128)]
    return ModelDesc(hidden=256, intermediate=512, vocabulary=2048, sliding_window=32, layers=layers,
                     assistant=True, assistant_hidden=256, assistant_intermediate=512,
                     assistant_layers=2, assistant_query_heads=4, seed=seed, weight_std=0.05)


def capacity_of(desc):
    return lambda li: min(MAX_CONTEXT, desc.sliding_window) if desc.layers[li].sliding else MAX_CONTEXT


@pytest.fixture(scope="module")
def model(torch_cuda):
    desc = tiny_desc()
    say("case: tiny runner create")
    runner = BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    yield desc, runner
    runner.close()


def reset_state(runner, positions, seed=11):
    runner.seed_random_cache(int(max(positions)), seed=seed, stddev=1 / math.sqrt(128))
    for slot, p in enumerate(positions):
        runner.set_slot_position(slot, int(p))


def read_caches(runner, desc):
    return [(runner.read(f"cache.{i}.k", np.uint16).copy(), runner.read(f"cache.{i}.v", np.uint16).copy())
            for i in range(len(desc.layers))]


def greedy_chain(runner, first, slots, depth):
    """Target greedy continuation of each slot from dry verifies (caps 0 commits nothing)."""
    chain = np.zeros((len(slots), depth + 1), np.int32)
    chain[:, 0] = first
    for t in range(depth):
        props = np.zeros((len(slots), depth), np.int32)
        props[:, : t + 1] = chain[:, : t + 1]
        res = runner.verify_greedy_proposals(props.tolist(), first, slots, [0] * len(slots))
        assert res.accepted_tokens == [0] * len(slots)
        pred = np.array(runner.last_predictions, np.int32).reshape(len(slots), depth)
        chain[:, t + 1] = pred[:, t]
    return chain


@pytest.mark.parametrize("T", [5, 8], ids=["depth5", "depth8"])  # the benchmark and the maximum depth
def test_verify_step_matches_oracle_and_commits(model, T):
    desc, runner = model
    positions_by_slot = [40, 100, 20, 31]       # wrapped and unwrapped sliding rings (window 32)
    reset_state(runner, positions_by_slot)
    slots = [2, 0, 3, 1]
    positions = np.array([positions_by_slot[s] for s in slots], np.int32)
    rng = np.random.default_rng(5)
    first = rng.integers(0, desc.vocabulary, 4).astype(np.int32)
    say(f"case: runner greedy chain (dry verifies), depth {T}")
    chain = greedy_chain(runner, first, slots, T)
    # proposals: slot patterns of ragged_batch_parity.cu:209-229 -- all correct, reject at 0, 1, 2
    proposals = chain[:, :T].copy()
    for r, reject_at in ((1, 0), (2, 1), (3, 2)):
        proposals[r, reject_at] = (proposals[r, reject_at] + 1) % desc.vocabulary
    before = read_caches(runner, desc)
    hidden_before = runner.read("target_hidden", np.uint16).reshape(BATCH, desc.hidden).copy()
    expect = verify_step(runner, desc, BATCH, capacity_of(desc), proposals, slots, positions)
    say("case: runner verify")
    res = runner.verify_greedy_proposals(proposals.tolist(), first.tolist(), slots)
    pred = np.array(runner.last_predictions, np.int32).reshape(4, T)
    # acceptance is exact given the target's own predictions
    acc, nxt = oracle.greedy_accept(proposals, first, pred)
    assert res.accepted_tokens == acc.tolist()
    assert res.next_tokens == nxt.tolist()
    assert res.accepted_tokens[1] == 0 and res.next_tokens[1] == first[1]
    say(f"  accepted={res.accepted_tokens} next={res.next_tokens}")
    # target predictions agree with the oracle's (fp32-order differences only move near-ties)
    logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(4 * T, -1)
    gap = logits.max(1) - logits[np.arange(4 * T), pred.reshape(-1)]
    mism = int(np.sum(pred.reshape(-1) != expect["predictions"]))
    say(f"  argmax mismatches vs oracle {mism}/{4 * T}, max gap {gap.max():.3e}")
    # a mismatch is a near-tie: within 2 bf16 ulps of the row maximum
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    assert mism <= max(1, 4 * T // 10)
    # this step's K/V rows agree with the oracle's
    for li in range(len(desc.layers)):
        got_k = runner.read(f"new.{li}.k", np.uint16)[: 4 * T * 2 * 128].reshape(4, T, 2, 128)
        ek = expect["k_new"][li]
        err = np.abs(oracle.bf16_to_f32(got_k) - oracle.bf16_to_f32(ek)).max()
        assert err <= 3e-2 * np.abs(oracle.bf16_to_f32(ek)).max(), (li, err)
    # commit: sliding rings hold accepted rows only; global caches hold all T rows
    for li, spec in enumerate(desc.layers):
        C = capacity_of(desc)(li)
        k_after = runner.read(f"cache.{li}.k", np.uint16).reshape(BATCH, 2, C, 128)
        v_after = runner.read(f"cache.{li}.v", np.uint16).reshape(BATCH, 2, C, 128)
        k_exp = before[li][0].reshape(BATCH, 2, C, 128).copy()
        v_exp = before[li][1].reshape(BATCH, 2, C, 128).copy()
        k_new = runner.read(f"new.{li}.k", np.uint16)[: 4 * T * 256].reshape(4, T, 2, 128)
        v_new = runner.read(f"new.{li}.v", np.uint16)[: 4 * T * 256].reshape(4, T, 2, 128)
        rows_kept = res.accepted_tokens if spec.sliding else [T] * 4
        oracle.commit_kv(k_exp, v_exp, k_new, v_new, slots, positions, rows_kept, C)
        bad = sorted({(int(a), int(b), int(c)) for a, b, c, _ in np.argwhere(k_after != k_exp)})
        if bad:
            old = before[li][0].reshape(BATCH, 2, C, 128)
            notes = []
            for sl, hh, row in bad[:8]:
                src = "old" if np.array_equal(k_after[sl, hh, row], old[sl, hh, row]) else "?"
                for rr in range(4):
                    for tt in range(T):
                        if np.array_equal(k_after[sl, hh, row], k_new[rr, tt, hh]):
                            src = f"new[r={rr},t={tt}]"
                notes.append((sl, hh, row, src))
            raise AssertionError((li, rows_kept, positions.tolist(), slots, notes))
        assert np.array_equal(v_after, v_exp), li
    # hidden hand-off and positions
    final_hidden = runner.read("final_hidden", np.uint16)[: 4 * T * desc.hidden].reshape(4 * T, desc.hidden)
    hidden_after = runner.read("target_hidden", np.uint16).reshape(BATCH, desc.hidden)
    for r, slot in enumerate(slots):
        a = res.accepted_tokens[r]
        want = final_hidden[r * T + a - 1] if a > 0 else hidden_before[slot]
        assert np.array_equal(hidden_after[slot], want)
        assert runner.slot_position(slot) == positions[r] + a


def test_graph_replay_matches_eager(model):
    desc, runner = model
    reset_state(runner, [50, 60, 70, 80], seed=12)
    rng = np.random.default_rng(9)
    props = rng.integers(0, desc.vocabulary, (4, 5)).tolist()
    first = [p[0] for p in props]
    slots = [0, 1, 2, 3]
    say("case: eager vs graph replays")
    names = ["final_hidden"] + [f"new.{li}.{kind}" for li in range(len(desc.layers)) for kind in ("k", "v")]
    runner.set_graphs(False)
    runner.verify_greedy_proposals(props, first, slots, [0] * 4)
    eager = list(runner.last_predictions)
    eager_tensors = [runner.read(n, np.uint16).copy() for n in names]
    runner.set_graphs(True)
    try:
        for replay in range(4):
            runner.verify_greedy_proposals(props, first, slots, [0] * 4)
            assert runner.last_predictions == eager, replay
            for name, want in zip(names, eager_tensors):
                assert np.array_equal(runner.read(name, np.uint16), want), (replay, name)
            # eager work of the runner's own between replays: a draft (never captured) that
            # overwrites the assistant's buffers, and a dry verify of another shape
            if runner.has_assistant():
                runner.draft_four(first, slots, first, 2)
            runner.verify_greedy_proposals([p[:3] for p in props[:2]], first[:2], [3, 2], [0, 0])
    finally:
        runner.set_graphs(False)


def fused_and_separate_quantization(runner, props, first, slots, names):
    """One dry verify with the producers quantising the next GEMM's operand themselves, one with
    the separate quantisation kernel: predictions and the named tensors of both."""
    out = []
    for fused in (True, False):
        runner.set_fused_quantization(fused)
        try:
            runner.verify_greedy_proposals(props, first, slots, [0] * len(slots))
            out.append((list(runner.last_predictions), [runner.read(n, np.uint16).copy() for n in names]))
        finally:
            runner.set_fused_quantization(0)
    return out


def test_fused_quantization_equals_the_separate_kernel(model):
    """The layer-end rows quantise the next GEMM's e4m3 operand themselves (a grid-wide amax
    agreement first); the result must equal the separate prepare kernel's bit for bit (same
    rounding of the same bf16 values with the same per-tensor scale)."""
    desc, runner = model
    reset_state(runner, [40, 55, 70, 90], seed=13)
    rng = np.random.default_rng(21)
    props = rng.integers(0, desc.vocabulary, (4, 5)).tolist()
    first = [p[0] for p in props]
    say("case: fused vs separate activation quantisation, tiny model")
    names = ["final_hidden"] + [f"new.{li}.k" for li in range(len(desc.layers))]
    (p_fused, t_fused), (p_sep, t_sep) = fused_and_separate_quantization(runner, props, first, [0, 1, 2, 3], names)
    assert p_fused == p_sep
    for name, a, b in zip(names, t_fused, t_sep):
        assert np.array_equal(a, b), name


def qkv_fusion_on_and_off(runner, props, first, slots, names):
    """One dry verify with the QKV post-processing inside the attention kernel, one with the
    separate kernel: predictions and the named tensors of both."""
    out = []
    for fused in (True, False):
        runner.set_qkv_fusion(fused)
        try:
            runner.verify_greedy_proposals(props, first, slots, [0] * len(slots))
            out.append((list(runner.last_predictions), [runner.read(n, np.uint16).copy() for n in names]))
        finally:
            runner.set_qkv_fusion(True)
    return out


def test_qkv_fusion_equals_the_separate_kernel(model):
    """Verify attention post-processes its own (request, kv head)'s QKV rows (split-K sum, Q/K
    norm, RoPE, V norm) with the QKV kernel's arithmetic: predictions, final hidden rows, this
    step's K/V rows and the global layer's cache rows equal the separate kernel's bit for bit."""
    desc, runner = model
    reset_state(runner, [40, 55, 70, 90], seed=15)
    rng = np.random.default_rng(23)
    props = rng.integers(0, desc.vocabulary, (4, 5)).tolist()
    first = [p[0] for p in props]
    say("case: fused vs separate QKV post-processing, tiny model")
    names = ["final_hidden"] + [f"new.{li}.{kind}" for li in range(len(desc.layers)) for kind in ("k", "v")]
    names += [f"cache.{li}.{kind}" for li, l in enumerate(desc.layers) if not l.sliding for kind in ("k", "v")]
    (p_fused, t_fused), (p_sep, t_sep) = qkv_fusion_on_and_off(runner, props, first, [2, 0, 3, 1], names)
    assert p_fused == p_sep
    for name, a, b in zip(names, t_fused, t_sep):
        assert np.array_equal(a, b), name


@pytest.mark.parametrize("mode", ["off", "all"])
def test_draft_query_fusion_equals_the_separate_kernel(torch_cuda, mode):
    """The assistant's decode attention post-processes its own query rows (norm, RoPE at
    p + step; bf16 projections unscaled, `all` mode with the per-tensor scale) with the QKV
    kernel's arithmetic: proposals and every intermediate the draft leaves equal the separate
    kernel's bit for bit, the global layer's two key chunks included."""
    desc = tiny_desc()
    desc.assistant_fp8_mode = mode
    say(f"case: fused vs separate assistant query post-processing, fp8 mode {mode}")
    runner = BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    try:
        names = ["assistant.queries", "assistant.attention_out", "assistant.previous_hidden",
                 "assistant.final_hidden"]
        out = []
        for fused in (True, False):
            reset_state(runner, [30, 60, 90, 120], seed=19)
            runner.set_qkv_fusion(fused)
            try:
                drafts = runner.draft_four([5, 6, 7, 8], [3, 1, 0, 2], [], 4)
                out.append((drafts, [runner.read(n, np.uint16).copy() for n in names]))
            finally:
                runner.set_qkv_fusion(True)
        assert out[0][0] == out[1][0]
        for name, a, b in zip(names, out[0][1], out[1][1]):
            assert np.array_equal(a, b), name
    finally:
        runner.close()


def test_fused_quantization_wait_timeout_is_an_error(model):
    """A layer-end workgroup whose wait for the agreed amax runs out sets a fault flag; the step
    raises instead of returning results from a partly quantised operand. Forced from the host with
    a zero wait bound (every waiting workgroup gives up at once, so no kernel ever spins); the
    next step runs normally, and a dry step leaves no state behind."""
    desc, runner = model
    reset_state(runner, [33, 47, 61, 75], seed=14)
    rng = np.random.default_rng(22)
    props = rng.integers(0, desc.vocabulary, (4, 5)).tolist()
    first = [p[0] for p in props]
    slots = [0, 1, 2, 3]
    say("case: fused quantisation wait bound of zero")
    runner.verify_greedy_proposals(props, first, slots, [0] * 4)
    before = list(runner.last_predictions)
    with pytest.raises(CaratError, match="fused activation quantisation timed out"):
        runner.set_fused_quantization(2)
        try:
            runner.verify_greedy_proposals(props, first, slots, [0] * 4)
        finally:
            runner.set_fused_quantization(0)
    with pytest.raises(CaratError, match="fused quantisation mode"):
        runner.set_fused_quantization(3)
    runner.verify_greedy_proposals(props, first, slots, [0] * 4)
    assert runner.last_predictions == before
    assert [runner.slot_position(s) for s in slots] == [33, 47, 61, 75]


def test_reference_error_messages(model):
    desc, runner = model
    reset_state(runner, [10, 10, 10, 0])
    ok = [[1, 2, 3]] * 2
    with pytest.raises(CaratError, match="invalid greedy verification batch"):
        runner.verify_greedy_proposals([[1] * 9], [1], [0])
    with pytest.raises(CaratError, match="invalid or repeated speculative slot"):
        runner.verify_greedy_proposals(ok, [1, 1], [0, 0])
    with pytest.raises(CaratError, match="speculative slot is empty or lacks context capacity"):
        runner.verify_greedy_proposals(ok, [1, 1], [0, 3])
    with pytest.raises(CaratError, match="speculative proposal contains an invalid token"):
        runner.verify_greedy_proposals([[1, 2, 3], [1, desc.vocabulary, 3]], [1, 1], [0, 1])
    with pytest.raises(CaratError, match="speculative acceptance caps do not match request count"):
        runner.verify_greedy_proposals(ok, [1, 1], [0, 1], [1])
    runner.set_slot_position(0, MAX_CONTEXT - 2)
    with pytest.raises(CaratError, match="lacks context capacity"):
        runner.verify_greedy_proposals([[1, 2, 3]], [1], [0])
    with pytest.raises(CaratError, match="assistant slot is empty or invalid"):
        runner.draft_four([1], [3])
    with pytest.raises(CaratError, match="forced assistant first tokens do not match draft batch"):
        runner.draft_four([1, 2], [0, 1], [5])


def check_draft_against_oracle(runner, desc, batch, capacity, last, slots, forced, depth, label,
                               fp8_mode="off", hidden_tolerance=2e-2):
    """draft_four vs the oracle's assistant chain (assistant_runner.cu:218-338), teacher-forced on
    the GPU's own tokens: every unforced step's token is the oracle argmax or a near-tie of the
    oracle's bf16 logits, the forced step returns the forced token, and the last step's
    post-projection (the hidden hand-off to the next step) agrees with the oracle's."""
    got = np.array(runner.draft_four(last, slots, forced or [], depth), np.int32)
    assert got.shape == (len(last), depth)
    exp = draft_steps(runner, desc, batch, capacity, last, slots, forced or None, depth, feed=got,
                      fp8_mode=fp8_mode)
    mismatches, total = 0, 0
    for d in range(depth):
        if exp["logits"][d] is None:
            assert got[:, d].tolist() == list(forced)
            continue
        logits = oracle.bf16_to_f32(exp["logits"][d]).astype(np.float64)
        rows = np.arange(len(last))
        gap = logits.max(1) - logits[rows, got[:, d]]
        mismatches += int(np.sum(got[:, d] != exp["tokens"][:, d]))
        total += len(last)
        # fp32 summation order only moves near-ties: within 2 bf16 ulps of the row maximum
        assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1)), (label, d, gap.max())
    say(f"  {label}: argmax mismatches {mismatches}/{total} (near-ties)")
    assert mismatches <= max(1, total // 20), label
    hidden = runner.read("assistant.previous_hidden", np.uint16).reshape(batch, desc.hidden)[: len(last)]
    g = oracle.bf16_to_f32(hidden).astype(np.float64)
    e = oracle.bf16_to_f32(exp["hidden"][-1]).astype(np.float64)
    err = np.abs(g - e).max() / np.abs(e).max()
    mean_err = np.abs(g - e).mean() / np.abs(e).max()
    say(f"  {label}: hidden hand-off max rel err {err:.2e}, mean {mean_err:.2e}")
    assert err <= hidden_tolerance, label
    assert mean_err <= hidden_tolerance / 5, label  # a systematic error would move every element
    return got


@pytest.mark.parametrize("depth", [1, 4, 8])
def test_draft_four_matches_oracle_chain(model, depth):
    desc, runner = model
    reset_state(runner, [30, 40, 50, 100], seed=13)  # slot 3 has wrapped its sliding ring
    last = [5, 6, 7, 8]
    slots = [3, 1, 0, 2]
    say(f"case: draft_four vs oracle chain, depth {depth}")
    free = check_draft_against_oracle(runner, desc, BATCH, capacity_of(desc), last, slots, None,
                                      depth, "unforced")
    again = runner.draft_four(last, slots, [], depth)
    assert free.tolist() == again  # deterministic
    forced = check_draft_against_oracle(runner, desc, BATCH, capacity_of(desc), last, slots,
                                        [11, 12, 13, 14], depth, "forced")
    assert forced[:, 0].tolist() == [11, 12, 13, 14]
    # a subset of the slots in another order reads the same caches
    check_draft_against_oracle(runner, desc, BATCH, capacity_of(desc), [9, 10], [2, 0], None,
                               depth, "two rows")


@pytest.mark.parametrize("mode", ["lm_head", "all"])
def test_draft_fp8_modes_match_oracle_chain(torch_cuda, mode):
    """AssistantFp8Mode (assistant_runner.cu:29-43, 147-160): the lm_head alone, or every assistant
    projection, as an e4m3 GEMM over per-tensor quantised weights with the input quantised from
    its own amax. The e4m3 copies are the oracle's per-tensor quantisation of the bf16 weights bit
    for bit (Fp8WeightArena::quantize); the drafts follow the oracle chain of the same mode."""
    desc = tiny_desc()
    desc.assistant_fp8_mode = mode
    say(f"case: tiny runner create, assistant fp8 mode {mode}")
    runner = BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    try:
        scales = runner.read("assistant.fp8_scales", np.float32)
        names = [("assistant.token_embedding", 0)]
        if mode == "all":
            names += [("assistant.pre_projection", 1), ("assistant.post_projection", 2)]
        for name, j in names:
            q, s = oracle.quantize_e4m3(runner.read(name, np.uint16))
            assert np.array_equal(runner.read(name + ".fp8", np.uint8), q), name
            assert scales[j] == np.float32(s), name
        for li in range(desc.assistant_layers):
            pre = f"assistant.layer.{li}."
            if mode == "all":
                ls = runner.read(pre + "fp8_scales", np.float32)
                for j, n in enumerate(("q", "o", "gate_up", "down")):
                    q, s = oracle.quantize_e4m3(runner.read(pre + n, np.uint16))
                    assert np.array_equal(runner.read(pre + n + ".fp8", np.uint8), q), (li, n)
                    assert ls[j] == np.float32(s), (li, n)
            else:
                with pytest.raises(CaratError, match="not allocated"):
                    runner.read(pre + "q.fp8", np.uint8)
        reset_state(runner, [30, 40, 50, 100], seed=13)
        last, slots = [5, 6, 7, 8], [3, 1, 0, 2]
        # The hand-off is held to 2e-2 of the maximum in lm_head mode (bf16 projections, as off).
        # In `all` mode each of a step's nine e4m3 projections quantises its input per tensor, and
        # an element whose bf16 input differs by one ulp between the GPU and the oracle can land
        # on the neighbouring e4m3 code (a 1/8-1/16 relative step of that element); the next
        # projections spread that over their outputs, so the chains drift apart by about 0.5% of
        # the maximum per element on average (measured: 2.7e-2 max, 5.2e-3 mean after one step):
        # 6e-2 of the maximum, mean 1.2e-2. test_draft_stages_given_the_gpu_inputs holds every
        # e4m3 stage to two bf16 ulps given the GPU's own stage inputs.
        for depth, forced in ((1, None), (1, [11, 12, 13, 14]), (4, None), (5, [11, 12, 13, 14])):
            say(f"case: draft_four {mode} vs oracle chain, depth {depth}, forced {forced is not None}")
            check_draft_against_oracle(runner, desc, BATCH, capacity_of(desc), last, slots, forced,
                                       depth, f"{mode} depth {depth}", fp8_mode=mode,
                                       hidden_tolerance=6e-2 if mode == "all" else 2e-2)
    finally:
        runner.close()


def close_rows(got, want, what, ulps=2):
    """bf16 rows equal up to `ulps` bf16 ulps of each row's maximum (fp32 summation order and the
    rounding of a norm's inputs are the only differences left once the inputs are the same)."""
    g = oracle.bf16_to_f32(got).astype(np.float64).reshape(want.shape[0], -1)
    e = oracle.bf16_to_f32(want).astype(np.float64).reshape(want.shape[0], -1)
    bound = ulps * 2.0 ** -8 * np.abs(e).max(1, keepdims=True)
    worst = float((np.abs(g - e) / bound).max())
    say(f"  {what}: max error {worst:.2f} of {ulps} ulps of the row maximum")
    assert worst <= 1.0, what


@pytest.mark.parametrize("mode", ["off", "lm_head", "all"])
def test_draft_stages_given_the_gpu_inputs(torch_cuda, mode):
    """Every projection of the last assistant layer of a draft step, and the step's lm_head and
    post-projection, recomputed by the oracle from the GPU's own inputs to that stage (the
    intermediates the step leaves behind): in `all` mode each stage quantises its input per tensor
    with the amax its producer published, so a stage that used another tensor's amax (or a stale
    operand) would be off by far more than the two bf16 ulps allowed here, which the chain test
    over several steps cannot resolve."""
    desc = tiny_desc()
    desc.assistant_fp8_mode = mode
    say(f"case: draft stages given GPU inputs, assistant fp8 mode {mode}")
    runner = BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    try:
        reset_state(runner, [30, 40, 50, 100], seed=17)
        last, slots = [5, 6, 7, 8], [3, 1, 0, 2]
        rows = len(last)
        got = np.array(runner.draft_four(last, slots, [], 1), np.int32)[:, 0]
        AH, H, eps = desc.assistant_hidden, desc.hidden, desc.rms_norm_epsilon
        rd = lambda name, width: runner.read(name, np.uint16).reshape(-1, width)[:rows]
        all8 = mode == "all"
        li = desc.assistant_layers - 1  # the last layer (global)
        pre = f"assistant.layer.{li}."
        spec = desc.layers[max(i for i, l in enumerate(desc.layers) if not l.sliding)]
        D, hkv, hq = spec.head_dimension, spec.kv_heads, desc.assistant_query_heads
        s8 = runner.read(pre + "fp8_scales", np.float32) if all8 else None

        def linear(x, n, j, shape):
            w = runner.read(pre + n, np.uint16).reshape(shape)
            if not all8:
                return oracle.bf16_linear(x, w)
            qx, sx = oracle.quantize_e4m3(x)
            return oracle.fp8_linear(qx, sx, runner.read(pre + n + ".fp8", np.uint8).reshape(shape), float(s8[j]))

        w = lambda n: runner.read(pre + n, np.uint16)
        layer_in = rd("assistant.hidden_b", AH)   # the last layer's input (the previous layer's output)
        normalized = rd("assistant.normalized", AH)
        close_rows(normalized, oracle.rms_norm(layer_in, w("input_norm"), eps=eps)[0], "input norm")
        context = np.array([runner.slot_position(s) - 1 for s in slots], np.int32)
        cos = runner.read("rope.global.cos", np.uint16).reshape(-1, D)
        sin = runner.read("rope.global.sin", np.uint16).reshape(-1, D)
        qp = linear(normalized, "q", 0, (hq * D, AH))
        q, _, _ = oracle.qkv_post(qp, w("q_norm"), w("q_norm"), cos, sin, context, hq, 0, D, False, eps)
        queries = rd("assistant.queries", hq * D)
        close_rows(queries, q.reshape(rows, -1), "q projection + norm + RoPE")
        attn = rd("assistant.attention_out", hq * D)
        o = linear(attn, "o", 1, (AH, hq * D))
        r1, pre_mlp, _ = oracle.rms_norm_add_and_norm(o, w("post_attention_norm"), layer_in,
                                                      w("pre_mlp_norm"), eps)
        close_rows(rd("assistant.first_residual", AH), r1, "o projection + residual")
        close_rows(rd("assistant.pre_mlp", AH), pre_mlp, "o projection + pre-MLP norm", ulps=3)
        pre_mlp = rd("assistant.pre_mlp", AH)
        act, _ = oracle.gelu_tanh_gate_rows(linear(pre_mlp, "gate_up", 2, (2 * desc.assistant_intermediate, AH)))
        activated = rd("assistant.activated", desc.assistant_intermediate)
        close_rows(activated, act, "gate/up + GELU gate")
        down = linear(activated, "down", 3, (AH, desc.assistant_intermediate))
        out = oracle.rms_norm_add_scale(down, w("post_mlp_norm"), rd("assistant.first_residual", AH),
                                        int(w("scalar")[0]), eps)
        close_rows(rd("assistant.hidden_a", AH), out, "down + post-MLP norm + residual")
        final = rd("assistant.final_hidden", AH)
        close_rows(final, oracle.rms_norm(rd("assistant.hidden_a", AH), runner.read("assistant.final_norm", np.uint16), eps=eps)[0], "final norm")
        # lm_head (+ argmax) and the post-projection from the GPU's final hidden rows
        if mode == "off":
            logits = oracle.bf16_linear(final, runner.read("assistant.token_embedding", np.uint16).reshape(desc.vocabulary, AH))
            want = oracle.argmax_bf16_rows(logits)
        else:
            scales = runner.read("assistant.fp8_scales", np.float32)
            want, logits = oracle.fp8_lm_head_argmax(
                final, runner.read("assistant.token_embedding.fp8", np.uint8).reshape(desc.vocabulary, AH),
                float(scales[0]))
        lg = oracle.bf16_to_f32(logits).astype(np.float64)
        gap = lg.max(1) - lg[np.arange(rows), got]
        assert np.all(gap <= 2 * 2 ** -7 * np.abs(lg).max(1)), "lm_head argmax"
        say(f"  lm_head argmax mismatches {int(np.sum(got != want))}/{rows}")
        post_w = runner.read("assistant.post_projection", np.uint16).reshape(H, AH)
        if all8:
            qx, sx = oracle.quantize_e4m3(final)
            post = oracle.fp8_linear(qx, sx, runner.read("assistant.post_projection.fp8", np.uint8).reshape(H, AH),
                                     float(runner.read("assistant.fp8_scales", np.float32)[2]))
        else:
            post = oracle.bf16_linear(final, post_w)
        close_rows(rd("assistant.previous_hidden", H), post, "post-projection")
    finally:
        runner.close()


def test_draft_fp8_mode_from_environment(torch_cuda, monkeypatch):
    """With no mode in the description the runner reads CARAT_ASSISTANT_FP8_MODE, as the
    reference's assistant runner does (assistant_runner.cu:31-44): unset is off, and a value other
    than off, lm_head or all is the reference's error."""
    desc = tiny_desc()
    monkeypatch.setenv("CARAT_ASSISTANT_FP8_MODE", "lm_head")
    say("case: assistant fp8 mode from the environment (lm_head)")
    with BatchModelRunner(desc, BATCH, MAX_CONTEXT) as runner:
        assert runner.read("assistant.token_embedding.fp8", np.uint8).size == desc.vocabulary * desc.assistant_hidden
        with pytest.raises(CaratError, match="not allocated"):
            runner.read("assistant.pre_projection.fp8", np.uint8)
    monkeypatch.setenv("CARAT_ASSISTANT_FP8_MODE", "on")
    with pytest.raises(CaratError, match="CARAT_ASSISTANT_FP8_MODE must be off, lm_head or all"):
        BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    monkeypatch.delenv("CARAT_ASSISTANT_FP8_MODE")
    with BatchModelRunner(desc, BATCH, MAX_CONTEXT) as runner:
        with pytest.raises(CaratError, match="not allocated"):
            runner.read("assistant.token_embedding.fp8", np.uint8)


def test_append_ragged_is_one_forced_decode_step(model):
    """append_ragged (batch_model_runner.cu:1544-1615) = a depth-1 verify of the input token: same
    next token and K/V row as the oracle composition, positions + 1, the reference's messages."""
    desc, runner = model
    positions_by_slot = [45, 70, 31, 100]
    reset_state(runner, positions_by_slot, seed=14)
    slots = [1, 3, 0]
    tokens = [17, 404, 1999]
    positions = np.array([positions_by_slot[s] for s in slots], np.int32)
    expect = verify_step(runner, desc, BATCH, capacity_of(desc), np.array(tokens, np.int32)[:, None],
                         slots, positions)
    say("case: append_ragged")
    nxt = runner.append_ragged(tokens, slots)
    logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(len(slots), -1)
    gap = logits.max(1) - logits[np.arange(len(slots)), nxt]
    # a mismatch with the oracle is a near-tie: within 2 bf16 ulps of the row maximum
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    assert int(np.sum(np.array(nxt) != expect["predictions"])) <= 1
    for r, slot in enumerate(slots):
        assert runner.slot_position(slot) == positions[r] + 1
    assert runner.slot_position(2) == positions_by_slot[2]
    # the new rows are committed at each slot's position (sliding ring and global cache)
    for li, spec in enumerate(desc.layers):
        C = capacity_of(desc)(li)
        k_after = runner.read(f"cache.{li}.k", np.uint16).reshape(BATCH, 2, C, 128)
        k_new = runner.read(f"new.{li}.k", np.uint16)[: len(slots) * 256].reshape(len(slots), 2, 128)
        for r, slot in enumerate(slots):
            assert np.array_equal(k_after[slot, :, positions[r] % C], k_new[r])
    with pytest.raises(CaratError, match="invalid ragged token batch"):
        runner.append_ragged([1, 2], [0])
    with pytest.raises(CaratError, match="invalid or repeated ragged slot"):
        runner.append_ragged([1, 2], [0, 0])
    with pytest.raises(CaratError, match="invalid or repeated ragged slot"):
        runner.append_ragged([desc.vocabulary], [0])
    runner.set_slot_position(2, 0)
    with pytest.raises(CaratError, match="ragged slot is empty or full"):
        runner.append_ragged([1], [2])


def test_stream_gemm_probe_leaves_the_verify_result_unchanged(model):
    desc, runner = model
    reset_state(runner, [40, 41, 42, 43], seed=13)
    rng = np.random.default_rng(10)
    props = rng.integers(0, desc.vocabulary, (4, 5)).tolist()
    first = [p[0] for p in props]
    slots = [0, 1, 2, 3]
    say("case: stream GEMM probe between two dry verifies")
    runner.verify_greedy_proposals(props, first, slots, [0] * 4)
    before = list(runner.last_predictions)
    for kind in ("qkv_gemm", "o_gemm", "gate_up_gemm", "down_gemm"):
        avg_ms, launches = runner.stream_gemm_probe(kind, passes=2)
        assert launches == 2 * len(desc.layers) and avg_ms > 0.0
    for kind, sliding in (("sliding_attention", True), ("global_attention", False)):
        avg_ms, launches = runner.stream_gemm_probe(kind, passes=2)
        assert launches == 2 * sum(l.sliding == sliding for l in desc.layers) and avg_ms > 0.0
    runner.verify_greedy_proposals(props, first, slots, [0] * 4)
    assert runner.last_predictions == before


def test_prefill_steps_match_oracle_and_one_call(model):
    """prefill_slot / prefill_slots_chunks (batch_model_runner.h:34-43): each forced step (short
    ones, and one of 30 rows -- a step holds up to the verify row budget, 32 here, bounded by the
    sliding ring) equals the oracle composition of that step over the caches as they stand (its
    K rows; its predictions in the step that completes the prompt, the only one that runs the
    lm_head), every row is committed, and one prefill_slot call reproduces chunked calls of the same step sizes
    bit for bit."""
    desc, runner = model
    rng = np.random.default_rng(17)
    prompt = rng.integers(0, desc.vocabulary, 45).astype(np.int32).tolist()
    runner.reset_slot(2)
    pos = 0
    token = None
    say("case: chunked prefill vs oracle steps (8, 7, 30 rows)")
    for T in (8, 7, 30):
        expect = verify_step(runner, desc, BATCH, capacity_of(desc), np.array([prompt[pos:pos + T]]),
                             [2], np.array([pos], np.int32))
        (token,) = runner.prefill_slots_chunks([2], [prompt], T)
        pred = np.array(runner.last_predictions, np.int32)
        assert len(pred) == T
        if pos + T < len(prompt):
            # no prompt completes in this step: the lm_head is skipped, predictions read -1
            assert np.all(pred == -1)
        else:
            logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(T, -1)
            gap = logits.max(1) - logits[np.arange(T), pred]
            mism = int(np.sum(pred != expect["predictions"]))
            say(f"  prefill argmax mismatches vs oracle {mism}/{T}, max gap {gap.max():.3e}")
            # a mismatch is a near-tie: within 2 bf16 ulps of the row maximum
            assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
            assert mism <= max(1, T // 10)
        for li, spec in enumerate(desc.layers):
            C = capacity_of(desc)(li)
            kc = runner.read(f"cache.{li}.k", np.uint16).reshape(BATCH, 2, C, 128)
            got = oracle.bf16_to_f32(np.stack([kc[2, :, (pos + t) % C] for t in range(T)]))
            want = oracle.bf16_to_f32(expect["k_new"][li][0])
            # fp8 activation noise: a few elements near e4m3 rounding boundaries move by a few
            # percent of the row maximum; the RMS error stays far below that
            assert np.abs(got - want).max() <= 5e-2 * np.abs(want).max(), (li, pos)
            assert np.sqrt(np.mean((got - want) ** 2)) <= 1e-2 * np.abs(want).max(), (li, pos)
        pos += T
        assert runner.slot_position(2) == pos
        if pos < len(prompt):
            assert token is None
    assert token == int(pred[-1])
    say("case: one prefill_slot call (steps 32 + 13) vs two chunked calls")
    runner.reset_slot(1)
    assert runner.prefill_slots_chunks([1], [prompt], 32) == [None]
    (chunked,) = runner.prefill_slots_chunks([1], [prompt], 32)
    assert runner.prefill_slot(3, prompt, 64) == chunked
    for li in range(len(desc.layers)):
        C = capacity_of(desc)(li)
        kc = runner.read(f"cache.{li}.k", np.uint16).reshape(BATCH, 2, C, 128)
        vc = runner.read(f"cache.{li}.v", np.uint16).reshape(BATCH, 2, C, 128)
        rows = [(p % C) for p in range(len(prompt))][-C:]
        assert np.array_equal(kc[3][:, rows], kc[1][:, rows]) and np.array_equal(vc[3][:, rows], vc[1][:, rows])
    assert runner.slot_position(3) == len(prompt)
    with pytest.raises(CaratError, match="invalid slot prefill shape"):
        runner.prefill_slot(1, [], 8)
    with pytest.raises(CaratError, match="slot prefill chunk does not extend resident context"):
        runner.prefill_slot_chunk(3, prompt, 8)
    with pytest.raises(CaratError, match="batched chunk does not extend resident context"):
        runner.prefill_slots_chunks([3], [prompt], 8)
    runner.reset_slot(1)
    with pytest.raises(CaratError, match="slot prompt contains an invalid token id"):
        runner.prefill_slot_chunk(1, [1, desc.vocabulary], 8)
    with pytest.raises(CaratError, match="batched chunk contains an invalid token id"):
        runner.prefill_slots_chunks([1], [[1, desc.vocabulary]], 8)
    with pytest.raises(CaratError, match="invalid slot prefill shape"):
        runner.prefill_slot_from_prefix(3, prompt, 10)  # slot 3 holds 45 tokens, not 10


def resident_rows(runner, desc, slot, position):
    """The slot's resident K/V ring rows of every layer and its hidden hand-off row."""
    out = []
    for li in range(len(desc.layers)):
        C = capacity_of(desc)(li)
        rows = sorted({p % C for p in range(max(0, position - C), position)})
        for kind in ("k", "v"):
            cache = runner.read(f"cache.{li}.{kind}", np.uint16).reshape(BATCH, 2, C, 128)
            out.append(cache[slot][:, rows].copy())
    out.append(runner.read("target_hidden", np.uint16).reshape(BATCH, -1)[slot].copy())
    return out


def test_suffix_prefill_layer_slices_and_clone(model):
    """prefill_slots_suffix and prefill_slots_suffix_layer_slice (batch_model_runner.cu:1127-1222,
    1356-1496) over the same cohort give the same predictions, resident K/V rows and hidden
    hand-off bit for bit, with dry verify steps on other slots between the layer slices (they
    share every per-step workspace); clone_slot (:1507-1541) copies a slot exactly."""
    desc, runner = model
    rng = np.random.default_rng(23)
    prompts = [rng.integers(0, desc.vocabulary, n).astype(np.int32).tolist() for n in (20, 45)]
    for slot in range(BATCH):
        runner.reset_slot(slot)
    say("case: batched suffix prefill on slots 0, 1")
    want = runner.prefill_slots_suffix([0, 1], prompts)
    assert [runner.slot_position(s) for s in (0, 1)] == [20, 45]
    rows = [resident_rows(runner, desc, s, n) for s, n in ((0, 20), (1, 45))]
    # a step-by-step reading of the same suffix: prefill_slots_chunks with no chunk limit
    for slot in (2, 3):
        runner.reset_slot(slot)
    assert runner.prefill_slots_chunks([2, 3], prompts, MAX_CONTEXT) == want
    say("case: layer-sliced suffix prefill on slots 2, 3, one layer per call")
    for slot in (2, 3):
        runner.reset_slot(slot)
    calls = 0
    while True:
        complete, got = runner.prefill_slots_suffix_layer_slice([2, 3], prompts, 1)
        calls += 1
        if complete:
            break
        assert runner.has_suffix_layer_slices() and runner.slot_position(2) == 0
        with pytest.raises(CaratError, match="layer-sliced suffix cohort changed while in flight"):
            runner.prefill_slots_suffix_layer_slice([3, 2], prompts, 1)
        with pytest.raises(CaratError, match="layer-sliced suffix prompt changed while in flight"):
            runner.prefill_slots_suffix_layer_slice([2, 3], [prompts[0], prompts[1][:-1]], 1)
        props = rng.integers(0, desc.vocabulary, (2, 5)).tolist()
        runner.verify_greedy_proposals(props, [p[0] for p in props], [0, 1], [0, 0])
    assert calls == len(desc.layers) and got == want and not runner.has_suffix_layer_slices()
    assert [runner.slot_position(s) for s in (2, 3)] == [20, 45]
    for slot, n, ref in ((2, 20, rows[0]), (3, 45, rows[1])):
        for a, b in zip(resident_rows(runner, desc, slot, n), ref):
            assert np.array_equal(a, b), slot
    say("case: layer-slice abort and errors")
    runner.reset_slot(2)
    assert runner.prefill_slots_suffix_layer_slice([2], [prompts[0]], 1) == (False, [])
    runner.abort_suffix_layer_slices()
    assert not runner.has_suffix_layer_slices()
    with pytest.raises(CaratError, match="layer-sliced suffix does not extend resident context"):
        runner.prefill_slots_suffix_layer_slice([3], [prompts[1]], 1)
    with pytest.raises(CaratError, match="batched suffix contains an invalid token id"):
        runner.prefill_slots_suffix([2], [[desc.vocabulary]])
    with pytest.raises(CaratError, match="batched suffix exceeds shared projection workspace"):
        runner.prefill_slots_suffix([2, 0], [[1] * 100, prompts[0] + [1] * 40])
    say("case: clone_slot")
    runner.reset_slot(2)
    copied = runner.clone_slot(1, 2)
    kv_width = [spec.kv_heads * spec.head_dimension for spec in desc.layers]
    assert copied == sum(2 * 2 * min(45, capacity_of(desc)(li)) * w for li, w in enumerate(kv_width))
    assert runner.slot_position(2) == 45
    for a, b in zip(resident_rows(runner, desc, 2, 45), rows[1]):
        assert np.array_equal(a, b)
    with pytest.raises(CaratError, match="invalid cache slot clone"):
        runner.clone_slot(1, 1)
    runner.reset_slot(0)
    with pytest.raises(CaratError, match="source cache slot is empty or full"):
        runner.clone_slot(0, 3)


def test_append_is_a_lock_step_decode(model):
    """append (batch_model_runner.cu:1006-1040): one token for every slot at the shared position
    equals the oracle composition of a depth-1 step, and every slot moves to the next position."""
    desc, runner = model
    runner.seed_random_cache(60, seed=29, stddev=1 / math.sqrt(128))
    assert runner.position() == 60
    tokens = np.random.default_rng(31).integers(0, desc.vocabulary, BATCH).astype(np.int32)
    expect = verify_step(runner, desc, BATCH, capacity_of(desc), tokens[:, None], list(range(BATCH)),
                         np.full(BATCH, 60, np.int32))
    say("case: append")
    got = np.array(runner.append(tokens.tolist()), np.int32)
    logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(BATCH, -1)
    gap = logits.max(1) - logits[np.arange(BATCH), got]
    mism = int(np.sum(got != expect["predictions"]))
    say(f"  append argmax mismatches vs oracle {mism}/{BATCH}, max gap {gap.max():.3e}")
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))  # near-ties only
    assert mism <= 1
    assert runner.position() == 61 and all(runner.slot_position(s) == 61 for s in range(BATCH))
    with pytest.raises(CaratError, match="token batch has the wrong size"):
        runner.append(tokens[:2].tolist())
    with pytest.raises(CaratError, match="token batch contains an invalid token id"):
        runner.append([0, 1, 2, desc.vocabulary])
    assert runner.position() == 61 and all(runner.slot_position(s) == 61 for s in range(BATCH))


def test_seed_empty_cache_for_benchmark(model):
    """seed_empty_cache_for_benchmark (batch_model_runner.cu:1845-1870): every cache row zeroed,
    every slot at `position`, the reference's message for an out-of-range position; a verify step
    over the zeroed caches then matches the oracle composition."""
    desc, runner = model
    runner.seed_random_cache(50, seed=15, stddev=1 / math.sqrt(128))
    runner.seed_empty_cache_for_benchmark(37)
    for li in range(len(desc.layers)):
        assert not runner.read(f"cache.{li}.k", np.uint16).any()
        assert not runner.read(f"cache.{li}.v", np.uint16).any()
    assert [runner.slot_position(s) for s in range(BATCH)] == [37] * BATCH
    with pytest.raises(CaratError, match="invalid benchmark cache position"):
        runner.seed_empty_cache_for_benchmark(MAX_CONTEXT)
    with pytest.raises(CaratError, match="invalid benchmark cache position"):
        runner.seed_empty_cache_for_benchmark(-1)
    rng = np.random.default_rng(23)
    T = 5
    props = rng.integers(0, desc.vocabulary, (BATCH, T)).astype(np.int32)
    slots = list(range(BATCH))
    positions = np.full(BATCH, 37, np.int32)
    expect = verify_step(runner, desc, BATCH, capacity_of(desc), props, slots, positions)
    say("case: verify over the zeroed benchmark cache")
    runner.verify_greedy_proposals(props.tolist(), props[:, 0].tolist(), slots, [0] * BATCH)
    pred = np.array(runner.last_predictions, np.int32)
    logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(BATCH * T, -1)
    gap = logits.max(1) - logits[np.arange(BATCH * T), pred]
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    assert int(np.sum(pred != expect["predictions"])) <= max(1, BATCH * T // 10)
