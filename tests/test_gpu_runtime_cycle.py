"""The runtime's speculative decode cycle on this runner, as the reference's scheduler drives it
(ContinuousScheduler::speculative_decode, native_runtime_main.cpp:583-678): prompts are made
resident with prefill_slots_suffix, then each cycle drafts four tokens (draft_four with the
pending token forced), caps acceptance (acceptance_cap), verifies (verify_greedy_proposals),
falls back to append_ragged where nothing was accepted, and commits (commit_speculation).

Checked over several cycles: every verify decision is a near-argmax of the oracle composition of
that step over the caches as they stand, acceptance and the next token follow from the step's own
predictions bit for bit (speculative_decode's contract), slot positions equal the resident token
counts, and the hidden hand-off feeds the next draft (row 0 is the forced token)."""
import math
import sys

import numpy as np
import pytest

from carat_amd.runner import BatchModelRunner, LayerSpec, ModelDesc, acceptance_cap, commit_speculation
from oracle import oracle
from tests.runner_oracle import verify_step

pytestmark = pytest.mark.gpu

BATCH = 4
MAX_CONTEXT = 128
DEPTH = 4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def tiny_desc():
    layers = [LayerSpec(True, 4, 2, 128), LayerSpec(True, 4, 2, 128), LayerSpec(False, 4, 2, 128)]
    return ModelDesc(hidden=256, intermediate=512, vocabulary=2048, sliding_window=32, layers=layers,
                     assistant=True, assistant_hidden=256, assistant_intermediate=512,
                     assistant_layers=2, assistant_query_heads=4, seed=5, weight_std=0.05)


class Slot:
    def __init__(self, prompt, max_tokens, stop_ids):
        self.cached = list(prompt)     # resident tokens
        self.token_to_append = None    # the pending (forced) token, not yet resident
        self.output = []
        self.max_tokens = max_tokens
        self.stop_ids = stop_ids
        self.done = False


def test_speculative_decode_cycles(torch_cuda):
    desc = tiny_desc()
    rng = np.random.default_rng(41)
    C = lambda li: min(MAX_CONTEXT, desc.sliding_window) if desc.layers[li].sliding else MAX_CONTEXT
    say("case: runtime cycle runner create")
    runner = BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    try:
        prompts = [rng.integers(0, desc.vocabulary, n).astype(np.int32).tolist() for n in (9, 23, 14, 30)]
        slots = list(range(BATCH))
        stop = [7]
        state = [Slot(p, 14, stop) for p in prompts]
        for s in slots:
            runner.reset_slot(s)
        say("case: prefill_slots_suffix of four prompts")
        first = runner.prefill_slots_suffix(slots, prompts)
        for s, tok in zip(state, first):
            s.token_to_append = tok
            s.output.append(tok)
        for cycle in range(6):
            active = [i for i in slots if not state[i].done]
            if not active:
                break
            # speculative_decode orders the cohort by position (ragged contexts)
            active.sort(key=lambda i: runner.slot_position(i))
            last = [state[i].cached[-1] for i in active]
            target_first = [state[i].token_to_append for i in active]
            say(f"case: cycle {cycle} draft for slots {active}")
            proposals = runner.draft_four(last, active, target_first, DEPTH)
            assert [row[0] for row in proposals] == target_first
            caps = [acceptance_cap(DEPTH, state[i].max_tokens - len(state[i].output), proposals[r],
                                   state[i].stop_ids) for r, i in enumerate(active)]
            positions = np.array([runner.slot_position(i) for i in active], np.int32)
            assert all(runner.slot_position(i) == len(state[i].cached) for i in active)
            expect = verify_step(runner, desc, BATCH, C, np.array(proposals, np.int32), active, positions)
            say(f"case: cycle {cycle} verify (caps {caps})")
            res = runner.verify_greedy_proposals(proposals, target_first, active, caps)
            pred = np.array(runner.last_predictions, np.int32).reshape(len(active), DEPTH)
            # every decision is a near-argmax of the oracle's logits for this step
            logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(len(active) * DEPTH, -1)
            flat = pred.reshape(-1)
            gap = logits.max(1) - logits[np.arange(flat.size), flat]
            assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))  # within 2 bf16 ulps of the row maximum
            # acceptance and next token follow from the step's own predictions, bit for bit
            acc, nxt = oracle.greedy_accept(np.array(proposals, np.int32), np.array(target_first, np.int32),
                                            flat, np.array(caps, np.int32))
            assert res.accepted_tokens == acc.tolist() and res.next_tokens == nxt.tolist()
            fallback = [r for r, a in enumerate(res.accepted_tokens) if a == 0]
            fallback_next = []
            if fallback:
                fallback_next = runner.append_ragged([target_first[r] for r in fallback],
                                                     [active[r] for r in fallback])
            for r, i in enumerate(active):
                s = state[i]
                a = res.accepted_tokens[r]
                nxt_tok = fallback_next[fallback.index(r)] if a == 0 else res.next_tokens[r]
                resident, emitted, next_token, stopped = commit_speculation(
                    s.token_to_append, proposals[r][1:a] if a > 1 else [], nxt_tok, s.stop_ids)
                s.cached += resident
                s.output += emitted
                s.token_to_append = next_token
                assert runner.slot_position(i) == len(s.cached), (cycle, i)
                if stopped or len(s.output) >= s.max_tokens:
                    s.done = True
        assert all(len(s.output) > 1 for s in state)
    finally:
        runner.close()


def test_bench_cycle_equals_the_python_cycle(torch_cuda):
    """carat_hip_bench_speculative_cycle (the benchmark's cycle in C++) makes the same decisions as
    the same cycle composed from the Python mirror: identical accepted counts, next forced tokens,
    last resident tokens and slot positions on two runners built from the same seed."""
    desc = tiny_desc()
    rng = np.random.default_rng(43)
    say("case: bench cycle (C++) vs python cycle")
    a = BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    b = BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    try:
        slots = list(range(BATCH))
        for r in (a, b):
            r.seed_random_cache(50, seed=3, stddev=1 / math.sqrt(128))
        forced = rng.integers(0, desc.vocabulary, BATCH).astype(np.int32)
        last = rng.integers(0, desc.vocabulary, BATCH).astype(np.int32)
        for cycle in range(3):
            planted = rng.integers(0, desc.vocabulary, (BATCH, DEPTH + 1)).astype(np.int32)
            planted[:, 0] = forced
            acc, nxt, lst, seconds = a.bench_speculative_cycle(last, slots, forced, planted, 3, [7])
            assert seconds > 0.0
            drafts = b.draft_four(last.tolist(), slots, forced.tolist(), DEPTH + 1)
            caps = [acceptance_cap(DEPTH + 1, 3, drafts[i], [7]) for i in range(BATCH)]
            res = b.verify_greedy_proposals(planted.tolist(), forced.tolist(), slots, caps)
            want_next, want_last = [], []
            for i in range(BATCH):
                k = res.accepted_tokens[i]
                resident, _, n, _ = commit_speculation(int(forced[i]), planted[i, 1:k].tolist(),
                                                       res.next_tokens[i], [7])
                want_next.append(n)
                want_last.append(resident[-1])
            assert acc.tolist() == res.accepted_tokens
            assert nxt.tolist() == want_next and lst.tolist() == want_last
            assert [a.slot_position(s) for s in slots] == [b.slot_position(s) for s in slots]
            forced, last = nxt, lst
        bad = planted.copy()
        bad[:, 0] = forced + 1
        with pytest.raises(Exception, match="planted proposals must start with the forced token"):
            a.bench_speculative_cycle(last, slots, forced, bad, 3, [7])
        # remaining = 0 caps every request at 0: nothing is accepted, and every request takes the
        # scheduler's fallback (append_ragged of its forced token), as the Python cycle does
        planted[:, 0] = forced
        before = [a.slot_position(s) for s in slots]
        acc, nxt, lst, _ = a.bench_speculative_cycle(last, slots, forced, planted, 0, [7])
        want = b.append_ragged(forced.tolist(), slots)
        assert acc.tolist() == [0] * BATCH
        assert nxt.tolist() == want and lst.tolist() == forced.tolist()
        assert [a.slot_position(s) for s in slots] == [p + 1 for p in before]
    finally:
        a.close()
        b.close()
