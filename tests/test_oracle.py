"""Pins the CPU oracle (oracle/carat_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible slip in the oracle (dropped term, wrong index, wrong tie
rule, wrong rounding) fails: golden vectors produced by the reference's own code, the reference's
own test fixtures, closed forms evaluated independently in float64, invariants and brute force.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "speculation_vectors.json"


@pytest.fixture(scope="module")
def golden():
    return json.loads(GOLDEN.read_text())


# ------------------------------------------------------------------ speculation helpers
def test_acceptance_cap_matches_reference_vectors(golden):
    for case in golden["acceptance_cap"]:
        got = oracle.acceptance_cap(case["depth"], case["remaining"], case["proposals"], case["stops"])
        assert got == case["expected"], case


def test_commit_speculation_matches_reference_vectors(golden):
    for case in golden["commit_speculation"]:
        resident, emitted, nxt, stopped = oracle.commit_speculation(
            case["forced"], case["drafts"], case["next"], case["stops"])
        e = case["expected"]
        assert (resident, emitted, nxt, stopped) == (e["resident"], e["emitted"], e["next"],
                                                     e["stopped"]), case


def test_speculation_known_answers():
    # tests/speculation_tests.cpp:15-60
    props = [10, 11, 12, 13]
    assert oracle.acceptance_cap(4, 10, props, []) == 4
    assert oracle.acceptance_cap(4, 2, props, []) == 2
    assert oracle.acceptance_cap(4, 0, props, []) == 0
    assert oracle.acceptance_cap(4, 10, props, [12]) == 3
    assert oracle.acceptance_cap(4, 10, props, [13, 11]) == 2
    assert oracle.acceptance_cap(4, 10, props, [10]) == 4
    assert oracle.acceptance_cap(4, 2, props, [12]) == 2
    assert oracle.commit_speculation(10, [11, 12], 20, [99]) == ([10, 11, 12], [11, 12, 20], 20, False)
    assert oracle.commit_speculation(10, [], 20, []) == ([10], [20], 20, False)
    assert oracle.commit_speculation(10, [11, 12], 20, [12]) == ([10, 11, 12], [11, 12], 20, True)


def test_reference_library_agrees_live():
    if oracle.ref() is None:
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    rng = np.random.default_rng(5)
    for _ in range(200):
        props = rng.integers(0, 12, size=rng.integers(0, 8)).tolist()
        stops = rng.choice(12, size=rng.integers(0, 4), replace=False).tolist()
        d, rem = int(rng.integers(1, 9)), int(rng.integers(0, 10))
        assert oracle.acceptance_cap(d, rem, props, stops) == oracle.ref_acceptance_cap(d, rem, props, stops)


# ------------------------------------------------------------------ greedy acceptance
def test_greedy_accept_speculative_parity_patterns():
    # ragged_batch_parity.cu:209-229: greedy chain e0..e5, four proposal patterns.
    e = [5, 7, 9, 11, 13, 15]
    rej = 6
    patterns = [[e[0], e[1], e[2], e[3]], [rej, e[1], e[2], e[3]], [e[0], rej, e[2], e[3]],
                [e[0], e[1], rej, e[3]]]
    proposals = np.array([patterns[r % 4] for r in range(16)], np.int32)
    first = np.full(16, e[0], np.int32)
    # target predictions of each row: row t predicts the token after proposal t; only rows whose
    # prefix is on the greedy chain matter.
    pred = np.array([[e[1], e[2], e[3], e[4]]] * 16, np.int32)
    acc, nxt = oracle.greedy_accept(proposals, first, pred)
    exp_acc = [4 if r % 4 == 0 else r % 4 - 1 for r in range(16)]
    exp_next = [e[4] if r % 4 == 0 else e[r % 4 - 1] for r in range(16)]
    assert acc.tolist() == exp_acc
    assert nxt.tolist() == exp_next


def test_greedy_accept_brute_force_invariants():
    # Every proposal/prediction pattern over a 3-token vocabulary at depth 3, with and without caps.
    import itertools

    T, V = 3, 3
    cases = list(itertools.product(range(V), repeat=T))
    props = np.array([c for c in cases for _ in cases], np.int32)
    preds = np.array([c for _ in cases for c in cases], np.int32)
    n = len(props)
    first = np.zeros(n, np.int32)
    for caps in (None, np.arange(n, dtype=np.int32) % (T + 2) - 1):
        acc, nxt = oracle.greedy_accept(props, first, preds, caps)
        for i in range(n):
            cap = T if caps is None else min(max(int(caps[i]), 0), T)
            expected = [0] + preds[i, : T - 1].tolist()  # token expected at each proposal index
            a = int(acc[i])
            assert 0 <= a <= cap
            assert props[i, :a].tolist() == expected[:a]
            if a < cap:
                assert props[i, a] != expected[a]
            assert nxt[i] == expected[a] if a < T else nxt[i] == preds[i, a - 1]


# ------------------------------------------------------------------ argmax
def test_argmax_known_answer():
    # cuda_ops_tests.cu:1137-1164
    vals = np.full((3, 513), -2.0, np.float32)
    vals[0, 17] = 9.0
    vals[1, 0] = 4.0
    vals[1, 401] = 4.0
    vals[2, 512] = 7.0
    assert oracle.argmax_bf16_rows(oracle.f32_to_bf16(vals)).tolist() == [17, 0, 512]


def test_argmax_matches_numpy_first_maximum():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((6, 50000)).astype(np.float32)
    bf = oracle.f32_to_bf16(logits)
    rounded = oracle.bf16_to_f32(bf)
    assert oracle.argmax_bf16_rows(bf).tolist() == np.argmax(rounded, axis=1).tolist()
    assert oracle.argmax_f32_rows_as_bf16(logits).tolist() == np.argmax(rounded, axis=1).tolist()


def test_argmax_special_values():
    inf = np.float32(np.inf)
    rows = np.array([
        [-inf, -inf, -inf, -inf],          # all -inf -> 0
        [np.nan, 1.0, np.nan, 1.0],         # NaN never wins, tie -> lower index
        [np.nan, np.nan, np.nan, np.nan],   # all NaN -> 0
        [-0.0, 0.0, -1.0, -0.0],            # -0 == +0 -> index 0
        [-inf, -5.0, -inf, -5.0],           # finite beats -inf
        [1.0, inf, inf, 3.0],               # +inf, tie -> lower
    ], np.float32)
    assert oracle.argmax_f32_rows_as_bf16(rows).tolist() == [0, 1, 0, 0, 1, 1]


# ------------------------------------------------------------------ conversions
def test_bf16_rounding_closed_form():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-30, 30, 100000))).astype(np.float32)
    x = np.concatenate([x, np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8)], np.float32)])
    got = oracle.bf16_to_f32(oracle.f32_to_bf16(x)).astype(np.float64)
    # nearest bf16 neighbours of each value, tie to even mantissa
    bits = x.view(np.uint32).astype(np.uint64)
    lo = (bits >> 16) << 16
    hi = lo + (1 << 16)
    lo_v = lo.astype(np.uint32).view(np.float32).astype(np.float64)
    hi_v = hi.astype(np.uint32).view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    dlo, dhi = np.abs(xd - lo_v), np.abs(hi_v - xd)
    even_lo = ((lo >> 16) & 1) == 0
    expect = np.where(dlo < dhi, lo_v, np.where(dhi < dlo, hi_v, np.where(even_lo, lo_v, hi_v)))
    assert np.array_equal(got, expect)
    assert oracle.bf16_to_f32(oracle.f32_to_bf16(np.array([1.0 + 2 ** -8], np.float32)))[0] == 1.0


def _e4m3_nearest(v: float) -> int:
    """Independent reference: search all finite codes for the nearest, ties to the even code."""
    table = oracle.e4m3_table()
    if math.isnan(v):
        return 0x7F
    sign = 0x80 if (v < 0 or (v == 0 and math.copysign(1, v) < 0)) else 0
    a = min(abs(v), 448.0)
    best, best_d = 0, None
    for code in range(0x7F):
        d = abs(float(table[code]) - a)
        if best_d is None or d < best_d or (d == best_d and code % 2 == 0 and best % 2 == 1):
            best, best_d = code, d
    return sign | best


def test_e4m3_conversion_against_nearest_search():
    table = oracle.e4m3_table()
    assert table[0x7E] == 448.0 and table[0x38] == 1.0 and table[0x01] == 2.0 ** -9
    assert np.isnan(table[0x7F]) and np.isnan(table[0xFF])
    rng = np.random.default_rng(3)
    vals = list((rng.standard_normal(3000) * np.exp(rng.uniform(-12, 7, 3000))).astype(np.float32))
    # midpoints between consecutive codes (ties) and just around them
    for code in range(0x7E):
        m = (float(table[code]) + float(table[code + 1])) / 2
        vals += [m, np.nextafter(np.float32(m), np.float32(0)), np.nextafter(np.float32(m), np.float32(1e9))]
    vals += [464.0, 470.0, 1e6, float("inf"), 2.0 ** -10, 3 * 2.0 ** -11, 0.0, -0.0]
    for v in vals:
        v = float(np.float32(v))
        assert oracle.f32_to_e4m3_scalar(v) == _e4m3_nearest(v), v
        assert oracle.f32_to_e4m3_scalar(-v) == _e4m3_nearest(-v), -v


def test_quantize_scale_closed_form():
    rng = np.random.default_rng(4)
    x = oracle.f32_to_bf16(rng.standard_normal(4096) * 3)
    q, s = oracle.quantize_e4m3(x)
    amax = float(np.abs(oracle.bf16_to_f32(x)).max())
    assert s == np.float32(np.float32(amax) / np.float32(448.0))
    decoded = oracle.e4m3_table()[q] * s
    assert np.abs(decoded).max() <= amax * (1 + 2 ** -3)
    zero_q, zero_s = oracle.quantize_e4m3(np.zeros(16, np.uint16))
    assert zero_s == 1.0 and not zero_q.any()


def test_fp8_linear_against_float64_matmul():
    rng = np.random.default_rng(5)
    qx = rng.integers(0, 256, (7, 256), dtype=np.uint8)
    qw = rng.integers(0, 256, (33, 256), dtype=np.uint8)
    qx[(qx & 0x7F) == 0x7F] = 0  # drop NaN codes
    qw[(qw & 0x7F) == 0x7F] = 0
    sx, sw = 0.37, 0.011
    table = oracle.e4m3_table().astype(np.float64)
    expect = (table[qx] @ table[qw].T) * np.float64(np.float32(sx) * np.float32(sw))
    got = oracle.fp8_linear_f32(qx, sx, qw, sw).astype(np.float64)
    assert np.allclose(got, expect, rtol=1e-6, atol=1e-6 * np.abs(expect).max())


# ------------------------------------------------------------------ channel / block_128 scaling
def _planted_blocks(rows, cols, block_rows, block_cols, rng):
    """bf16 matrix whose (block_rows x block_cols) blocks each hold one planted maximum of a
    distinct magnitude, so that every block's amax (and scale) is known in closed form."""
    x = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    nb, kb = -(-rows // block_rows), -(-cols // block_cols)
    amax = np.zeros((nb, kb))
    for i in range(nb):
        for j in range(kb):
            big = 2.0 + i * 3.5 + j * 1.25  # bf16-exact values > 1
            r = i * block_rows + (i + j) % min(block_rows, rows - i * block_rows)
            c = j * block_cols + (2 * i + j) % min(block_cols, cols - j * block_cols)
            x[r, c] = -big if (i + j) % 2 else big
            amax[i, j] = big
    return oracle.f32_to_bf16(x), amax


def _dequantised(q, scale_of_element):
    return oracle.e4m3_table().astype(np.float64)[q] * scale_of_element


def test_row_quantisation_closed_form():
    rng = np.random.default_rng(21)
    x, amax = _planted_blocks(9, 300, 1, 300, rng)
    x[4] = 0  # an all-zero row takes the 2^-24 floor and quantises to zeros
    q, s = oracle.quantize_e4m3_rows(x)
    expect = np.float32(amax[:, 0]).astype(np.float32) / np.float32(448.0)
    expect[4] = np.float32(2.0 ** -24)
    assert np.array_equal(s, expect)
    assert not q[4].any()
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    # q = e4m3(x / scale) with a true float32 division; the planted maximum lands on +-448
    direct = np.array([[oracle.f32_to_e4m3_scalar(float(np.float32(v) / s[r])) for v in xf[r]]
                       for r in range(9)], np.uint8)
    assert np.array_equal(q, direct)
    assert np.all(np.isin(q[np.abs(xf) == amax[:, :1]], [0x7E, 0xFE]))
    rel = np.abs(_dequantised(q, s[:, None].astype(np.float64)) - xf)
    assert np.all(rel <= np.abs(xf) * 2 ** -4 + s[:, None] * 2 ** -9 * 0.5 + 1e-30)


def test_weight_block128_quantisation_layout():
    rng = np.random.default_rng(22)
    for n, k in ((200, 300), (128, 512), (37, 129)):
        w, amax = _planted_blocks(n, k, 128, 128, rng)
        q, s = oracle.quantize_e4m3_weight_block128(w)
        nb, kb = amax.shape
        kbp = (kb + 3) // 4 * 4
        assert s.shape == (nb * kbp,)
        grid = s.reshape(nb, kbp)
        assert np.array_equal(grid[:, :kb], (amax.astype(np.float32) / np.float32(448.0)))
        assert not grid[:, kb:].any()  # padding columns stay zero
        per_element = np.repeat(np.repeat(grid[:, :kb].astype(np.float64), 128, 0), 128, 1)[:n, :k]
        xf = oracle.bf16_to_f32(w).astype(np.float64)
        assert np.all(np.abs(_dequantised(q, per_element) - xf) <= np.abs(xf) * 2 ** -4 + per_element * 2 ** -10)


def test_activation_block128_quantisation_layout():
    rng = np.random.default_rng(23)
    x, amax = _planted_blocks(5, 384, 1, 128, rng)
    q, s = oracle.quantize_e4m3_activation_block128(x)
    # [k block][row]
    assert np.array_equal(s.reshape(3, 5), (amax.T.astype(np.float32) / np.float32(448.0)))
    per_element = np.repeat(s.reshape(3, 5).T.astype(np.float64), 128, 1)
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    assert np.all(np.abs(_dequantised(q, per_element) - xf) <= np.abs(xf) * 2 ** -4 + per_element * 2 ** -10)


@pytest.mark.parametrize("scaling", [1, 2])
def test_scaled_fp8_linear_against_dequantised_float64_matmul(scaling):
    """Scales factor out of each block's dot product, so the block-scaled sum equals the float64
    product of the dequantised operands; a transposed or shifted scale index fails this."""
    rng = np.random.default_rng(24 + scaling)
    m, k, n = 6, 384, 260
    x = oracle.f32_to_bf16(rng.standard_normal((m, k)) * np.exp(rng.uniform(-2, 2, (m, 1))))
    w = oracle.f32_to_bf16(rng.standard_normal((n, k)) * 0.05 * np.exp(rng.uniform(-2, 2, (n, 1))))
    qw, sw = oracle.quantize_weight_scaled(w, scaling)
    qx, sx = oracle.quantize_activation_scaled(x, scaling)
    if scaling == 1:
        xs, ws = sx[:, None].astype(np.float64), sw[:, None].astype(np.float64)
    else:
        kb = k // 128
        xs = np.repeat(sx.reshape(kb, m).T.astype(np.float64), 128, 1)
        ws = np.repeat(np.repeat(sw.reshape(-1, (kb + 3) // 4 * 4)[:, :kb].astype(np.float64), 128, 0), 128, 1)[:n]
    expect = _dequantised(qx, xs) @ _dequantised(qw, ws).T
    got = oracle.fp8_linear_scaled(qx, sx, qw, sw, scaling, f32=True).astype(np.float64)
    assert np.allclose(got, expect, rtol=1e-6, atol=1e-6 * np.abs(expect).max())
    # and the quantised product stays close to the bf16 one (the scales are not misapplied)
    exact = oracle.bf16_to_f32(x).astype(np.float64) @ oracle.bf16_to_f32(w).astype(np.float64).T
    assert np.abs(got - exact).max() <= 0.08 * np.abs(exact).max()
    bf = oracle.bf16_to_f32(oracle.fp8_linear_scaled(qx, sx, qw, sw, scaling)).astype(np.float64)
    assert np.all(np.abs(bf - got) <= np.abs(got) * 2 ** -8 * 1.01 + 1e-30)


# ------------------------------------------------------------------ row ops
def _bf(x):
    return oracle.bf16_to_f32(oracle.f32_to_bf16(x)).astype(np.float64)


def test_bf16_linear_against_float64_matmul():
    rng = np.random.default_rng(8)
    for m, k, n in ((1, 64, 3), (7, 256, 33), (24, 1024, 40)):
        x = oracle.f32_to_bf16(rng.standard_normal((m, k)))
        w = oracle.f32_to_bf16(rng.standard_normal((n, k)) * 0.05)
        exp = oracle.bf16_to_f32(x).astype(np.float64) @ oracle.bf16_to_f32(w).astype(np.float64).T
        got = oracle.bf16_to_f32(oracle.bf16_linear(x, w)).astype(np.float64)
        # one bf16 rounding of the float64 value (ties and double-rounding aside)
        assert np.all(np.abs(got - exp) <= np.abs(exp) * 2 ** -8 * 1.01 + 1e-12)


def test_rms_norm_closed_form():
    rng = np.random.default_rng(6)
    x = oracle.f32_to_bf16(rng.standard_normal((5, 384)))
    w = oracle.f32_to_bf16(1 + 0.1 * rng.standard_normal(384))
    res = oracle.f32_to_bf16(rng.standard_normal((5, 384)))
    xf, wf, rf = (oracle.bf16_to_f32(a).astype(np.float64) for a in (x, w, res))
    inv = 1 / np.sqrt((xf ** 2).mean(1, keepdims=True) + 1e-6)
    out, amax = oracle.rms_norm(x, w)
    assert np.allclose(oracle.bf16_to_f32(out), xf * inv * wf, rtol=2 ** -8, atol=1e-6)
    assert np.array_equal(amax, np.abs(oracle.bf16_to_f32(out)).max(1))
    out_r, _ = oracle.rms_norm(x, w, res)
    assert np.allclose(oracle.bf16_to_f32(out_r), xf * inv * wf + rf, rtol=2 ** -7, atol=2 ** -7)
    # fused add-and-norm equals the two steps (cuda_ops_tests.cu:66-136 checks the same identity)
    r1, y, a2 = oracle.rms_norm_add_and_norm(x, w, res, w)
    assert np.array_equal(r1, out_r)
    y2, _ = oracle.rms_norm(r1, w)
    assert np.array_equal(y, y2)
    scalar = int(oracle.f32_to_bf16(np.array([0.5], np.float32))[0])
    scaled = oracle.rms_norm_add_scale(x, w, res, scalar)
    assert np.array_equal(oracle.bf16_to_f32(scaled), oracle.bf16_to_f32(out_r) * 0.5)


def test_gelu_gate_closed_form():
    rng = np.random.default_rng(7)
    packed = oracle.f32_to_bf16(rng.standard_normal((4, 512)) * 2)
    pf = oracle.bf16_to_f32(packed).astype(np.float64)
    g, u = pf[:, :256], pf[:, 256:]
    gelu = 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)))
    out, amax = oracle.gelu_tanh_gate_rows(packed)
    assert np.allclose(oracle.bf16_to_f32(out), gelu * u, rtol=2 ** -7, atol=1e-5)
    assert np.array_equal(amax, np.abs(oracle.bf16_to_f32(out)).max(1))


def test_embedding_closed_form():
    rng = np.random.default_rng(8)
    w = oracle.f32_to_bf16(rng.standard_normal((50, 64)))
    out = oracle.embedding(w, [3, 49, 0], math.sqrt(5376))
    s = _bf(np.float32(math.sqrt(5376)))
    assert np.array_equal(oracle.bf16_to_f32(out), _bf(oracle.bf16_to_f32(w)[[3, 49, 0]] * s).astype(np.float32))


def test_rope_table_closed_form_and_partial_rotary():
    cos, sin = oracle.rope_table(128, False, 64)
    pos = np.arange(64)[:, None]
    i = np.arange(128)[None, :] % 64
    freq = (10000.0 ** (-2.0 * i / 128)).astype(np.float32)
    ang = (pos.astype(np.float32) * freq).astype(np.float64)
    assert np.abs(oracle.bf16_to_f32(cos) - np.cos(ang)).max() <= 2 ** -8
    assert np.abs(oracle.bf16_to_f32(sin) - np.sin(ang)).max() <= 2 ** -8
    gcos, gsin = oracle.rope_table(128, True, 64)
    idx = np.arange(128) % 64
    assert (oracle.bf16_to_f32(gcos)[:, idx >= 16] == 1.0).all()
    assert (oracle.bf16_to_f32(gsin)[:, idx >= 16] == 0.0).all()
    assert oracle.bf16_to_f32(gsin)[5, 1] != 0.0


def test_qkv_post_rotation_invariants():
    rng = np.random.default_rng(9)
    hq, hkv, d = 4, 2, 128
    packed = oracle.f32_to_bf16(rng.standard_normal((3, (hq + 2 * hkv) * d)))
    ones = oracle.f32_to_bf16(np.ones(d, np.float32))
    cos, sin = oracle.rope_table(d, False, 32)
    q0, k0, v0 = oracle.qkv_post(packed, ones, ones, cos, sin, [0, 0, 0], hq, hkv, d)
    # position 0: cos = 1, sin = 0 -> plain bf16 RMSNorm
    pf = oracle.bf16_to_f32(packed).reshape(3, hq + 2 * hkv, d).astype(np.float64)
    normed = pf / np.sqrt((pf ** 2).mean(-1, keepdims=True) + 1e-6)
    assert np.allclose(oracle.bf16_to_f32(q0), normed[:, :hq], rtol=2 ** -7, atol=1e-6)
    assert np.allclose(oracle.bf16_to_f32(v0), normed[:, hq + hkv:], rtol=2 ** -7, atol=1e-6)
    # later positions rotate each (i, i + D/2) pair: pair norms are preserved
    q5, k5, _ = oracle.qkv_post(packed, ones, ones, cos, sin, [5, 17, 31], hq, hkv, d)
    for a, b in ((q0, q5), (k0, k5)):
        fa, fb = oracle.bf16_to_f32(a).astype(np.float64), oracle.bf16_to_f32(b).astype(np.float64)
        na = fa[..., :64] ** 2 + fa[..., 64:] ** 2
        nb = fb[..., :64] ** 2 + fb[..., 64:] ** 2
        assert np.allclose(na, nb, rtol=3e-2, atol=1e-3)
        assert not np.array_equal(fa, fb)


def _rope_closed_form(normalized, position, dimension, theta, rotating_pairs):
    """Rotate-half RoPE of qkv.cu:410-416 in float64: for i < D/2 with frequency
    f_i = theta^(-2i/D), out[i] = n[i]cos(p f_i) - n[i+D/2]sin(p f_i) and
    out[i+D/2] = n[i+D/2]cos(p f_i) + n[i]sin(p f_i); pairs i >= rotating_pairs stay as they are."""
    half = dimension // 2
    out = normalized.copy()
    for i in range(min(half, rotating_pairs)):
        angle = position * theta ** (-2.0 * i / dimension)
        c, s = math.cos(angle), math.sin(angle)
        a, b = normalized[..., i], normalized[..., i + half]
        out[..., i] = a * c - b * s
        out[..., i + half] = b * c + a * s
    return out


@pytest.mark.parametrize("proportional", [False, True], ids=["sliding", "global_partial"])
@pytest.mark.parametrize("key_equals_value", [False, True], ids=["kv", "k_eq_v"])
def test_qkv_post_closed_form_rotation(proportional, key_equals_value):
    """Known answers for qkv.cu:387-530 at nonzero positions: weighted per-head RMSNorm, then the
    rotate-half rotation in its stated sense (a flipped sign moves values by ~|n sin|), partial
    rotary of D/8 pairs in global layers (qkv.cu:52-55), V = unweighted RMSNorm of the V input,
    which is the K input in K=V mode."""
    rng = np.random.default_rng(21)
    hq, hkv, d = 4, 2, 128
    rows = 4
    width = (hq + hkv * (1 if key_equals_value else 2)) * d
    packed = oracle.f32_to_bf16(rng.standard_normal((rows, width)) * 3.0)
    qw = oracle.f32_to_bf16(1.0 + 0.5 * rng.standard_normal(d))
    kw = oracle.f32_to_bf16(1.0 + 0.5 * rng.standard_normal(d))
    positions = np.array([17, 1, 300, 4095], np.int32)
    cos, sin = oracle.rope_table(d, proportional, 4096)
    q, k, v = oracle.qkv_post(packed, qw, kw, cos, sin, positions, hq, hkv, d, key_equals_value)
    f = lambda a: oracle.bf16_to_f32(a).astype(np.float64)
    heads = f(packed).reshape(rows, -1, d)
    rms = lambda x: x / np.sqrt((x ** 2).mean(-1, keepdims=True) + 1e-6)
    theta, pairs = (1e6, d // 8) if proportional else (1e4, d // 2)
    k_in = heads[:, hq:hq + hkv]
    v_in = k_in if key_equals_value else heads[:, hq + hkv:]
    for r in range(rows):
        eq = _rope_closed_form(rms(heads[r, :hq]) * f(qw), int(positions[r]), d, theta, pairs)
        ek = _rope_closed_form(rms(k_in[r]) * f(kw), int(positions[r]), d, theta, pairs)
        for got, exp in ((f(q[r]), eq), (f(k[r]), ek)):
            # bf16 rounding of the normalized value, of cos/sin and of the output: a few bf16 ulps
            assert np.abs(got - exp).max() <= 4 * 2 ** -8 * np.abs(exp).max(), r
        assert np.allclose(f(v[r]), rms(v_in[r]), rtol=2 ** -7, atol=1e-6)
    # the same values with the opposite rotation sense are far off at position 17
    wrong = _rope_closed_form(rms(heads[0, :hq]) * f(qw), -17, d, theta, pairs)
    assert np.abs(f(q[0]) - wrong).max() > 0.3
    if proportional:  # pairs past D/8 do not rotate: the output is the rounded normalized value
        idx = np.r_[pairs:d // 2, d // 2 + pairs:d]
        n = oracle.f32_to_bf16(rms(heads[2, :hq]) * f(qw))
        assert np.array_equal(q[2][..., idx], n[..., idx])


# ------------------------------------------------------------------ attention
def _rand_bf16(rng, shape, scale=1.0):
    return oracle.f32_to_bf16(rng.standard_normal(shape) * scale)


def test_sliding_attention_equals_reference_ring_formulation():
    """The logical-window oracle on a full ring equals the reference's ring+backup formulation
    (prefill_gemm_attention.cu:126-298 as restated by its own test, cuda_ops_tests.cu:1630-1779)."""
    rng = np.random.default_rng(10)
    R, T, hq, hkv, d, C = 3, 5, 4, 2, 32, 16
    positions = np.array([40, 47, 16 + 11], np.int32)  # all >= C - 1: the ring is full
    slots = np.array([2, 0, 1], np.int32)
    k_old = _rand_bf16(rng, (3, hkv, C, d))
    v_old = _rand_bf16(rng, (3, hkv, C, d))
    k_new = _rand_bf16(rng, (R, T, hkv, d))
    v_new = _rand_bf16(rng, (R, T, hkv, d))
    q = _rand_bf16(rng, (R, T, hq, d), 0.5)
    got = oracle.bf16_to_f32(oracle.verify_attention(q, k_old, v_old, k_new, v_new, slots, positions, C, C))
    # reference layout: the ring holds the proposals, the overwritten rows sit in the backup
    k_ring = k_old[slots].copy()
    v_ring = v_old[slots].copy()
    k_backup = np.empty((R, hkv, T, d), np.uint16)
    v_backup = np.empty((R, hkv, T, d), np.uint16)
    for r in range(R):
        for t in range(T):
            phys = (positions[r] + t) % C
            k_backup[r, :, t] = k_ring[r, :, phys]
            v_backup[r, :, t] = v_ring[r, :, phys]
            k_ring[r, :, phys] = k_new[r, t]
            v_ring[r, :, phys] = v_new[r, t]
    ref = oracle.ring_backup_attention(q.transpose(0, 2, 1, 3), k_ring, v_ring, k_backup, v_backup,
                                       positions, hkv, C).transpose(0, 2, 1, 3)
    assert np.abs(got - ref).max() <= 2 ** -7 * np.abs(ref).max() + 1e-6


def _softmax_attention(q, keys, values):
    s = keys @ q
    s = s - s.max()
    p = np.exp(s)
    return (p / p.sum()) @ values


def test_global_and_sliding_attention_brute_force():
    rng = np.random.default_rng(11)
    R, T, hq, hkv, d, C = 2, 3, 4, 2, 16, 64
    positions = np.array([5, 40], np.int32)
    slots = np.array([1, 0], np.int32)
    kc = _rand_bf16(rng, (2, hkv, C, d))
    vc = _rand_bf16(rng, (2, hkv, C, d))
    kn = _rand_bf16(rng, (R, T, hkv, d))
    vn = _rand_bf16(rng, (R, T, hkv, d))
    q = _rand_bf16(rng, (R, T, hq, d), 0.5)
    f = lambda a: oracle.bf16_to_f32(a).astype(np.float64)
    for window in (0, 9):
        got = f(oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, C, window))
        for r in range(R):
            p = positions[r]
            for t in range(T):
                for h in range(hq):
                    kvh = h // (hq // hkv)
                    qpos = p + t
                    lo = 0 if window == 0 else max(0, qpos - window + 1)
                    keys, vals = [], []
                    for j in range(lo, qpos + 1):
                        if j >= p:
                            keys.append(f(kn[r, j - p, kvh])), vals.append(f(vn[r, j - p, kvh]))
                        else:
                            keys.append(f(kc[slots[r], kvh, j % C])), vals.append(f(vc[slots[r], kvh, j % C]))
                    exp = _softmax_attention(f(q[r, t, h]), np.array(keys), np.array(vals))
                    assert np.allclose(got[r, t, h], exp, rtol=2 ** -7, atol=2 ** -8)


def test_decode_attention_brute_force():
    rng = np.random.default_rng(12)
    B, hq, hkv, d, C = 3, 4, 2, 16, 32
    kc = _rand_bf16(rng, (4, hkv, C, d))
    vc = _rand_bf16(rng, (4, hkv, C, d))
    q = _rand_bf16(rng, (B, hq, d), 0.5)
    slots = np.array([3, 0, 2], np.int32)
    positions = np.array([4, 31, 100], np.int32)
    f = lambda a: oracle.bf16_to_f32(a).astype(np.float64)
    got = f(oracle.decode_attention(q, kc, vc, slots, positions, hkv, C))
    for b in range(B):
        valid = min(positions[b] + 1, C)
        for h in range(hq):
            kvh = h // 2
            exp = _softmax_attention(f(q[b, h]), f(kc[slots[b], kvh, :valid]), f(vc[slots[b], kvh, :valid]))
            assert np.allclose(got[b, h], exp, rtol=2 ** -7, atol=2 ** -8)


def test_commit_kv_net_effect_of_backup_and_restore():
    """orc_commit_kv equals the reference's sequence: backup rows, write all T proposals,
    restore rows t >= accepted (ops.cu:827-871)."""
    rng = np.random.default_rng(13)
    R, T, hkv, d, C = 3, 5, 2, 8, 16
    cache_k = rng.integers(0, 60000, (3, hkv, C, d)).astype(np.uint16)
    cache_v = rng.integers(0, 60000, (3, hkv, C, d)).astype(np.uint16)
    kn = rng.integers(0, 60000, (R, T, hkv, d)).astype(np.uint16)
    vn = rng.integers(0, 60000, (R, T, hkv, d)).astype(np.uint16)
    slots = np.array([1, 2, 0], np.int32)
    positions = np.array([14, 3, 30], np.int32)
    accepted = np.array([0, 5, 2], np.int32)
    ref_k, ref_v = cache_k.copy(), cache_v.copy()
    for r in range(R):
        backup_k = [ref_k[slots[r], :, (positions[r] + t) % C].copy() for t in range(T)]
        backup_v = [ref_v[slots[r], :, (positions[r] + t) % C].copy() for t in range(T)]
        for t in range(T):
            ref_k[slots[r], :, (positions[r] + t) % C] = kn[r, t]
            ref_v[slots[r], :, (positions[r] + t) % C] = vn[r, t]
        for t in range(accepted[r], T):
            ref_k[slots[r], :, (positions[r] + t) % C] = backup_k[t]
            ref_v[slots[r], :, (positions[r] + t) % C] = backup_v[t]
    got_k, got_v = cache_k.copy(), cache_v.copy()
    oracle.commit_kv(got_k, got_v, kn, vn, slots, positions, accepted, C)
    assert np.array_equal(got_k, ref_k) and np.array_equal(got_v, ref_v)


def _e4m3_pow2_kv(rng, shape):
    """e4m3 codes of N(0,1)-ish values, finite codes only."""
    codes = oracle.f32_to_e4m3(rng.standard_normal(shape).astype(np.float32) * 2.0)
    return codes


def test_fp8_attention_equals_bf16_attention_on_exact_dequantised_values():
    """With power-of-two scales e4m3(x)*scale is exact in bf16 and scaling by 2^k commutes with
    every fp32 sum, so the e4m3 oracle must equal the bf16 oracle on the dequantised K/V bit for
    bit (global window, ragged positions including position 0)."""
    rng = np.random.default_rng(31)
    R, T, hq, hkv, d, C = 3, 5, 4, 2, 32, 48
    positions = np.array([0, 7, 40], np.int32)
    slots = np.array([2, 0, 1], np.int32)
    table = oracle.e4m3_table().astype(np.float32)
    kc, vc = _e4m3_pow2_kv(rng, (3, hkv, C, d)), _e4m3_pow2_kv(rng, (3, hkv, C, d))
    kn, vn = _e4m3_pow2_kv(rng, (R, T, hkv, d)), _e4m3_pow2_kv(rng, (R, T, hkv, d))
    q = _rand_bf16(rng, (R, T, hq, d), 0.25)
    for k_scale, v_scale in ((0.25, 2.0), (1.0, 0.0625)):
        deq = lambda codes, s: oracle.f32_to_bf16(table[codes] * np.float32(s))
        for codes, s in ((kc, k_scale), (vc, v_scale), (kn, k_scale), (vn, v_scale)):
            assert np.array_equal(oracle.bf16_to_f32(deq(codes, s)), table[codes] * np.float32(s))
        got = oracle.verify_attention_fp8(q, kc, vc, kn, vn, k_scale, v_scale, slots, positions, C)
        exp = oracle.verify_attention(q, deq(kc, k_scale), deq(vc, v_scale), deq(kn, k_scale),
                                      deq(vn, v_scale), slots, positions, C, 0)
        assert np.array_equal(got, exp)


def test_fp8_attention_brute_force():
    """Any scales: float64 softmax over e4m3(k)*s_k with output sum p*e4m3(v)*s_v."""
    rng = np.random.default_rng(32)
    R, T, hq, hkv, d, C = 2, 3, 4, 1, 16, 24
    positions = np.array([3, 20], np.int32)
    slots = np.array([1, 0], np.int32)
    table = oracle.e4m3_table().astype(np.float64)
    kc, vc = _e4m3_pow2_kv(rng, (2, hkv, C, d)), _e4m3_pow2_kv(rng, (2, hkv, C, d))
    kn, vn = _e4m3_pow2_kv(rng, (R, T, hkv, d)), _e4m3_pow2_kv(rng, (R, T, hkv, d))
    q = _rand_bf16(rng, (R, T, hq, d), 0.3)
    ks, vs = 0.0371, 0.113
    got = oracle.bf16_to_f32(oracle.verify_attention_fp8(q, kc, vc, kn, vn, ks, vs, slots,
                                                         positions, C)).astype(np.float64)
    qf = oracle.bf16_to_f32(q).astype(np.float64)
    for r in range(R):
        p = int(positions[r])
        for t in range(T):
            keys = [table[kc[slots[r], 0, j]] if j < p else table[kn[r, j - p, 0]] for j in range(p + t + 1)]
            vals = [table[vc[slots[r], 0, j]] if j < p else table[vn[r, j - p, 0]] for j in range(p + t + 1)]
            for h in range(hq):
                exp = _softmax_attention(qf[r, t, h], np.array(keys) * ks, np.array(vals) * vs)
                assert np.allclose(got[r, t, h], exp, rtol=2 ** -7, atol=2 ** -8 * np.abs(exp).max())
