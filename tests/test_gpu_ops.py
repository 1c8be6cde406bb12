"""Kernel parity on the GPU: every HIP entry point of include/carat_hip.h against the CPU oracle on
the same seeded inputs.

Bars: integer/index results (argmax, acceptance, e4m3 codes) are bit-exact; floating-point outputs
carry the tolerance written in each test (attention: max |err| <= 2e-2 * max |ref|, the
bound stated for attention outputs against an fp32-accumulated reference).
"""
import math
import sys

import numpy as np
import pytest

from carat_amd import _lib
from oracle import oracle

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev(torch_cuda):
    return torch_cuda


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def to_host(t):
    return t.cpu().numpy()


def stream_of(torch):
    return torch.cuda.current_stream().cuda_stream


def bf16_rel_err(got_bf16, ref_bf16):
    g = oracle.bf16_to_f32(got_bf16).astype(np.float64)
    r = oracle.bf16_to_f32(ref_bf16).astype(np.float64)
    return np.abs(g - r).max() / max(np.abs(r).max(), 1e-30)


# ------------------------------------------------------------------ conversions
def test_e4m3_conversion_exhaustive_over_bf16(dev):
    torch = dev
    say("case: e4m3 conversion, all 65536 bf16 patterns x 4 scales")
    patterns = np.arange(65536, dtype=np.uint16)
    base = oracle.bf16_to_f32(patterns)
    finite = np.isfinite(base)
    for scale in (1.0, 1 / 3.7, 17.3, 2.0 ** -7):
        vals = (base[finite] * np.float32(scale)).astype(np.float32)
        x = to_dev(torch, vals)
        out = torch.empty(vals.size, dtype=torch.uint8, device="cuda")
        _lib.check(_lib.lib().carat_hip_f32_to_e4m3(_lib.ptr(x), _lib.ptr(out), vals.size,
                                                   _lib.ptr(stream_of(torch))))
        torch.cuda.synchronize()
        got = to_host(out)
        expect = oracle.f32_to_e4m3(vals)
        bad = np.nonzero(got != expect)[0]
        assert bad.size == 0, (scale, vals[bad[:5]], got[bad[:5]], expect[bad[:5]])


# ------------------------------------------------------------------ argmax + acceptance
def planted_config1(rng, requests=24, tokens=5, vocab=262144, p=0.7):
    """Benchmark config 1: N(0,1) fp32 logits; draft d_{j+1} = argmax(row j) w.p. p (geometric
    acceptance), else a random non-argmax id. proposal[0] = forced = target_first."""
    logits = rng.standard_normal((requests * tokens, vocab), dtype=np.float32)
    arg = oracle.argmax_f32_rows_as_bf16(logits).reshape(requests, tokens)
    proposals = np.zeros((requests, tokens), np.int32)
    first = rng.integers(0, vocab, requests).astype(np.int32)
    proposals[:, 0] = first
    for r in range(requests):
        matching = True
        for j in range(tokens - 1):
            want = int(arg[r, j])
            if matching and rng.random() < p:
                proposals[r, j + 1] = want
            else:
                matching = False
                other = int(rng.integers(0, vocab - 1))
                proposals[r, j + 1] = other if other < want else other + 1
    return logits, proposals, first


@pytest.mark.parametrize("vocab", [262144, 4096])
def test_argmax_accept_config1(dev, vocab):
    torch = dev
    rng = np.random.default_rng(100 + vocab)
    say(f"case: argmax+accept config1 vocab={vocab}")
    logits, proposals, first = planted_config1(rng, vocab=vocab)
    caps = rng.integers(-1, 7, 24).astype(np.int32)
    expect_pred = oracle.argmax_f32_rows_as_bf16(logits)
    for use_caps in (False, True):
        exp_acc, exp_next = oracle.greedy_accept(proposals, first, expect_pred.reshape(24, 5),
                                                 caps if use_caps else None)
        d_logits = to_dev(torch, logits)
        d_prop, d_first = to_dev(torch, proposals), to_dev(torch, first)
        d_caps = to_dev(torch, caps) if use_caps else None
        pred = torch.zeros(120, dtype=torch.int32, device="cuda")
        acc = torch.zeros(24, dtype=torch.int32, device="cuda")
        nxt = torch.zeros(24, dtype=torch.int32, device="cuda")
        for repeat in range(2):  # the kernel re-arms its keys/counters: a second call must agree
            _lib.check(_lib.lib().carat_hip_argmax_accept(
                _lib.ptr(d_logits), None, 24, 5, vocab, _lib.ptr(d_prop), _lib.ptr(d_first),
                _lib.ptr(d_caps), _lib.ptr(pred), _lib.ptr(acc), _lib.ptr(nxt),
                _lib.ptr(stream_of(torch))))
            torch.cuda.synchronize()
            assert np.array_equal(to_host(pred), expect_pred)
            assert np.array_equal(to_host(acc), exp_acc)
            assert np.array_equal(to_host(nxt), exp_next)


@pytest.mark.parametrize("requests,tokens,vocab", [(7, 3, 8192), (30, 8, 40000), (1, 1, 262144)])
def test_argmax_accept_shapes_in_sequence(dev, requests, tokens, vocab):
    """Request/token counts other than config 1's, bf16 and fp32 logits alternating, called
    three times each, with ragged last chunks (40000): the shared partial-key workspace leaves
    nothing behind that a later call of another shape could pick up."""
    torch = dev
    rng = np.random.default_rng(requests * 1000 + tokens)
    say(f"case: argmax+accept requests={requests} tokens={tokens} vocab={vocab}")
    logits, proposals, first = planted_config1(rng, requests, tokens, vocab)
    caps = rng.integers(-1, tokens + 2, requests).astype(np.int32)
    for f32 in (True, False, True):
        if f32:
            expect_pred = oracle.argmax_f32_rows_as_bf16(logits)
            d_f32, d_bf16 = to_dev(torch, logits), None
        else:
            bf = oracle.f32_to_bf16(logits)
            expect_pred = oracle.argmax_bf16_rows(bf)
            d_f32, d_bf16 = None, to_dev(torch, bf.view(np.int16))
        exp_acc, exp_next = oracle.greedy_accept(proposals, first,
                                                 expect_pred.reshape(requests, tokens), caps)
        d_prop, d_first, d_caps = to_dev(torch, proposals), to_dev(torch, first), to_dev(torch, caps)
        pred = torch.zeros(requests * tokens, dtype=torch.int32, device="cuda")
        acc = torch.zeros(requests, dtype=torch.int32, device="cuda")
        nxt = torch.zeros(requests, dtype=torch.int32, device="cuda")
        for repeat in range(3):
            _lib.check(_lib.lib().carat_hip_argmax_accept(
                _lib.ptr(d_f32), _lib.ptr(d_bf16), requests, tokens, vocab, _lib.ptr(d_prop),
                _lib.ptr(d_first), _lib.ptr(d_caps), _lib.ptr(pred), _lib.ptr(acc), _lib.ptr(nxt),
                _lib.ptr(stream_of(torch))))
            torch.cuda.synchronize()
            assert np.array_equal(to_host(pred), expect_pred), (f32, repeat)
            assert np.array_equal(to_host(acc), exp_acc), (f32, repeat)
            assert np.array_equal(to_host(nxt), exp_next), (f32, repeat)


def test_argmax_bf16_known_answer_and_specials(dev):
    torch = dev
    say("case: argmax bf16 KAT + special values")
    vals = np.full((3, 513), -2.0, np.float32)
    vals[0, 17] = 9.0
    vals[1, 0] = 4.0
    vals[1, 401] = 4.0
    vals[2, 512] = 7.0
    inf = np.float32(np.inf)
    specials = np.full((6, 513), -inf, np.float32)
    specials[1, :] = np.nan
    specials[1, 300] = 1.0
    specials[1, 400] = 1.0
    specials[2, :] = np.nan
    specials[3, :] = -0.0
    specials[3, 7] = 0.0
    specials[4, 9] = -5.0
    specials[5, 100] = inf
    specials[5, 200] = inf
    allv = np.concatenate([vals, specials]).astype(np.float32)
    pad = np.full((allv.shape[0], 520), -inf, np.float32)  # vocabulary multiple of 8
    pad[:, :513] = allv
    bf = oracle.f32_to_bf16(pad)
    expect = oracle.argmax_bf16_rows(bf)
    assert expect[:3].tolist() == [17, 0, 512]
    d = to_dev(torch, bf.view(np.int16))
    pred = torch.zeros(9, dtype=torch.int32, device="cuda")
    _lib.check(_lib.lib().carat_hip_argmax_accept(None, _lib.ptr(d), 9, 1, 520, None, None, None,
                                                 _lib.ptr(pred), None, None,
                                                 _lib.ptr(stream_of(torch))))
    torch.cuda.synchronize()
    assert to_host(pred).tolist() == expect.tolist()
    assert expect[3:].tolist() == [0, 300, 0, 0, 9, 100]


# ------------------------------------------------------------------ GEMMs
def rand_fp8(rng, shape, std=0.02):
    w = oracle.f32_to_bf16(rng.standard_normal(shape) * std)
    return oracle.quantize_e4m3(w)


def run_fp8_linear(torch, x_bf16, amax, qw, sw, epilogue, splits=1):
    m, k = x_bf16.shape
    n = qw.shape[0]
    d_x = to_dev(torch, x_bf16.view(np.int16))
    d_amax = to_dev(torch, np.array([amax], np.float32))
    d_w = to_dev(torch, qw)
    d_sw = to_dev(torch, np.array([sw], np.float32))
    y = torch.zeros((m, n // 2 if epilogue == 3 else n), dtype=torch.int16, device="cuda")
    y_amax = torch.zeros(1, dtype=torch.float32, device="cuda")
    part = torch.zeros((splits, m, n), dtype=torch.float32, device="cuda")
    pred = torch.zeros(m, dtype=torch.int32, device="cuda")
    _lib.check(_lib.lib().carat_hip_fp8_linear(
        _lib.ptr(d_x), m, k, _lib.ptr(d_amax), _lib.ptr(d_w), n, _lib.ptr(d_sw), epilogue, splits,
        _lib.ptr(y), _lib.ptr(y_amax), _lib.ptr(part), _lib.ptr(pred), _lib.ptr(stream_of(torch))))
    torch.cuda.synchronize()
    return (to_host(y).view(np.uint16), float(to_host(y_amax)[0]), to_host(part), to_host(pred))


# n selects the packed weight layout: 256/512 one tile per wave, 16384 four (the lm_head shape).
# m > 128 runs several 128-row token blocks (prefill steps): on the one-tile layouts a workgroup
# then takes four layout blocks.
@pytest.mark.parametrize("m,k,n", [(120, 5376, 256), (24, 1024, 512), (1, 256, 256), (192, 512, 256),
                                   (120, 1024, 16384), (300, 512, 256), (1024, 1024, 512),
                                   (300, 512, 16384)])
def test_fp8_linear_matches_oracle(dev, m, k, n):
    torch = dev
    rng = np.random.default_rng(m * 7 + k + n)
    say(f"case: fp8 linear m={m} k={k} n={n}")
    x = oracle.f32_to_bf16(rng.standard_normal((m, k)))
    amax = float(np.abs(oracle.bf16_to_f32(x)).max())
    qw, sw = rand_fp8(rng, (n, k))
    qx, sx = oracle.quantize_e4m3(x)
    ref32 = oracle.fp8_linear_f32(qx, sx, qw, sw).astype(np.float64)
    ref = oracle.f32_to_bf16(ref32)
    y, y_amax, _, _ = run_fp8_linear(torch, x, amax, qw, sw, 0)
    # fp32 accumulation order differs from the float64 oracle: <= 1 bf16 ulp of the value
    gf = oracle.bf16_to_f32(y).astype(np.float64)
    # atol: fp32 accumulation of K products (cancellation near zero), far below a bf16 ulp of max
    assert np.all(np.abs(gf - ref32) <= np.abs(ref32) * 2 ** -7 + 1e-3 * np.abs(ref32).max())
    assert y_amax == np.abs(gf).max()
    # split-K partial sums reproduce the same accumulation up to fp32 reassociation
    splits = 2
    _, _, part, _ = run_fp8_linear(torch, x, amax, qw, sw, 1, splits)
    summed = part.sum(0).astype(np.float64) * np.float32(sx * sw)
    # the fp8 MFMA's internal accumulation is not IEEE fp32 summation: agree to ~1e-5 of the scale
    assert np.allclose(summed, ref32, rtol=1e-3, atol=1e-4 * np.abs(ref32).max())


# 120 x 8192: one-tile layout, one token block; 1008 x 32768: four-tile layout with eight token
# blocks at two workgroups per CU (a prefill step whose prompt completes)
@pytest.mark.parametrize("m,k,n", [(120, 1024, 8192), (1008, 512, 32768)])
def test_fp8_lm_head_argmax_is_bit_exact_on_its_own_logits(dev, m, k, n):
    torch = dev
    rng = np.random.default_rng(21)
    say(f"case: fp8 lm_head argmax m={m} k={k} n={n}")
    x = oracle.f32_to_bf16(rng.standard_normal((m, k)))
    amax = float(np.abs(oracle.bf16_to_f32(x)).max())
    qw, sw = rand_fp8(rng, (n, k))
    logits, _, _, _ = run_fp8_linear(torch, x, amax, qw, sw, 0)
    _, _, _, pred = run_fp8_linear(torch, x, amax, qw, sw, 2)
    # "bit-exact given identical logits": the fused argmax equals the argmax of the same logits
    assert np.array_equal(pred, oracle.argmax_bf16_rows(logits))
    # and the logits match the oracle's lm_head within one bf16 ulp
    o_pred, o_logits = oracle.fp8_lm_head_argmax(x, qw, sw)
    o32 = oracle.bf16_to_f32(o_logits).astype(np.float64)
    g32 = oracle.bf16_to_f32(logits).astype(np.float64)
    assert np.all(np.abs(g32 - o32) <= np.abs(o32) * 2 ** -7 + 1e-3 * np.abs(o32).max())
    # against the oracle's own argmax, a mismatch is a near-tie (2 bf16 ulps of the row maximum)
    gap = o32.max(1) - o32[np.arange(len(pred)), pred]
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(o32).max(1))


# 256 and 8192: 4-wave blocks of two tiles per wave; 21504 (the verify shape): 3-wave blocks of
# four tiles per wave; at 1008 rows (a prefill step) eight token blocks, two workgroups per CU
@pytest.mark.parametrize("inter,m", [(256, 120), (8192, 120), (21504, 120), (21504, 1008)])
def test_fp8_gelu_gate_epilogue(dev, inter, m):
    torch = dev
    rng = np.random.default_rng(22)
    k = 512
    say(f"case: fp8 gate/up + GELU epilogue inter={inter} m={m}")
    x = oracle.f32_to_bf16(rng.standard_normal((m, k)))
    amax = float(np.abs(oracle.bf16_to_f32(x)).max())
    qw, sw = rand_fp8(rng, (2 * inter, k), 0.05)
    y, y_amax, _, _ = run_fp8_linear(torch, x, amax, qw, sw, 3)
    qx, sx = oracle.quantize_e4m3(x)
    packed = oracle.fp8_linear(qx, sx, qw, sw)
    ref, _ = oracle.gelu_tanh_gate_rows(packed)
    assert bf16_rel_err(y, ref) <= 2e-2
    assert y_amax == np.abs(oracle.bf16_to_f32(y)).max()


def test_bf16_linear_matches_float64(dev):
    torch = dev
    rng = np.random.default_rng(23)
    m, k, n = 24, 1024, 512
    say("case: bf16 linear")
    x = oracle.f32_to_bf16(rng.standard_normal((m, k)))
    w = oracle.f32_to_bf16(rng.standard_normal((n, k)) * 0.02)
    ref = oracle.bf16_to_f32(x).astype(np.float64) @ oracle.bf16_to_f32(w).astype(np.float64).T
    d_x, d_w = to_dev(torch, x.view(np.int16)), to_dev(torch, w.view(np.int16))
    y = torch.zeros((m, n), dtype=torch.int16, device="cuda")
    _lib.check(_lib.lib().carat_hip_bf16_linear(_lib.ptr(d_x), m, k, _lib.ptr(d_w), n, 0, 1,
                                               _lib.ptr(y), None, None, None,
                                               _lib.ptr(stream_of(torch))))
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(to_host(y).view(np.uint16)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2 ** -7 + 1e-3 * np.abs(ref).max())


# ------------------------------------------------------------------ attention
def attention_case(rng, mode, requests, tokens, hq, hkv, d, capacity, positions, fp8=False):
    slots = rng.permutation(requests).astype(np.int32)
    scale = 1 / math.sqrt(d)
    kc = oracle.f32_to_bf16(rng.standard_normal((requests, hkv, capacity, d), dtype=np.float32) * np.float32(scale))
    vc = oracle.f32_to_bf16(rng.standard_normal((requests, hkv, capacity, d), dtype=np.float32) * np.float32(scale))
    kn = oracle.f32_to_bf16(rng.standard_normal((requests, tokens, hkv, d), dtype=np.float32) * np.float32(scale))
    vn = oracle.f32_to_bf16(rng.standard_normal((requests, tokens, hkv, d), dtype=np.float32) * np.float32(scale))
    q = oracle.f32_to_bf16(rng.standard_normal((requests, tokens, hq, d), dtype=np.float32) * np.float32(scale))
    return slots, kc, vc, kn, vn, q


def run_attention(torch, mode, q, kc, vc, kn, vn, slots, positions, capacity, window, max_keys,
                  fp8=False, k_scale=1.0, v_scale=1.0, chunk=0):
    r, t, hq, d = q.shape
    hkv = kc.shape[1]
    as_dev = (lambda a: to_dev(torch, a)) if fp8 else (lambda a: to_dev(torch, a.view(np.int16)))
    d_q = to_dev(torch, q.view(np.int16))
    d_kc, d_vc, d_kn, d_vn = as_dev(kc), as_dev(vc), as_dev(kn), as_dev(vn)
    d_slots, d_pos = to_dev(torch, slots), to_dev(torch, positions.astype(np.int32))
    out = torch.zeros(q.shape, dtype=torch.int16, device="cuda")
    amax = torch.zeros(1, dtype=torch.float32, device="cuda")
    _lib.check(_lib.lib().carat_hip_verify_attention(
        mode, _lib.ptr(d_q), _lib.ptr(d_kc), _lib.ptr(d_vc), _lib.ptr(d_kn), _lib.ptr(d_vn),
        int(fp8), _lib.ctypes.c_float(k_scale), _lib.ctypes.c_float(v_scale), _lib.ptr(d_slots),
        _lib.ptr(d_pos), r, t, hq, hkv, d, capacity, window, max_keys, _lib.ptr(out),
        _lib.ptr(amax), chunk, _lib.ptr(stream_of(torch))))
    torch.cuda.synchronize()
    got = to_host(out).view(np.uint16)
    assert float(to_host(amax)[0]) == np.abs(oracle.bf16_to_f32(got)).max()
    return got


def attention_err(got, ref):
    g = oracle.bf16_to_f32(got).astype(np.float64)
    r = oracle.bf16_to_f32(ref).astype(np.float64)
    return np.abs(g - r).max() / np.abs(r).max()


@pytest.mark.parametrize("chunk", [0, 256])
def test_deep_prefill_step_attention(dev, chunk):
    """A forced (prefill) step of 200 rows per request: 400 query rows per kv head in 13 query
    tiles, each streaming only the keys its rows see (the causal triangle, the sliding band), over
    a wrapped ring, an unwrapped ring from position 0 and the global cache."""
    torch = dev
    rng = np.random.default_rng(71 + chunk)
    R, T, hq, hkv, d = 3, 200, 8, 4, 128
    say(f"case: deep sliding step T={T} chunk={chunk}")
    C = 256
    positions = np.array([0, 700, 37], np.int32)
    slots, kc, vc, kn, vn, q = attention_case(rng, 0, R, T, hq, hkv, d, C, positions)
    got = run_attention(torch, 0, q, kc, vc, kn, vn, slots, positions, C, C, C + T - 1, chunk=chunk)
    assert attention_err(got, oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, C, C)) <= 2e-2
    say(f"case: deeper sliding step T=300 chunk={chunk}")
    positions3 = np.array([0, 900, 41], np.int32)
    slots3, kc3, vc3, kn3, vn3, q3 = attention_case(rng, 0, R, 300, hq, hkv, d, 512, positions3)
    got = run_attention(torch, 0, q3, kc3, vc3, kn3, vn3, slots3, positions3, 512, 512, 512 + 299, chunk=chunk)
    assert attention_err(got, oracle.verify_attention(q3, kc3, vc3, kn3, vn3, slots3, positions3, 512, 512)) <= 2e-2
    say(f"case: deep global step T={T} chunk={chunk}")
    C = 1024
    positions = np.array([0, 600, 301], np.int32)
    slots, kc, vc, kn, vn, q = attention_case(rng, 1, R, T, hq, hkv, d, C, positions)
    got = run_attention(torch, 1, q, kc, vc, kn, vn, slots, positions, C, 0, C, chunk=chunk)
    assert attention_err(got, oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, C, 0)) <= 2e-2


# 0: one workgroup per pair; 256 / 512: five / three key chunks per pair and the merge
@pytest.mark.parametrize("chunk", [0, 256, 512])
def test_sliding_verify_attention_config2(dev, chunk):
    """Config 2: 24 slots, T=5, 32/16 heads x 128, ring 1024, contexts U[256, 8192] (mixed
    wrapped / unwrapped slots in one launch)."""
    torch = dev
    rng = np.random.default_rng(31 + chunk)
    R, T, hq, hkv, d, C = 24, 5, 32, 16, 128, 1024
    positions = rng.integers(256, 8192, R).astype(np.int32)
    positions[:3] = [256, 1019, 1020]  # unwrapped, boundary cases
    say(f"case: sliding attention config2 chunk={chunk} positions={positions[:6]}")
    slots, kc, vc, kn, vn, q = attention_case(rng, 0, R, T, hq, hkv, d, C, positions)
    got = run_attention(torch, 0, q, kc, vc, kn, vn, slots, positions, C, C, C + T - 1, chunk=chunk)
    ref = oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, C, C)
    err = attention_err(got, ref)
    say(f"  max err / max ref = {err:.3e}")
    assert err <= 2e-2
    ref_rounded = oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, C, C, True)
    assert attention_err(got, ref_rounded) <= 5e-2


def test_sliding_attention_reference_ring_fixture(dev):
    """cuda_ops_tests.cu:1630-1779 fixture (2 requests, 2/1 heads, ring 16, D 16 -> here D 128 is
    the smallest instantiated head_dim, so the fixture's values are tiled) checked against the
    reference's ring+backup formulation."""
    torch = dev
    say("case: reference ring fixture")
    for T in (4, 8):
        R, hq, hkv, C, d = 2, 2, 1, 16, 128
        positions = np.array([11 + 16, 13 + 16], np.int32)  # the fixture's ring is full
        qv = np.array([((i * 7) % 19 - 9) / 32.0 for i in range(R * hq * T * d)], np.float32)
        kv = np.array([((i * 5) % 23 - 11) / 48.0 for i in range(R * hkv * C * d)], np.float32)
        vv = np.array([((i * 11) % 29 - 14) / 24.0 for i in range(R * hkv * C * d)], np.float32)
        bk = np.array([((i * 13) % 17 - 8) / 40.0 for i in range(R * hkv * T * d)], np.float32)
        bv = np.array([((i * 3) % 31 - 15) / 20.0 for i in range(R * hkv * T * d)], np.float32)
        q_hm = oracle.f32_to_bf16(qv).reshape(R, hq, T, d)
        ring_k = oracle.f32_to_bf16(kv).reshape(R, hkv, C, d)
        ring_v = oracle.f32_to_bf16(vv).reshape(R, hkv, C, d)
        back_k = oracle.f32_to_bf16(bk).reshape(R, hkv, T, d)
        back_v = oracle.f32_to_bf16(bv).reshape(R, hkv, T, d)
        ref = oracle.ring_backup_attention(q_hm, ring_k, ring_v, back_k, back_v, positions, hkv, C)
        # this kernel's inputs: the ring before the write (backup rows restored) + new rows
        old_k, old_v = ring_k.copy(), ring_v.copy()
        new_k = np.empty((R, T, hkv, d), np.uint16)
        new_v = np.empty((R, T, hkv, d), np.uint16)
        for r in range(R):
            for t in range(T):
                phys = (positions[r] + t) % C
                new_k[r, t] = ring_k[r, :, phys]
                new_v[r, t] = ring_v[r, :, phys]
                old_k[r, :, phys] = back_k[r, :, t]
                old_v[r, :, phys] = back_v[r, :, t]
        got = run_attention(torch, 0, q_hm.transpose(0, 2, 1, 3).copy(), old_k, old_v, new_k, new_v,
                            np.arange(R, dtype=np.int32), positions, C, C, C + T - 1)
        g = oracle.bf16_to_f32(got).transpose(0, 2, 1, 3)
        assert np.abs(g - ref).max() <= 0.015  # the reference test's own tolerance


@pytest.mark.parametrize("fp8", [False, True])
def test_global_verify_attention_config3(dev, fp8):
    torch = dev
    rng = np.random.default_rng(41 + int(fp8))
    R, T, hq, hkv, d, C = 24, 5, 32, 16, 128, 8192
    positions = rng.integers(1024, 8192 - T, R).astype(np.int32)
    say(f"case: global attention config3 fp8={fp8}")
    slots, kc, vc, kn, vn, q = attention_case(rng, 1, R, T, hq, hkv, d, C, positions)
    if not fp8:
        got = run_attention(torch, 1, q, kc, vc, kn, vn, slots, positions, C, 0, C)
        ref = oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, C, 0)
    else:
        kf = oracle.bf16_to_f32(kc)
        vf = oracle.bf16_to_f32(vc)
        ks = float(np.abs(kf).max() / 448.0)
        vs = float(np.abs(vf).max() / 448.0)
        enc = lambda a, s: oracle.f32_to_e4m3((oracle.bf16_to_f32(a) / np.float32(s))).reshape(a.shape)
        qk, qv, qkn, qvn = enc(kc, ks), enc(vc, vs), enc(kn, ks), enc(vn, vs)
        got = run_attention(torch, 1, q, qk, qv, qkn, qvn, slots, positions, C, 0, C, fp8=True,
                            k_scale=ks, v_scale=vs)
        ref = oracle.verify_attention_fp8(q, qk, qv, qkn, qvn, ks, vs, slots, positions, C)
    err = attention_err(got, ref)
    say(f"  max err / max ref = {err:.3e}")
    assert err <= 2e-2


def test_decode_attention(dev):
    torch = dev
    rng = np.random.default_rng(51)
    B, hq, hkv, d = 24, 32, 16, 128
    for C in (1024, 8192):
        positions = rng.integers(0, 2 * C, B).astype(np.int32)
        positions[0] = 0
        say(f"case: decode attention C={C}")
        slots = rng.permutation(B).astype(np.int32)
        s = 1 / math.sqrt(d)
        kc = oracle.f32_to_bf16(rng.standard_normal((B, hkv, C, d), dtype=np.float32) * np.float32(s))
        vc = oracle.f32_to_bf16(rng.standard_normal((B, hkv, C, d), dtype=np.float32) * np.float32(s))
        q = oracle.f32_to_bf16(rng.standard_normal((B, 1, hq, d)) * s)
        dummy = np.zeros((B, 1, hkv, d), np.uint16)
        got = run_attention(torch, 2, q, kc, vc, dummy, dummy, slots, positions, C, 0, C)
        ref = oracle.decode_attention(q[:, 0], kc, vc, slots, positions, hkv, C)
        assert attention_err(got[:, 0], ref) <= 2e-2


# ------------------------------------------------------------------ row ops / QKV
# 600 rows runs the 512-thread variant used for prefill steps
@pytest.mark.parametrize("rows", [120, 600])
def test_row_op_chains_match_oracle(dev, rows):
    torch = dev
    rng = np.random.default_rng(61 + rows)
    width, splits = 5376, 3
    say("case: row kernel (embedding / partials / input chains)")
    lib = _lib.lib()
    f = lambda a: to_dev(torch, a.view(np.int16) if a.dtype == np.uint16 else a)
    w1 = oracle.f32_to_bf16(1 + 0.1 * rng.standard_normal(width))
    w2 = oracle.f32_to_bf16(1 + 0.1 * rng.standard_normal(width))
    res = oracle.f32_to_bf16(rng.standard_normal((rows, width)))
    scalar = oracle.f32_to_bf16(np.array([0.75], np.float32))
    part = rng.standard_normal((splits, rows, width)).astype(np.float32)
    amax_in, wsc = 3.5, 0.7
    d_w1, d_w2, d_res, d_scalar, d_part = f(w1), f(w2), f(res), f(scalar), f(part)
    d_amax_in = to_dev(torch, np.array([amax_in], np.float32))
    d_wsc = to_dev(torch, np.array([wsc], np.float32))
    v_out = torch.zeros((rows, width), dtype=torch.int16, device="cuda")
    r1 = torch.zeros_like(v_out)
    y = torch.zeros_like(v_out)
    y_amax = torch.zeros(1, dtype=torch.float32, device="cuda")
    a = _lib.RowArgs()
    a.source, a.rows, a.width, a.eps = 1, rows, width, 1e-6
    a.partials, a.splits, a.x_amax, a.w_scale = _lib.ptr(d_part).value, splits, _lib.ptr(d_amax_in).value, _lib.ptr(d_wsc).value
    a.v_out, a.w1, a.residual, a.scalar = _lib.ptr(v_out).value, _lib.ptr(d_w1).value, _lib.ptr(d_res).value, _lib.ptr(d_scalar).value
    a.r1_out, a.w2, a.y_out, a.y_amax = _lib.ptr(r1).value, _lib.ptr(d_w2).value, _lib.ptr(y).value, _lib.ptr(y_amax).value
    _lib.check(lib.carat_hip_row_op(_lib.ctypes.byref(a), _lib.ptr(stream_of(torch))))
    torch.cuda.synchronize()
    scale = np.float32(np.float32(amax_in) / np.float32(448.0)) * np.float32(wsc)
    v_ref = oracle.f32_to_bf16(part.sum(0, dtype=np.float32) * scale)
    got_v = to_host(v_out).view(np.uint16)
    assert np.abs(oracle.bf16_to_f32(got_v) - oracle.bf16_to_f32(v_ref)).max() <= 2 ** -7 * np.abs(oracle.bf16_to_f32(v_ref)).max()
    # downstream stages from the GPU's own v (so the check isolates the norm chain)
    r1_ref = oracle.rms_norm_add_scale(got_v, w1, res, int(scalar[0]))
    got_r1 = to_host(r1).view(np.uint16)
    got_y = to_host(y).view(np.uint16)
    ulp = lambda a, b: np.abs(a.astype(np.int32) - b.astype(np.int32)).max()
    # r1 = bf16(norm(v) w1 + residual) cancels; bound the error by the operands' magnitude
    vf = oracle.bf16_to_f32(got_v).astype(np.float64)
    inv = 1 / np.sqrt((vf ** 2).mean(1, keepdims=True) + 1e-6)
    operand = (np.abs(vf * inv * oracle.bf16_to_f32(w1)) + np.abs(oracle.bf16_to_f32(res))) * 0.75
    diff = np.abs(oracle.bf16_to_f32(got_r1).astype(np.float64) - oracle.bf16_to_f32(r1_ref))
    assert np.all(diff <= operand * 2 ** -6 + 1e-30)
    y_ref2, _ = oracle.rms_norm(got_r1, w2)
    assert ulp(got_y, y_ref2) <= 1
    assert float(to_host(y_amax)[0]) == np.abs(oracle.bf16_to_f32(got_y)).max()
    # embedding source + input norm
    vocab = 1000
    emb = oracle.f32_to_bf16(rng.standard_normal((vocab, width)))
    tokens = rng.integers(0, vocab, rows).astype(np.int32)
    d_emb, d_tok = f(emb), to_dev(torch, tokens)
    b = _lib.RowArgs()
    b.source, b.rows, b.width, b.eps = 0, rows, width, 1e-6
    b.embedding, b.tokens, b.vocabulary, b.embed_scale = _lib.ptr(d_emb).value, _lib.ptr(d_tok).value, vocab, math.sqrt(width)
    b.v_out, b.w2, b.y_out, b.y_amax = _lib.ptr(v_out).value, _lib.ptr(d_w2).value, _lib.ptr(y).value, None
    _lib.check(lib.carat_hip_row_op(_lib.ctypes.byref(b), _lib.ptr(stream_of(torch))))
    torch.cuda.synchronize()
    e_ref = oracle.embedding(emb, tokens, math.sqrt(width))
    assert np.array_equal(to_host(v_out).view(np.uint16), e_ref)
    n_ref, _ = oracle.rms_norm(e_ref, w2)
    assert ulp(to_host(y).view(np.uint16), n_ref) <= 1


@pytest.mark.parametrize("kv_heads,dim,keq", [(16, 128, False), (4, 512, True), (16, 256, False)])
def test_qkv_post_matches_oracle(dev, kv_heads, dim, keq):
    torch = dev
    rng = np.random.default_rng(71 + dim)
    R, T, hq = 6, 5, 32
    rows = R * T
    say(f"case: qkv post D={dim} kv={kv_heads} k_eq_v={keq}")
    width = hq * dim + kv_heads * dim * (1 if keq else 2)
    packed = oracle.f32_to_bf16(rng.standard_normal((rows, width)))
    qn = oracle.f32_to_bf16(1 + 0.1 * rng.standard_normal(dim))
    kn = oracle.f32_to_bf16(1 + 0.1 * rng.standard_normal(dim))
    positions = rng.integers(0, 1000, R).astype(np.int32)
    cos, sin = oracle.rope_table(dim, keq, 1100)
    rowpos = (positions[:, None] + np.arange(T)[None, :]).reshape(-1).astype(np.int32)
    q_ref, k_ref, v_ref = oracle.qkv_post(packed, qn, kn, cos, sin, rowpos, hq, kv_heads, dim, keq)
    f = lambda a: to_dev(torch, a.view(np.int16) if a.dtype == np.uint16 else a)
    q = torch.zeros((rows, hq, dim), dtype=torch.int16, device="cuda")
    k = torch.zeros((rows, kv_heads, dim), dtype=torch.int16, device="cuda")
    v = torch.zeros_like(k)
    # keep every device input alive until the kernel has run
    d_packed, d_qn, d_kn, d_cos, d_sin, d_pos = f(packed), f(qn), f(kn), f(cos), f(sin), f(positions)
    _lib.check(_lib.lib().carat_hip_qkv_post(
        _lib.ptr(d_packed), rows, T, hq, kv_heads, dim, int(keq), _lib.ctypes.c_float(1e-6),
        _lib.ptr(d_qn), _lib.ptr(d_kn), _lib.ptr(d_cos), _lib.ptr(d_sin),
        _lib.ptr(d_pos), None, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), None, None, 0,
        _lib.ptr(stream_of(torch))))
    torch.cuda.synchronize()
    def close(got, ref):
        # norm + RoPE rounding points as the reference; rsqrt and summation order differ, and
        # n*cos + rot*sin cancels: 1/64 relative plus a floor at 1/1024 of the row rms
        g = oracle.bf16_to_f32(got.view(np.uint16)).astype(np.float64)
        r = oracle.bf16_to_f32(ref).astype(np.float64)
        rms = np.sqrt((r ** 2).mean(-1, keepdims=True))
        return np.all(np.abs(g - r) <= np.abs(r) * 2 ** -6 + rms * 2 ** -10)
    assert close(to_host(q), q_ref)
    assert close(to_host(k), k_ref)
    assert close(to_host(v), v_ref)


@pytest.mark.parametrize("chunk", [0, 256])
def test_native_gemma4_attention_shapes(dev, chunk):
    """Native Gemma-4 shapes (gemma4_config.cpp:174-203): sliding D 256 with 32/16 heads; global
    D 512 with 32/4 heads -- 40 query rows per kv head, all in one workgroup whose four waves
    split D -- with and without key chunks (and the same D-split kernel over a wrapped sliding
    ring); the assistant's D 512 decode."""
    torch = dev
    rng = np.random.default_rng(61 + chunk)
    R, T = 6, 5
    say(f"case: native sliding D=256 chunk={chunk}")
    C = 1024
    positions = rng.integers(256, 3000, R).astype(np.int32)
    slots, kc, vc, kn, vn, q = attention_case(rng, 0, R, T, 32, 16, 256, C, positions)
    got = run_attention(torch, 0, q, kc, vc, kn, vn, slots, positions, C, C, C + T - 1, chunk=chunk)
    assert attention_err(got, oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, C, C)) <= 2e-2
    say(f"case: native global D=512 (40 query rows) chunk={chunk}")
    C = 1536
    positions = rng.integers(300, C - T, R).astype(np.int32)
    slots, kc, vc, kn, vn, q = attention_case(rng, 1, R, T, 32, 4, 512, C, positions)
    got = run_attention(torch, 1, q, kc, vc, kn, vn, slots, positions, C, 0, C, chunk=chunk)
    assert attention_err(got, oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, C, 0)) <= 2e-2
    say(f"case: sliding ring at D=512 with 40 query rows chunk={chunk}")
    C = 1024
    positions = rng.integers(256, 3000, R).astype(np.int32)
    slots, kc, vc, kn, vn, q = attention_case(rng, 0, R, T, 32, 4, 512, C, positions)
    got = run_attention(torch, 0, q, kc, vc, kn, vn, slots, positions, C, C, C + T - 1, chunk=chunk)
    assert attention_err(got, oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, C, C)) <= 2e-2
    say(f"case: native decode D=512 chunk={chunk}")
    B, d = 6, 512
    s = 1 / math.sqrt(d)
    kc = oracle.f32_to_bf16(rng.standard_normal((B, 4, C, d), dtype=np.float32) * np.float32(s))
    vc = oracle.f32_to_bf16(rng.standard_normal((B, 4, C, d), dtype=np.float32) * np.float32(s))
    q = oracle.f32_to_bf16(rng.standard_normal((B, 1, 32, d)) * s)
    positions = rng.integers(0, C, B).astype(np.int32)
    slots = rng.permutation(B).astype(np.int32)
    dummy = np.zeros((B, 1, 4, d), np.uint16)
    got = run_attention(torch, 2, q, kc, vc, dummy, dummy, slots, positions, C, 0, C, chunk=chunk)
    assert attention_err(got[:, 0], oracle.decode_attention(q[:, 0], kc, vc, slots, positions, 4, C)) <= 2e-2


def random_attention_cases(seed, count):
    """Seeded random verify / decode attention configurations: mode, heads per kv head, head
    dimension, ring capacity and window, tokens per request, positions (0, just below and past a
    wrap, random), request count, key chunking and, for global layers, e4m3 K/V."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        mode = int(rng.choice([0, 1, 2]))
        d = int(rng.choice([128, 128, 256, 512] if mode == 1 else [128, 128, 256]))
        hkv = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 2, 4, 8]))
        requests = int(rng.integers(1, 5))
        tokens = 1 if mode == 2 else int(rng.choice([1, 2, 5, 8, 17, 40]))
        if mode == 0:
            capacity = int(rng.choice([64, 256, 1024]))
            window = int(rng.choice([capacity, max(16, capacity // 2)]))
            tokens = min(tokens, capacity)
            positions = rng.integers(0, 3 * capacity, requests)
            positions[0] = int(rng.choice([0, capacity - 1, capacity, window - 1]))
        elif mode == 1:
            capacity = int(rng.choice([256, 1024, 2048]))
            window = 0
            positions = rng.integers(0, capacity - tokens + 1, requests)
            positions[0] = int(rng.choice([0, capacity - tokens]))
        else:
            capacity = int(rng.choice([256, 1024]))
            window = 0
            positions = rng.integers(0, 2 * capacity, requests)
        fp8 = mode == 1 and d == 128 and bool(rng.integers(0, 2))
        chunk = int(rng.choice([0, 256]))
        cases.append((i, mode, d, hkv, group, requests, tokens, capacity, window,
                      positions.astype(np.int32), fp8, chunk))
    return cases


@pytest.mark.parametrize("seed", [101, 202])
def test_attention_random_shapes(dev, seed):
    """Twenty seeded random configurations per seed through the op-level entry point against the
    oracle (max |err| <= 2e-2 * max |ref|): sliding rings with windows at and below their
    capacity, positions at 0 and around a wrap, 1-40 tokens per request, 1-8 query heads per kv
    head, D 128/256/512, single and split key ranges, bf16 and e4m3 K/V."""
    torch = dev
    for (i, mode, d, hkv, group, requests, tokens, capacity, window, positions, fp8,
         chunk) in random_attention_cases(seed, 20):
        hq = hkv * group
        rng = np.random.default_rng(seed * 1000 + i)
        say(f"case: seed {seed} #{i} mode={mode} D={d} heads={hq}/{hkv} R={requests} T={tokens} "
            f"C={capacity} window={window} positions={positions.tolist()} fp8={fp8} chunk={chunk}")
        slots, kc, vc, kn, vn, q = attention_case(rng, mode, requests, tokens, hq, hkv, d, capacity,
                                                  positions)
        if mode == 0:
            got = run_attention(torch, 0, q, kc, vc, kn, vn, slots, positions, capacity, window,
                                window + tokens - 1, chunk=chunk)
            ref = oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, capacity, window)
        elif mode == 1 and fp8:
            ks = float(np.abs(oracle.bf16_to_f32(kc)).max() / 448.0)
            vs = float(np.abs(oracle.bf16_to_f32(vc)).max() / 448.0)
            enc = lambda a, s: oracle.f32_to_e4m3(oracle.bf16_to_f32(a) / np.float32(s)).reshape(a.shape)
            qk, qv, qkn, qvn = enc(kc, ks), enc(vc, vs), enc(kn, ks), enc(vn, vs)
            got = run_attention(torch, 1, q, qk, qv, qkn, qvn, slots, positions, capacity, 0, capacity,
                                fp8=True, k_scale=ks, v_scale=vs, chunk=chunk)
            ref = oracle.verify_attention_fp8(q, qk, qv, qkn, qvn, ks, vs, slots, positions, capacity)
        elif mode == 1:
            got = run_attention(torch, 1, q, kc, vc, kn, vn, slots, positions, capacity, 0, capacity,
                                chunk=chunk)
            ref = oracle.verify_attention(q, kc, vc, kn, vn, slots, positions, capacity, 0)
        else:
            dummy = np.zeros((requests, 1, hkv, d), np.uint16)
            got = run_attention(torch, 2, q, kc, vc, dummy, dummy, slots, positions, capacity, 0,
                                capacity, chunk=chunk)[:, 0]
            ref = oracle.decode_attention(q[:, 0], kc, vc, slots, positions, hkv, capacity)
        err = attention_err(got, ref)
        say(f"  max err / max ref = {err:.3e}")
        assert err <= 2e-2, i


def random_gemm_cases(seed, count):
    """Seeded random fp8 GEMM calls: rows around the token-block edges (1-32 rows take two-tile
    blocks, up to 128 one block, more several), K from one 128-byte step to 16, feature counts
    that select the one-, two- and four-tile layouts, and every epilogue (bf16 store with amax,
    split-K partials, GELU gate, argmax)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        epilogue = int(rng.choice([0, 1, 3, 2]))
        m = int(rng.choice([1, 3, 16, 31, 32, 33, 100, 120, 128, 129, 200, 300]))
        k = int(rng.choice([128, 384, 1024, 2048]))
        if epilogue == 3:
            n = int(rng.choice([128, 256, 1024, 8192, 16384]))
        else:
            n = int(rng.choice([64, 192, 320, 512, 1024, 8192, 16384]))
        while m * n * k > 2_000_000_000:  # keep the float64 oracle quick
            n //= 2
        steps = k // 128
        splits = int(rng.choice([s for s in (1, 2, 3, 4) if steps % s == 0])) if epilogue == 1 else 1
        cases.append((i, epilogue, m, k, n, splits))
    return cases


@pytest.mark.parametrize("seed", [303, 404])
def test_fp8_gemm_random_shapes(dev, seed):
    """Sixteen seeded random fp8 GEMM calls per seed through the op-level entry point against the
    oracle's float64 GEMM over the same e4m3 bytes: bf16 outputs within one bf16 ulp (plus 1e-3
    of the maximum), split-K partials within fp32 reassociation, the GELU gate within 2e-2, and
    the fused argmax bit-exact on the kernel's own logits and a near-tie of the oracle's."""
    torch = dev
    for i, epilogue, m, k, n, splits in random_gemm_cases(seed, 16):
        rng = np.random.default_rng(seed * 1000 + i)
        say(f"case: seed {seed} #{i} epilogue={epilogue} m={m} k={k} n={n} splits={splits}")
        x = oracle.f32_to_bf16(rng.standard_normal((m, k)))
        amax = float(np.abs(oracle.bf16_to_f32(x)).max())
        qw, sw = rand_fp8(rng, (n, k), 0.05 if epilogue == 3 else 0.02)
        qx, sx = oracle.quantize_e4m3(x)
        if epilogue == 3:
            y, y_amax, _, _ = run_fp8_linear(torch, x, amax, qw, sw, 3)
            ref, _ = oracle.gelu_tanh_gate_rows(oracle.fp8_linear(qx, sx, qw, sw))
            assert bf16_rel_err(y, ref) <= 2e-2, i
            assert y_amax == np.abs(oracle.bf16_to_f32(y)).max(), i
            continue
        ref32 = oracle.fp8_linear_f32(qx, sx, qw, sw).astype(np.float64)
        if epilogue == 1:
            _, _, part, _ = run_fp8_linear(torch, x, amax, qw, sw, 1, splits)
            summed = part.sum(0).astype(np.float64) * np.float32(sx * sw)
            assert np.allclose(summed, ref32, rtol=1e-3, atol=1e-4 * np.abs(ref32).max()), i
            continue
        y, y_amax, _, _ = run_fp8_linear(torch, x, amax, qw, sw, 0)
        gf = oracle.bf16_to_f32(y).astype(np.float64)
        assert np.all(np.abs(gf - ref32) <= np.abs(ref32) * 2 ** -7 + 1e-3 * np.abs(ref32).max()), i
        assert y_amax == np.abs(gf).max(), i
        if epilogue == 2:
            _, _, _, pred = run_fp8_linear(torch, x, amax, qw, sw, 2)
            assert np.array_equal(pred, oracle.argmax_bf16_rows(y)), i
            gap = ref32.max(1) - ref32[np.arange(m), pred]
            assert np.all(gap <= 2 * 2 ** -7 * np.abs(ref32).max(1)), i
