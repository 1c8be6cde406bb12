"""Fp8Scaling::channel and ::block_128 on the GPU (include/carat/linear.h:27): the weight arena's
quantisation (Fp8WeightArena::quantize, device_weights.cu:222-256), the scaled projections
(run_decode_linear + Fp8Linear::run, layer_runner.cu:220-238, linear.cu:300-420, 706-717) and a
verify step of a runner built on channel / block-scaled weights, against the oracle.

Bars: e4m3 codes and scales bit-exact; GEMM outputs within one bf16 ulp of the float64-accumulated
oracle plus 1e-3 of the output's maximum (fp32 accumulation order); argmax bit-exact on the GPU's
own logits and a near-tie (2 bf16 ulps of the row maximum) against the oracle's.
"""
import math
import sys

import numpy as np
import pytest

from carat_amd import _lib
from carat_amd.runner import BatchModelRunner, LayerSpec, ModelDesc
from oracle import oracle
from tests.runner_oracle import verify_step

pytestmark = pytest.mark.gpu

SCALINGS = {"channel": 1, "block_128": 2}


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def stream_of(torch):
    return _lib.ptr(torch.cuda.current_stream().cuda_stream)


def quantize_on_gpu(torch, w_bf16, scaling):
    n, k = w_bf16.shape
    count = _lib.ctypes.c_uint64()
    _lib.check(_lib.lib().carat_hip_fp8_weight_scale_elements(scaling, n, k, _lib.ctypes.byref(count)))
    d_w = to_dev(torch, w_bf16.view(np.int16))
    q = torch.zeros((n, k), dtype=torch.uint8, device="cuda")
    s = torch.full((count.value,), -1.0, dtype=torch.float32, device="cuda")
    _lib.check(_lib.lib().carat_hip_quantize_weight_fp8(_lib.ptr(d_w), n, k, scaling, _lib.ptr(q),
                                                        _lib.ptr(s), stream_of(torch)))
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


@pytest.mark.parametrize("scaling", [0, 1, 2], ids=["tensor", "channel", "block_128"])
@pytest.mark.parametrize("n,k", [(200, 300), (1024, 5376), (37, 129)])
def test_weight_quantisation_is_bit_exact(torch_cuda, scaling, n, k):
    rng = np.random.default_rng(n + k + scaling)
    say(f"case: weight quantisation scaling={scaling} n={n} k={k}")
    w = oracle.f32_to_bf16(rng.standard_normal((n, k)) * 0.02 * np.exp(rng.uniform(-3, 3, (n, 1))))
    if scaling == 1:
        w[n // 2] = 0  # a zero row takes the 2^-24 floor
    q, s = quantize_on_gpu(torch_cuda, w, scaling)
    eq, es = oracle.quantize_weight_scaled(w, scaling)
    assert np.array_equal(s, es)  # includes the zeroed padding of the block scales
    assert np.array_equal(q, eq)


def run_scaled_linear(torch, x_bf16, qw, sw, scaling, epilogue, splits=1):
    m, k = x_bf16.shape
    n = qw.shape[0]
    d_x = to_dev(torch, x_bf16.view(np.int16))
    d_w, d_s = to_dev(torch, qw), to_dev(torch, sw)
    y = torch.zeros((m, n // 2 if epilogue == 3 else n), dtype=torch.int16, device="cuda")
    part = torch.zeros((splits, m, n), dtype=torch.float32, device="cuda")
    pred = torch.zeros(m, dtype=torch.int32, device="cuda")
    _lib.check(_lib.lib().carat_hip_fp8_linear_scaled(
        _lib.ptr(d_x), m, k, scaling, _lib.ptr(d_w), n, _lib.ptr(d_s), epilogue, splits, _lib.ptr(y),
        _lib.ptr(part), _lib.ptr(pred), stream_of(torch)))
    torch.cuda.synchronize()
    return y.cpu().numpy().view(np.uint16), part.cpu().numpy(), pred.cpu().numpy()


def scaled_inputs(rng, m, k, n, scaling, rows_spread=2.0):
    # rows (and weight rows) of different magnitudes, so a misapplied scale shows
    x = oracle.f32_to_bf16(rng.standard_normal((m, k)) * np.exp(rng.uniform(-rows_spread, rows_spread, (m, 1))))
    w = oracle.f32_to_bf16(rng.standard_normal((n, k)) * 0.02 * np.exp(rng.uniform(-2, 2, (n, 1))))
    qw, sw = oracle.quantize_weight_scaled(w, scaling)
    qx, sx = oracle.quantize_activation_scaled(x, scaling)
    ref32 = oracle.fp8_linear_scaled(qx, sx, qw, sw, scaling, f32=True).astype(np.float64)
    return x, qw, sw, ref32


# the runner's layouts: one tile per wave (256, 512), four (16384, the lm_head's); m > 128 runs
# several token blocks (four layout blocks per workgroup on the one-tile layouts)
@pytest.mark.parametrize("scaling", [1, 2], ids=["channel", "block_128"])
@pytest.mark.parametrize("m,k,n", [(120, 5376, 256), (24, 1024, 512), (1, 256, 256), (300, 512, 256),
                                   (120, 1024, 16384)])
def test_scaled_fp8_linear_matches_oracle(torch_cuda, scaling, m, k, n):
    rng = np.random.default_rng(m * 5 + k + n + scaling)
    say(f"case: scaled fp8 linear scaling={scaling} m={m} k={k} n={n}")
    x, qw, sw, ref32 = scaled_inputs(rng, m, k, n, scaling)
    y, _, _ = run_scaled_linear(torch_cuda, x, qw, sw, scaling, 0)
    got = oracle.bf16_to_f32(y).astype(np.float64)
    assert np.all(np.abs(got - ref32) <= np.abs(ref32) * 2 ** -7 + 1e-3 * np.abs(ref32).max())
    # split-K partials carry the full scale: their sum is the output before rounding
    _, part, _ = run_scaled_linear(torch_cuda, x, qw, sw, scaling, 1, 2)
    summed = part.sum(0).astype(np.float64)
    assert np.allclose(summed, ref32, rtol=1e-3, atol=1e-4 * np.abs(ref32).max())


@pytest.mark.parametrize("scaling", [1, 2], ids=["channel", "block_128"])
@pytest.mark.parametrize("m,n", [(120, 8192), (1008, 32768)])
def test_scaled_lm_head_argmax(torch_cuda, scaling, m, n):
    rng = np.random.default_rng(m + n + scaling)
    k = 1024
    say(f"case: scaled fp8 lm_head argmax scaling={scaling} m={m} n={n}")
    x, qw, sw, ref32 = scaled_inputs(rng, m, k, n, scaling, rows_spread=1.0)
    logits, _, _ = run_scaled_linear(torch_cuda, x, qw, sw, scaling, 0)
    _, _, pred = run_scaled_linear(torch_cuda, x, qw, sw, scaling, 2)
    assert np.array_equal(pred, oracle.argmax_bf16_rows(logits))
    o32 = oracle.bf16_to_f32(oracle.f32_to_bf16(ref32)).astype(np.float64)
    gap = o32.max(1) - o32[np.arange(m), pred]
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(o32).max(1))


@pytest.mark.parametrize("scaling", [1, 2], ids=["channel", "block_128"])
@pytest.mark.parametrize("inter,m", [(256, 120), (21504, 120), (21504, 1008)])
def test_scaled_gelu_gate_epilogue(torch_cuda, scaling, inter, m):
    rng = np.random.default_rng(inter + m + scaling)
    k = 512
    say(f"case: scaled gate/up + GELU scaling={scaling} inter={inter} m={m}")
    x, qw, sw, ref32 = scaled_inputs(rng, m, k, 2 * inter, scaling, rows_spread=1.0)
    y, _, _ = run_scaled_linear(torch_cuda, x, qw, sw, scaling, 3)
    ref, _ = oracle.gelu_tanh_gate_rows(oracle.f32_to_bf16(ref32))
    g = oracle.bf16_to_f32(y).astype(np.float64)
    r = oracle.bf16_to_f32(ref).astype(np.float64)
    # per row: the rows' magnitudes differ by design
    err = np.abs(g - r).max(1) / np.maximum(np.abs(r).max(1), 1e-30)
    assert err.max() <= 2e-2


# ------------------------------------------------------------------ runner
BATCH = 4
MAX_CONTEXT = 128


def tiny_desc(scaling):
    layers = [LayerSpec(True, 4, 2, 128), LayerSpec(True, 4, 2, 128), LayerSpec(False, 4, 2, 128)]
    return ModelDesc(hidden=256, intermediate=512, vocabulary=2048, sliding_window=32, layers=layers,
                     seed=7, weight_std=0.05, fp8_scaling=scaling)


@pytest.mark.parametrize("scaling", ["channel", "block_128"])
def test_runner_weights_carry_the_arena_scales(torch_cuda, scaling):
    """The runner's own weights: its e4m3 bytes and scale tables are the quantisation of a bf16
    weight, i.e. dequantising reproduces a tensor whose re-quantisation gives the same bytes."""
    desc = tiny_desc(scaling)
    say(f"case: scaled runner weights {scaling}")
    runner = BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    try:
        mode = SCALINGS[scaling]
        for name, n, k in (("layer.0.qkv", 4 * 128 + 2 * 2 * 128, 256), ("layer.2.down", 256, 512),
                           ("token_embedding", 2048, 256)):
            q = runner.read(name + (".fp8" if name == "token_embedding" else ""), np.uint8).reshape(n, k)
            s = runner.read(name + ".scale_table", np.float32)
            count = _lib.ctypes.c_uint64()
            _lib.check(_lib.lib().carat_hip_fp8_weight_scale_elements(mode, n, k, _lib.ctypes.byref(count)))
            assert s.size == count.value
            if mode == 1:
                per = s.astype(np.float64)[:, None]
            else:
                kbp = s.size // ((n + 127) // 128)
                per = np.repeat(np.repeat(s.reshape(-1, kbp)[:, : (k + 127) // 128].astype(np.float64), 128, 0),
                                128, 1)[:n, :k]
            # every row / block holds a code of magnitude 448 (its maximum) and nothing above
            mag = oracle.e4m3_table()[q & 0x7F]
            if mode == 1:
                assert np.all(mag.max(1) == 448.0), name
            deq = oracle.e4m3_table().astype(np.float64)[q] * per
            rq, rs = oracle.quantize_weight_scaled(oracle.f32_to_bf16(deq), mode)
            assert np.array_equal(rq, q), name
    finally:
        runner.close()


@pytest.mark.parametrize("scaling", ["channel", "block_128"])
def test_scaled_verify_step_matches_oracle(torch_cuda, scaling):
    desc = tiny_desc(scaling)
    say(f"case: scaled runner verify {scaling}")
    runner = BatchModelRunner(desc, BATCH, MAX_CONTEXT)
    try:
        positions_by_slot = [40, 100, 20, 31]
        runner.seed_random_cache(max(positions_by_slot), seed=13, stddev=1 / math.sqrt(128))
        for slot, p in enumerate(positions_by_slot):
            runner.set_slot_position(slot, p)
        slots = [2, 0, 3, 1]
        positions = np.array([positions_by_slot[s] for s in slots], np.int32)
        T = 5
        rng = np.random.default_rng(9)
        proposals = rng.integers(0, desc.vocabulary, (4, T)).astype(np.int32)
        first = rng.integers(0, desc.vocabulary, 4).astype(np.int32)
        capacity_of = lambda li: min(MAX_CONTEXT, desc.sliding_window) if desc.layers[li].sliding else MAX_CONTEXT
        expect = verify_step(runner, desc, BATCH, capacity_of, proposals, slots, positions)
        res = runner.verify_greedy_proposals(proposals.tolist(), first.tolist(), slots, [0] * 4)
        assert res.accepted_tokens == [0] * 4
        pred = np.array(runner.last_predictions, np.int32).reshape(4 * T)
        logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(4 * T, -1)
        gap = logits.max(1) - logits[np.arange(4 * T), pred]
        mism = int(np.sum(pred != expect["predictions"]))
        say(f"  argmax mismatches vs oracle {mism}/{4 * T}, max gap {gap.max():.3e}")
        assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
        assert mism <= 2
        for li in range(len(desc.layers)):
            got_k = runner.read(f"new.{li}.k", np.uint16)[: 4 * T * 2 * 128].reshape(4, T, 2, 128)
            ek = oracle.bf16_to_f32(expect["k_new"][li])
            err = np.abs(oracle.bf16_to_f32(got_k) - ek).max()
            assert err <= 3e-2 * np.abs(ek).max(), (li, err)
        hid = oracle.bf16_to_f32(runner.read("final_hidden", np.uint16)[: 4 * T * desc.hidden]
                                 .reshape(4 * T, desc.hidden)).astype(np.float64)
        want = oracle.bf16_to_f32(expect["final_hidden"]).astype(np.float64)
        assert np.abs(hid - want).max() <= 3e-2 * np.abs(want).max()
    finally:
        runner.close()
