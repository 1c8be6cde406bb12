"""The runner over a Gemma-4-format checkpoint (DeviceWeightArena::load + Fp8WeightArena::quantize,
cuda/device_weights.cu:125-263, over WeightPlan::gemma4 / gemma4_assistant), at D 128 shapes and
at the native geometry (sliding D 256, global D 512 with one kv head and K = V): every execution
weight read back from the device equals the checkpoint bytes (bf16) or the oracle's per-tensor
e4m3 quantisation of them, bit for bit, and a verify step over the loaded weights matches the
oracle composition of the same step."""
import math
import sys

import numpy as np
import pytest

from carat_amd.runner import BatchModelRunner
from oracle import oracle
from tests import checkpoint_fixture as fx
from tests.runner_oracle import verify_step

pytestmark = pytest.mark.gpu

BATCH = 4
MAX_CONTEXT = 128


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", params=[False, True], ids=["d128", "native"])
def loaded(torch_cuda, tmp_path_factory, request):
    root = tmp_path_factory.mktemp("ckpt")
    model, a_dir, cfg, tensors, a_tensors = fx.tiny_checkpoint(root, shards=2, k_eq_v=True,
                                                               native=request.param)
    say(f"case: runner from a 2-shard checkpoint with an assistant (native={request.param})")
    runner = BatchModelRunner.from_checkpoint(str(model), BATCH, MAX_CONTEXT, str(a_dir))
    yield runner, cfg, tensors, a_tensors
    runner.close()


def test_loaded_weights_are_the_checkpoint_bytes(loaded):
    runner, cfg, tensors, a_tensors = loaded
    t = cfg["text_config"]
    H = t["hidden_size"]
    emb = tensors["model.language_model.embed_tokens.weight"]
    assert np.array_equal(runner.read("token_embedding", np.uint16).reshape(emb.shape), emb)
    q, s = oracle.quantize_e4m3(emb)
    assert np.array_equal(runner.read("token_embedding.fp8", np.uint8).reshape(emb.shape), q)
    assert runner.read("token_embedding.scale", np.float32)[0] == np.float32(s)
    assert np.array_equal(runner.read("final_norm", np.uint16), tensors["model.language_model.norm.weight"])
    for li, kind in enumerate(t["layer_types"]):
        p = f"model.language_model.layers.{li}."
        parts = [tensors[p + "self_attn.q_proj.weight"], tensors[p + "self_attn.k_proj.weight"]]
        if kind == "sliding_attention":
            parts.append(tensors[p + "self_attn.v_proj.weight"])
        mats = {"qkv": np.concatenate(parts),
                "o": tensors[p + "self_attn.o_proj.weight"],
                "gate_up": np.concatenate([tensors[p + "mlp.gate_proj.weight"],
                                           tensors[p + "mlp.up_proj.weight"]]),
                "down": tensors[p + "mlp.down_proj.weight"]}
        scales = runner.read(f"layer.{li}.scales", np.float32)
        for j, (name, m) in enumerate(mats.items()):
            q, s = oracle.quantize_e4m3(m)
            got = runner.read(f"layer.{li}.{name}", np.uint8).reshape(m.shape)
            assert np.array_equal(got, q), (li, name)
            assert scales[j] == np.float32(s), (li, name)
        norms = {"input_norm": "input_layernorm.weight", "q_norm": "self_attn.q_norm.weight",
                 "k_norm": "self_attn.k_norm.weight",
                 "post_attention_norm": "post_attention_layernorm.weight",
                 "pre_mlp_norm": "pre_feedforward_layernorm.weight",
                 "post_mlp_norm": "post_feedforward_layernorm.weight", "scalar": "layer_scalar"}
        for name, src in norms.items():
            assert np.array_equal(runner.read(f"layer.{li}.{name}", np.uint16), tensors[p + src]), (li, name)
    # assistant: bf16 weights packed for the GEMM, read back in logical order
    checks = {"assistant.token_embedding": "model.embed_tokens.weight",
              "assistant.pre_projection": "pre_projection.weight",
              "assistant.post_projection": "post_projection.weight",
              "assistant.final_norm": "model.norm.weight"}
    for li in range(2):
        p = f"model.layers.{li}."
        checks.update({f"assistant.layer.{li}.q": p + "self_attn.q_proj.weight",
                       f"assistant.layer.{li}.o": p + "self_attn.o_proj.weight",
                       f"assistant.layer.{li}.down": p + "mlp.down_proj.weight",
                       f"assistant.layer.{li}.q_norm": p + "self_attn.q_norm.weight",
                       f"assistant.layer.{li}.scalar": p + "layer_scalar"})
        gate_up = np.concatenate([a_tensors[p + "mlp.gate_proj.weight"], a_tensors[p + "mlp.up_proj.weight"]])
        assert np.array_equal(runner.read(f"assistant.layer.{li}.gate_up", np.uint16).reshape(gate_up.shape),
                              gate_up), li
    for name, src in checks.items():
        want = a_tensors[src]
        assert np.array_equal(runner.read(name, np.uint16).reshape(want.shape), want), name


def test_verify_step_over_checkpoint_weights(loaded):
    runner, cfg, tensors, _ = loaded
    desc = runner._desc
    T = 5
    runner.seed_random_cache(60, seed=21, stddev=1 / math.sqrt(128))
    positions_by_slot = [40, 60, 20, 31]
    for slot, pos in enumerate(positions_by_slot):
        runner.set_slot_position(slot, pos)
    slots = [1, 3, 0, 2]
    positions = np.array([positions_by_slot[s] for s in slots], np.int32)
    rng = np.random.default_rng(8)
    proposals = rng.integers(0, desc.vocabulary, (4, T)).astype(np.int32)
    first = proposals[:, 0].copy()
    capacity = lambda li: min(MAX_CONTEXT, desc.sliding_window) if desc.layers[li].sliding else MAX_CONTEXT
    expect = verify_step(runner, desc, BATCH, capacity, proposals, slots, positions)
    say("case: verify over checkpoint weights (dry)")
    res = runner.verify_greedy_proposals(proposals.tolist(), first.tolist(), slots, [0] * 4)
    assert res.accepted_tokens == [0] * 4
    pred = np.array(runner.last_predictions, np.int32)
    logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(4 * T, -1)
    gap = logits.max(1) - logits[np.arange(4 * T), pred]
    mism = int(np.sum(pred != expect["predictions"]))
    say(f"  argmax mismatches vs oracle {mism}/{4 * T}, max gap {gap.max():.3e}")
    # a mismatch is a near-tie: within 2 bf16 ulps of the row maximum
    assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    assert mism <= max(1, 4 * T // 10)
    drafts = runner.draft_four(first.tolist(), slots, first.tolist(), 4)
    assert [row[0] for row in drafts] == first.tolist()


def plan_segments(cfg, tensors, a_tensors):
    """Execution segments of the reference's WeightPlan::gemma4 / gemma4_assistant
    (weight_plan.cpp:37-127) built from the checkpoint tensors: {(assistant, name): bf16 array}."""
    t = cfg["text_config"]
    out = {(False, "token_embedding"): tensors["model.language_model.embed_tokens.weight"],
           (False, "final_norm"): tensors["model.language_model.norm.weight"]}
    single = {"input_norm": "input_layernorm.weight", "q_norm": "self_attn.q_norm.weight",
              "k_norm": "self_attn.k_norm.weight", "o": "self_attn.o_proj.weight",
              "post_attention_norm": "post_attention_layernorm.weight",
              "pre_mlp_norm": "pre_feedforward_layernorm.weight", "down": "mlp.down_proj.weight",
              "post_mlp_norm": "post_feedforward_layernorm.weight", "scalar": "layer_scalar"}
    for li, kind in enumerate(t["layer_types"]):
        p = f"model.language_model.layers.{li}."
        for name, src in single.items():
            out[(False, f"layer.{li}.{name}")] = tensors[p + src]
        parts = [tensors[p + "self_attn.q_proj.weight"], tensors[p + "self_attn.k_proj.weight"]]
        if kind == "sliding_attention":
            parts.append(tensors[p + "self_attn.v_proj.weight"])
        out[(False, f"layer.{li}.qkv")] = np.concatenate(parts)
        out[(False, f"layer.{li}.gate_up")] = np.concatenate(
            [tensors[p + "mlp.gate_proj.weight"], tensors[p + "mlp.up_proj.weight"]])
    out.update({(True, "token_embedding"): a_tensors["model.embed_tokens.weight"],
                (True, "pre_projection"): a_tensors["pre_projection.weight"],
                (True, "post_projection"): a_tensors["post_projection.weight"],
                (True, "final_norm"): a_tensors["model.norm.weight"]})
    a_single = dict(single, q="self_attn.q_proj.weight")
    del a_single["k_norm"]
    li = 0
    while f"model.layers.{li}.input_layernorm.weight" in a_tensors:
        p = f"model.layers.{li}."
        for name, src in a_single.items():
            out[(True, f"layer.{li}.{name}")] = a_tensors[p + src]
        out[(True, f"layer.{li}.gate_up")] = np.concatenate(
            [a_tensors[p + "mlp.gate_proj.weight"], a_tensors[p + "mlp.up_proj.weight"]])
        li += 1
    return out


def test_runner_from_device_weights_equals_checkpoint_runner(loaded, torch_cuda):
    """Gemma4BatchModelRunner(config, DeviceWeightArena, ..., Fp8WeightArena) over device-resident
    plan segments: with bf16 segments only, every weight and a verify step equal the checkpoint
    runner's bit for bit; with the arena's own e4m3 segments and scales (here: the oracle's
    quantisation at twice the scale, as a weight_scale_multiplier of 2 gives), those are used."""
    torch = torch_cuda
    runner, cfg, tensors, a_tensors = loaded
    desc = runner._desc
    host = plan_segments(cfg, tensors, a_tensors)
    dev = {k: torch.from_numpy(np.ascontiguousarray(v).view(np.int16)).cuda() for k, v in host.items()}
    addresses = {k: v.data_ptr() for k, v in dev.items()}
    say("case: runner from device-resident bf16 segments")
    other = BatchModelRunner.from_device_weights(desc, addresses, BATCH, MAX_CONTEXT)
    try:
        names = ["token_embedding", "token_embedding.fp8", "token_embedding.scale", "final_norm",
                 "assistant.token_embedding", "assistant.layer.0.gate_up"]
        for li in range(len(desc.layers)):
            names += [f"layer.{li}.{n}" for n in ("qkv", "o", "gate_up", "down", "scales", "q_norm")]
        for name in names:
            assert np.array_equal(other.read(name, np.uint8), runner.read(name, np.uint8)), name
        for r in (runner, other):
            r.seed_random_cache(60, seed=22, stddev=1 / math.sqrt(128))
        props = np.random.default_rng(9).integers(0, desc.vocabulary, (4, 5)).tolist()
        first = [p[0] for p in props]
        a = runner.verify_greedy_proposals(props, first, [0, 1, 2, 3], [0] * 4)
        pa = list(runner.last_predictions)
        b = other.verify_greedy_proposals(props, first, [0, 1, 2, 3], [0] * 4)
        assert a == b and other.last_predictions == pa
    finally:
        other.close()
    say("case: runner from device-resident e4m3 segments with their own scales")
    fp8 = {}
    keep = []
    for (assistant, name), m in host.items():
        if assistant or not (name == "token_embedding" or name.split(".")[-1] in ("qkv", "o", "gate_up", "down")):
            continue
        amax = float(np.abs(oracle.bf16_to_f32(m)).max())
        q, s = oracle.quantize_e4m3(m, amax * 2.0)
        dq = torch.from_numpy(np.ascontiguousarray(q)).cuda()
        ds = torch.tensor([s], dtype=torch.float32, device="cuda")
        keep += [dq, ds]
        fp8[(False, name)] = (dq.data_ptr(), ds.data_ptr(), q, s)
    other = BatchModelRunner.from_device_weights(desc, addresses, BATCH, MAX_CONTEXT,
                                                 {k: v[:2] for k, v in fp8.items()})
    try:
        q, s = fp8[(False, "token_embedding")][2:]
        assert np.array_equal(other.read("token_embedding.fp8", np.uint8), q.reshape(-1))
        assert other.read("token_embedding.scale", np.float32)[0] == np.float32(s)
        for li in range(len(desc.layers)):
            scales = other.read(f"layer.{li}.scales", np.float32)
            for j, n in enumerate(("qkv", "o", "gate_up", "down")):
                q, s = fp8[(False, f"layer.{li}.{n}")][2:]
                assert np.array_equal(other.read(f"layer.{li}.{n}", np.uint8), q.reshape(-1)), (li, n)
                assert scales[j] == np.float32(s)
    finally:
        other.close()
    with pytest.raises(Exception, match="device weights have no segment final_norm"):
        BatchModelRunner.from_device_weights(
            desc, {k: v for k, v in addresses.items() if k != (False, "final_norm")}, BATCH, MAX_CONTEXT)
    # a segment shorter than the description expects is refused before any copy reads past it
    short = dict(addresses)
    qkv = (False, "layer.0.qkv")
    short[qkv] = (addresses[qkv], dev[qkv].numel() * 2 - 128)
    with pytest.raises(Exception, match=r"device weight layer\.0\.qkv has \d+ bytes, the runner expects"):
        BatchModelRunner.from_device_weights(desc, short, BATCH, MAX_CONTEXT)
    sized = {k: (v, dev[k].numel() * 2) for k, v in addresses.items()}
    BatchModelRunner.from_device_weights(desc, sized, BATCH, MAX_CONTEXT).close()


def test_assistant_fp8_arena_from_device_weights(loaded, torch_cuda, monkeypatch):
    """Gemma4BatchModelRunner(..., assistant_weights, assistant_fp8_weights) in the assistant's FP8
    modes (assistant_runner.cu:29-43): the runner takes the assistant's e4m3 segments and scales
    from the assistant FP8 arena (here the oracle's quantisation at twice the scale, so they
    differ from what the runner would compute), and fails with the reference's error when a mode
    is set and the arena is absent."""
    torch = torch_cuda
    runner, cfg, tensors, a_tensors = loaded
    desc = runner._desc
    host = plan_segments(cfg, tensors, a_tensors)
    dev = {k: torch.from_numpy(np.ascontiguousarray(v).view(np.int16)).cuda() for k, v in host.items()}
    addresses = {k: v.data_ptr() for k, v in dev.items()}
    monkeypatch.setenv("CARAT_ASSISTANT_FP8_MODE", "all")
    with pytest.raises(Exception, match="assistant FP8 mode requires quantized assistant weights"):
        BatchModelRunner.from_device_weights(desc, addresses, BATCH, MAX_CONTEXT)
    fp8, keep = {}, []
    for (assistant, name), m in host.items():
        if not assistant or m.ndim != 2 or "norm" in name:
            continue
        amax = float(np.abs(oracle.bf16_to_f32(m)).max())
        q, s = oracle.quantize_e4m3(m, amax * 2.0)
        dq = torch.from_numpy(np.ascontiguousarray(q)).cuda()
        ds = torch.tensor([s], dtype=torch.float32, device="cuda")
        keep += [dq, ds]
        fp8[(True, name)] = (dq.data_ptr(), ds.data_ptr(), q.size, q, s)
    say("case: runner from device weights with the assistant FP8 arena (mode all, from the environment)")
    other = BatchModelRunner.from_device_weights(desc, addresses, BATCH, MAX_CONTEXT,
                                                 {k: v[:3] for k, v in fp8.items()})
    try:
        scales = other.read("assistant.fp8_scales", np.float32)
        for j, name in enumerate(("token_embedding", "pre_projection", "post_projection")):
            q, s = fp8[(True, name)][3:]
            assert np.array_equal(other.read(f"assistant.{name}.fp8", np.uint8), q.reshape(-1)), name
            assert scales[j] == np.float32(s), name
        for li in range(desc.assistant_layers):
            ls = other.read(f"assistant.layer.{li}.fp8_scales", np.float32)
            for j, n in enumerate(("q", "o", "gate_up", "down")):
                q, s = fp8[(True, f"layer.{li}.{n}")][3:]
                assert np.array_equal(other.read(f"assistant.layer.{li}.{n}.fp8", np.uint8), q.reshape(-1))
                assert ls[j] == np.float32(s)
        other.seed_random_cache(60, seed=23, stddev=1 / math.sqrt(128))
        drafts = other.draft_four([1, 2, 3, 4], [0, 1, 2, 3], [5, 6, 7, 8], 4)
        assert [row[0] for row in drafts] == [5, 6, 7, 8]
    finally:
        other.close()


@pytest.mark.parametrize("scaling", ["channel", "block_128"])
def test_scaled_fp8_weights_from_device_segments(loaded, torch_cuda, scaling):
    """Fp8WeightArena::quantize with Fp8Scaling::channel / ::block_128 (device_weights.cu:222-256):
    from bf16 device segments the runner quantises each projection and the lm_head itself, bit for
    bit the oracle's quantisation of the checkpoint bytes; given an arena, it takes the arena's
    e4m3 bytes and scale arrays (here the oracle's at twice the input, so the scales differ from
    the runner's own), and a verify step over them runs."""
    import dataclasses

    torch = torch_cuda
    runner, cfg, tensors, a_tensors = loaded
    desc = dataclasses.replace(runner._desc, fp8_scaling=scaling)
    mode = {"channel": 1, "block_128": 2}[scaling]
    host = plan_segments(cfg, tensors, a_tensors)
    dev = {k: torch.from_numpy(np.ascontiguousarray(v).view(np.int16)).cuda() for k, v in host.items()}
    addresses = {k: v.data_ptr() for k, v in dev.items()}
    names = ["token_embedding"] + [f"layer.{li}.{n}" for li in range(len(desc.layers))
                                   for n in ("qkv", "o", "gate_up", "down")]

    def fp8_name(name):
        return name + (".fp8" if name == "token_embedding" else "")

    say(f"case: {scaling} runner quantising bf16 device segments")
    other = BatchModelRunner.from_device_weights(desc, addresses, BATCH, MAX_CONTEXT)
    try:
        for name in names:
            q, s = oracle.quantize_weight_scaled(host[(False, name)], mode)
            assert np.array_equal(other.read(fp8_name(name), np.uint8), q.reshape(-1)), name
            assert np.array_equal(other.read(name + ".scale_table", np.float32), s), name
    finally:
        other.close()
    say(f"case: {scaling} runner over an arena's e4m3 segments and scale arrays")
    fp8, keep = {}, []
    for name in names:
        m = host[(False, name)]
        q, s = oracle.quantize_weight_scaled(oracle.f32_to_bf16(oracle.bf16_to_f32(m) * 2.0), mode)
        dq = torch.from_numpy(np.ascontiguousarray(q)).cuda()
        ds = torch.from_numpy(s).cuda()
        keep += [dq, ds]
        fp8[(False, name)] = (dq.data_ptr(), ds.data_ptr(), q, s)
    other = BatchModelRunner.from_device_weights(desc, addresses, BATCH, MAX_CONTEXT,
                                                 {k: v[:2] for k, v in fp8.items()})
    try:
        for name in names:
            q, s = fp8[(False, name)][2:]
            assert np.array_equal(other.read(fp8_name(name), np.uint8), q.reshape(-1)), name
            assert np.array_equal(other.read(name + ".scale_table", np.float32), s), name
        other.seed_random_cache(60, seed=24, stddev=1 / math.sqrt(128))
        props = np.random.default_rng(10).integers(0, desc.vocabulary, (4, 5))
        positions = np.full(4, 60, np.int32)
        expect = verify_step(other, desc, BATCH, lambda li: min(MAX_CONTEXT, desc.sliding_window)
                             if desc.layers[li].sliding else MAX_CONTEXT, props, [0, 1, 2, 3], positions)
        other.verify_greedy_proposals(props.tolist(), props[:, 0].tolist(), [0, 1, 2, 3], [0] * 4)
        pred = np.array(other.last_predictions, np.int32)
        logits = oracle.bf16_to_f32(expect["logits"]).astype(np.float64).reshape(len(pred), -1)
        gap = logits.max(1) - logits[np.arange(len(pred)), pred]
        assert np.all(gap <= 2 * 2 ** -7 * np.abs(logits).max(1))
    finally:
        other.close()
