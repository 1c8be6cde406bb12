"""Oracle compositions of the runner's verify step and assistant draft (test helpers).

verify_step restates cuda/batch_model_runner.cu:1617-1810 with cuda/layer_runner.cu:241-354,
730-1041; draft_steps restates cuda/assistant_runner.cu:162-338 (with batch_model_runner.cu:
1813-1836 for its arguments). Both use the oracle primitives on the weights and caches read back
from a BatchModelRunner.
"""
import math

import numpy as np

from oracle import oracle


SCALINGS = {"tensor": 0, "channel": 1, "block_128": 2}


def layer_weights(runner, i, scaling=0):
    names = ["input_norm", "q_norm", "k_norm", "post_attention_norm", "pre_mlp_norm",
             "post_mlp_norm", "scalar"]
    w = {n: runner.read(f"layer.{i}.{n}", np.uint16) for n in names}
    tensor_scales = runner.read(f"layer.{i}.scales", np.float32)
    for j, n in enumerate(("qkv", "o", "gate_up", "down")):
        w[n] = runner.read(f"layer.{i}.{n}", np.uint8)
        # the weight's scales: one float (tensor), or its channel / block_128 table
        w[n + ".scales"] = (tensor_scales[j:j + 1] if scaling == 0 else
                            runner.read(f"layer.{i}.{n}.scale_table", np.float32))
    w["scales"] = tensor_scales
    return w


def projection(x, qw, sw, scaling):
    """run_decode_linear (layer_runner.cu:220-238) under the arena's Fp8Scaling: the activation
    quantised per tensor / row / 1 x 128 block, then Fp8Linear::run."""
    qx, sx = oracle.quantize_activation_scaled(x, scaling)
    return oracle.fp8_linear_scaled(qx, sx, qw, sw, scaling)


def verify_step(runner, desc, batch, capacity_of, proposals, slots, positions, head_rows=None):
    """Returns dict(final_hidden, logits, predictions, k_new[l], v_new[l], attention[l]).

    With `head_rows` (flat row indices r * T + t), the lm_head and argmax run on those rows only
    and `logits` / `predictions` hold them in that order (the full-vocabulary head over every row
    of a 1008-row step is too slow for the CPU oracle)."""
    proposals = np.asarray(proposals, np.int32)
    R, T = proposals.shape
    H = desc.hidden
    rows = R * T
    emb = runner.read("token_embedding", np.uint16).reshape(desc.vocabulary, H)
    emb_q = runner.read("token_embedding.fp8", np.uint8).reshape(desc.vocabulary, H)
    scaling = SCALINGS[getattr(desc, "fp8_scaling", "tensor")]
    emb_s = (runner.read("token_embedding.scale", np.float32)[:1] if scaling == 0 else
             runner.read("token_embedding.scale_table", np.float32))
    final_norm = runner.read("final_norm", np.uint16)
    rowpos = (np.asarray(positions, np.int32)[:, None] + np.arange(T, dtype=np.int32)[None, :]).reshape(-1)
    hidden = oracle.embedding(emb, proposals.reshape(-1), math.sqrt(H))
    weights = [layer_weights(runner, i, scaling) for i in range(len(desc.layers))]
    x, _ = oracle.rms_norm(hidden, weights[0]["input_norm"], eps=desc.rms_norm_epsilon)
    out = {"k_new": [], "v_new": [], "attention": []}
    for li, spec in enumerate(desc.layers):
        w = weights[li]
        D, hq, hkv = spec.head_dimension, spec.query_heads, spec.kv_heads
        C = capacity_of(li)
        packed = projection(x, w["qkv"].reshape(-1, H), w["qkv.scales"], scaling)
        cos = runner.read("rope.sliding.cos" if spec.sliding else "rope.global.cos", np.uint16).reshape(-1, D)
        sin = runner.read("rope.sliding.sin" if spec.sliding else "rope.global.sin", np.uint16).reshape(-1, D)
        q, k, v = oracle.qkv_post(packed, w["q_norm"], w["k_norm"], cos, sin, rowpos, hq, hkv, D,
                                  spec.key_equals_value, desc.rms_norm_epsilon)
        out["k_new"].append(k.reshape(R, T, hkv, D))
        out["v_new"].append(v.reshape(R, T, hkv, D))
        kc = runner.read(f"cache.{li}.k", np.uint16).reshape(batch, hkv, C, D)
        vc = runner.read(f"cache.{li}.v", np.uint16).reshape(batch, hkv, C, D)
        window = min(desc.sliding_window, C) if spec.sliding else 0
        attn = oracle.verify_attention(q.reshape(R, T, hq, D), kc, vc, k.reshape(R, T, hkv, D),
                                       v.reshape(R, T, hkv, D), slots, positions, C, window)
        out["attention"].append(attn)
        proj = projection(attn.reshape(rows, hq * D), w["o"].reshape(H, hq * D), w["o.scales"], scaling)
        r1, pre, _ = oracle.rms_norm_add_and_norm(proj, w["post_attention_norm"], hidden,
                                                  w["pre_mlp_norm"], desc.rms_norm_epsilon)
        gu = projection(pre, w["gate_up"].reshape(2 * desc.intermediate, H), w["gate_up.scales"], scaling)
        act, _ = oracle.gelu_tanh_gate_rows(gu)
        down = projection(act, w["down"].reshape(H, desc.intermediate), w["down.scales"], scaling)
        hidden = oracle.rms_norm_add_scale(down, w["post_mlp_norm"], r1, int(w["scalar"][0]),
                                           desc.rms_norm_epsilon)
        nxt = weights[li + 1]["input_norm"] if li + 1 < len(desc.layers) else final_norm
        x, _ = oracle.rms_norm(hidden, nxt, eps=desc.rms_norm_epsilon)
    out["final_hidden"] = x
    head_x = x if head_rows is None else x[np.asarray(head_rows)]
    if scaling == 0:
        pred, logits = oracle.fp8_lm_head_argmax(head_x, emb_q, float(emb_s[0]))
    else:  # batch_model_runner.cu:840-853: the final hidden quantised per row / block
        logits = projection(head_x, emb_q, emb_s, scaling)
        pred = oracle.argmax_bf16_rows(logits)
    out["predictions"] = pred
    out["logits"] = logits
    return out


def _shared_layers(desc):
    """batch_model_runner.cu shared_sliding_layer / shared_global_layer: the target's last sliding
    and last global layers, whose caches the assistant reads."""
    last_sliding = max(i for i, l in enumerate(desc.layers) if l.sliding)
    last_global = max(i for i, l in enumerate(desc.layers) if not l.sliding)
    return last_sliding, last_global


def draft_steps(runner, desc, batch, capacity_of, last_tokens, slots, forced=None, depth=4,
                feed=None, fp8_mode="off"):
    """One draft_four call (assistant_runner.cu:218-338) in AssistantFp8Mode `fp8_mode`: "off"
    runs every projection in bf16; "lm_head" runs the lm_head, and "all" every projection, as an
    e4m3 GEMM over the runner's e4m3 weight copies with the input quantised per tensor from its
    own amax (run_linear, :147-160: quantize_bf16_to_fp8_e4m3 then Fp8Linear).

    Per step: input = [embedding(token) * bf16(sqrt(H)) | previous hidden], pre-projection, the
    assistant layers (run_layer, :162-208: q-only projection, query RMSNorm + RoPE at position
    context + step, decode attention over the target's last sliding / global cache with
    valid = min(context + 1, C), o, norms, gate/up GELU, down), final norm, lm_head + argmax
    (the forced token instead at step 0 when given, :306-312), post-projection -> previous hidden.
    context = slot position - 1 (batch_model_runner.cu:1820-1828). With `feed` ([rows][depth]),
    step d > 0 takes feed[:, d - 1] as its input token instead of the oracle's own output
    (teacher forcing), so a GPU chain can be checked step by step.

    Returns dict(tokens [rows][depth], logits [depth] (None at a forced step), hidden [depth]).
    """
    H = desc.hidden
    AH = desc.assistant_hidden
    rows = len(last_tokens)
    slots = np.asarray(slots, np.int32)
    context = np.array([runner.slot_position(int(s)) - 1 for s in slots], np.int32)
    emb = runner.read("token_embedding", np.uint16).reshape(desc.vocabulary, H)
    a_emb = runner.read("assistant.token_embedding", np.uint16).reshape(desc.vocabulary, AH)
    pre_w = runner.read("assistant.pre_projection", np.uint16).reshape(AH, 2 * H)
    post_w = runner.read("assistant.post_projection", np.uint16).reshape(H, AH)
    final_norm = runner.read("assistant.final_norm", np.uint16)
    previous = runner.read("target_hidden", np.uint16).reshape(batch, H)[slots]
    all8 = fp8_mode == "all"
    if fp8_mode != "off":
        scales8 = runner.read("assistant.fp8_scales", np.float32)
        a_emb8 = runner.read("assistant.token_embedding.fp8", np.uint8).reshape(desc.vocabulary, AH)
    if all8:
        pre_w8 = runner.read("assistant.pre_projection.fp8", np.uint8).reshape(AH, 2 * H)
        post_w8 = runner.read("assistant.post_projection.fp8", np.uint8).reshape(H, AH)

    def linear(x, w, w8=None, s8=None):
        if w8 is None:
            return oracle.bf16_linear(x, w)
        qx, sx = oracle.quantize_e4m3(x)
        return oracle.fp8_linear(qx, sx, w8, float(s8))

    last_sliding, last_global = _shared_layers(desc)
    layers = []
    for li in range(desc.assistant_layers):
        pre = f"assistant.layer.{li}."
        glob = li == desc.assistant_layers - 1
        target = last_global if glob else last_sliding
        spec = desc.layers[target]
        D, hkv, hq = spec.head_dimension, spec.kv_heads, desc.assistant_query_heads
        C = capacity_of(target)
        w = {n: runner.read(pre + n, np.uint16) for n in
             ("input_norm", "q_norm", "post_attention_norm", "pre_mlp_norm", "post_mlp_norm", "scalar")}
        w["q"] = runner.read(pre + "q", np.uint16).reshape(hq * D, AH)
        w["o"] = runner.read(pre + "o", np.uint16).reshape(AH, hq * D)
        w["gate_up"] = runner.read(pre + "gate_up", np.uint16).reshape(2 * desc.assistant_intermediate, AH)
        w["down"] = runner.read(pre + "down", np.uint16).reshape(AH, desc.assistant_intermediate)
        for n in ("q", "o", "gate_up", "down"):
            w[n + "8"] = (runner.read(pre + n + ".fp8", np.uint8).reshape(w[n].shape) if all8 else None)
        w["s8"] = runner.read(pre + "fp8_scales", np.float32) if all8 else [None] * 4
        kind = "global" if glob else "sliding"
        w["cos"] = runner.read(f"rope.{kind}.cos", np.uint16).reshape(-1, D)
        w["sin"] = runner.read(f"rope.{kind}.sin", np.uint16).reshape(-1, D)
        w["k"] = runner.read(f"cache.{target}.k", np.uint16).reshape(batch, hkv, C, D)
        w["v"] = runner.read(f"cache.{target}.v", np.uint16).reshape(batch, hkv, C, D)
        layers.append((w, D, hkv, hq, C))
    tokens = np.asarray(last_tokens, np.int32)
    out = {"tokens": np.zeros((rows, depth), np.int32), "logits": [], "hidden": []}
    for d in range(depth):
        x = oracle.embedding(emb, tokens, math.sqrt(H))
        h = linear(np.concatenate([x, previous], axis=1), pre_w, pre_w8 if all8 else None,
                   scales8[1] if all8 else None)
        for w, D, hkv, hq, C in layers:
            n, _ = oracle.rms_norm(h, w["input_norm"], eps=desc.rms_norm_epsilon)
            qp = linear(n, w["q"], w["q8"], w["s8"][0])
            q, _, _ = oracle.qkv_post(qp, w["q_norm"], w["q_norm"], w["cos"], w["sin"], context + d,
                                      hq, 0, D, False, desc.rms_norm_epsilon)
            attn = oracle.decode_attention(q, w["k"], w["v"], slots, context, hkv, C)
            o = linear(attn.reshape(rows, hq * D), w["o"], w["o8"], w["s8"][1])
            r1, pre_mlp, _ = oracle.rms_norm_add_and_norm(o, w["post_attention_norm"], h,
                                                          w["pre_mlp_norm"], desc.rms_norm_epsilon)
            act, _ = oracle.gelu_tanh_gate_rows(linear(pre_mlp, w["gate_up"], w["gate_up8"], w["s8"][2]))
            down = linear(act, w["down"], w["down8"], w["s8"][3])
            h = oracle.rms_norm_add_scale(down, w["post_mlp_norm"], r1, int(w["scalar"][0]),
                                          desc.rms_norm_epsilon)
        fh, _ = oracle.rms_norm(h, final_norm, eps=desc.rms_norm_epsilon)
        if d == 0 and forced is not None:
            step_tokens = np.asarray(forced, np.int32)
            out["logits"].append(None)
        elif fp8_mode != "off":
            step_tokens, logits = oracle.fp8_lm_head_argmax(fh, a_emb8, float(scales8[0]))
            out["logits"].append(logits)
        else:
            logits = oracle.bf16_linear(fh, a_emb)
            step_tokens = oracle.argmax_bf16_rows(logits)
            out["logits"].append(logits)
        out["tokens"][:, d] = step_tokens
        previous = linear(fh, post_w, post_w8 if all8 else None, scales8[2] if all8 else None)
        out["hidden"].append(previous)
        tokens = step_tokens if feed is None else np.asarray(feed, np.int32)[:, d]
    return out
