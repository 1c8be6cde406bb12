"""ctypes wrapper of the CPU oracle (libcarat_oracle.so) and of the reference's own speculation
helpers compiled into _ref/ -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module, as the
checker or the timed CPU baseline. The HIP product never imports it.
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "libcarat_oracle.so"
REF_SO = HERE / "_ref" / "libref_speculation.so"


def build() -> None:
    """Compiles the oracle (and, when /root/reference is present, oracle/_ref)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_LIB = None
_REF = None


def lib():
    global _LIB
    if _LIB is None:
        if not ORACLE_SO.exists():
            build()
        _LIB = ctypes.CDLL(str(ORACLE_SO))
        _LIB.orc_quantize_e4m3.restype = c_float
        _LIB.orc_bf16_to_f32.restype = c_float
        _LIB.orc_e4m3_to_f32.restype = c_float
        _LIB.orc_f32_to_bf16.restype = ctypes.c_uint16
        _LIB.orc_f32_to_bf16.argtypes = [c_float]
        _LIB.orc_f32_to_e4m3.restype = ctypes.c_uint8
        _LIB.orc_f32_to_e4m3.argtypes = [c_float]
    return _LIB


def ref():
    """The reference's speculation.cpp (compiled here from /root/reference), or None."""
    global _REF
    if _REF is None and REF_SO.exists():
        _REF = ctypes.CDLL(str(REF_SO))
    return _REF


class _Pointer(c_void_p):
    """A void* that keeps the array it points into alive for the duration of the call."""


def p(a) -> c_void_p:
    if a is None:
        return c_void_p(0)
    pointer = _Pointer(a.ctypes.data)
    pointer.keep = a
    return pointer


def c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ conversions
def f32_to_bf16(x) -> np.ndarray:
    x = c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_array(p(x), p(out), c_int64(x.size))
    return out


def bf16_to_f32(x) -> np.ndarray:
    x = c(x, np.uint16)
    out = np.empty(x.shape, np.float32)
    lib().orc_bf16_to_f32_array(p(x), p(out), c_int64(x.size))
    return out


def f32_to_e4m3_scalar(v: float) -> int:
    return int(lib().orc_f32_to_e4m3(float(v)))


def e4m3_table() -> np.ndarray:
    return np.array([lib().orc_e4m3_to_f32(i) for i in range(256)], np.float32)


def f32_to_e4m3(x) -> np.ndarray:
    x = c(x, np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().orc_f32_to_e4m3_array(p(x), p(out), c_int64(x.size))
    return out


# ------------------------------------------------------------------ speculation
def acceptance_cap(depth, remaining, proposals, stop_ids) -> int:
    pr = c(proposals, np.int32)
    st = c(list(stop_ids), np.int32)
    return lib().orc_acceptance_cap(depth, remaining, p(pr), len(pr), p(st), len(st))


def commit_speculation(forced, drafts, next_token, stop_ids):
    d = c(drafts, np.int32)
    st = c(list(stop_ids), np.int32)
    res = np.zeros(len(d) + 1, np.int32)
    em = np.zeros(len(d) + 1, np.int32)
    nr, ne, nx = c_int(), c_int(), ctypes.c_int32()
    stopped = lib().orc_commit_speculation(forced, p(d), len(d), next_token, p(st), len(st), p(res),
                                           ctypes.byref(nr), p(em), ctypes.byref(ne), ctypes.byref(nx))
    return res[: nr.value].tolist(), em[: ne.value].tolist(), int(nx.value), bool(stopped)


def ref_acceptance_cap(depth, remaining, proposals, stop_ids) -> int:
    pr = c(proposals, np.int32)
    st = c(list(stop_ids), np.int32)
    return ref().ref_acceptance_cap(depth, remaining, p(pr), len(pr), p(st), len(st))


def ref_commit_speculation(forced, drafts, next_token, stop_ids):
    d = c(drafts, np.int32)
    st = c(list(stop_ids), np.int32)
    res = np.zeros(len(d) + 1, np.int32)
    em = np.zeros(len(d) + 1, np.int32)
    nr, ne, nx = c_int(), c_int(), ctypes.c_int32()
    stopped = ref().ref_commit_speculation(forced, p(d), len(d), next_token, p(st), len(st), p(res),
                                           ctypes.byref(nr), p(em), ctypes.byref(ne), ctypes.byref(nx))
    return res[: nr.value].tolist(), em[: ne.value].tolist(), int(nx.value), bool(stopped)


def greedy_accept(proposals, target_first, predictions, caps=None):
    pr = c(proposals, np.int32)
    r, t = pr.shape
    first = c(target_first, np.int32)
    pred = c(predictions, np.int32)
    cp = None if caps is None else c(caps, np.int32)
    acc = np.zeros(r, np.int32)
    nxt = np.zeros(r, np.int32)
    lib().orc_greedy_accept(r, t, p(pr), p(first), p(pred), p(cp), p(acc), p(nxt))
    return acc, nxt


# ------------------------------------------------------------------ argmax
def argmax_bf16_rows(logits_bf16) -> np.ndarray:
    x = c(logits_bf16, np.uint16)
    out = np.zeros(x.shape[0], np.int32)
    lib().orc_argmax_bf16_rows(p(x), x.shape[0], c_int64(x.shape[1]), p(out))
    return out


def argmax_f32_rows_as_bf16(logits) -> np.ndarray:
    x = c(logits, np.float32)
    out = np.zeros(x.shape[0], np.int32)
    lib().orc_argmax_f32_rows_as_bf16(p(x), x.shape[0], c_int64(x.shape[1]), p(out))
    return out


# ------------------------------------------------------------------ fp8
def quantize_e4m3(x_bf16, amax=None):
    x = c(x_bf16, np.uint16)
    q = np.empty(x.shape, np.uint8)
    if amax is None:
        s = lib().orc_quantize_e4m3(p(x), c_int64(x.size), c_float(1.0), p(q))
        return q, float(s)
    s = c_float()
    lib().orc_quantize_e4m3_with_amax(p(x), c_int64(x.size), c_float(amax), c_float(1.0), p(q),
                                      ctypes.byref(s))
    return q, float(s.value)


def fp8_linear(qx, sx, qw, sw) -> np.ndarray:
    qx = c(qx, np.uint8)
    qw = c(qw, np.uint8)
    m, k = qx.shape
    n = qw.shape[0]
    out = np.empty((m, n), np.uint16)
    lib().orc_fp8_linear(p(qx), c_float(sx), p(qw), c_float(sw), m, k, n, p(out))
    return out


def fp8_linear_f32(qx, sx, qw, sw) -> np.ndarray:
    qx = c(qx, np.uint8)
    qw = c(qw, np.uint8)
    m, k = qx.shape
    n = qw.shape[0]
    out = np.empty((m, n), np.float32)
    lib().orc_fp8_linear_f32(p(qx), c_float(sx), p(qw), c_float(sw), m, k, n, p(out))
    return out


def bf16_linear(x_bf16, w_bf16) -> np.ndarray:
    x = c(x_bf16, np.uint16)
    w = c(w_bf16, np.uint16)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.uint16)
    lib().orc_bf16_linear(p(x), p(w), m, k, n, p(out))
    return out


SCALING = {"tensor": 0, "channel": 1, "block_128": 2}


def quantize_e4m3_rows(x_bf16):
    """quantize_bf16_rows (Fp8Scaling::channel): q, scales[rows]."""
    x = c(x_bf16, np.uint16)
    rows, width = x.shape
    q = np.empty(x.shape, np.uint8)
    s = np.empty(rows, np.float32)
    lib().orc_quantize_e4m3_rows(p(x), rows, width, p(q), p(s))
    return q, s


def quantize_e4m3_weight_block128(w_bf16):
    """quantize_bf16_weight_to_fp8_block_128: q, scales[ceil(n/128) * kbp] (flat)."""
    w = c(w_bf16, np.uint16)
    n, k = w.shape
    q = np.empty(w.shape, np.uint8)
    lib().orc_fp8_weight_block_scale_elements.restype = c_int64
    s = np.empty(lib().orc_fp8_weight_block_scale_elements(n, k), np.float32)
    lib().orc_quantize_e4m3_weight_block128(p(w), n, k, p(q), p(s))
    return q, s


def quantize_e4m3_activation_block128(x_bf16):
    """quantize_bf16_activation_to_fp8_block_128: q, scales[ceil(k/128)][rows] (flat)."""
    x = c(x_bf16, np.uint16)
    rows, k = x.shape
    q = np.empty(x.shape, np.uint8)
    s = np.empty(((k + 127) // 128) * rows, np.float32)
    lib().orc_quantize_e4m3_activation_block128(p(x), rows, k, p(q), p(s))
    return q, s


def quantize_weight_scaled(w_bf16, scaling):
    """Fp8WeightArena::quantize of one segment under `scaling` (0/1/2): q, scales (flat)."""
    if scaling == 0:
        q, s = quantize_e4m3(w_bf16)
        return q, np.array([s], np.float32)
    return quantize_e4m3_rows(w_bf16) if scaling == 1 else quantize_e4m3_weight_block128(w_bf16)


def quantize_activation_scaled(x_bf16, scaling):
    """run_decode_linear's activation quantisation under `scaling` (0/1/2): q, scales (flat)."""
    if scaling == 0:
        q, s = quantize_e4m3(x_bf16)
        return q, np.array([s], np.float32)
    return quantize_e4m3_rows(x_bf16) if scaling == 1 else quantize_e4m3_activation_block128(x_bf16)


def fp8_linear_scaled(qx, sx, qw, sw, scaling, f32=False) -> np.ndarray:
    """Fp8Linear::run under `scaling` (0 tensor, 1 channel, 2 block_128)."""
    qx = c(qx, np.uint8)
    qw = c(qw, np.uint8)
    if scaling == 0:
        f = fp8_linear_f32 if f32 else fp8_linear
        return f(qx, float(np.ravel(sx)[0]), qw, float(np.ravel(sw)[0]))
    m, k = qx.shape
    n = qw.shape[0]
    out = np.empty((m, n), np.float32 if f32 else np.uint16)
    fn = lib().orc_fp8_linear_scaled_f32 if f32 else lib().orc_fp8_linear_scaled
    fn(p(qx), p(c(sx, np.float32)), p(qw), p(c(sw, np.float32)), m, k, n, scaling, p(out))
    return out


def fp8_lm_head_argmax(x_bf16, qw, sw):
    x = c(x_bf16, np.uint16)
    qw = c(qw, np.uint8)
    m, k = x.shape
    n = qw.shape[0]
    out = np.zeros(m, np.int32)
    logits = np.empty((m, n), np.uint16)
    lib().orc_fp8_lm_head_argmax(p(x), m, k, p(qw), c_float(sw), n, p(out), p(logits))
    return out, logits


# ------------------------------------------------------------------ row ops
def rms_norm(x, w, residual=None, eps=1e-6):
    x = c(x, np.uint16)
    rows, width = x.shape
    out = np.empty_like(x)
    amax = np.zeros(rows, np.float32)
    lib().orc_rms_norm(p(x), p(c(w, np.uint16)), p(None if residual is None else c(residual, np.uint16)),
                       p(out), p(amax), rows, width, c_float(eps))
    return out, amax


def rms_norm_add_and_norm(x, w, residual, next_w, eps=1e-6):
    x = c(x, np.uint16)
    rows, width = x.shape
    r1 = np.empty_like(x)
    y = np.empty_like(x)
    amax = np.zeros(rows, np.float32)
    lib().orc_rms_norm_add_and_norm(p(x), p(c(w, np.uint16)), p(c(residual, np.uint16)),
                                    p(c(next_w, np.uint16)), p(r1), p(y), p(amax), rows, width,
                                    c_float(eps))
    return r1, y, amax


def rms_norm_add_scale(x, w, residual, scalar_bf16: int, eps=1e-6):
    x = c(x, np.uint16)
    rows, width = x.shape
    out = np.empty_like(x)
    lib().orc_rms_norm_add_scale(p(x), p(c(w, np.uint16)), p(c(residual, np.uint16)),
                                 ctypes.c_uint16(int(scalar_bf16)), p(out), rows, width, c_float(eps))
    return out


def gelu_tanh_gate_rows(packed):
    x = c(packed, np.uint16)
    rows, width2 = x.shape
    out = np.empty((rows, width2 // 2), np.uint16)
    amax = np.zeros(rows, np.float32)
    lib().orc_gelu_tanh_gate_rows(p(x), p(out), p(amax), rows, width2 // 2)
    return out, amax


def embedding(weight, tokens, scale):
    w = c(weight, np.uint16)
    t = c(tokens, np.int32)
    out = np.zeros((len(t), w.shape[1]), np.uint16)
    lib().orc_embedding(p(w), p(t), p(out), len(t), w.shape[0], w.shape[1], c_float(scale))
    return out


def rope_table(dimension, proportional, positions):
    cos = np.empty((positions, dimension), np.uint16)
    sin = np.empty((positions, dimension), np.uint16)
    lib().orc_rope_table(dimension, int(proportional), positions, p(cos), p(sin))
    return cos, sin


def qkv_post(packed, q_norm, k_norm, cos, sin, positions, query_heads, kv_heads, dimension,
             key_equals_value=False, eps=1e-6):
    x = c(packed, np.uint16)
    rows = x.shape[0]
    q = np.empty((rows, query_heads, dimension), np.uint16)
    k = np.empty((rows, kv_heads, dimension), np.uint16)
    v = np.empty((rows, kv_heads, dimension), np.uint16)
    lib().orc_qkv_post(p(x), p(c(q_norm, np.uint16)), p(c(k_norm, np.uint16)), p(c(cos, np.uint16)),
                       p(c(sin, np.uint16)), p(c(positions, np.int32)), rows, query_heads, kv_heads,
                       dimension, int(key_equals_value), c_float(eps), p(q), p(k), p(v))
    return q, k, v


# ------------------------------------------------------------------ attention
def verify_attention(q, k_cache, v_cache, k_new, v_new, slots, positions, capacity, window,
                     round_like_reference=False):
    q = c(q, np.uint16)
    r, t, hq, d = q.shape
    hkv = k_new.shape[2]
    out = np.empty_like(q)
    lib().orc_verify_attention(p(q), p(c(k_cache, np.uint16)), p(c(v_cache, np.uint16)),
                               p(c(k_new, np.uint16)), p(c(v_new, np.uint16)), p(c(slots, np.int32)),
                               p(c(positions, np.int32)), r, t, hq, hkv, d, capacity, window,
                               int(round_like_reference), p(out))
    return out


def verify_attention_fp8(q, k_cache, v_cache, k_new, v_new, k_scale, v_scale, slots, positions,
                         capacity):
    q = c(q, np.uint16)
    r, t, hq, d = q.shape
    hkv = k_new.shape[2]
    out = np.empty_like(q)
    lib().orc_verify_attention_fp8(p(q), p(c(k_cache, np.uint8)), p(c(v_cache, np.uint8)),
                                   p(c(k_new, np.uint8)), p(c(v_new, np.uint8)), c_float(k_scale),
                                   c_float(v_scale), p(c(slots, np.int32)), p(c(positions, np.int32)),
                                   r, t, hq, hkv, d, capacity, p(out))
    return out


def ring_backup_attention(q_head_major, k_ring, v_ring, k_backup, v_backup, positions, kv_heads,
                          capacity):
    q = c(q_head_major, np.uint16)
    r, hq, t, d = q.shape
    out = np.empty(q.shape, np.float32)
    lib().orc_ring_backup_attention(p(q), p(c(k_ring, np.uint16)), p(c(v_ring, np.uint16)),
                                    p(c(k_backup, np.uint16)), p(c(v_backup, np.uint16)),
                                    p(c(positions, np.int32)), r, t, hq, kv_heads, d, capacity, p(out))
    return out


def decode_attention(q, k_cache, v_cache, slots, positions, kv_heads, capacity,
                     round_like_reference=False):
    q = c(q, np.uint16)
    b, hq, d = q.shape
    out = np.empty_like(q)
    lib().orc_decode_attention(p(q), p(c(k_cache, np.uint16)), p(c(v_cache, np.uint16)),
                               p(c(slots, np.int32)), p(c(positions, np.int32)), b, hq, kv_heads, d,
                               capacity, int(round_like_reference), p(out))
    return out


def commit_kv(k_cache, v_cache, k_new, v_new, slots, positions, accepted, capacity):
    r, t, hkv, d = k_new.shape
    lib().orc_commit_kv(p(k_cache), p(v_cache), p(c(k_new, np.uint16)), p(c(v_new, np.uint16)),
                        p(c(slots, np.int32)), p(c(positions, np.int32)), p(c(accepted, np.int32)),
                        r, t, hkv, d, capacity)
