"""Python mirror of the reference runner interface over the C ABI.

Names, argument meaning and error behaviour follow include/carat/batch_model_runner.h:22-77 and
src/runtime/speculation.h:11-27 of the reference: invalid batches raise with the reference's
messages (wrapped in CaratError, a RuntimeError).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Iterable, Sequence

import numpy as np

from ._lib import CaratError, LayerDesc, ModelDesc as _CModelDesc, check, lib, ptr


@dataclass
class LayerSpec:
    sliding: bool = True
    query_heads: int = 32
    kv_heads: int = 16
    head_dimension: int = 128
    key_equals_value: bool = False


@dataclass
class ModelDesc:
    hidden: int = 5376
    intermediate: int = 21504
    vocabulary: int = 262144
    sliding_window: int = 1024
    rms_norm_epsilon: float = 1e-6
    layers: list[LayerSpec] = field(default_factory=list)
    assistant: bool = False
    assistant_hidden: int = 1024
    assistant_intermediate: int = 8192
    assistant_layers: int = 4
    assistant_query_heads: int = 32
    seed: int = 1
    weight_std: float = 0.02
    # AssistantFp8Mode (assistant_runner.cu:29-43): None reads CARAT_ASSISTANT_FP8_MODE as the
    # reference does (unset: off); else "off", "lm_head" or "all"
    assistant_fp8_mode: str | None = None
    # Fp8Scaling of the target's e4m3 weights (include/carat/linear.h:27): "tensor", "channel"
    # or "block_128"
    fp8_scaling: str = "tensor"

    @staticmethod
    def gemma4_benchmark(with_assistant: bool = True) -> "ModelDesc":
        layers = [LayerSpec(sliding=(i % 6) != 5) for i in range(60)]
        return ModelDesc(layers=layers, assistant=with_assistant)

    @staticmethod
    def gemma4_31b(with_assistant: bool = True) -> "ModelDesc":
        """The native Gemma-4 31B attention geometry (gemma4_config.cpp:174-203): sliding layers
        D 256 with 32/16 heads, every sixth layer global with D 512, 32/4 heads and K = V."""
        layers = [LayerSpec(sliding=True, query_heads=32, kv_heads=16, head_dimension=256)
                  if (i % 6) != 5 else
                  LayerSpec(sliding=False, query_heads=32, kv_heads=4, head_dimension=512,
                            key_equals_value=True) for i in range(60)]
        return ModelDesc(layers=layers, assistant=with_assistant)

    def to_c(self):
        arr = (LayerDesc * len(self.layers))()
        for i, l in enumerate(self.layers):
            arr[i] = LayerDesc(int(l.sliding), l.query_heads, l.kv_heads, l.head_dimension,
                               int(l.key_equals_value))
        d = _CModelDesc()
        d.hidden, d.intermediate, d.vocabulary = self.hidden, self.intermediate, self.vocabulary
        d.sliding_window, d.rms_norm_epsilon = self.sliding_window, self.rms_norm_epsilon
        d.layer_count, d.layers = len(self.layers), arr
        d.assistant = int(self.assistant)
        d.assistant_hidden, d.assistant_intermediate = self.assistant_hidden, self.assistant_intermediate
        d.assistant_layers, d.assistant_query_heads = self.assistant_layers, self.assistant_query_heads
        d.seed, d.weight_std = self.seed, self.weight_std
        modes = {None: 0, "off": 1, "lm_head": 2, "all": 3}
        if self.assistant_fp8_mode not in modes:
            raise ValueError("assistant_fp8_mode must be None, 'off', 'lm_head' or 'all'")
        d.assistant_fp8_mode = modes[self.assistant_fp8_mode]
        scalings = {"tensor": 0, "channel": 1, "block_128": 2}
        if self.fp8_scaling not in scalings:
            raise ValueError("fp8_scaling must be 'tensor', 'channel' or 'block_128'")
        d.fp8_scaling = scalings[self.fp8_scaling]
        return d, arr


@dataclass
class GreedyVerificationResult:
    accepted_tokens: list[int]
    next_tokens: list[int]


def describe_checkpoint(model_dir: str, assistant_dir: str | None = None
                        ) -> tuple[ModelDesc, int, int]:
    """Validates a checkpoint without reading weight data: (model description, target plan
    bytes, assistant plan bytes). Raises CaratError with the reference's messages."""
    c_desc = _CModelDesc()
    enc = model_dir.encode()
    aenc = None if assistant_dir is None else assistant_dir.encode()
    check(lib().carat_hip_checkpoint_describe(enc, aenc, ctypes.byref(c_desc), None, 0, None, None))
    layers = (LayerDesc * c_desc.layer_count)()
    target_bytes = ctypes.c_uint64()
    assistant_bytes = ctypes.c_uint64()
    check(lib().carat_hip_checkpoint_describe(enc, aenc, ctypes.byref(c_desc), layers,
                                              c_desc.layer_count, ctypes.byref(target_bytes),
                                              ctypes.byref(assistant_bytes)))
    desc = ModelDesc(
        hidden=c_desc.hidden, intermediate=c_desc.intermediate, vocabulary=c_desc.vocabulary,
        sliding_window=c_desc.sliding_window, rms_norm_epsilon=c_desc.rms_norm_epsilon,
        layers=[LayerSpec(bool(l.sliding), l.query_heads, l.kv_heads, l.head_dimension,
                          bool(l.key_equals_value)) for l in layers],
        assistant=bool(c_desc.assistant), assistant_hidden=c_desc.assistant_hidden,
        assistant_intermediate=c_desc.assistant_intermediate,
        assistant_layers=c_desc.assistant_layers, assistant_query_heads=c_desc.assistant_query_heads)
    return desc, target_bytes.value, assistant_bytes.value


def _i32(values: Iterable[int]) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(list(values), dtype=np.int32))


class BatchModelRunner:
    """Gemma4BatchModelRunner (batch_model_runner.h:22-77) on one MI355X."""

    def __init__(self, desc: ModelDesc, batch: int, maximum_context: int):
        self._desc = desc
        c_desc, self._layers_keepalive = desc.to_c()
        handle = ctypes.c_void_p()
        check(lib().carat_hip_runner_create(ctypes.byref(c_desc), batch, maximum_context,
                                            ctypes.byref(handle)))
        self._handle = handle
        self.last_predictions: list[int] = []  # per row of the last step; -1 for a prefill step no prompt completes

    @classmethod
    def from_checkpoint(cls, model_dir: str, batch: int, maximum_context: int,
                        assistant_dir: str | None = None) -> "BatchModelRunner":
        """The runner over a Gemma-4 safetensors checkpoint (weight_plan.cpp / device_weights.cu)."""
        desc, _, _ = describe_checkpoint(model_dir, assistant_dir)
        self = cls.__new__(cls)
        self._desc = desc
        self._layers_keepalive = None
        handle = ctypes.c_void_p()
        check(lib().carat_hip_runner_create_from_checkpoint(
            model_dir.encode(), None if assistant_dir is None else assistant_dir.encode(), batch,
            maximum_context, ctypes.byref(handle)))
        self._handle = handle
        self.last_predictions = []
        return self

    def bench_speculative_cycle(self, last_tokens, slots, forced, planted, remaining, stop_ids=()):
        """One scheduler cycle in C++ (carat_hip_bench_speculative_cycle): draft, caps, verify of
        `planted`, commit. Returns (accepted, next forced tokens, last resident tokens, seconds)."""
        planted = np.ascontiguousarray(planted, dtype=np.int32)
        requests, depth = planted.shape
        stops = _i32(stop_ids)
        acc = np.zeros(requests, np.int32)
        nxt = np.zeros(requests, np.int32)
        last = np.zeros(requests, np.int32)
        seconds = ctypes.c_double()
        check(lib().carat_hip_bench_speculative_cycle(
            self._handle, requests, depth, ptr(_i32(last_tokens)), ptr(_i32(slots)), ptr(_i32(forced)),
            ptr(planted), remaining, ptr(stops) if stops.size else None, int(stops.size), ptr(acc),
            ptr(nxt), ptr(last), ctypes.byref(seconds)))
        return acc, nxt, last, seconds.value

    SEGMENT_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                  ctypes.POINTER(ctypes.c_uint64))

    @classmethod
    def from_device_weights(cls, desc: ModelDesc, segments: dict, batch: int, maximum_context: int,
                            fp8_segments: dict | None = None) -> "BatchModelRunner":
        """The runner over weights already on the device (DeviceWeightArena / Fp8WeightArena,
        device_weights.h:15-52). `segments` maps (assistant, name) to the device address of the
        bf16 execution segment the reference's WeightPlan calls `name`, or to (address, byte
        size); `fp8_segments` (optional) maps it to (e4m3 segment address, device address of its
        fp32 scale[, byte size]). A byte size that differs from the runner's is an error."""
        fp8_segments = fp8_segments or {}

        def lookup(_context, assistant, fp8, name, scale, size):
            key = (bool(assistant), name.decode())
            entry = fp8_segments.get(key) if fp8 else segments.get(key)
            if entry is None:
                return None
            if fp8:
                scale[0] = entry[1]
                if len(entry) > 2:
                    size[0] = entry[2]
                return entry[0]
            if isinstance(entry, tuple):
                size[0] = entry[1]
                return entry[0]
            return entry

        callback = cls.SEGMENT_FN(lookup)
        self = cls.__new__(cls)
        self._desc = desc
        c_desc, self._layers_keepalive = desc.to_c()
        handle = ctypes.c_void_p()
        check(lib().carat_hip_runner_create_from_device_weights(
            ctypes.byref(c_desc), callback, None, batch, maximum_context, ctypes.byref(handle)))
        self._handle = handle
        self.last_predictions = []
        return self

    def close(self) -> None:
        if getattr(self, "_handle", None):
            lib().carat_hip_runner_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ------------------------------------------------------------------ reference interface
    def verify_greedy_proposals(self, proposals: Sequence[Sequence[int]],
                                target_first_tokens: Sequence[int], slots: Sequence[int],
                                maximum_accepted_tokens: Sequence[int] = ()) -> GreedyVerificationResult:
        requests = len(proposals)
        depth = len(proposals[0]) if requests else 0
        if any(len(p) != depth for p in proposals):
            raise CaratError("invalid or repeated speculative slot")
        flat = _i32(t for p in proposals for t in p)
        first = _i32(target_first_tokens)
        slot_arr = _i32(slots)
        caps = _i32(maximum_accepted_tokens) if len(maximum_accepted_tokens) else None
        if len(first) != requests or len(slot_arr) != requests:
            raise CaratError("invalid greedy verification batch")
        if caps is not None and len(caps) != requests:
            raise CaratError("speculative acceptance caps do not match request count")
        accepted = np.zeros(max(requests, 1), np.int32)
        nxt = np.zeros(max(requests, 1), np.int32)
        pred = np.zeros(max(requests * depth, 1), np.int32)
        check(lib().carat_hip_runner_verify(self._handle, requests, depth, ptr(flat), ptr(first),
                                            ptr(slot_arr), ptr(caps), ptr(accepted), ptr(nxt),
                                            ptr(pred)))
        self.last_predictions = pred[: requests * depth].tolist()
        return GreedyVerificationResult(accepted[:requests].tolist(), nxt[:requests].tolist())

    def append_ragged(self, token_ids: Sequence[int], slots: Sequence[int]) -> list[int]:
        """batch_model_runner.h:55: one decode step per (token, slot); returns the next tokens."""
        tokens = _i32(token_ids)
        slot_arr = _i32(slots)
        if len(tokens) != len(slot_arr) or len(tokens) == 0:
            raise CaratError("invalid ragged token batch")
        out = np.zeros(max(len(tokens), 1), np.int32)
        check(lib().carat_hip_runner_append_ragged(self._handle, len(tokens), ptr(tokens),
                                                   ptr(slot_arr), ptr(out)))
        return out[: len(tokens)].tolist()

    def draft_four(self, last_tokens: Sequence[int], slots: Sequence[int],
                   forced_first_tokens: Sequence[int] = (), depth: int = 4) -> list[list[int]]:
        last = _i32(last_tokens)
        slot_arr = _i32(slots)
        forced = _i32(forced_first_tokens) if len(forced_first_tokens) else None
        if len(last) != len(slot_arr) or len(last) == 0:
            raise CaratError("assistant is not configured or draft batch is invalid")
        if forced is not None and len(forced) != len(last):
            raise CaratError("forced assistant first tokens do not match draft batch")
        out = np.zeros((len(last), max(depth, 1)), np.int32)
        check(lib().carat_hip_runner_draft(self._handle, len(last), depth, ptr(last), ptr(slot_arr),
                                           ptr(forced), ptr(out)))
        return out[:, :depth].tolist()

    def has_assistant(self) -> bool:
        v = ctypes.c_int()
        check(lib().carat_hip_runner_has_assistant(self._handle, ctypes.byref(v)))
        return bool(v.value)

    def reset_slot(self, slot: int) -> None:
        check(lib().carat_hip_runner_reset_slot(self._handle, slot))

    def seed_empty_cache_for_benchmark(self, position: int) -> None:
        check(lib().carat_hip_runner_seed_empty_cache_for_benchmark(self._handle, position))

    def batch(self) -> int:
        v = ctypes.c_int()
        check(lib().carat_hip_runner_batch(self._handle, ctypes.byref(v)))
        return v.value

    def position(self) -> int:
        v = ctypes.c_int()
        check(lib().carat_hip_runner_position(self._handle, ctypes.byref(v)))
        return v.value

    def slot_position(self, slot: int) -> int:
        v = ctypes.c_int()
        check(lib().carat_hip_runner_slot_position(self._handle, slot, ctypes.byref(v)))
        return v.value

    # ------------------------------------------------------------------ helpers (no reference twin)
    def seed_random_cache(self, position: int, seed: int = 1, stddev: float = 1.0) -> None:
        check(lib().carat_hip_runner_seed_random_cache(self._handle, position, ctypes.c_uint64(seed),
                                                       ctypes.c_float(stddev)))

    def set_slot_position(self, slot: int, position: int) -> None:
        check(lib().carat_hip_runner_set_slot_position(self._handle, slot, position))

    def tensor_bytes(self, name: str) -> int:
        p = ctypes.c_void_p()
        n = ctypes.c_size_t()
        check(lib().carat_hip_runner_tensor(self._handle, name.encode(), ctypes.byref(p),
                                            ctypes.byref(n)))
        return n.value

    def read(self, name: str, dtype) -> np.ndarray:
        n = self.tensor_bytes(name)
        out = np.empty(n // np.dtype(dtype).itemsize, dtype=dtype)
        check(lib().carat_hip_runner_copy_tensor(self._handle, name.encode(), ptr(out),
                                                 ctypes.c_size_t(out.nbytes), 0))
        return out

    def write(self, name: str, values: np.ndarray) -> None:
        values = np.ascontiguousarray(values)
        check(lib().carat_hip_runner_copy_tensor(self._handle, name.encode(), ptr(values),
                                                 ctypes.c_size_t(values.nbytes), 1))

    def set_graphs(self, enabled: bool) -> None:
        check(lib().carat_hip_runner_set_graphs(self._handle, int(enabled)))

    def set_qkv_fusion(self, enabled: bool) -> None:
        """Whether verify attention post-processes its own QKV rows (default) or the separate
        QKV kernel runs first; the same results bit for bit."""
        check(lib().carat_hip_runner_set_qkv_fusion(self._handle, int(enabled)))

    def set_fused_quantization(self, mode: int) -> None:
        """0 (default) separate quantisation kernel, 1 fused into the layer-end rows, 2 fused with a
        zero wait bound (error-path test)."""
        check(lib().carat_hip_runner_set_fused_quantization(self._handle, int(mode)))

    PROBES = {"qkv_gemm": 0, "o_gemm": 1, "gate_up_gemm": 2, "down_gemm": 3, "lm_head_gemm": 4,
              "sliding_attention": 5, "global_attention": 6}

    def set_probe(self, kind: str | None) -> None:
        check(lib().carat_hip_runner_set_probe(self._handle, -1 if kind is None else self.PROBES[kind]))

    def read_probe(self) -> tuple[float, int]:
        total = ctypes.c_float()
        launches = ctypes.c_int()
        check(lib().carat_hip_runner_read_probe(self._handle, ctypes.byref(total), ctypes.byref(launches)))
        return total.value, launches.value

    def stream_gemm_probe(self, kind: str, passes: int = 1) -> tuple[float, int]:
        """Mean ms per launch of one per-layer kernel kind (an fp8 GEMM or the sliding / global
        verify attention), launched back to back over every layer that has it."""
        avg = ctypes.c_float()
        launches = ctypes.c_int()
        check(lib().carat_hip_runner_stream_gemm_probe(self._handle, self.PROBES[kind], passes,
                                                       ctypes.byref(avg), ctypes.byref(launches)))
        return avg.value, launches.value

    def prefill_slot(self, slot: int, token_ids: Sequence[int], chunk_tokens: int = 1024) -> int:
        """prefill_slot (batch_model_runner.h:34): the greedy next token after the prompt."""
        toks = _i32(token_ids)
        out = ctypes.c_int32()
        check(lib().carat_hip_runner_prefill_slot(self._handle, slot, ptr(toks), len(toks), chunk_tokens,
                                                  ctypes.byref(out)))
        self._read_predictions()
        return out.value

    def prefill_slots_chunks(self, slots: Sequence[int], token_ids: Sequence[Sequence[int]],
                             chunk_tokens: int) -> list[int | None]:
        """prefill_slots_chunks (batch_model_runner.h:40-43): None where the prompt is not yet
        fully resident."""
        flat = _i32([t for row in token_ids for t in row])
        offsets = _i32(np.concatenate([[0], np.cumsum([len(r) for r in token_ids])]).astype(int))
        out = np.zeros(len(slots), np.int32)
        check(lib().carat_hip_runner_prefill_slots_chunks(self._handle, len(slots), ptr(_i32(slots)),
                                                          ptr(offsets), ptr(flat), chunk_tokens, ptr(out)))
        self._read_predictions()
        return [None if v < 0 else int(v) for v in out]

    def prefill_slot_from_prefix(self, slot: int, token_ids: Sequence[int], cached_prefix_tokens: int,
                                 chunk_tokens: int = 1024) -> int:
        """prefill_slot_from_prefix (batch_model_runner.h:36-37)."""
        toks = _i32(token_ids)
        out = ctypes.c_int32()
        check(lib().carat_hip_runner_prefill_slot_from_prefix(self._handle, slot, ptr(toks), len(toks),
                                                              cached_prefix_tokens, chunk_tokens,
                                                              ctypes.byref(out)))
        self._read_predictions()
        return out.value

    def prefill_slot_chunk(self, slot: int, token_ids: Sequence[int], chunk_tokens: int) -> int | None:
        """prefill_slot_chunk (batch_model_runner.h:38-39): None until the prompt is resident."""
        toks = _i32(token_ids)
        out = ctypes.c_int32()
        check(lib().carat_hip_runner_prefill_slot_chunk(self._handle, slot, ptr(toks), len(toks),
                                                        chunk_tokens, ctypes.byref(out)))
        self._read_predictions()
        return None if out.value < 0 else out.value

    @staticmethod
    def _pack(token_ids: Sequence[Sequence[int]]):
        flat = _i32([t for row in token_ids for t in row])
        offsets = _i32(np.concatenate([[0], np.cumsum([len(r) for r in token_ids])]).astype(int))
        return flat, offsets

    def prefill_slots_suffix(self, slots: Sequence[int], token_ids: Sequence[Sequence[int]]) -> list[int]:
        """prefill_slots_suffix (batch_model_runner.h:44-45)."""
        flat, offsets = self._pack(token_ids)
        out = np.zeros(len(slots), np.int32)
        check(lib().carat_hip_runner_prefill_slots_suffix(self._handle, len(slots), ptr(_i32(slots)),
                                                          ptr(offsets), ptr(flat), ptr(out)))
        self._read_predictions()
        return out.tolist()

    def prefill_slots_suffix_layer_slice(self, slots: Sequence[int], token_ids: Sequence[Sequence[int]],
                                         maximum_layers: int) -> tuple[bool, list[int]]:
        """prefill_slots_suffix_layer_slice (batch_model_runner.h:46-50): (complete, predictions)."""
        flat, offsets = self._pack(token_ids)
        out = np.zeros(len(slots), np.int32)
        complete = ctypes.c_int()
        check(lib().carat_hip_runner_prefill_slots_suffix_layer_slice(
            self._handle, len(slots), ptr(_i32(slots)), ptr(offsets), ptr(flat), maximum_layers,
            ctypes.byref(complete), ptr(out)))
        return (True, out.tolist()) if complete.value else (False, [])

    def abort_suffix_layer_slices(self) -> None:
        check(lib().carat_hip_runner_abort_suffix_layer_slices(self._handle))

    def has_suffix_layer_slices(self) -> bool:
        out = ctypes.c_int()
        check(lib().carat_hip_runner_has_suffix_layer_slices(self._handle, ctypes.byref(out)))
        return bool(out.value)

    def clone_slot(self, source_slot: int, destination_slot: int) -> int:
        """clone_slot (batch_model_runner.h:53): KV bytes copied."""
        out = ctypes.c_uint64()
        check(lib().carat_hip_runner_clone_slot(self._handle, source_slot, destination_slot,
                                                ctypes.byref(out)))
        return out.value

    def append(self, token_ids: Sequence[int]) -> list[int]:
        """append (batch_model_runner.h:33): one lock-step decode token for every slot."""
        toks = _i32(token_ids)
        out = np.zeros(len(toks), np.int32)
        check(lib().carat_hip_runner_append(self._handle, ptr(toks), len(toks), ptr(out)))
        self._read_predictions()
        return out.tolist()

    def _read_predictions(self) -> None:
        count = ctypes.c_int()
        check(lib().carat_hip_runner_last_predictions(self._handle, None, 0, ctypes.byref(count)))
        buf = np.zeros(max(count.value, 1), np.int32)
        check(lib().carat_hip_runner_last_predictions(self._handle, ptr(buf), count.value,
                                                      ctypes.byref(count)))
        self.last_predictions = buf[: count.value].tolist()

    def timing(self) -> tuple[float, float]:
        v = ctypes.c_float()
        d = ctypes.c_float()
        check(lib().carat_hip_runner_timing(self._handle, ctypes.byref(v), ctypes.byref(d)))
        return v.value, d.value


def _c_i32(values: Iterable[int]):
    """A ctypes int32 array (at least one element, so the pointer is never null) and its length:
    the host helpers run once per request per step, so they avoid numpy's allocation cost."""
    v = [int(x) for x in values]
    return (ctypes.c_int32 * max(len(v), 1))(*v), len(v)


def acceptance_cap(depth: int, remaining: int, proposals: Sequence[int], stop_ids: Iterable[int]) -> int:
    """speculation.h:11-12."""
    props, n = _c_i32(proposals)
    stops, m = _c_i32(stop_ids)
    out = ctypes.c_int()
    check(lib().carat_hip_acceptance_cap(depth, remaining, props, n, stops, m, ctypes.byref(out)))
    return out.value


def commit_speculation(forced_token: int, accepted_drafts: Sequence[int], next_token: int,
                       stop_ids: Iterable[int]):
    """speculation.h:24-27 -> (resident_tokens, emitted_tokens, next_token, stopped)."""
    drafts, n = _c_i32(accepted_drafts)
    stops, m = _c_i32(stop_ids)
    resident = (ctypes.c_int32 * (n + 1))()
    emitted = (ctypes.c_int32 * (n + 1))()
    nr, ne, nxt, stopped = ctypes.c_int(), ctypes.c_int(), ctypes.c_int32(), ctypes.c_int()
    check(lib().carat_hip_commit_speculation(int(forced_token), drafts, n, int(next_token), stops, m,
                                             resident, ctypes.byref(nr), emitted, ctypes.byref(ne),
                                             ctypes.byref(nxt), ctypes.byref(stopped)))
    return (resident[: nr.value], emitted[: ne.value], int(nxt.value), bool(stopped.value))
