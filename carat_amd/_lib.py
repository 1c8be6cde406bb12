"""ctypes binding of libcarat_hip.so (the C ABI declared in include/carat_hip.h).

The product path is the HIP library: importing this module fails loudly when the library is
missing, and nothing here falls back to a CPU implementation.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint16, c_uint64, c_void_p
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libcarat_hip.so"

# Every symbol declared in include/carat_hip.h (checked by tests/test_abi.py).
EXPORTED = [
    "carat_hip_last_error", "carat_hip_device_count", "carat_hip_synchronize",
    "carat_hip_acceptance_cap", "carat_hip_commit_speculation",
    "carat_hip_gemma4_benchmark_desc", "carat_hip_runner_create", "carat_hip_runner_destroy",
    "carat_hip_checkpoint_describe", "carat_hip_runner_create_from_checkpoint",
    "carat_hip_runner_prefill_slot", "carat_hip_runner_prefill_slots_chunks",
    "carat_hip_runner_prefill_slot_from_prefix", "carat_hip_runner_prefill_slot_chunk",
    "carat_hip_runner_prefill_slots_suffix", "carat_hip_runner_prefill_slots_suffix_layer_slice",
    "carat_hip_runner_abort_suffix_layer_slices", "carat_hip_runner_has_suffix_layer_slices",
    "carat_hip_runner_clone_slot", "carat_hip_runner_append",
    "carat_hip_runner_last_predictions", "carat_hip_runner_create_from_device_weights",
    "carat_hip_runner_verify", "carat_hip_runner_append_ragged", "carat_hip_runner_draft",
    "carat_hip_runner_has_assistant",
    "carat_hip_runner_batch", "carat_hip_runner_position", "carat_hip_runner_slot_position",
    "carat_hip_runner_reset_slot", "carat_hip_runner_seed_empty_cache_for_benchmark",
    "carat_hip_runner_seed_random_cache", "carat_hip_runner_set_slot_position",
    "carat_hip_runner_tensor", "carat_hip_runner_copy_tensor", "carat_hip_runner_set_graphs",
    "carat_hip_runner_set_fused_quantization", "carat_hip_runner_set_qkv_fusion",
    "carat_hip_runner_timing", "carat_hip_runner_set_probe", "carat_hip_runner_read_probe",
    "carat_hip_runner_stream_gemm_probe", "carat_hip_bench_speculative_cycle",
    "carat_hip_argmax_accept", "carat_hip_argmax_accept_noalloc", "carat_hip_gemm_plan", "carat_hip_fp8_linear",
    "carat_hip_fp8_linear_scaled", "carat_hip_fp8_weight_scale_elements", "carat_hip_quantize_weight_fp8",
    "carat_hip_bf16_linear", "carat_hip_verify_attention", "carat_hip_row_op",
    "carat_hip_qkv_post", "carat_hip_rope_table", "carat_hip_f32_to_e4m3",
]


class LayerDesc(ctypes.Structure):
    _fields_ = [("sliding", c_int), ("query_heads", c_int), ("kv_heads", c_int),
                ("head_dimension", c_int), ("key_equals_value", c_int)]


class ModelDesc(ctypes.Structure):
    _fields_ = [("hidden", c_int), ("intermediate", c_int), ("vocabulary", c_int),
                ("sliding_window", c_int), ("rms_norm_epsilon", c_float), ("layer_count", c_int),
                ("layers", POINTER(LayerDesc)), ("assistant", c_int), ("assistant_hidden", c_int),
                ("assistant_intermediate", c_int), ("assistant_layers", c_int),
                ("assistant_query_heads", c_int), ("seed", c_uint64), ("weight_std", c_float),
                ("assistant_fp8_mode", c_int), ("fp8_scaling", c_int)]


class RowArgs(ctypes.Structure):
    _fields_ = [("source", c_int), ("rows", c_int), ("width", c_int), ("eps", c_float),
                ("embedding", c_void_p), ("tokens", c_void_p), ("vocabulary", c_int),
                ("embed_scale", c_float), ("partials", c_void_p), ("splits", c_int),
                ("x_amax", c_void_p), ("w_scale", c_void_p), ("x", c_void_p), ("v_out", c_void_p),
                ("w1", c_void_p), ("residual", c_void_p), ("scalar", c_void_p),
                ("r1_out", c_void_p), ("w2", c_void_p), ("y_out", c_void_p), ("y_amax", c_void_p)]


class CaratError(RuntimeError):
    pass


def load(path: Path | str = LIBRARY_PATH) -> ctypes.CDLL:
    path = Path(path)
    if not path.exists():
        raise CaratError(f"{path} is missing: build it with `python -m carat_amd.build` "
                         "(the HIP path has no fallback)")
    lib = ctypes.CDLL(str(path))
    lib.carat_hip_last_error.restype = c_char_p
    lib.carat_hip_runner_destroy.restype = None
    for name in EXPORTED:
        getattr(lib, name)  # every declared entry point must resolve
    return lib


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def check(status: int) -> None:
    if status != 0:
        raise CaratError(lib().carat_hip_last_error().decode())


class _Pointer(c_void_p):
    """A void* that keeps the tensor/array it points into alive while it is referenced."""


def ptr(x) -> c_void_p:
    """Device/host address of a torch tensor or numpy array (or an int address / None)."""
    if x is None:
        return c_void_p(0)
    if isinstance(x, int):
        return c_void_p(x)
    pointer = _Pointer(x.data_ptr() if hasattr(x, "data_ptr") else x.ctypes.data)
    pointer.keep = x
    return pointer
