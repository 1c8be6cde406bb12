"""The C-ABI library loads on the CPU, exports every entry point include/carat_hip.h declares, and
its host-only entry points (speculation helpers, validation, RoPE tables) behave like the
reference. No kernel is launched here."""
import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest

from carat_amd import _lib, runner
from oracle import oracle

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    header = (ROOT / "include" / "carat_hip.h").read_text()
    return sorted(set(re.findall(r"\b(carat_hip_\w+)\s*\(", header)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(_lib.EXPORTED) == names


def test_speculation_helpers_match_reference_vectors():
    golden = json.loads((ROOT / "tests" / "golden" / "speculation_vectors.json").read_text())
    for case in golden["acceptance_cap"]:
        got = runner.acceptance_cap(case["depth"], case["remaining"], case["proposals"], case["stops"])
        assert got == case["expected"], case
    for case in golden["commit_speculation"]:
        e = case["expected"]
        got = runner.commit_speculation(case["forced"], case["drafts"], case["next"], case["stops"])
        assert got == (e["resident"], e["emitted"], e["next"], e["stopped"]), case


def test_rope_table_matches_oracle():
    for dim, prop in ((128, False), (128, True), (256, False), (512, True)):
        cos = np.empty((300, dim), np.uint16)
        sin = np.empty((300, dim), np.uint16)
        _lib.check(_lib.lib().carat_hip_rope_table(dim, int(prop), 300, _lib.ptr(cos), _lib.ptr(sin)))
        ocos, osin = oracle.rope_table(dim, prop, 300)
        # same double-precision evaluation -> identical tables
        assert np.array_equal(cos, ocos) and np.array_equal(sin, osin)


def test_errors_come_back_as_messages():
    lib = _lib.lib()
    out = ctypes.c_int()
    status = lib.carat_hip_acceptance_cap(4, 4, None, 3, None, 0, ctypes.byref(out))
    assert status != 0
    assert b"invalid acceptance cap arguments" in lib.carat_hip_last_error()
    with pytest.raises(_lib.CaratError):
        _lib.check(lib.carat_hip_runner_batch(None, ctypes.byref(out)))


def test_gemm_plan_is_the_runner_dispatch():
    """The layouts and split-K factors the runner uses at the verify shapes (host-only query)."""
    lib = _lib.lib()

    def plan(n, k, fp8, gate_up):
        f, w, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _lib.check(lib.carat_hip_gemm_plan(n, k, fp8, gate_up, ctypes.byref(f), ctypes.byref(w),
                                           ctypes.byref(s)))
        return f.value, w.value, s.value

    assert plan(8192, 5376, 1, 0) == (1, 4, 2)       # qkv
    assert plan(5376, 4096, 1, 0) == (1, 3, 2)       # o (3-wave blocks: 224 workgroups)
    assert plan(43008, 5376, 1, 1) == (4, 3, 1)      # gate/up (GELU epilogue: no split-K)
    assert plan(5376, 21504, 1, 0) == (1, 4, 3)      # down
    assert plan(262144, 5376, 1, 0) == (4, 4, 1)     # lm_head
    with pytest.raises(_lib.CaratError):
        _lib.check(lib.carat_hip_gemm_plan(100, 5376, 1, 0, None, None, None))


def test_noalloc_argmax_rejects_shapes_beyond_its_scratch():
    """The size check runs before any device call, so it is testable without a GPU."""
    lib = _lib.lib()
    # 512 requests x 8 rows x 32 fp32 chunks = 131072 keys > 65536
    status = lib.carat_hip_argmax_accept_noalloc(ctypes.c_void_p(16), None, 512, 8, 262144, None,
                                                 None, None, None, None, None, None)
    assert status != 0
    assert b"exceed the fixed scratch of 65536" in lib.carat_hip_last_error()
