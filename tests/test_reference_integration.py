"""The reference's own serving loop compiles against the drop-in (CPU; needs the reference tree).

native_runtime_main.cpp -- ContinuousScheduler with its speculative_decode cycle
(native_runtime_main.cpp:583-678), which constructs and drives Gemma4BatchModelRunner -- is
compiled unchanged with the reference's warning flags as errors (CMakeLists.txt:156, 199-205 host
compile), with carat_amd/binding ahead of the reference's include/ so that
"carat/batch_model_runner.h" is the MI355X runner. The reference-side binding of the
constructor (carat_amd/binding/batch_model_runner_binding.cpp) compiles the same way. Every
C-ABI symbol the two objects need is exported by libcarat_hip.so, and the constructor the
scheduler calls is the one the binding defines. (A full executable link also needs the
reference's CUDA arenas and HTTP server, which stay in the reference.)"""
import subprocess
from pathlib import Path

import pytest

from carat_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
REF = Path("/root/reference")
FLAGS = ["-std=c++20", "-c", "-Wall", "-Wextra", "-Wpedantic", "-Wconversion", "-Wshadow", "-Werror"]

pytestmark = pytest.mark.skipif(not (REF / "src" / "native_runtime_main.cpp").exists(),
                                reason="the reference tree is not present")


def compile_object(source: Path, out: Path) -> None:
    includes = [ROOT / "carat_amd" / "binding", ROOT / "include", REF / "include", REF / "src",
                REF / "support" / "include"]
    cmd = ["g++", *FLAGS, *[f"-I{p}" for p in includes], str(source), "-o", str(out)]
    result = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert result.returncode == 0, result.stderr[-4000:]


def symbols(args, path):
    out = subprocess.run(["nm", *args, str(path)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_scheduler_compiles_against_the_drop_in(tmp_path):
    scheduler = tmp_path / "native_runtime_main.o"
    binding = tmp_path / "binding.o"
    compile_object(REF / "src" / "native_runtime_main.cpp", scheduler)
    compile_object(ROOT / "carat_amd" / "binding" / "batch_model_runner_binding.cpp", binding)
    needed = {s for s in symbols(["-u"], scheduler) | symbols(["-u"], binding) if s.startswith("carat_hip_")}
    assert {"carat_hip_runner_verify", "carat_hip_runner_draft", "carat_hip_runner_append_ragged",
            "carat_hip_runner_create_from_device_weights"} <= needed
    exported = symbols(["-D", "--defined-only"], _lib.LIBRARY_PATH)
    assert needed <= exported, sorted(needed - exported)
    # the reference constructor (batch_model_runner.h:24-28) the scheduler calls is the binding's
    ctor = [s for s in symbols(["-u"], scheduler) if "Gemma4BatchModelRunnerC" in s and "Gemma4Config" in s]
    assert ctor and set(ctor) <= symbols(["--defined-only"], binding), ctor
