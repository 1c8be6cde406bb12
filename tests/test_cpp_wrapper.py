"""The C++ drop-in header (include/carat_hip_runner.hpp) compiled with g++ against the library:
the reference's speculation helpers against its golden vectors on the CPU, and (GPU) a tiny
runner driven through the reference's class interface."""
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

from carat_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def build(tmp_path):
    lib_dir = _lib.LIBRARY_PATH.parent
    exe = tmp_path / "wrapper_check"
    subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Werror", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "cpp" / "wrapper_check.cpp"), f"-L{lib_dir}", "-lcarat_hip",
                    f"-Wl,-rpath,{lib_dir}", "-o", str(exe)], check=True, capture_output=True, text=True)
    return exe


def write_vectors(path):
    golden = json.loads((ROOT / "tests" / "golden" / "speculation_vectors.json").read_text())
    ls = lambda v: f"{len(v)} {' '.join(map(str, v))}".strip()
    lines = []
    for c in golden["acceptance_cap"]:
        lines.append(f"cap {c['depth']} {c['remaining']} {ls(c['proposals'])} {ls(c['stops'])} {c['expected']}")
    for c in golden["commit_speculation"]:
        e = c["expected"]
        lines.append(f"commit {c['forced']} {ls(c['drafts'])} {c['next']} {ls(c['stops'])} "
                     f"{ls(e['resident'])} {ls(e['emitted'])} {e['next']} {int(e['stopped'])}")
    path.write_text("\n".join(lines) + "\n")
    return len(lines)


def test_cpp_wrapper_speculation_helpers(tmp_path):
    exe = build(tmp_path)
    n = write_vectors(tmp_path / "vectors.txt")
    out = subprocess.run([str(exe), "vectors", str(tmp_path / "vectors.txt")], capture_output=True,
                         text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    assert f"{n} speculation cases, 0 failures" in out.stdout


def gpu_initialised_here() -> bool:
    """Whether this process has opened the GPU: the HIP runtime opens /dev/kfd when it
    initialises (torch's lazy CUDA init, or any HIP call through the library)."""
    torch = sys.modules.get("torch")
    if torch is not None and torch.cuda.is_initialized():
        return True
    fd_dir = Path("/proc/self/fd")
    for fd in fd_dir.iterdir() if fd_dir.exists() else ():
        try:
            if os.readlink(fd) == "/dev/kfd":
                return True
        except OSError:
            continue
    return False


@pytest.mark.gpu
def test_cpp_wrapper_runner(tmp_path):
    # The runner program is started as a child process; a process that has initialised the GPU
    # must not fork and exec another program, so this test has to run before any GPU call here.
    if gpu_initialised_here():
        pytest.fail("test_cpp_wrapper_runner must run before this pytest process touches the GPU: "
                    "run it first or in a process of its own")
    exe = build(tmp_path)
    print("case: C++ wrapper runner program", flush=True)
    out = subprocess.run([str(exe), "runner"], capture_output=True, text=True, timeout=110)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "runner checks done, 0 failures" in out.stdout
