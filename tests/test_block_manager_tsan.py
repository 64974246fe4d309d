"""Native multithreaded stress of the C++ BlockManager under ThreadSanitizer.

tests/native/bm_stress.cpp restates the reference's loom models
(src/block_manager.rs:304-548: unique ownership, refcount preventing early
reclaim, stale handles after reallocation, generation == 1 + allocations,
OutOfBlocks on exhaustion) as randomized stress runs over the C ABI.  It is
built here from zealot_amd/csrc/block_manager.cpp and status.cpp alone with
g++ -fsanitize=thread and must finish with no failed invariant and no
ThreadSanitizer report.  CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = [os.path.join(ROOT, "tests", "native", "bm_stress.cpp"),
       os.path.join(ROOT, "zealot_amd", "csrc", "block_manager.cpp"),
       os.path.join(ROOT, "zealot_amd", "csrc", "status.cpp")]


def _build(tmp_path, sanitize):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = str(tmp_path / f"bm_stress_{sanitize or 'plain'}")
    flags = ["-std=c++17", "-O1", "-g", "-pthread", "-Wall", "-Wextra"]
    if sanitize:
        flags.append(f"-fsanitize={sanitize}")
    r = subprocess.run([gxx, *flags, *SRC, "-o", exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def _run(exe, threads, iters):
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66 second_deadlock_stack=1")
    r = subprocess.run([exe, str(threads), str(iters)], capture_output=True, text=True, env=env, timeout=600)
    return r


def test_block_manager_stress_under_tsan(tmp_path):
    exe = _build(tmp_path, "thread")
    r = _run(exe, 8, 3000)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr[-4000:])
    assert "0 failures" in r.stdout


def test_block_manager_stress_plain_build_more_iterations(tmp_path):
    """The same invariants without the sanitizer's slowdown: more iterations
    and threads than the TSan run."""
    exe = _build(tmp_path, None)
    r = _run(exe, 16, 50000)
    assert r.returncode == 0, (r.stdout, r.stderr[-4000:])
    assert "0 failures" in r.stdout
