"""The library's host C++ -- block allocator and tables (block_table.cpp),
the engine step machine (pkv_sched.cpp) and the compaction planner
(compact_plan.cpp) -- built with g++ and AddressSanitizer +
UndefinedBehaviorSanitizer (leak detection on) and driven through their
entry points by tests/sanitize/host_check.cpp on seeded random workloads.
The driver also checks the allocator against a model of block_table.rs, the
planner by executing its plans, and the scheduler's block accounting; any
sanitizer report or failed check fails the test.  CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ai-engine_amd", "csrc")
SOURCES = [os.path.join(ROOT, "tests", "sanitize", "host_check.cpp"),
           os.path.join(CSRC, "block_table.cpp"), os.path.join(CSRC, "pkv_sched.cpp"),
           os.path.join(CSRC, "compact_plan.cpp")]


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_host_code_under_address_and_ub_sanitizers(tmp_path):
    exe = str(tmp_path / "host_check")
    build = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
             "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
             # the runtimes linked in, so no library load order matters
             "-static-libasan", "-static-libubsan",
             f"-I{os.path.join(ROOT, 'include')}", *SOURCES, "-o", exe]
    r = subprocess.run(build, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe, "200"], capture_output=True, text=True, timeout=300, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert "0 failures" in r.stdout, out[-2000:]
