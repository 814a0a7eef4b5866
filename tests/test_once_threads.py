"""Thread safety of the library's host-side memo (helixml_amd/csrc/hx_once.h), which caches the
kernel LDS grants and device properties the dispatch code queries: a host-only program calls it
from 8 threads, built with ThreadSanitizer; any reported data race, a key computed twice or a
wrong value fails the test. (The GPU-side callers cannot run here; the memo is the shared part.)"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ needed")
def test_once_map_is_race_free_under_tsan(tmp_path):
    exe = tmp_path / "once_threads"
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=thread", "-pthread",
                        f"-I{ROOT / 'helixml_amd' / 'csrc'}", str(ROOT / "tests" / "cpp" / "once_threads.cpp"),
                        "-o", str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120,
                       env={"TSAN_OPTIONS": "halt_on_error=1 exitcode=66"})
    print(r.stdout, r.stderr[-3000:])
    assert "ThreadSanitizer" not in r.stderr
    assert r.returncode == 0
