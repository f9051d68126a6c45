"""The page pool's claim logic (fastdms_amd/csrc/fdms_pool.h) replayed on the
host: the subtract-then-undo interleaving that handed one page out twice, a
swap that finds the counter moved, and a multi-threaded stress with real
atomics (tests/pool_claim_replay.cpp)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_claim_units_replays(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "pool_claim_replay"
    subprocess.run([gxx, "-std=c++17", "-O1", "-pthread", "-I", str(ROOT / "fastdms_amd" / "csrc"),
                    str(ROOT / "tests" / "pool_claim_replay.cpp"), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0 and res.stdout.strip() == "ok", res.stdout + res.stderr
