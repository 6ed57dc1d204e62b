"""The host C++ under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only): the residency
policy (urbilateria_amd/csrc/urb_residency.cpp) and the oracle (oracle/urb_oracle.cpp), each
linked into a driver under tests/sanitize/ and built with g++ into a temporary directory."""

import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


def _build_and_run(name, sources, extra=()):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, name)
        cmd = ["g++", "-std=c++17", "-O1", "-g", *SAN, *extra, "-o", exe,
               *[os.path.join(ROOT, s) for s in sources], "-lpthread"]
        b = subprocess.run(cmd, capture_output=True, text=True)
        assert b.returncode == 0, b.stderr
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
                   UBSAN_OPTIONS="print_stacktrace=1")
        r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
        assert "ERROR" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
        return r.stdout


def test_residency_policy_is_clean_under_asan_and_ubsan():
    out = _build_and_run("lru_driver", ["tests/sanitize/lru_driver.cpp",
                                        "urbilateria_amd/csrc/urb_residency.cpp"])
    assert "lru driver ok" in out


def test_oracle_is_clean_under_asan_and_ubsan():
    out = _build_and_run("oracle_driver", ["tests/sanitize/oracle_driver.cpp",
                                           "oracle/urb_oracle.cpp"],
                         ["-mavx2", "-mfma", "-ffp-contract=off"])
    assert "oracle driver ok" in out
