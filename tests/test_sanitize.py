"""Host sanitizer runs (CPU only): the packed NF4 file parser under a fuzz
harness, and the oracle's own tests against an oracle build, both with
AddressSanitizer and UndefinedBehaviorSanitizer (tests/sanitize/Makefile).
A sanitizer report aborts the process, so a clean exit is the check."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")


def _make(target):
    subprocess.run(["make", "-s", "-C", SAN, target], check=True)


def _gcc_lib(name):
    return subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True,
                          text=True, check=True).stdout.strip()


def test_nf4_file_parser_fuzz_under_asan_ubsan():
    _make("_build/nf4_fuzz")
    r = subprocess.run([os.path.join(SAN, "_build", "nf4_fuzz")], capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failures" in r.stdout


def test_oracle_tests_under_asan_ubsan():
    _make("_build/liboracle_san.so")
    env = dict(os.environ,
               LD_PRELOAD=f"{_gcc_lib('libasan.so')}:{_gcc_lib('libubsan.so')}",
               ASAN_OPTIONS="detect_leaks=0",
               QH_ORACLE_LIB=os.path.join(SAN, "_build", "liboracle_san.so"))
    tests = [os.path.join(ROOT, "tests", f) for f in
             ("test_oracle.py", "test_oracle_block.py", "test_golden.py")]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        *tests], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=900)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert " passed" in r.stdout
