"""The host layer and the oracle under AddressSanitizer + UndefinedBehaviorSanitizer.

Builds soverign-grad_amd/host `make sanitize` (test_host_san: the host layer
and tests/cpp/test_host.cpp with -fsanitize=address,undefined, host code only)
and oracle `make sanitize` (liboracle_san.so), then runs:

- test_host_san cpu over the reference-written checkpoints (including every
  truncation and single-byte change of a .sgrd and a .safetensors file);
- tests/test_oracle.py against liboracle_san.so in a child interpreter that
  preloads the sanitizer runtimes.

Any sanitizer report fails the test (-fno-sanitize-recover: UBSan aborts).
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

import helpers

HOST = helpers.PKG_DIR / "host"
ORACLE = helpers.ROOT / "oracle"
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:allocator_may_return_null=1:abort_on_error=1",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


def _runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and Path(p).exists() else None


ASAN, UBSAN = _runtime("libasan.so"), _runtime("libubsan.so")
pytestmark = pytest.mark.skipif(ASAN is None or UBSAN is None, reason="gcc sanitizer runtimes not installed")


def _make(d):
    r = subprocess.run(["make", "-j8", "-C", str(d), "sanitize"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]


def _clean(out):
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-6000:]


def test_host_layer_under_sanitizers(tmp_path):
    _make(HOST)
    env = dict(os.environ, **SAN_ENV)
    r = subprocess.run([str(HOST / "test_host_san"), "cpu", str(helpers.GOLDEN_DIR / "persist"), str(tmp_path)],
                       capture_output=True, text=True, timeout=300, env=env)
    print(r.stdout[-3000:])
    _clean(r.stdout + r.stderr)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout, r.stdout[-3000:] + r.stderr[-3000:]
    assert "damaged checkpoint files" in r.stdout and "reference-written modules" in r.stdout


def test_oracle_under_sanitizers():
    _make(ORACLE)
    lib = ORACLE / "liboracle_san.so"
    env = dict(os.environ, **SAN_ENV, LD_PRELOAD=f"{ASAN}:{UBSAN}", SGQ_ORACLE_LIB=str(lib))
    probe = ("import sys; sys.path.insert(0, %r); from oracle.oracle import Oracle; Oracle(); "
             "print(any('liboracle_san.so' in l for l in open('/proc/self/maps')))" % str(helpers.ROOT))
    r = subprocess.run([sys.executable, "-c", probe], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0 and r.stdout.strip() == "True", r.stdout + r.stderr
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        str(helpers.ROOT / "tests" / "test_oracle.py")],
                       capture_output=True, text=True, timeout=600, env=env, cwd=str(helpers.ROOT))
    print(r.stdout[-2000:])
    _clean(r.stdout + r.stderr)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
