"""Runs the C++ host layer's host-only tests (tests/cpp/test_host.cpp, `cpu` mode):
allocator, tensors, module state_dict, .sgrd and .safetensors formats."""
import subprocess

import pytest

import helpers

BIN = helpers.PKG_DIR / "host" / "test_host"


def test_host_layer_cpu():
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    r = subprocess.run([str(BIN), "cpu", str(helpers.GOLDEN_DIR / "persist")], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL PASSED" in r.stdout
