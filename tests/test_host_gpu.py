"""Runs the C++ host layer's GPU tests (tests/cpp/test_host.cpp, `gpu` mode):
the reference's quantization checks on CPU and CUDA devices, fused forward vs
dequantize+matmul+bias, the persistence bridge (.sgrd/.safetensors/
load_state_dict repack; modules saved by the reference itself, loaded on the
GPU and checked against its forward), Module::to, concurrent forwards, the HIP pool."""
import os
import subprocess

import pytest

import helpers

pytestmark = pytest.mark.gpu

BIN = helpers.PKG_DIR / "host" / "test_host"


def test_host_layer_gpu(dev):
    assert BIN.exists(), f"{BIN} is not built"
    # Loads the reference-written checkpoints of tests/golden/persist; with
    # SGQ_PERSIST_OUT set, also saves GPU-quantized modules there.
    args = [str(BIN), "gpu", str(helpers.GOLDEN_DIR / "persist")]
    if os.environ.get("SGQ_PERSIST_OUT"):
        args.append(os.environ["SGQ_PERSIST_OUT"])
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL PASSED" in r.stdout
