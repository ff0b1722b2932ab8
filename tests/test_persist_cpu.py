"""Checkpoint interchange with the reference (host-only; no GPU).

tests/golden/persist/ holds quantized modules saved by the reference itself
(tests/golden/make_persist.py: QuantizedLinear / QuantizedLinear4Bit built with
from_float, saved with serialization::save_module and safetensors::save_module,
src/serialization.cpp:14-47,103-105, src/safetensors.cpp:174-234,288-290).

- The host layer's loaders read them (tests/cpp/test_host.cpp `cpu` mode with
  the fixture directory) and its writers save the same module trees again.
- The reference (oracle/_ref, compiled from its own sources in the development
  container) loads the host-written files with its strict load_module into a
  fresh module and runs its forward: the output must equal, bit for bit, the
  forward of the module it saved itself (same codes, same scales, same bias).
- tests/golden/persist/host/, when present, holds the same weights quantized by
  this library on the GPU (from_float) and saved by the host layer
  (test_host `gpu` mode with an output directory); the reference loads those too.
"""
import json
import subprocess

import numpy as np
import pytest

import helpers

BIN = helpers.PKG_DIR / "host" / "test_host"
PERSIST = helpers.GOLDEN_DIR / "persist"
INDEX = json.loads((PERSIST / "index.json").read_text())["weights"]


def _io(ref, w):
    io = PERSIST / w["io"]
    return {k: ref.read_entry(io, k) for k in ("W", "b", "x", "y")}


@pytest.fixture(scope="module")
def host_written(tmp_path_factory):
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    out = tmp_path_factory.mktemp("host_written")
    r = subprocess.run([str(BIN), "cpu", str(PERSIST), str(out)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "reference-written modules" in r.stdout and "ALL PASSED" in r.stdout
    return out


@pytest.mark.parametrize("w", INDEX, ids=[w["name"] for w in INDEX])
@pytest.mark.parametrize("ext", [".sgrd", ".safetensors"])
def test_reference_loads_host_written(ref, host_written, w, ext):
    path = host_written / f"{w['name']}{ext}"
    pre = f"{w['prefix']}." if w["prefix"] else ""
    assert ref.list_entries(path) == sorted(pre + k for k in ("bias", "qdata", "scales"))
    io = _io(ref, w)
    y = ref.load_qlinear_forward(path, w["bits"], w["K"], w["N"], io["x"], w["group_size"] or 32, w["prefix"])
    assert helpers.same_bits(y, io["y"])


@pytest.mark.parametrize("w", INDEX, ids=[w["name"] for w in INDEX])
def test_reference_files_agree_with_oracle(ref, oracle, w):
    """The reference-written codes and scales are the oracle's quantization of
    W bit for bit, and the reference module's forward is the oracle's."""
    path = PERSIST / w["files"][0]
    pre = f"{w['prefix']}." if w["prefix"] else ""
    io = _io(ref, w)
    q, s = ref.read_entry(path, pre + "qdata"), ref.read_entry(path, pre + "scales")
    if w["bits"] == 8:
        qo, so = oracle.quantize_int8(io["W"], 1)
        yo = oracle.quantized_matmul_int8(io["x"], qo, so, 1, io["b"])
    else:
        qo, so = oracle.quantize_int4(io["W"], w["group_size"])
        yo = oracle.quantized_matmul_int4(io["x"], qo, so, w["group_size"], io["b"])
    assert helpers.same_bits(q, qo) and helpers.same_bits(s.reshape(-1), so.reshape(-1))
    assert helpers.same_bits(io["y"], yo)


GPU_WRITTEN = PERSIST / "host"


@pytest.mark.skipif(not GPU_WRITTEN.exists(), reason="no GPU-written checkpoints committed")
@pytest.mark.parametrize("w", INDEX, ids=[w["name"] for w in INDEX])
@pytest.mark.parametrize("ext", [".sgrd", ".safetensors"])
def test_reference_loads_gpu_quantized_modules(ref, w, ext):
    path = GPU_WRITTEN / f"{w['name']}{ext}"
    io = _io(ref, w)
    pre = f"{w['prefix']}." if w["prefix"] else ""
    # Codes and scales quantized on the GPU equal the reference's own.
    for k in ("qdata", "scales", "bias"):
        assert helpers.same_bits(ref.read_entry(path, pre + k), ref.read_entry(PERSIST / w["files"][0], pre + k)), k
    y = ref.load_qlinear_forward(path, w["bits"], w["K"], w["N"], io["x"], w["group_size"] or 32, w["prefix"])
    assert helpers.same_bits(y, io["y"])
