"""Writes tests/golden/persist/: checkpoints saved by the reference itself.

Run in the development container only (it needs oracle/_ref/libsgref.so, built
by `make -C oracle ref` from the reference's own sources):

    python tests/golden/make_persist.py

For each weight below, the reference's own nn::QuantizedLinear (per-channel
INT8) or nn::QuantizedLinear4Bit is built with from_float from a seeded fp32
weight and bias (include/sovereigngrad/nn.hpp:946-954, 984-992) and saved with
serialization::save_module (.sgrd, src/serialization.cpp:14-47,103-105) and
safetensors::save_module (.safetensors, src/safetensors.cpp:174-230,288-290),
either alone or as submodule "proj" of a parent module (keys "proj.qdata").
A companion <weight>.io.sgrd, written by the reference's save_checkpoint
(src/serialization.cpp:14-47),
holds the float weight W, the bias b, an input x, the reference module's own
forward y = x . dequantize(W) + b (nn.hpp:956-958, 994-996) after loading its
saved file back, and `meta` = [bits, K, N, group_size, M, nested].  The files
are data only.
"""
from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.oracle import Reference  # noqa: E402

spec = importlib.util.spec_from_file_location("sgq_synth", ROOT / "soverign-grad_amd" / "synth.py")
synth = importlib.util.module_from_spec(spec)
spec.loader.exec_module(synth)

OUT = Path(__file__).with_name("persist")

# name, bits, K, N, group, batch rows, submodule name ("" = the layer itself)
WEIGHTS = [
    ("q8_pc_64x48", 8, 64, 48, 0, 5, ""),
    ("q8_pc_nested_40x72", 8, 40, 72, 0, 3, "proj"),
    ("q4_g32_64x48", 4, 64, 48, 32, 5, ""),
    ("q4_g128_96x256", 4, 96, 256, 128, 4, ""),
    ("q4_g32_nested_48x40", 4, 48, 40, 32, 2, "proj"),
]


def main() -> None:
    ref = Reference()
    OUT.mkdir(exist_ok=True)
    index = []
    for i, (name, bits, K, N, G, M, child) in enumerate(WEIGHTS):
        assert child in ("", "proj")  # the readers know the submodule by this one name
        seed = synth.config_seed(200 + i)
        W = synth.normal((K, N), seed, synth.STREAM_W, 0.0, 0.02)
        b = synth.normal((N,), seed, synth.STREAM_BIAS, 0.0, 0.02)
        x = synth.normal((M, K), seed, synth.STREAM_X, 0.0, 1.0)
        files = []
        y_first = None
        for ext in (".sgrd", ".safetensors"):
            path = OUT / f"{name}{ext}"
            ref.save_qlinear(path, bits, W, G if bits == 4 else 32, b, child)
            # The reference reads its own file back into a fresh module.
            y = ref.load_qlinear_forward(path, bits, K, N, x, G if bits == 4 else 32, child)
            if y_first is None:
                y_first = y
            assert np.array_equal(y.view(np.uint32), y_first.view(np.uint32)), "formats disagree"
            files.append(path.name)
        pre = f"{child}." if child else ""
        q = ref.read_entry(OUT / files[0], pre + "qdata")
        s = ref.read_entry(OUT / files[0], pre + "scales")
        # meta: bits, K, N, group size, batch rows, nested under "proj" (1) or not (0)
        meta = np.array([bits, K, N, G, M, 1 if child else 0], np.float32)
        io = {"W": W, "b": b.reshape(1, N), "x": x, "y": y_first, "meta": meta}
        ref.save_entries(OUT / f"{name}.io.sgrd", io)
        for k, t in io.items():  # the reference reads it back bit for bit
            back = ref.read_entry(OUT / f"{name}.io.sgrd", k)
            assert np.array_equal(back.view(np.uint32), np.ascontiguousarray(t).view(np.uint32)), k
        index.append({"name": name, "bits": bits, "K": K, "N": N, "group_size": G, "M": M, "prefix": child,
                      "files": files, "io": f"{name}.io.sgrd", "scale_count": int(s.size),
                      "codes_min": float(q.min()), "codes_max": float(q.max())})
    (OUT / "index.json").write_text(json.dumps({"generator": "tests/golden/make_persist.py", "weights": index},
                                               indent=1))
    total = sum(p.stat().st_size for p in OUT.iterdir())
    print(f"wrote {len(index)} weights into {OUT} ({total} bytes)")


if __name__ == "__main__":
    main()
