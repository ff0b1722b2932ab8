"""Writes tests/golden/golden.npz + golden.json from the compiled reference.

Run in the development container only (it needs oracle/_ref/libsgref.so, built
by `make -C oracle ref` from the reference's own sources):

    python tests/golden/make_golden.py

Every expected output comes from the reference's own functions
(quantization::quantize_int8/_int4, dequantize_*, quantized_matmul_*, silu /
mul composed as SwiGLU::forward composes them, rms_norm, softmax, embedding,
and LLaMABlock::forward written out with QuantizedLinear4Bit projections; see
oracle/ref_shim.cpp).  Inputs are seeded (soverign-grad_amd/synth.py) or
hand-built special values.  The fixtures are data only: inputs and the
reference's outputs.
"""
from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.oracle import BLOCK_PROJ, Reference, block_shapes  # noqa: E402

spec = importlib.util.spec_from_file_location("sgq_synth", ROOT / "soverign-grad_amd" / "synth.py")
synth = importlib.util.module_from_spec(spec)
spec.loader.exec_module(synth)

OUT_NPZ = Path(__file__).with_name("golden.npz")
OUT_JSON = Path(__file__).with_name("golden.json")


def special_values() -> np.ndarray:
    # max |x| = 127 makes inv_scale == 1 and scale == 1 for INT8, so rounding
    # ties, -0.0 results and clamping are visible directly in the codes.
    v = [127.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 0.49999997, -0.49999997, 126.5, -126.5, -0.3, -0.0, 0.0,
         1e-40, -1e-40, 1e-9, -1e-9, 64.25, -64.75]
    return np.array(v, dtype=np.float32)


def main() -> None:
    ref = Reference()
    arrays = {}
    cases = []
    rng_seed = synth.config_seed(100)

    def add(kind, params, **tensors):
        idx = len(cases)
        names = {}
        for k, v in tensors.items():
            key = f"c{idx}_{k}"
            arrays[key] = np.ascontiguousarray(v)
            names[k] = key
        cases.append({"kind": kind, "params": params, "arrays": names})

    def x_of(shape, stream, std=1.0):
        nonlocal rng_seed
        rng_seed += 1
        return synth.normal(shape, rng_seed, stream, 0.0, std)

    # ---- INT8 quantize + dequantize -------------------------------------
    for shape in [(16, 32), (33, 70), (1, 5), (7, 1), (3, 0), (24, 48)]:
        x = x_of(shape, 0)
        for scheme in (0, 1):
            q, s = ref.quantize_int8(x, scheme)
            d = ref.dequantize_int8(q.reshape(shape), s, scheme) if x.size else np.zeros(shape, np.float32)
            add("quantize_int8", {"shape": list(shape), "scheme": scheme}, x=x, q=q, s=s, deq=d)
    x1 = x_of((40,), 0)
    for scheme in (0, 1):
        q, s = ref.quantize_int8(x1, scheme)  # rank 1 always per-tensor
        add("quantize_int8", {"shape": [40], "scheme": scheme}, x=x1, q=q, s=s)

    sv = special_values()
    for scheme in (0, 1):
        x = sv.reshape(4, 5)
        q, s = ref.quantize_int8(x, scheme)
        add("quantize_int8", {"shape": [4, 5], "scheme": scheme, "special": True}, x=x, q=q, s=s)
    for special in ([np.nan, 1.0, -2.0, 0.25], [np.inf, 1.0, -2.0, -0.25], [-np.inf, 3.0, np.nan, 0.0],
                    [0.0, 0.0, 0.0, 0.0], [np.nan, np.nan, np.nan, np.nan]):
        x = np.array(special, dtype=np.float32).reshape(2, 2)
        for scheme in (0, 1):
            q, s = ref.quantize_int8(x, scheme)
            add("quantize_int8", {"shape": [2, 2], "scheme": scheme, "special": True}, x=x, q=q, s=s)

    # ---- INT4 quantize + dequantize --------------------------------------
    for shape, g in [((16, 32), 32), ((64, 256), 128), ((32, 16), 16), ((5, 13), 7), ((3, 11), 8),
                     ((8, 24), 0), ((4, 9), -5), ((16, 40), 24), ((2, 100), 64), ((1, 3), 32)]:
        x = x_of(shape, 0)
        q, s = ref.quantize_int4(x, g)
        d = ref.dequantize_int4(q, s, g if g > 0 else 32)
        add("quantize_int4", {"shape": list(shape), "group_size": g}, x=x, q=q, s=s, deq=d)
    x = np.array([7.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, -0.3, 6.5, -6.5, -0.0, 1e-40, np.nan, 1.0, -7.0, 4.0],
                 dtype=np.float32).reshape(2, 8)
    for g in (8, 16, 4):
        q, s = ref.quantize_int4(x, g)
        add("quantize_int4", {"shape": [2, 8], "group_size": g, "special": True}, x=x, q=q, s=s)
    x = np.array([np.inf, 1.0, -1.0, 0.5, -np.inf, 2.0, 3.0, 4.0], dtype=np.float32).reshape(2, 4)
    q, s = ref.quantize_int4(x, 4)
    add("quantize_int4", {"shape": [2, 4], "group_size": 4, "special": True}, x=x, q=q, s=s)

    # ---- forward: quantized_matmul ---------------------------------------
    for (M, K, N, scheme, with_bias) in [(1, 32, 16, 1, True), (4, 32, 16, 0, True), (9, 130, 77, 0, True),
                                         (37, 130, 77, 1, False), (40, 128, 96, 0, True), (1, 300, 70, 1, False),
                                         (17, 64, 64, 0, False), (8, 512, 64, 1, True)]:
        W = x_of((K, N), 0, 0.02)
        xx = x_of((M, K), 1)
        b = x_of((1, N), 2, 0.02) if with_bias else None
        q, s = ref.quantize_int8(W, scheme)
        y = ref.quantized_matmul_int8(xx, q, s, scheme, b)
        t = dict(x=xx, q=q, s=s, y=y)
        if b is not None:
            t["bias"] = b
        add("linear_int8", {"M": M, "K": K, "N": N, "scheme": scheme}, **t)
    for (M, K, N, g, with_bias) in [(1, 256, 256, 128, False), (4, 32, 16, 16, True), (8, 128, 96, 32, True),
                                    (3, 13, 5, 7, False), (16, 64, 40, 24, False), (33, 64, 128, 128, True),
                                    (1, 512, 128, 128, False), (5, 100, 12, 8, True)]:
        W = x_of((K, N), 0, 0.02)
        xx = x_of((M, K), 1)
        b = x_of((1, N), 2, 0.02) if with_bias else None
        q, s = ref.quantize_int4(W, g)
        y = ref.quantized_matmul_int4(xx, q, s, g, b)
        t = dict(x=xx, q=q, s=s, y=y)
        if b is not None:
            t["bias"] = b
        add("linear_int4", {"M": M, "K": K, "N": N, "group_size": g}, **t)

    # ---- silu and the gated MLP half of SwiGLU (nn.hpp:151-154) ------------
    sx = np.array([0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 3.0, -3.0, 10.0, -10.0, 20.0, -20.0, 88.0, -88.0, 89.0, -89.0,
                   104.0, -104.0, 1e-30, -1e-30, 1e-40, -1e-40, np.inf, -np.inf, np.nan, 1e30, -1e30],
                  dtype=np.float32)
    sx = np.concatenate([sx, x_of((64,), 0, 4.0)])
    add("silu", {"n": int(sx.size)}, x=sx, y=ref.silu(sx))
    for (M, K, N, bits, gs, with_bias) in [(1, 64, 32, 4, 32, True), (5, 96, 40, 4, 8, False),
                                           (8, 128, 64, 4, 128, True), (20, 64, 48, 4, 16, True),
                                           (3, 64, 36, 8, 0, True), (17, 40, 24, 8, 1, False)]:
        xx = x_of((M, K), 1)
        Wg, Wu = x_of((K, N), 0, 0.05), x_of((K, N), 0, 0.05)
        bg = x_of((1, N), 2, 0.5) if with_bias else None
        bu = x_of((1, N), 2, 0.5) if with_bias else None
        if bits == 4:
            qg, sg = ref.quantize_int4(Wg, gs)
            qu, su = ref.quantize_int4(Wu, gs)
            g = ref.quantized_matmul_int4(xx, qg, sg, gs, bg)
            u = ref.quantized_matmul_int4(xx, qu, su, gs, bu)
            params = {"M": M, "K": K, "N": N, "group_size": gs}
        else:
            qg, sg = ref.quantize_int8(Wg, gs)
            qu, su = ref.quantize_int8(Wu, gs)
            g = ref.quantized_matmul_int8(xx, qg, sg, gs, bg)
            u = ref.quantized_matmul_int8(xx, qu, su, gs, bu)
            params = {"M": M, "K": K, "N": N, "scheme": gs}
        h = ref.mul(ref.silu(g), u)
        t = dict(x=xx, qg=qg, sg=sg, qu=qu, su=su, y=h)
        if bg is not None:
            t["bias_gate"], t["bias_up"] = bg, bu
        add(f"swiglu_int{bits}", params, **t)

    # ---- rms_norm, softmax, embedding and the quantized LLaMA block ---------
    for (B, D, std) in [(2, 1, 1.0), (3, 3, 1.0), (2, 4, 2.0), (2, 7, 1.0), (3, 8, 1.0), (2, 9, 3.0), (2, 12, 1.0),
                        (2, 15, 1.0), (2, 16, 0.1), (3, 31, 1.0), (2, 97, 3.0), (2, 2048, 1.0)]:
        xx = x_of((B, D), 1, std)
        g = (1.0 + x_of((D,), 2, 0.1)).astype(np.float32)
        add("rms_norm", {"B": B, "D": D, "eps": 1e-5}, x=xx, g=g, y=ref.rms_norm(xx, g, 1e-5))
    xs = np.array([[0.0] * 6, [1e18, -1e18, 3.0, 0.0, 1.0, 2.0], [np.inf, 1.0, 2.0, 3.0, 4.0, 5.0],
                   [1e-30, -1e-30, 1e-38, 0.0, -0.0, 5e-39]], np.float32)
    gs6 = np.array([1.0, -1.0, 0.5, 2.0, 1.0, 3.0], np.float32)
    add("rms_norm", {"B": 4, "D": 6, "eps": 1e-5, "special": True}, x=xs, g=gs6, y=ref.rms_norm(xs, gs6, 1e-5))
    for (R, C) in [(1, 1), (3, 7), (4, 37), (2, 300)]:
        sc = x_of((R, C), 1, 3.0)
        add("softmax", {"R": R, "C": C}, x=sc, y=ref.softmax_rows(sc))
    sc = x_of((4, 9), 1, 3.0)
    sc[0, 3:] = -1e9
    sc[1, :] = 2.5
    sc[2, 1:] = -1e9
    sc[3, 0] = 80.0
    add("softmax", {"R": 4, "C": 9, "special": True}, x=sc, y=ref.softmax_rows(sc))
    ew = x_of((11, 24), 0)
    idx = np.array([0, 10, 3, -1, 11, 2.9, -0.5, 7, 7, 5.5], np.float32)
    add("embedding", {"V": 11, "E": 24}, idx=idx, w=ew, y=ref.embedding(idx, ew))
    for (L, D, H, G, heads, with_bias) in [(1, 32, 64, 32, 4, True), (5, 64, 160, 32, 4, True),
                                           (9, 128, 256, 128, 8, True), (12, 64, 96, 16, 2, False),
                                           (17, 32, 64, 32, 1, True)]:
        xx = x_of((L, D), 1)
        t = {"x": xx}
        proj = []
        for name, (K, N) in zip(BLOCK_PROJ, block_shapes(D, H)):
            W = x_of((K, N), 0, 0.05)
            q, s_ = ref.quantize_int4(W, G)
            b = x_of((N,), 2, 0.02) if with_bias else None
            proj.append((q, s_, b))
            t[f"q_{name}"], t[f"s_{name}"] = q, s_
            if b is not None:
                t[f"b_{name}"] = b
        g1 = (1.0 + x_of((D,), 2, 0.1)).astype(np.float32)
        g2 = (1.0 + x_of((D,), 2, 0.1)).astype(np.float32)
        scale = np.float32(1.0) / np.sqrt(np.float32(D // heads))  # CausalSelfAttention, nn.hpp:518
        t.update(g1=g1, g2=g2, attn_scale=np.array([scale], np.float32))
        t["y"] = ref.qllama_block_int4(xx, proj, g1, g2, 1e-5, float(scale), G)
        add("qllama_block_int4", {"L": L, "D": D, "H": H, "group_size": G, "heads": heads, "eps": 1e-5}, **t)

    np.savez_compressed(OUT_NPZ, **arrays)
    OUT_JSON.write_text(json.dumps({"generator": "tests/golden/make_golden.py", "cases": cases}, indent=1))
    print(f"wrote {len(cases)} cases, {OUT_NPZ.stat().st_size} bytes")


if __name__ == "__main__":
    main()
