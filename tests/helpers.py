"""Shared test helpers: package loader, golden fixtures, numpy models of the
device layouts, error metrics."""
from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "soverign-grad_amd"
GOLDEN_DIR = Path(__file__).resolve().parent / "golden"
SGQ_HEADER = ROOT / "include" / "sgq.h"

if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_sgq():
    """Imports soverign-grad_amd/ as the package `soverign_grad_amd`."""
    name = "soverign_grad_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def load_synth():
    load_sgq()
    import soverign_grad_amd.synth as synth  # noqa: E402

    return synth


def load_golden():
    meta = json.loads((GOLDEN_DIR / "golden.json").read_text())
    arrays = np.load(GOLDEN_DIR / "golden.npz", allow_pickle=False)
    out = []
    for c in meta["cases"]:
        out.append({"kind": c["kind"], "params": c["params"], **{k: arrays[v] for k, v in c["arrays"].items()}})
    return out


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    return a.shape == b.shape and np.array_equal(bits(a), bits(b))


def same_value_allow_zero_sign(a: np.ndarray, b: np.ndarray) -> bool:
    """Bitwise equal except that +0.0 and -0.0 count as equal (NaN == NaN)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    if a.shape != b.shape:
        return False
    ba, bb = bits(a).copy(), bits(b).copy()
    ba[a == 0] = 0
    bb[b == 0] = 0
    return np.array_equal(ba, bb)


def rel_err(y: np.ndarray, yref: np.ndarray) -> float:
    """max|y - yref| / max|yref| (the parity metric of the forward)."""
    y = np.asarray(y, np.float64)
    yref = np.asarray(yref, np.float64)
    den = np.max(np.abs(yref)) if yref.size else 0.0
    num = np.max(np.abs(y - yref)) if y.size else 0.0
    if den == 0.0:
        return float(num)
    return float(num / den)


# ---- numpy models of the device layouts (see csrc/sgq_internal.h) ---------

def _ceil(a, b):
    return (a + b - 1) // b


def i8_geom(K, N):
    """(Kpad, RQ, NS): rows padded to 16, row quads, strips of 4 columns."""
    Kpad = _ceil(K, 16) * 16
    return Kpad, Kpad // 4, _ceil(N, 4)


def i4_geom(K, N, G):
    G = G if G > 0 else 32
    Kpad = _ceil(K, 16) * 16
    tiled = N % 8 == 0 and G % 8 == 0
    NS = N // 8
    spc = G // 8 if (tiled and N % G == 0) else 1
    nsc = _ceil(NS, spc) if tiled else 0
    return dict(G=G, Kpad=Kpad, RQ=Kpad // 4, NS=NS, tiled=tiled, spc=spc, nsc=nsc)


def model_pack_i8(codes: np.ndarray) -> np.ndarray:
    """INT8 strip-major: chunk (strip j, row quad rq) at (j*RQ + rq)*16;
    dword d = column 4*j+d; byte r = row 4*rq+r."""
    K, N = codes.shape
    Kpad, RQ, NS = i8_geom(K, N)
    full = np.zeros((Kpad, NS * 4), np.int8)
    full[:K, :N] = codes.astype(np.int8)
    t = full.reshape(RQ, 4, NS, 4)  # rq, r, j, d
    t = t.transpose(2, 0, 3, 1)  # j, rq, d, r
    return np.ascontiguousarray(t).view(np.uint8).reshape(-1)


def i4_koct_geom(K, N, G):
    """(offset, KB, NB) of the k-octet copy that follows the strips: the
    strips' bytes rounded up to 256, k blocks of 32 rows, column blocks of 16."""
    g = i4_geom(K, N, G)
    return _ceil(g["NS"] * g["RQ"] * 16, 256) * 256, _ceil(g["Kpad"], 32), _ceil(g["NS"], 2)


def i4_packed_bytes(K, N, G):
    g = i4_geom(K, N, G)
    if not g["tiled"]:
        return (K * N + 1) // 2
    off, KB, NB = i4_koct_geom(K, N, G)
    return off + NB * KB * 256


def _nibble_words(t: np.ndarray) -> np.ndarray:
    """Eight codes along the last axis as one uint32, code i in nibble i."""
    nib = (t & 0xF).astype(np.uint32)
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    return np.bitwise_or.reduce(nib << shifts, axis=-1).astype(np.uint32)


def model_pack_i4_strips(codes: np.ndarray, G: int) -> np.ndarray:
    """INT4 strip-major: chunk (strip j, row quad rq) at (j*RQ + rq)*16;
    dword r = row 4*rq+r; nibble e = column 8*j+e (low nibble first)."""
    K, N = codes.shape
    g = i4_geom(K, N, G)
    full = np.zeros((g["Kpad"], N), np.int64)
    full[:K, :N] = codes.astype(np.int64)
    t = full.reshape(g["RQ"], 4, g["NS"], 8)  # rq, r, j, e
    t = t.transpose(2, 0, 1, 3)  # j, rq, r, e
    return np.ascontiguousarray(_nibble_words(t)).view(np.uint8).reshape(-1)


def model_pack_i4_koct(codes: np.ndarray, G: int) -> np.ndarray:
    """The k-octet copy: block (column block cb, k block kb) of 256 bytes at
    (cb*KB + kb)*256; dword 16*g + c = column 16*cb + c, rows 32*kb + 8*g + i
    in nibble i."""
    K, N = codes.shape
    _, KB, NB = i4_koct_geom(K, N, G)
    full = np.zeros((KB * 32, NB * 16), np.int64)
    full[:K, :N] = codes.astype(np.int64)
    t = full.reshape(KB, 4, 8, NB, 16)  # kb, g, i, cb, c
    t = t.transpose(3, 0, 1, 4, 2)  # cb, kb, g, c, i
    return np.ascontiguousarray(_nibble_words(t)).view(np.uint8).reshape(-1)


def model_pack_i4_tiled(codes: np.ndarray, G: int) -> np.ndarray:
    """The whole INT4 strip-major buffer: the strips, zeros up to the k-octet
    copy's offset, then the k-octet copy."""
    K, N = codes.shape
    strips = model_pack_i4_strips(codes, G)
    off, _, _ = i4_koct_geom(K, N, G)
    return np.concatenate([strips, np.zeros(off - strips.size, np.uint8), model_pack_i4_koct(codes, G)])


def model_pack_i4_flat(codes: np.ndarray) -> np.ndarray:
    flat = codes.reshape(-1).astype(np.int64) & 0xF
    if flat.size % 2:
        flat = np.concatenate([flat, [0]])
    return (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8)


def model_devscales_i4(scales: np.ndarray, K: int, N: int, G: int) -> np.ndarray:
    g = i4_geom(K, N, G)
    out = np.zeros((g["nsc"], g["Kpad"]), np.float32)
    for sc in range(g["nsc"]):
        n = sc * g["spc"] * 8
        if n < N:
            idx = (np.arange(K, dtype=np.int64) * N + n) // g["G"]
            out[sc, :K] = scales[idx]
    return out.reshape(-1)


def header_symbols() -> list:
    import re

    text = SGQ_HEADER.read_text()
    return sorted(set(re.findall(r"\b(sgq_[a-z0-9_]+)\s*\(", text)))
