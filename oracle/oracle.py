"""ctypes front end of the CPU oracle.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module.  It loads:

  oracle/liboracle.so    the C restatement of the reference path (sgq_oracle.c);
  oracle/_ref/libsgref.so  the reference's own sources compiled in place
                         (oracle/Makefile target `ref`), when it has been built.

Both expose the same operations, returned as numpy arrays, so a test can run a
case through either and compare.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Tuple

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
# SGQ_ORACLE_LIB selects another build of sgq_oracle.c (the sanitizer build,
# oracle/liboracle_san.so, loaded by tests/test_sanitize_cpu.py).
ORACLE_LIB = Path(os.environ.get("SGQ_ORACLE_LIB", ORACLE_DIR / "liboracle.so"))
REF_LIB = ORACLE_DIR / "_ref" / "libsgref.so"

_i64, _int, _vp, _dbl = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_double


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# Projections of a LLaMA block, in the order the block functions take them.
BLOCK_PROJ = ("q", "k", "v", "out", "gate", "up", "down")


def block_shapes(D: int, H: int):
    """[K, N] of each projection of BLOCK_PROJ for model width D and MLP width H."""
    return [(D, D), (D, D), (D, D), (D, D), (D, H), (D, H), (H, D)]


def _ptrs(arrays):
    """A C array of pointers to the given float32 arrays (None -> NULL), plus
    the converted arrays, which the caller keeps alive across the call."""
    conv = [None if a is None else _f32(a) for a in arrays]
    arr = (_vp * len(conv))(*[None if a is None else a.ctypes.data for a in conv])
    return arr, conv


def _block_args(proj):
    """proj: 7 (codes[K,N], scales, bias or None) in BLOCK_PROJ order."""
    if len(proj) != 7:
        raise ValueError("a block has 7 projections")
    q, kq = _ptrs([p[0] for p in proj])
    s, ks = _ptrs([p[1] for p in proj])
    b, kb = _ptrs([p[2] if len(p) > 2 else None for p in proj])
    return q, s, b, (kq, ks, kb)


class Oracle:
    """The C restatement (sgq_oracle.c)."""

    def __init__(self, path: Path = ORACLE_LIB):
        if not path.exists():
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = ctypes.CDLL(str(path))
        L.oracle_quantize_int8_per_tensor.argtypes = [_vp, _i64, _vp, _vp]
        L.oracle_quantize_int8_per_channel.argtypes = [_vp, _i64, _i64, _vp, _vp]
        L.oracle_dequantize_int8.argtypes = [_vp, _vp, _i64, _i64, _int, _vp]
        L.oracle_int4_num_groups.argtypes = [_i64, _i64]
        L.oracle_int4_num_groups.restype = _i64
        L.oracle_quantize_int4.argtypes = [_vp, _i64, _i64, _vp, _vp]
        L.oracle_dequantize_int4.argtypes = [_vp, _vp, _i64, _i64, _i64, _vp]
        L.oracle_matmul.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64]
        L.oracle_add_row_bias.argtypes = [_vp, _vp, _i64, _i64]
        L.oracle_quantized_matmul_int8.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _int, _vp, _vp]
        L.oracle_quantized_matmul_int4.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp]
        L.oracle_matmul_f64.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64]
        L.oracle_silu.argtypes = [_vp, _i64, _vp]
        L.oracle_mul.argtypes = [_vp, _vp, _i64, _vp]
        L.oracle_swiglu_int8.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _int, _vp]
        L.oracle_swiglu_int4.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp]
        L.oracle_rms_norm.argtypes = [_vp, _i64, _i64, _vp, ctypes.c_float, _vp]
        L.oracle_softmax_rows.argtypes = [_vp, _i64, _i64, _vp]
        L.oracle_embedding.argtypes = [_vp, _i64, _vp, _i64, _i64, _vp]
        L.oracle_causal_attention.argtypes = [_vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp]
        L.oracle_qllama_block_int4.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, ctypes.c_float,
                                               ctypes.c_float, _i64, _vp]

    # quantize_int8: per-tensor for scheme 0 or rank < 2 (src/quantization.cpp:22)
    def quantize_int8(self, x: np.ndarray, scheme: int) -> Tuple[np.ndarray, np.ndarray]:
        x = _f32(x)
        q = np.empty_like(x)
        if scheme == 0 or x.ndim < 2:
            s = np.empty(1, np.float32)
            self.lib.oracle_quantize_int8_per_tensor(_p(x), x.size, _p(q), _p(s))
        else:
            rows = x.shape[0]
            s = np.empty(rows, np.float32)
            self.lib.oracle_quantize_int8_per_channel(_p(x), rows, x.size // rows, _p(q), _p(s))
        return q, s

    def dequantize_int8(self, q: np.ndarray, s: np.ndarray, scheme: int) -> np.ndarray:
        q, s = _f32(q), _f32(s)
        out = np.empty_like(q)
        rows = q.shape[0] if q.ndim >= 2 else 1
        per_tensor = 1 if (scheme == 0 or s.size == 1) else 0
        self.lib.oracle_dequantize_int8(_p(q), _p(s), rows, q.size // max(rows, 1), per_tensor, _p(out))
        return out

    def quantize_int4(self, x: np.ndarray, group_size: int = 32) -> Tuple[np.ndarray, np.ndarray]:
        x = _f32(x)
        q = np.empty_like(x)
        s = np.empty(self.lib.oracle_int4_num_groups(x.size, group_size), np.float32)
        self.lib.oracle_quantize_int4(_p(x), x.size, group_size, _p(q), _p(s))
        return q, s

    def dequantize_int4(self, q: np.ndarray, s: np.ndarray, group_size: int) -> np.ndarray:
        q, s = _f32(q), _f32(s)
        out = np.empty_like(q)
        g = group_size if group_size > 0 else 32
        self.lib.oracle_dequantize_int4(_p(q), _p(s), q.size, g, s.size, _p(out))
        return out

    def matmul(self, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        a, b = _f32(a), _f32(b)
        out = np.empty((a.shape[0], b.shape[1]), np.float32)
        self.lib.oracle_matmul(_p(a), _p(b), _p(out), a.shape[0], a.shape[1], b.shape[1])
        return out

    def quantized_matmul_int8(self, x, q, s, scheme: int, bias=None) -> np.ndarray:
        x, q, s = _f32(x), _f32(q), _f32(s)
        out = np.empty((x.shape[0], q.shape[1]), np.float32)
        per_tensor = 1 if (scheme == 0 or s.size == 1) else 0
        b = None if bias is None else _f32(bias).reshape(-1)
        self.lib.oracle_quantized_matmul_int8(_p(x), x.shape[0], x.shape[1], q.shape[1], _p(q), _p(s), per_tensor,
                                              _p(b), _p(out))
        return out

    def quantized_matmul_int4(self, x, q, s, group_size: int, bias=None) -> np.ndarray:
        x, q, s = _f32(x), _f32(q), _f32(s)
        out = np.empty((x.shape[0], q.shape[1]), np.float32)
        b = None if bias is None else _f32(bias).reshape(-1)
        self.lib.oracle_quantized_matmul_int4(_p(x), x.shape[0], x.shape[1], q.shape[1], _p(q), _p(s), group_size,
                                              _p(b), _p(out))
        return out

    def silu(self, x) -> np.ndarray:
        x = _f32(x)
        out = np.empty_like(x)
        self.lib.oracle_silu(_p(x), x.size, _p(out))
        return out

    def mul(self, a, b) -> np.ndarray:
        a, b = _f32(a), _f32(b)
        out = np.empty_like(a)
        self.lib.oracle_mul(_p(a), _p(b), a.size, _p(out))
        return out

    def swiglu_int8(self, x, qg, sg, qu, su, scheme: int, bias_gate=None, bias_up=None) -> np.ndarray:
        """silu(x . deq(Wg) + bg) * (x . deq(Wu) + bu), nn.hpp:151-154 on quantized weights."""
        x, qg, sg, qu, su = _f32(x), _f32(qg), _f32(sg), _f32(qu), _f32(su)
        out = np.empty((x.shape[0], qg.shape[1]), np.float32)
        bg = None if bias_gate is None else _f32(bias_gate).reshape(-1)
        bu = None if bias_up is None else _f32(bias_up).reshape(-1)
        per_tensor = 1 if (scheme == 0 or sg.size == 1) else 0
        self.lib.oracle_swiglu_int8(_p(x), x.shape[0], x.shape[1], qg.shape[1], _p(qg), _p(sg), _p(bg), _p(qu),
                                    _p(su), _p(bu), per_tensor, _p(out))
        return out

    def rms_norm(self, x, g, eps: float = 1e-5) -> np.ndarray:
        x, g = _f32(x), _f32(g).reshape(-1)
        out = np.empty_like(x)
        D = x.shape[-1]
        self.lib.oracle_rms_norm(_p(x), x.size // max(D, 1), D, _p(g), eps, _p(out))
        return out

    def softmax_rows(self, x) -> np.ndarray:
        x = _f32(x)
        out = np.empty_like(x)
        self.lib.oracle_softmax_rows(_p(x), x.size // max(x.shape[-1], 1), x.shape[-1], _p(out))
        return out

    def embedding(self, idx, w) -> np.ndarray:
        idx, w = _f32(idx).reshape(-1), _f32(w)
        out = np.empty((idx.size, w.shape[1]), np.float32)
        self.lib.oracle_embedding(_p(idx), idx.size, _p(w), w.shape[0], w.shape[1], _p(out))
        return out

    def causal_attention(self, q, k, v, scale: float) -> np.ndarray:
        q, k, v = _f32(q), _f32(k), _f32(v)
        out = np.empty_like(q)
        self.lib.oracle_causal_attention(_p(q), _p(k), _p(v), q.shape[0], q.shape[1], scale, _p(out))
        return out

    def qllama_block_int4(self, x, proj, g1, g2, eps: float, attn_scale: float, group_size: int) -> np.ndarray:
        """LLaMABlock::forward on x[L, D] with quantized projections; proj as in _block_args."""
        x = _f32(x)
        L, D = x.shape
        H = _f32(proj[4][0]).shape[1]
        qa, sa, ba, keep = _block_args(proj)
        g1, g2 = _f32(g1).reshape(-1), _f32(g2).reshape(-1)
        out = np.empty_like(x)
        self.lib.oracle_qllama_block_int4(_p(x), L, D, H, qa, sa, ba, _p(g1), _p(g2), eps, attn_scale, group_size,
                                          _p(out))
        del keep
        return out

    def swiglu_int4(self, x, qg, sg, qu, su, group_size: int, bias_gate=None, bias_up=None) -> np.ndarray:
        x, qg, sg, qu, su = _f32(x), _f32(qg), _f32(sg), _f32(qu), _f32(su)
        out = np.empty((x.shape[0], qg.shape[1]), np.float32)
        bg = None if bias_gate is None else _f32(bias_gate).reshape(-1)
        bu = None if bias_up is None else _f32(bias_up).reshape(-1)
        self.lib.oracle_swiglu_int4(_p(x), x.shape[0], x.shape[1], qg.shape[1], _p(qg), _p(sg), _p(bg), _p(qu),
                                    _p(su), _p(bu), group_size, _p(out))
        return out

    def matmul_f64(self, a: np.ndarray, b: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
        a, b = _f32(a), _f32(b)
        c = np.empty((a.shape[0], b.shape[1]), np.float64)
        cabs = np.empty_like(c)
        self.lib.oracle_matmul_f64(_p(a), _p(b), _p(c), _p(cabs), a.shape[0], a.shape[1], b.shape[1])
        return c, cabs


class Reference:
    """The reference's own code, compiled by oracle/Makefile (`ref` target)."""

    def __init__(self, path: Path = REF_LIB):
        if not path.exists():
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref` where the reference is mounted")
        L = self.lib = ctypes.CDLL(str(path))
        L.ref_quantize_int8.argtypes = [_vp, _i64, _i64, _int, _int, _vp, _vp]
        L.ref_quantize_int8.restype = _i64
        L.ref_quantize_int4.argtypes = [_vp, _i64, _i64, _int, _i64, _vp, _vp]
        L.ref_quantize_int4.restype = _i64
        L.ref_dequantize_int8.argtypes = [_vp, _vp, _i64, _i64, _i64, _int, _vp]
        L.ref_dequantize_int4.argtypes = [_vp, _vp, _i64, _i64, _i64, _i64, _vp]
        L.ref_quantized_matmul_int8.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _int, _vp, _vp]
        L.ref_quantized_matmul_int4.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp]
        L.ref_matmul.argtypes = [_vp, _vp, _i64, _i64, _i64, _vp]
        L.ref_time_quantized_matmul.argtypes = [_int, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _int, _i64, _vp, _int,
                                                ctypes.POINTER(_dbl), _vp]
        L.ref_omp_max_threads.restype = _int
        L.ref_time_phases.argtypes = [_int, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _int, _i64, _vp, _int,
                                      ctypes.POINTER(_dbl)]
        L.ref_set_threads.argtypes = [_int]
        L.ref_set_threads.restype = _int
        L.ref_silu.argtypes = [_vp, _i64, _vp]
        L.ref_rms_norm.argtypes = [_vp, _i64, _i64, _vp, ctypes.c_float, _vp]
        L.ref_softmax.argtypes = [_vp, _i64, _i64, _vp]
        L.ref_embedding.argtypes = [_vp, _i64, _vp, _i64, _i64, _vp]
        L.ref_qllama_block_int4.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, ctypes.c_float,
                                            ctypes.c_float, _i64, _vp]
        L.ref_mul.argtypes = [_vp, _vp, _i64, _vp]
        L.ref_save_qlinear.argtypes = [_int, ctypes.c_char_p, _int, _vp, _i64, _i64, _i64, _vp, ctypes.c_char_p]
        L.ref_load_qlinear_forward.argtypes = [_int, ctypes.c_char_p, _int, _i64, _i64, _i64, ctypes.c_char_p, _vp,
                                               _i64, _vp]
        L.ref_read_entry.argtypes = [_int, ctypes.c_char_p, ctypes.c_char_p, _vp, _i64, ctypes.POINTER(_i64),
                                     ctypes.POINTER(_int)]
        L.ref_read_entry.restype = _i64
        L.ref_save_entries.argtypes = [_int, ctypes.c_char_p, _int, _vp, _vp, _vp, _vp]
        L.ref_list_entries.argtypes = [_int, ctypes.c_char_p, ctypes.c_char_p, _i64]
        L.ref_list_entries.restype = _i64

    @staticmethod
    def _rc(x: np.ndarray):
        if x.ndim >= 2:
            return x.shape[0], x.size // max(x.shape[0], 1), 2
        return 1, x.size, 1

    def quantize_int8(self, x: np.ndarray, scheme: int):
        x = _f32(x)
        rows, cols, rank = self._rc(x)
        q = np.empty_like(x)
        s = np.empty(max(rows, 1), np.float32)
        n = self.lib.ref_quantize_int8(_p(x), rows, cols, rank, scheme, _p(q), _p(s))
        if n < 0:
            raise RuntimeError("reference quantize_int8 raised")
        return q, s[:n].copy()

    def quantize_int4(self, x: np.ndarray, group_size: int = 32):
        x = _f32(x)
        rows, cols, rank = self._rc(x)
        g = group_size if group_size > 0 else 32
        q = np.empty_like(x)
        s = np.empty(max((x.size + g - 1) // g, 1), np.float32)
        n = self.lib.ref_quantize_int4(_p(x), rows, cols, rank, group_size, _p(q), _p(s))
        if n < 0:
            raise RuntimeError("reference quantize_int4 raised")
        return q, s[:n].copy()

    def dequantize_int8(self, q, s, scheme: int):
        q, s = _f32(q), _f32(s)
        out = np.empty_like(q)
        rows = q.shape[0]
        if self.lib.ref_dequantize_int8(_p(q), _p(s), s.size, rows, q.size // rows, scheme, _p(out)) != 0:
            raise RuntimeError("reference dequantize_int8 raised")
        return out

    def dequantize_int4(self, q, s, group_size: int):
        q, s = _f32(q), _f32(s)
        out = np.empty_like(q)
        rows = q.shape[0]
        if self.lib.ref_dequantize_int4(_p(q), _p(s), s.size, rows, q.size // rows, group_size, _p(out)) != 0:
            raise RuntimeError("reference dequantize_int4 raised")
        return out

    def matmul(self, a, b):
        a, b = _f32(a), _f32(b)
        out = np.empty((a.shape[0], b.shape[1]), np.float32)
        if self.lib.ref_matmul(_p(a), _p(b), a.shape[0], a.shape[1], b.shape[1], _p(out)) != 0:
            raise RuntimeError("reference matmul raised")
        return out

    def quantized_matmul_int8(self, x, q, s, scheme: int, bias=None):
        x, q, s = _f32(x), _f32(q), _f32(s)
        out = np.empty((x.shape[0], q.shape[1]), np.float32)
        b = None if bias is None else _f32(bias).reshape(-1)
        rc = self.lib.ref_quantized_matmul_int8(_p(x), x.shape[0], x.shape[1], q.shape[1], _p(q), _p(s), s.size,
                                                scheme, _p(b), _p(out))
        if rc != 0:
            raise RuntimeError("reference quantized_matmul_int8 raised")
        return out

    def quantized_matmul_int4(self, x, q, s, group_size: int, bias=None):
        x, q, s = _f32(x), _f32(q), _f32(s)
        out = np.empty((x.shape[0], q.shape[1]), np.float32)
        b = None if bias is None else _f32(bias).reshape(-1)
        rc = self.lib.ref_quantized_matmul_int4(_p(x), x.shape[0], x.shape[1], q.shape[1], _p(q), _p(s), s.size,
                                                group_size, _p(b), _p(out))
        if rc != 0:
            raise RuntimeError("reference quantized_matmul_int4 raised")
        return out

    def time_quantized_matmul(self, bits: int, x, q, s, scheme: int, group_size: int, bias, reps: int):
        """Per-call seconds of the reference forward (dequantize + matmul + bias)."""
        x, q, s = _f32(x), _f32(q), _f32(s)
        b = None if bias is None else _f32(bias).reshape(-1)
        secs = (_dbl * reps)()
        out = np.empty((x.shape[0], q.shape[1]), np.float32)
        rc = self.lib.ref_time_quantized_matmul(bits, _p(x), x.shape[0], x.shape[1], q.shape[1], _p(q), _p(s),
                                                s.size, scheme, group_size, _p(b), reps, secs, _p(out))
        if rc != 0:
            raise RuntimeError("reference forward raised")
        return list(secs), out

    def silu(self, x):
        x = _f32(x)
        out = np.empty_like(x)
        if self.lib.ref_silu(_p(x), x.size, _p(out)) != 0:
            raise RuntimeError("reference silu raised")
        return out

    def mul(self, a, b):
        a, b = _f32(a), _f32(b)
        out = np.empty_like(a)
        if self.lib.ref_mul(_p(a), _p(b), a.size, _p(out)) != 0:
            raise RuntimeError("reference mul raised")
        return out

    def rms_norm(self, x, g, eps: float = 1e-5):
        x, g = _f32(x), _f32(g).reshape(-1)
        out = np.empty_like(x)
        D = x.shape[-1]
        if self.lib.ref_rms_norm(_p(x), x.size // max(D, 1), D, _p(g), eps, _p(out)) != 0:
            raise RuntimeError("reference rms_norm raised")
        return out

    def softmax_rows(self, x):
        x = _f32(x)
        out = np.empty_like(x)
        if self.lib.ref_softmax(_p(x), x.size // max(x.shape[-1], 1), x.shape[-1], _p(out)) != 0:
            raise RuntimeError("reference softmax raised")
        return out

    def embedding(self, idx, w):
        idx, w = _f32(idx).reshape(-1), _f32(w)
        out = np.empty((idx.size, w.shape[1]), np.float32)
        if self.lib.ref_embedding(_p(idx), idx.size, _p(w), w.shape[0], w.shape[1], _p(out)) != 0:
            raise RuntimeError("reference embedding raised")
        return out

    def qllama_block_int4(self, x, proj, g1, g2, eps: float, attn_scale: float, group_size: int):
        x = _f32(x)
        L, D = x.shape
        H = _f32(proj[4][0]).shape[1]
        qa, sa, ba, keep = _block_args(proj)
        g1, g2 = _f32(g1).reshape(-1), _f32(g2).reshape(-1)
        out = np.empty_like(x)
        if self.lib.ref_qllama_block_int4(_p(x), L, D, H, qa, sa, ba, _p(g1), _p(g2), eps, attn_scale, group_size,
                                          _p(out)) != 0:
            raise RuntimeError("reference block raised")
        del keep
        return out

    # ---- persistence (format 0: .sgrd, 1: .safetensors) -------------------

    @staticmethod
    def _fmt(path) -> int:
        return 1 if str(path).endswith(".safetensors") else 0

    def save_qlinear(self, path, bits: int, W, group_size: int = 32, bias=None, child: str = "") -> None:
        """The reference's QuantizedLinear (bits 8, per-channel) or
        QuantizedLinear4Bit (bits 4) built by from_float(W, bias) and saved
        with save_module, optionally as submodule `child` of a parent module."""
        W = _f32(W)
        b = None if bias is None else _f32(bias).reshape(-1)
        rc = self.lib.ref_save_qlinear(self._fmt(path), str(path).encode(), bits, _p(W), W.shape[0], W.shape[1],
                                       group_size, _p(b), child.encode())
        if rc != 0:
            raise RuntimeError(f"reference save_module raised for {path}")

    def load_qlinear_forward(self, path, bits: int, K: int, N: int, x, group_size: int = 32, child: str = ""):
        """A fresh reference module of shape [K, N] loaded from `path` with the
        strict load_module, then its forward on x."""
        x = _f32(x)
        out = np.empty((x.shape[0], N), np.float32)
        rc = self.lib.ref_load_qlinear_forward(self._fmt(path), str(path).encode(), bits, K, N, group_size,
                                               child.encode(), _p(x), x.shape[0], _p(out))
        if rc != 0:
            raise RuntimeError(f"reference load_module / forward raised for {path}")
        return out

    def read_entry(self, path, name: str):
        """One tensor of a checkpoint read with the reference's loader."""
        shape = (_i64 * 8)()
        rank = _int(0)
        n = self.lib.ref_read_entry(self._fmt(path), str(path).encode(), name.encode(), None, 0, shape,
                                    ctypes.byref(rank))
        if n == -2:
            raise KeyError(name)
        if n < 0:
            raise RuntimeError(f"reference loader raised for {path}")
        out = np.empty(max(n, 1), np.float32)
        self.lib.ref_read_entry(self._fmt(path), str(path).encode(), name.encode(), _p(out), n, shape,
                                ctypes.byref(rank))
        return out[:n].reshape([shape[i] for i in range(rank.value)])

    def save_entries(self, path, tensors: dict) -> None:
        """Raw fp32 tensors saved with the reference's save_checkpoint /
        safetensors::save_file."""
        names = sorted(tensors)
        arrs = [_f32(tensors[k]) for k in names]
        shapes = [np.array(a.shape if a.ndim else (1,), np.int64) for a in arrs]
        c_names = (ctypes.c_char_p * len(names))(*[k.encode() for k in names])
        c_data = (ctypes.c_void_p * len(names))(*[a.ctypes.data for a in arrs])
        c_shapes = (ctypes.c_void_p * len(names))(*[sh.ctypes.data for sh in shapes])
        c_ranks = (_int * len(names))(*[len(sh) for sh in shapes])
        rc = self.lib.ref_save_entries(self._fmt(path), str(path).encode(), len(names), c_names, c_data, c_shapes,
                                       c_ranks)
        if rc != 0:
            raise RuntimeError(f"reference save raised for {path}")

    def list_entries(self, path):
        buf = ctypes.create_string_buffer(1 << 16)
        n = self.lib.ref_list_entries(self._fmt(path), str(path).encode(), buf, len(buf))
        if n < 0:
            raise RuntimeError(f"reference loader raised for {path}")
        return sorted(e for e in buf.value.decode().split("\n") if e)

    def omp_max_threads(self) -> int:
        return int(self.lib.ref_omp_max_threads())

    def set_threads(self, n: int) -> int:
        """OpenMP threads for later calls; returns the previous maximum."""
        return int(self.lib.ref_set_threads(int(n)))

    def time_phases(self, bits: int, x, q, s, scheme: int, group_size: int, bias, reps: int):
        """Per-call seconds of (dequantize, matmul, bias add) of the reference forward."""
        x, q, s = _f32(x), _f32(q), _f32(s)
        b = None if bias is None else _f32(bias).reshape(-1)
        secs = (_dbl * (3 * reps))()
        rc = self.lib.ref_time_phases(bits, _p(x), x.shape[0], x.shape[1], q.shape[1], _p(q), _p(s), s.size, scheme,
                                      group_size, _p(b), reps, secs)
        if rc != 0:
            raise RuntimeError("reference forward raised")
        return [tuple(secs[3 * r: 3 * r + 3]) for r in range(reps)]


def reference_available() -> bool:
    return REF_LIB.exists()
