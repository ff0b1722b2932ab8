"""GPU parity over a seeded spread of forward shapes.

Sixty-four (bits, M, K, N, group or scheme, bias) draws from fixed menus that
cross every dispatch rule of the forward: one to 256 rows (GEMV row groups, the
skinny MFMA kernels' whole-K, super-block and split-K forms, the GEMM tiles),
K with and without a tail inside a 16- or 32-row block, N that is or is not a
multiple of 8, 16 or the group (strip layout, its k-octet copy with a
half-empty column block, the flat INT4 layout), INT4 groups 24..128 and INT8
per tensor and per channel.  Each output is checked against the oracle's
dequantize-then-matmul on the same quantized weight, to the forward's 1e-5.
Twenty-four more draws run the gated MLP the same way.  The draws are fixed
by the seed, so a failure names a reproducible case.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
MS = [1, 2, 3, 4, 5, 6, 8, 9, 12, 16, 17, 24, 32, 33, 40, 64]
KS = [64, 100, 512, 1000, 2048, 2064, 4096]
NS = [8, 24, 136, 1001, 1024, 2048, 3000, 4096, 6144]
GS = [0, 24, 32, 64, 128]
# Prefill-sized draws, where the GEMMs take over.
MS_L = [48, 64, 96, 128, 200, 256]
KS_L = [1024, 2048, 4096]
NS_L = [2048, 4096]


def _draws(n_small=48, n_large=16, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for ms, ks, ns, n, max_work in ((MS, KS, NS, n_small, 1 << 28), (MS_L, KS_L, NS_L, n_large, 1 << 32)):
        drawn = 0
        while drawn < n:
            bits = int(rng.choice([4, 8]))
            M, K, N = int(rng.choice(ms)), int(rng.choice(ks)), int(rng.choice(ns))
            if M * K * N > max_work:
                continue
            g = int(rng.choice(GS)) if bits == 4 else int(rng.integers(0, 2))
            bias = bool(rng.integers(0, 2))
            out.append((bits, M, K, N, g, bias, len(out)))
            drawn += 1
    return out


CASES = _draws()


def _path(sgq, bits, M, K, N, g):
    lib = sgq.load_library()
    path, ks = ctypes.c_int(), ctypes.c_int()
    assert lib.sgq_linear_plan(bits, M, K, N, g if bits == 4 else 0, 0, ctypes.byref(path), ctypes.byref(ks)) == 0
    return path.value, ks.value


def test_draws_cross_the_dispatch(sgq):
    paths = {_path(sgq, b, M, K, N, g) for b, M, K, N, g, _, _ in CASES}
    kinds = {p for p, _ in paths}
    assert {0, 1, 2, 3, 4} <= kinds, paths  # GEMV, three-term GEMM, fp32-MFMA GEMM, flat INT4, skinny MFMA


@pytest.mark.parametrize("bits,M,K,N,g,bias,i", CASES, ids=[f"d{c[6]}_{c[0]}b_{c[1]}x{c[2]}x{c[3]}" for c in CASES])
def test_random_shape(sgq, dev, oracle, synth, bits, M, K, N, g, bias, i):
    path, ks = _path(sgq, bits, M, K, N, g)
    print(f"  case {i}: bits={bits} M={M} K={K} N={N} g={g} bias={bias} path={path} k_splits={ks}", flush=True)
    seed = synth.config_seed(100 + i)
    W = synth.normal((K, N), seed, synth.STREAM_W, 0.0, 0.02)
    x = synth.normal((M, K), seed, synth.STREAM_X, 0.0, 1.0)
    b = synth.normal((1, N), seed, synth.STREAM_BIAS, 0.0, 0.02) if bias else None
    Wd = torch.from_numpy(np.ascontiguousarray(W, np.float32)).to(dev)
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev)
    bd = torch.from_numpy(np.ascontiguousarray(b, np.float32)).to(dev) if bias else None
    # Rows of the forward are independent: past 64 rows the oracle checks the
    # first and last eight (its single-threaded matmul would take minutes).
    rows = np.r_[0:M] if M <= 64 else np.r_[0:8, M - 8:M]
    if bits == 8:
        qw = sgq.quantize_int8(Wd, g)
        y = sgq.quantized_matmul_int8(xd, qw, bd)
        q, s = oracle.quantize_int8(W, g)
        yref = oracle.quantized_matmul_int8(x[rows], q, s, g, b)
    else:
        qw = sgq.quantize_int4(Wd, g)
        y = sgq.quantized_matmul_int4(xd, qw, bd)
        q, s = oracle.quantize_int4(W, g)
        yref = oracle.quantized_matmul_int4(x[rows], q, s, g, b)
    torch.cuda.synchronize()
    e = rel_err(y.cpu().numpy()[rows], yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


def _swiglu_draws(n=24, seed=20261203, max_work=1 << 27):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        bits = int(rng.choice([4, 8]))
        M, K, N = int(rng.choice(MS + [96, 128])), int(rng.choice(KS)), int(rng.choice(NS))
        if M * K * N > max_work:
            continue
        g = int(rng.choice(GS)) if bits == 4 else int(rng.integers(0, 2))
        out.append((bits, M, K, N, g, bool(rng.integers(0, 2)), len(out)))
    return out


SWIGLU_CASES = _swiglu_draws()


@pytest.mark.parametrize("bits,M,K,N,g,bias,i", SWIGLU_CASES,
                         ids=[f"s{c[6]}_{c[0]}b_{c[1]}x{c[2]}x{c[3]}" for c in SWIGLU_CASES])
def test_random_swiglu(sgq, dev, oracle, synth, bits, M, K, N, g, bias, i):
    """The gated MLP, silu(x Wg + bg) * (x Wu + bu), on the same kind of draws."""
    print(f"  case {i}: bits={bits} M={M} K={K} N={N} g={g} bias={bias}", flush=True)
    seed = synth.config_seed(300 + i)
    Wg = synth.normal((K, N), seed, synth.STREAM_W, 0.0, 0.02)
    Wu = synth.normal((K, N), seed, synth.STREAM_W2, 0.0, 0.02)
    x = synth.normal((M, K), seed, synth.STREAM_X, 0.0, 1.0)
    bg = synth.normal((1, N), seed, synth.STREAM_BIAS, 0.0, 0.02) if bias else None
    bu = synth.normal((1, N), seed, synth.STREAM_BIAS2, 0.0, 0.02) if bias else None

    def dev_(a):
        return None if a is None else torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)

    if bits == 8:
        wg, wu = sgq.quantize_int8(dev_(Wg), g), sgq.quantize_int8(dev_(Wu), g)
        (qg, sg), (qu, su) = oracle.quantize_int8(Wg, g), oracle.quantize_int8(Wu, g)
        href = oracle.swiglu_int8(x, qg, sg, qu, su, g, bg, bu)
    else:
        wg, wu = sgq.quantize_int4(dev_(Wg), g), sgq.quantize_int4(dev_(Wu), g)
        (qg, sg), (qu, su) = oracle.quantize_int4(Wg, g), oracle.quantize_int4(Wu, g)
        href = oracle.swiglu_int4(x, qg, sg, qu, su, g, bg, bu)
    h = sgq.quantized_swiglu(dev_(x), wg, wu, dev_(bg), dev_(bu))
    torch.cuda.synchronize()
    e = rel_err(h.cpu().numpy(), href)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL
