"""GPU parity of the skinny INT4 forward on the bf16 matrix cores (k_skinny3):
batches of 5..16 rows over weights wide enough for it (sgq_linear_plan path 4),
against the oracle's dequantize-then-matmul on the same quantized weights
(src/quantization.cpp:199-206), and of the gated MLP that runs both of its
projections through the same kernel.

Bar: max|y - y_ref| / max|y_ref| <= 1e-5 (fp32 accumulate in another order).
"""
import ctypes

import numpy as np
import pytest
import torch

import helpers
from helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
SKINNY = 4  # sgq_linear_plan path of k_skinny3


def _to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _path(sgq, M, K, N, G):
    lib = sgq.load_library()
    path, ks = ctypes.c_int(), ctypes.c_int()
    assert lib.sgq_linear_plan(4, M, K, N, G, 0, ctypes.byref(path), ctypes.byref(ks)) == 0
    return path.value


def _weights(synth, K, N, seed, G):
    cs = synth.config_seed(seed)
    W = synth.normal((K, N), cs, synth.STREAM_W, 0.0, 0.02)
    b = synth.normal((1, N), cs, synth.STREAM_BIAS, 0.0, 0.02)
    return W, b


_QUANT = {}


def _quantized(sgq, dev, oracle, synth, K, N, G, seed):
    """Weight, bias, device weight and the oracle's codes and scales of one
    shape, made once for all batch sizes."""
    key = (K, N, G, seed)
    if key not in _QUANT:
        _QUANT.clear()
        W, b = _weights(synth, K, N, seed, G)
        _QUANT[key] = (W, b, sgq.quantize_int4(_to_dev(W, dev), G), oracle.quantize_int4(W, G))
    return _QUANT[key]


# Shapes whose width fills the device with 32- or 64-column workgroups:
# the BASELINE gate/up (4096->11008) and NanoLLaMA q/k/v and gate/up widths,
# groups 64 and 32 (fewer strips per scale column), a K that ends inside a
# 32-row k block, and a long K.
@pytest.mark.parametrize("M", [5, 8, 12, 16])
@pytest.mark.parametrize("K,N,G", [(4096, 11008, 128), (2048, 6144, 128), (2048, 5632, 128), (4096, 8192, 64),
                                   (2048, 5120, 32), (4112, 6144, 128), (11008, 5632, 128)])
def test_skinny_shapes(sgq, dev, oracle, synth, M, K, N, G):
    path = _path(sgq, M, K, N, G)
    print(f"  case M={M} K={K} N={N} G={G} path={path}", flush=True)
    assert path == SKINNY
    W, b, qw, (q, s) = _quantized(sgq, dev, oracle, synth, K, N, G, 61)
    x = synth.normal((M, K), synth.config_seed(61), synth.STREAM_X, 0.0, 1.0)
    y = _np(sgq.quantized_matmul_int4(_to_dev(x, dev), qw, _to_dev(b, dev)))
    yref = oracle.quantized_matmul_int4(x, q, s, G, b)
    e = rel_err(y, yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


def test_skinny_boundaries(sgq, dev):
    # Four rows, narrow weights and groups whose scale column holds a single
    # strip stay on the GEMV; the batches above take the MFMA kernel.
    assert _path(sgq, 4, 4096, 11008, 128) == 0
    assert _path(sgq, 17, 4096, 11008, 128) == 1
    assert _path(sgq, 8, 5632, 2048, 128) == 0
    assert _path(sgq, 8, 2048, 6144, 8) == 0
    for M in range(5, 17):
        assert _path(sgq, M, 4096, 11008, 128) == SKINNY


# x that is not 16-byte aligned, or whose rows are not a multiple of four
# floats, takes the kernel's one-float loads.
@pytest.mark.parametrize("K,offset", [(2048, 1), (2050, 0), (2051, 3)])
def test_skinny_unaligned_x(sgq, dev, oracle, synth, K, offset):
    M, N, G = 8, 6144, 128
    assert _path(sgq, M, K, N, G) == SKINNY
    W, b = _weights(synth, K, N, 62, G)
    flat = synth.normal((M * K + offset,), synth.config_seed(62), synth.STREAM_X, 0.0, 1.0)
    x = _to_dev(flat, dev)[offset:].view(M, K)
    print(f"  case K={K} offset={offset} aligned={x.data_ptr() % 16 == 0}", flush=True)
    qw = sgq.quantize_int4(_to_dev(W, dev), G)
    y = _np(sgq.quantized_matmul_int4(x, qw, _to_dev(b, dev)))
    q, s = oracle.quantize_int4(W, G)
    yref = oracle.quantized_matmul_int4(flat[offset:].reshape(M, K), q, s, G, b)
    e = rel_err(y, yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


@pytest.mark.parametrize("kind", ["abs", "silu"])
def test_skinny_same_sign_activations(sgq, dev, oracle, synth, kind):
    # Same-sign inputs at long K: no cancellation between terms to hide an
    # error in the split of x * s.
    M, K, N, G = 16, 11008, 5632, 128
    W, _ = _weights(synth, K, N, 63, G)
    z = synth.normal((M, K), synth.config_seed(63), synth.STREAM_X, 0.0, 1.0)
    if kind == "abs":
        x = np.abs(z).astype(np.float32)
    else:
        zz = (2.0 * z).astype(np.float32)
        x = (zz / (np.float32(1.0) + np.exp(-zz))).astype(np.float32)
    qw = sgq.quantize_int4(_to_dev(W, dev), G)
    y = _np(sgq.quantized_matmul_int4(_to_dev(x, dev), qw))
    q, s = oracle.quantize_int4(W, G)
    e = rel_err(y, oracle.quantized_matmul_int4(x, q, s, G))
    print(f"  case x={kind} rel_err={e:.3e}", flush=True)
    assert e <= TOL


@pytest.mark.parametrize("k0", [0, 1000, 2047])
def test_skinny_split_sums_to_rounded_product(sgq, dev, k0):
    # One nonzero activation per row (column k0) and codes of 1 in weight row
    # k0: every output is h + m + l of x * s, each partial sum exact, so
    # y == float32(x * s) bit for bit whatever the accumulation's rounding.
    # A split of the unrounded product (an fma fused into the split) would
    # miss by an ulp in about a quarter of them.
    M, K, N, G = 8, 2048, 6144, 128
    assert _path(sgq, M, K, N, G) == SKINNY
    rng = np.random.default_rng(2000 + k0)
    x = np.zeros((M, K), np.float32)
    x[:, k0] = (rng.standard_normal(M) * 10.0 ** rng.uniform(-3, 3, M)).astype(np.float32)
    q = rng.integers(-7, 8, (K, N)).astype(np.float32)
    q[k0, :] = 1.0
    s = rng.uniform(1e-3, 1.0, K * N // G).astype(np.float32)
    qw = sgq.pack_int4(_to_dev(q, dev), _to_dev(s, dev), G)
    s_kn = s[(k0 * N + np.arange(N)) // G]
    y = _np(sgq.quantized_matmul_int4(_to_dev(x, dev), qw))
    want = x[:, k0:k0 + 1] * s_kn[None, :].astype(np.float32)
    assert want.dtype == np.float32
    assert helpers.same_bits(y, want), np.count_nonzero(y != want)


def test_skinny_infinite_activation(sgq, dev, oracle, synth):
    # inf * s split into three bf16 planes is inf - inf; the kernel hands a
    # non-finite total to the reference's k-order sum, so infinities and NaNs
    # land where the reference's x . (q * s) puts them.
    M, K, N, G = 8, 2048, 6144, 128
    W, _ = _weights(synth, K, N, 65, G)
    x = synth.normal((M, K), synth.config_seed(65), synth.STREAM_X, 0.0, 1.0)
    x[0, 17] = np.inf
    x[M - 1, 600] = -np.inf
    x[1, 3] = np.inf
    x[1, 900] = -np.inf
    x[2, 1000] = np.nan
    q, s = oracle.quantize_int4(W, G)
    qw = sgq.quantize_int4(_to_dev(W, dev), G)
    y = _np(sgq.quantized_matmul_int4(_to_dev(x, dev), qw))
    yref = oracle.quantized_matmul_int4(x, q, s, G)
    assert np.isinf(yref).any() and np.isnan(yref).any()
    assert np.array_equal(np.isnan(y), np.isnan(yref))
    assert np.array_equal(np.isposinf(y), np.isposinf(yref))
    assert np.array_equal(np.isneginf(y), np.isneginf(yref))
    fin = np.isfinite(yref)
    assert np.max(np.abs(y[fin].astype(np.float64) - yref[fin])) <= TOL * np.max(np.abs(yref[fin]))


def test_skinny_rows_independent_and_deterministic(sgq, dev, synth):
    # A row's sums do not depend on the other rows of the batch (each is its
    # own row of the MFMA tile), and repeated calls give identical bits.
    K, N, G = 4096, 11008, 128
    W, _ = _weights(synth, K, N, 66, G)
    x = _to_dev(synth.normal((16, K), synth.config_seed(66), synth.STREAM_X, 0.0, 1.0), dev)
    qw = sgq.quantize_int4(_to_dev(W, dev), G)
    y16 = sgq.quantized_matmul_int4(x, qw).clone()
    for M in (5, 9, 13):
        assert torch.equal(sgq.quantized_matmul_int4(x[:M].contiguous(), qw), y16[:M])
    for _ in range(3):
        assert torch.equal(sgq.quantized_matmul_int4(x, qw), y16)


@pytest.mark.parametrize("M,K,N", [(8, 2048, 5632), (16, 4096, 11008)])
def test_skinny_swiglu(sgq, dev, oracle, synth, M, K, N):
    # The gated MLP runs gate and up through the same kernel: its sums equal
    # two forward calls', so the fused output matches the two projections
    # followed by the oracle's silu and mul to rounding, and the oracle's
    # gated MLP within the forward's bar.
    G = 128
    assert _path(sgq, M, K, N, G) == SKINNY
    cs = synth.config_seed(67)
    Wg = synth.normal((K, N), cs, synth.STREAM_W, 0.0, 0.02)
    Wu = synth.normal((K, N), cs, synth.STREAM_W2, 0.0, 0.02)
    bg = synth.normal((1, N), cs, synth.STREAM_BIAS, 0.0, 0.02)
    bu = synth.normal((1, N), cs, synth.STREAM_BIAS2, 0.0, 0.02)
    x = synth.normal((M, K), cs, synth.STREAM_X, 0.0, 1.0)
    xd = _to_dev(x, dev)
    wg, wu = sgq.quantize_int4(_to_dev(Wg, dev), G), sgq.quantize_int4(_to_dev(Wu, dev), G)
    bgd, bud = _to_dev(bg, dev), _to_dev(bu, dev)
    h = _np(sgq.quantized_swiglu(xd, wg, wu, bgd, bud))
    g = _np(sgq.quantized_matmul_int4(xd, wg, bgd))
    u = _np(sgq.quantized_matmul_int4(xd, wu, bud))
    e2 = rel_err(h, oracle.mul(oracle.silu(g), u))
    qg, sg = oracle.quantize_int4(Wg, G)
    qu, su = oracle.quantize_int4(Wu, G)
    e = rel_err(h, oracle.swiglu_int4(x, qg, sg, qu, su, G, bg, bu))
    print(f"  case M={M} K={K} N={N} vs two calls {e2:.3e} vs oracle {e:.3e}", flush=True)
    assert e2 <= 2e-7
    assert e <= TOL
