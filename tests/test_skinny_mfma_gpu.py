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
@pytest.mark.parametrize("M", [3, 4, 5, 8, 12, 16])
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
    # Two rows, narrow weights of little work and groups whose scale column
    # holds a single strip stay on the GEMV; 3..32 rows over wide weights, and
    # narrow ones from (M rounded up to 8) * K * N = 2^28 and 5 rows, take the
    # MFMA kernel; 33 rows the GEMM.
    assert _path(sgq, 2, 4096, 11008, 128) == 0
    assert _path(sgq, 3, 4096, 11008, 128) == SKINNY
    assert _path(sgq, 4, 2048, 6144, 128) == SKINNY
    assert _path(sgq, 33, 4096, 11008, 128) == 1
    assert _path(sgq, 8, 5632, 2048, 128) == 0
    assert _path(sgq, 8, 2048, 6144, 8) == 0
    assert _path(sgq, 4, 11008, 4096, 128) == 0
    assert _path(sgq, 8, 11008, 4096, 128) == SKINNY
    assert _path(sgq, 16, 11008, 4096, 128) == SKINNY
    for M in range(3, 33):
        assert _path(sgq, M, 4096, 11008, 128) == SKINNY


def _splits(sgq, M, K, N, G):
    lib = sgq.load_library()
    path, ks = ctypes.c_int(), ctypes.c_int()
    assert lib.sgq_linear_plan(4, M, K, N, G, 0, ctypes.byref(path), ctypes.byref(ks)) == 0
    return ks.value


# The super-block form: two row blocks over wide weights (17..32 rows; a K
# longer than 8192 rows splits even there), and narrow weights whose K is
# split into ranges added by the reduce kernel; K tails inside a super-block
# and a group of 32 (two column blocks per workgroup).
@pytest.mark.parametrize("M,K,N,G,ks", [(17, 4096, 11008, 128, 1), (24, 4096, 11008, 128, 1),
                                        (32, 4096, 11008, 128, 1), (24, 2048, 6144, 128, 1),
                                        (20, 2048, 5120, 32, 1), (17, 4112, 6144, 128, 1),
                                        (24, 16384, 11008, 128, 2), (12, 11008, 4096, 128, 4),
                                        (16, 11008, 4096, 128, 4), (17, 11008, 4096, 128, 4),
                                        (32, 11008, 4096, 128, 4), (32, 4096, 4096, 128, 4),
                                        (16, 11024, 4096, 128, 4), (32, 8192, 3072, 32, 4)])
def test_skinny_superblock_shapes(sgq, dev, oracle, synth, M, K, N, G, ks):
    path = _path(sgq, M, K, N, G)
    print(f"  case M={M} K={K} N={N} G={G} path={path} k_splits={_splits(sgq, M, K, N, G)}", flush=True)
    assert path == SKINNY and _splits(sgq, M, K, N, G) == ks
    W, b, qw, (q, s) = _quantized(sgq, dev, oracle, synth, K, N, G, 71)
    x = synth.normal((M, K), synth.config_seed(71), synth.STREAM_X, 0.0, 1.0)
    y = _np(sgq.quantized_matmul_int4(_to_dev(x, dev), qw, _to_dev(b, dev)))
    yref = oracle.quantized_matmul_int4(x, q, s, G, b)
    e = rel_err(y, yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


# x that is not 16-byte aligned, or whose rows are not a multiple of four
# floats, takes the kernel's one-float loads (both forms, split K).
@pytest.mark.parametrize("M,K,N,offset", [(8, 2048, 6144, 1), (8, 2050, 6144, 0), (8, 2051, 6144, 3),
                                          (17, 2050, 6144, 0), (24, 2051, 6144, 3), (16, 11008, 4096, 1),
                                          (20, 11010, 4096, 0)])
def test_skinny_unaligned_x(sgq, dev, oracle, synth, M, K, N, offset):
    G = 128
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
@pytest.mark.parametrize("M,N", [(16, 5632), (16, 4096), (32, 5632)])
def test_skinny_same_sign_activations(sgq, dev, oracle, synth, kind, M, N):
    # Same-sign inputs at long K: no cancellation between terms to hide an
    # error in the split of x * s (whole K, split K, two row blocks).
    K, G = 11008, 128
    assert _path(sgq, M, K, N, G) == SKINNY
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


@pytest.mark.parametrize("M,K,N", [(8, 2048, 6144), (24, 2048, 6144), (16, 11008, 4096)])
def test_skinny_infinite_activation(sgq, dev, oracle, synth, M, K, N):
    # inf * s split into three bf16 planes is inf - inf; the kernel hands a
    # non-finite total (of its K range) to the reference's k-order sum, so
    # infinities and NaNs land where the reference's x . (q * s) puts them.
    G = 128
    assert _path(sgq, M, K, N, G) == SKINNY
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


@pytest.mark.parametrize("K,N,Ms", [(4096, 11008, (5, 9, 13, 16)), (4096, 11008, (17, 24, 29, 32)),
                                     (11008, 4096, (12, 16, 17, 25, 32))])
def test_skinny_rows_independent_and_deterministic(sgq, dev, synth, K, N, Ms):
    # A row's sums do not depend on the other rows of the batch (each is its
    # own row of the MFMA tile; the K ranges and wavefronts of a form do not
    # depend on M), and repeated calls give identical bits.
    G = 128
    W, _ = _weights(synth, K, N, 66, G)
    x = _to_dev(synth.normal((Ms[-1], K), synth.config_seed(66), synth.STREAM_X, 0.0, 1.0), dev)
    qw = sgq.quantize_int4(_to_dev(W, dev), G)
    y = sgq.quantized_matmul_int4(x, qw).clone()
    for M in Ms[:-1]:
        assert torch.equal(sgq.quantized_matmul_int4(x[:M].contiguous(), qw), y[:M])
    for _ in range(3):
        assert torch.equal(sgq.quantized_matmul_int4(x, qw), y)


@pytest.mark.parametrize("M,K,N", [(8, 2048, 5632), (16, 4096, 11008), (24, 2048, 5632), (16, 11008, 4096),
                                   (32, 4096, 4096)])
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
