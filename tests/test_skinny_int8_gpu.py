"""GPU parity of the INT8 forward on the bf16 matrix cores (k_skinny8):
batches of 5..128 rows with enough work for it (sgq_linear_plan path 4),
per-tensor and per-channel, against the oracle's dequantize-then-matmul on the
same quantized weights (src/quantization.cpp:189-197), and of the INT8 gated
MLP that runs both of its projections through the same kernel.

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
SKINNY = 4  # sgq_linear_plan path of the skinny MFMA kernels


def _to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _path(sgq, M, K, N):
    lib = sgq.load_library()
    path, ks = ctypes.c_int(), ctypes.c_int()
    assert lib.sgq_linear_plan(8, M, K, N, 0, 0, ctypes.byref(path), ctypes.byref(ks)) == 0
    return path.value, ks.value


_QUANT = {}


def _quantized(sgq, dev, oracle, synth, K, N, scheme, seed):
    """Weight, bias, device weight and the oracle's codes and scales of one
    shape, made once for all batch sizes."""
    key = (K, N, scheme, seed)
    if key not in _QUANT:
        _QUANT.clear()
        cs = synth.config_seed(seed)
        W = synth.normal((K, N), cs, synth.STREAM_W, 0.0, 0.02)
        b = synth.normal((1, N), cs, synth.STREAM_BIAS, 0.0, 0.02)
        _QUANT[key] = (W, b, sgq.quantize_int8(_to_dev(W, dev), scheme), oracle.quantize_int8(W, scheme))
    return _QUANT[key]


def test_skinny_int8_boundaries(sgq, dev):
    # Four rows and little work stay on the GEMV; above 16 rows, shapes with
    # M * K * N > 2^29 take the GEMM.
    assert _path(sgq, 4, 4096, 4096) == (0, 1)
    assert _path(sgq, 8, 2048, 2048) == (0, 1)
    assert _path(sgq, 32, 1024, 1024) == (0, 1)
    assert _path(sgq, 129, 1024, 1024)[0] == 1
    assert _path(sgq, 33, 4096, 4096)[0] == 1
    assert _path(sgq, 128, 2048, 2056)[0] == 1
    for M in (5, 8, 16):
        assert _path(sgq, M, 4096, 4096) == (SKINNY, 1)
    assert _path(sgq, 17, 1024, 1024) == (0, 1)
    for M in (64, 100, 128):
        assert _path(sgq, M, 1024, 1024) == (SKINNY, 1)
    for M in (9, 16, 17, 64):
        assert _path(sgq, M, 2048, 2048) == (SKINNY, 1)
    assert _path(sgq, 16, 11008, 4096) == (SKINNY, 1)


# C1 (1024 -> 1024 + bias at 128 rows), one and two row blocks, ragged M,
# a K that ends inside a 32-row k block and one not a multiple of four, an N
# that ends inside a strip, and a wide and a long weight.
@pytest.mark.parametrize("scheme", [0, 1])
@pytest.mark.parametrize("M,K,N", [(128, 1024, 1024), (100, 1024, 1024), (65, 1024, 1024), (17, 2048, 2048),
                                   (48, 2048, 2048), (5, 4096, 4096), (8, 4096, 4096), (13, 4096, 4096),
                                   (16, 4096, 4096), (16, 4096, 11008), (16, 11008, 4096), (96, 1040, 1000),
                                   (40, 2051, 1034), (12, 4100, 4098), (32, 4096, 4096), (128, 2048, 2048),
                                   (128, 4096, 1024)])
def test_skinny_int8_shapes(sgq, dev, oracle, synth, scheme, M, K, N):
    assert _path(sgq, M, K, N) == (SKINNY, 1)
    W, b, qw, (q, s) = _quantized(sgq, dev, oracle, synth, K, N, scheme, 81)
    x = synth.normal((M, K), synth.config_seed(81), synth.STREAM_X, 0.0, 1.0)
    print(f"  case scheme={scheme} M={M} K={K} N={N}", flush=True)
    y = _np(sgq.quantized_matmul_int8(_to_dev(x, dev), qw, _to_dev(b, dev)))
    yref = oracle.quantized_matmul_int8(x, q, s, scheme, b)
    e = rel_err(y, yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


# x that is not 16-byte aligned takes the kernel's one-float loads.
@pytest.mark.parametrize("scheme", [0, 1])
@pytest.mark.parametrize("M,K,N,offset", [(128, 1024, 1024, 1), (8, 4096, 4096, 3), (40, 2048, 2048, 2)])
def test_skinny_int8_unaligned_x(sgq, dev, oracle, synth, scheme, M, K, N, offset):
    assert _path(sgq, M, K, N) == (SKINNY, 1)
    W, b, qw, (q, s) = _quantized(sgq, dev, oracle, synth, K, N, scheme, 82)
    flat = synth.normal((M * K + offset,), synth.config_seed(82), synth.STREAM_X, 0.0, 1.0)
    x = _to_dev(flat, dev)[offset:].view(M, K)
    print(f"  case M={M} K={K} offset={offset} aligned={x.data_ptr() % 16 == 0}", flush=True)
    y = _np(sgq.quantized_matmul_int8(x, qw, _to_dev(b, dev)))
    e = rel_err(y, oracle.quantized_matmul_int8(flat[offset:].reshape(M, K), q, s, scheme, b))
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


@pytest.mark.parametrize("kind", ["abs", "silu"])
@pytest.mark.parametrize("scheme", [0, 1])
def test_skinny_int8_same_sign_activations(sgq, dev, oracle, synth, kind, scheme):
    # Same-sign inputs at long K: no cancellation between terms to hide an
    # error in the split of x (or x * s).
    M, K, N = 16, 11008, 4096
    assert _path(sgq, M, K, N) == (SKINNY, 1)
    W, _, qw, (q, s) = _quantized(sgq, dev, oracle, synth, K, N, scheme, 83)
    z = synth.normal((M, K), synth.config_seed(83), synth.STREAM_X, 0.0, 1.0)
    if kind == "abs":
        x = np.abs(z).astype(np.float32)
    else:
        zz = (2.0 * z).astype(np.float32)
        x = (zz / (np.float32(1.0) + np.exp(-zz))).astype(np.float32)
    y = _np(sgq.quantized_matmul_int8(_to_dev(x, dev), qw))
    e = rel_err(y, oracle.quantized_matmul_int8(x, q, s, scheme))
    print(f"  case x={kind} scheme={scheme} rel_err={e:.3e}", flush=True)
    assert e <= TOL


@pytest.mark.parametrize("M,K,N", [(8, 4096, 4096), (40, 2048, 2048)])
def test_skinny_int8_split_sums_to_rounded_product(sgq, dev, M, K, N):
    # One nonzero activation per row (column k0), per-channel scales and
    # codes of 1 in weight row k0: every output is h + m + l of x * s[k0],
    # each partial sum exact, so y == float32(x * s[k0]) bit for bit.
    k0 = 1234
    assert _path(sgq, M, K, N) == (SKINNY, 1)
    rng = np.random.default_rng(3000 + M)
    x = np.zeros((M, K), np.float32)
    x[:, k0] = (rng.standard_normal(M) * 10.0 ** rng.uniform(-3, 3, M)).astype(np.float32)
    q = rng.integers(-127, 128, (K, N)).astype(np.float32)
    q[k0, :] = 1.0
    s = rng.uniform(1e-3, 1.0, K).astype(np.float32)
    qw = sgq.pack_int8(_to_dev(q, dev), _to_dev(s, dev), 1)
    y = _np(sgq.quantized_matmul_int8(_to_dev(x, dev), qw))
    want = np.repeat(x[:, k0:k0 + 1] * s[k0], N, axis=1).astype(np.float32)
    assert helpers.same_bits(y, want), np.count_nonzero(y != want)


@pytest.mark.parametrize("scheme", [0, 1])
@pytest.mark.parametrize("M,K,N", [(8, 4096, 4096), (128, 1024, 1024)])
def test_skinny_int8_infinite_activation(sgq, dev, oracle, synth, scheme, M, K, N):
    # inf split into three bf16 planes is inf - inf; the kernel hands a
    # non-finite total to the reference's k-order sum, so infinities and NaNs
    # land where the reference's x . (q * s) puts them.
    W, _, qw, (q, s) = _quantized(sgq, dev, oracle, synth, K, N, scheme, 84)
    x = synth.normal((M, K), synth.config_seed(84), synth.STREAM_X, 0.0, 1.0)
    x[0, 17] = np.inf
    x[M - 1, 600] = -np.inf
    x[1, 3] = np.inf
    x[1, 900] = -np.inf
    x[2, 1000] = np.nan
    y = _np(sgq.quantized_matmul_int8(_to_dev(x, dev), qw))
    yref = oracle.quantized_matmul_int8(x, q, s, scheme)
    assert np.isinf(yref).any() and np.isnan(yref).any()
    assert np.array_equal(np.isnan(y), np.isnan(yref))
    assert np.array_equal(np.isposinf(y), np.isposinf(yref))
    assert np.array_equal(np.isneginf(y), np.isneginf(yref))
    fin = np.isfinite(yref)
    assert np.max(np.abs(y[fin].astype(np.float64) - yref[fin])) <= TOL * np.max(np.abs(yref[fin]))


@pytest.mark.parametrize("K,N,Ms", [(4096, 4096, (5, 9, 16)), (2048, 2048, (9, 16, 17, 40, 64)),
                                     (1024, 1024, (65, 100, 128))])
def test_skinny_int8_rows_independent_and_deterministic(sgq, dev, synth, K, N, Ms):
    # A row's sums do not depend on the other rows of the batch (each is its
    # own row of an MFMA tile; the wavefronts' k blocks and their order do not
    # depend on M or the row blocks per workgroup), and repeated calls give
    # identical bits.
    cs = synth.config_seed(85)
    W = synth.normal((K, N), cs, synth.STREAM_W, 0.0, 0.02)
    x = _to_dev(synth.normal((Ms[-1], K), cs, synth.STREAM_X, 0.0, 1.0), dev)
    qw = sgq.quantize_int8(_to_dev(W, dev), 1)
    y = sgq.quantized_matmul_int8(x, qw).clone()
    for M in Ms[:-1]:
        assert _path(sgq, M, K, N) == (SKINNY, 1)
        assert torch.equal(sgq.quantized_matmul_int8(x[:M].contiguous(), qw), y[:M])
    for _ in range(3):
        assert torch.equal(sgq.quantized_matmul_int8(x, qw), y)


@pytest.mark.parametrize("scheme", [0, 1])
@pytest.mark.parametrize("M,K,N", [(8, 4096, 4096), (128, 1024, 1024)])
def test_skinny_int8_swiglu(sgq, dev, oracle, synth, scheme, M, K, N):
    # The INT8 gated MLP runs gate and up through the same kernel as two
    # forward calls: equal to them followed by the oracle's silu and mul to
    # rounding, and to the oracle's gated MLP within the forward's bar.
    assert _path(sgq, M, K, N) == (SKINNY, 1)
    cs = synth.config_seed(86)
    Wg = synth.normal((K, N), cs, synth.STREAM_W, 0.0, 0.02)
    Wu = synth.normal((K, N), cs, synth.STREAM_W2, 0.0, 0.02)
    bg = synth.normal((1, N), cs, synth.STREAM_BIAS, 0.0, 0.02)
    bu = synth.normal((1, N), cs, synth.STREAM_BIAS2, 0.0, 0.02)
    x = synth.normal((M, K), cs, synth.STREAM_X, 0.0, 1.0)
    xd = _to_dev(x, dev)
    wg, wu = sgq.quantize_int8(_to_dev(Wg, dev), scheme), sgq.quantize_int8(_to_dev(Wu, dev), scheme)
    bgd, bud = _to_dev(bg, dev), _to_dev(bu, dev)
    h = _np(sgq.quantized_swiglu(xd, wg, wu, bgd, bud))
    g = _np(sgq.quantized_matmul_int8(xd, wg, bgd))
    u = _np(sgq.quantized_matmul_int8(xd, wu, bud))
    e2 = rel_err(h, oracle.mul(oracle.silu(g), u))
    qg, sg = oracle.quantize_int8(Wg, scheme)
    qu, su = oracle.quantize_int8(Wu, scheme)
    e = rel_err(h, oracle.swiglu_int8(x, qg, sg, qu, su, scheme, bg, bu))
    print(f"  case scheme={scheme} M={M} vs two calls {e2:.3e} vs oracle {e:.3e}", flush=True)
    assert e2 <= 2e-7
    assert e <= TOL
