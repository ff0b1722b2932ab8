"""GPU parity of the fused dequantize + matmul forward.

Outputs must be within max|y - y_ref| / max|y_ref| <= 1e-5 of the CPU
dequantize-then-matmul (fp32 accumulate; the kernels accumulate in a different
order, so bits are not expected to match).  y_ref comes from the golden
fixtures (compiled reference) or the oracle on the same quantized weights.
"""
import ctypes

import numpy as np
import pytest
import torch

import helpers
from helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5  # max relative error of the forward against the CPU reference


def _to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def test_golden_linear(sgq, dev, golden):
    n = 0
    for c in golden:
        if c["kind"] not in ("linear_int8", "linear_int4"):
            continue
        p = c["params"]
        print(f"  case {c['kind']} {p}", flush=True)
        x = _to_dev(c["x"], dev)
        b = _to_dev(c["bias"], dev) if "bias" in c else None
        if c["kind"] == "linear_int8":
            qw = sgq.pack_int8(_to_dev(c["q"], dev), _to_dev(c["s"], dev), p["scheme"])
            y = sgq.quantized_matmul_int8(x, qw, b)
        else:
            qw = sgq.pack_int4(_to_dev(c["q"], dev), _to_dev(c["s"], dev), p["group_size"])
            y = sgq.quantized_matmul_int4(x, qw, b)
        e = rel_err(_np(y), c["y"])
        assert e <= TOL, (p, e)
        n += 1
    assert n >= 16


def _case(sgq, dev, oracle, synth, bits_, M, K, N, G=128, scheme=0, bias=False, seed=1, rows=None):
    W = synth.normal((K, N), synth.config_seed(seed), synth.STREAM_W, 0.0, 0.02)
    x = synth.normal((M, K), synth.config_seed(seed), synth.STREAM_X, 0.0, 1.0)
    b = synth.normal((1, N), synth.config_seed(seed), synth.STREAM_BIAS, 0.0, 0.02) if bias else None
    xd = _to_dev(x, dev)
    bd = _to_dev(b, dev) if bias else None
    if bits_ == 8:
        qw = sgq.quantize_int8(_to_dev(W, dev), scheme)
        y = sgq.quantized_matmul_int8(xd, qw, bd)
        q, s = oracle.quantize_int8(W, scheme)
        sub = x if rows is None else x[rows]
        yref = oracle.quantized_matmul_int8(sub, q, s, scheme, b)
    else:
        qw = sgq.quantize_int4(_to_dev(W, dev), G)
        y = sgq.quantized_matmul_int4(xd, qw, bd)
        q, s = oracle.quantize_int4(W, G)
        sub = x if rows is None else x[rows]
        yref = oracle.quantized_matmul_int4(sub, q, s, G, b)
    yg = _np(y)
    if rows is not None:
        yg = yg[rows]
    return yg, yref


# BASELINE configs 1-5 (config 4 checked on a row subset: rows of the GEMM are independent)
@pytest.mark.parametrize(
    "name,bits_,M,K,N,G,scheme,bias,seed",
    [
        ("C1_int8_pt_bias_M128", 8, 128, 1024, 1024, 0, 0, True, 0),
        ("C2_int4_g128_M1", 4, 1, 4096, 4096, 128, 0, False, 1),
        ("C3_gate_M1", 4, 1, 4096, 11008, 128, 0, False, 2),
        ("C3_gate_M2", 4, 2, 4096, 11008, 128, 0, False, 2),
        ("C3_down_M2", 4, 2, 11008, 4096, 128, 0, False, 2),
        ("C3_gate_M4", 4, 4, 4096, 11008, 128, 0, False, 2),
        ("C3_gate_M8", 4, 8, 4096, 11008, 128, 0, False, 2),
        ("C3_gate_M16", 4, 16, 4096, 11008, 128, 0, False, 2),
        ("C3_down_M1", 4, 1, 11008, 4096, 128, 0, False, 2),
        ("C3_down_M4", 4, 4, 11008, 4096, 128, 0, False, 2),
        ("C3_down_M8", 4, 8, 11008, 4096, 128, 0, False, 2),
        ("C3_down_M16", 4, 16, 11008, 4096, 128, 0, False, 2),
        ("C5_qkv_M8", 4, 8, 2048, 6144, 128, 0, False, 4),
        ("C5_o_M8", 4, 8, 2048, 2048, 128, 0, False, 4),
        ("C5_up_M8", 4, 8, 2048, 5632, 128, 0, False, 4),
        ("C5_down_M8", 4, 8, 5632, 2048, 128, 0, False, 4),
    ],
)
def test_configs(sgq, dev, oracle, synth, name, bits_, M, K, N, G, scheme, bias, seed):
    print(f"  case {name}", flush=True)
    y, yref = _case(sgq, dev, oracle, synth, bits_, M, K, N, G, scheme, bias, seed)
    e = rel_err(y, yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


def test_config4_gemm_rows(sgq, dev, oracle, synth):
    M = 2048
    rows = np.r_[0:16, 1000:1016, 2032:2048]
    print("  case C4_int8_pt_M2048 (48 rows vs oracle)", flush=True)
    y, yref = _case(sgq, dev, oracle, synth, 8, M, 4096, 4096, 0, 0, False, 3, rows=rows)
    e = rel_err(y, yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


def test_config4_gemm_all_rows_vs_fp64(sgq, dev, oracle, synth):
    """C4 in full: all 2048 rows of the M=2048 INT8 per-tensor GEMM within 1e-5
    of an fp64 product of x with the reference's fp32 weights q * s (beside the
    48-row oracle check above)."""
    M, K, N = 2048, 4096, 4096
    W = synth.normal((K, N), synth.config_seed(3), synth.STREAM_W, 0.0, 0.02)
    x = synth.normal((M, K), synth.config_seed(3), synth.STREAM_X, 0.0, 1.0)
    print("  case C4_int8_pt_M2048 (all rows vs fp64)", flush=True)
    qw = sgq.quantize_int8(_to_dev(W, dev), 0)
    y = _np(sgq.quantized_matmul_int8(_to_dev(x, dev), qw))
    q, s = oracle.quantize_int8(W, 0)
    w32 = oracle.dequantize_int8(q, s, 0)
    y64 = x.astype(np.float64) @ np.asarray(w32, np.float64)
    e = rel_err(y, y64)
    print(f"    rel_err vs fp64 over {M} rows: {e:.3e}", flush=True)
    assert e <= TOL


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("K,N", [(4096, 4096), (11008, 4096), (4096, 11008)])
@pytest.mark.parametrize("kind", ["abs", "silu"])
def test_same_sign_activations(sgq, dev, oracle, synth, M, K, N, kind):
    """The one- and two-row INT4 GEMV accumulates offset-binary codes u = q + 8
    and subtracts 8 * sum(x * s) per lane.  With activations of one sign (|x|,
    or silu outputs, as the down projection sees them) at long K, that
    correction is as large as it gets; the result must still be within 1e-5 of
    the reference's dequantize-then-matmul."""
    W = synth.normal((K, N), synth.config_seed(40), synth.STREAM_W, 0.0, 0.02)
    z = synth.normal((M, K), synth.config_seed(40), synth.STREAM_X, 0.0, 1.0)
    if kind == "abs":
        x = np.abs(z).astype(np.float32)
    else:
        zz = (2.0 * z).astype(np.float32)
        x = (zz / (np.float32(1.0) + np.exp(-zz))).astype(np.float32)
    print(f"  case M={M} K={K} N={N} x={kind}", flush=True)
    qw = sgq.quantize_int4(_to_dev(W, dev), 128)
    y = _np(sgq.quantized_matmul_int4(_to_dev(x, dev), qw))
    q, s = oracle.quantize_int4(W, 128)
    yref = oracle.quantized_matmul_int4(x, q, s, 128)
    e = rel_err(y, yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


# Batches of 17..64 rows with too much work for the GEMV take the GEMM's 32-
# and 64-row tiles (split K), or for INT4 up to 32 rows the skinny MFMA
# kernel's super-block form; every row against the oracle.
@pytest.mark.parametrize("M", [17, 24, 32, 33, 48, 64])
@pytest.mark.parametrize("bits_,K,N,G,scheme", [(4, 4096, 11008, 128, 0), (4, 11008, 4096, 128, 0),
                                                (8, 4096, 8192, 0, 0), (8, 4096, 8192, 0, 1)])
def test_skinny_gemm_tiles(sgq, dev, oracle, synth, M, bits_, K, N, G, scheme):
    lib = sgq.load_library()
    path, ks = ctypes.c_int(), ctypes.c_int()
    assert lib.sgq_linear_plan(bits_, M, K, N, G, 256, ctypes.byref(path), ctypes.byref(ks)) == 0
    print(f"  case M={M} K={K} N={N} bits={bits_} path={path.value} k_splits={ks.value}", flush=True)
    assert path.value == (4 if bits_ == 4 and M <= 32 else 1)  # skinny MFMA kernel, or the three-term GEMM
    y, yref = _case(sgq, dev, oracle, synth, bits_, M, K, N, G, scheme, True, 17)
    e = rel_err(y, yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


# Prefill-sized GEMMs, checked on a row subset (first, middle and last rows).
@pytest.mark.parametrize(
    "name,bits_,M,K,N,G,scheme",
    [
        ("C3_down_prefill_int4_g128", 4, 512, 11008, 4096, 128, 0),  # long K
        ("C3_gate_prefill_int4_g128_ragged_M", 4, 300, 4096, 11008, 128, 0),  # partial last row tile
        ("int4_g256_M384", 4, 384, 2048, 2048, 256, 0),  # two 128-column tiles per scale column
        ("int4_g64_M256", 4, 256, 2048, 1024, 64, 0),  # group not a multiple of 128: the fp32 GEMM
        ("int8_pc_prefill", 8, 1024, 4096, 11008, 0, 1),
    ],
)
def test_prefill_gemm_rows(sgq, dev, oracle, synth, name, bits_, M, K, N, G, scheme):
    print(f"  case {name}", flush=True)
    rows = np.r_[0:16, M // 2 - 8:M // 2 + 8, M - 16:M]
    y, yref = _case(sgq, dev, oracle, synth, bits_, M, K, N, G, scheme, True, 13, rows=rows)
    e = rel_err(y, yref)
    print(f"    rel_err={e:.3e}", flush=True)
    assert e <= TOL


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 9, 15, 16, 17, 31, 33, 64, 129])
@pytest.mark.parametrize("bits_", [8, 4])
def test_batch_sizes(sgq, dev, oracle, synth, M, bits_):
    y, yref = _case(sgq, dev, oracle, synth, bits_, M, 320, 192, 32, 1, True, 7)
    assert rel_err(y, yref) <= TOL


@pytest.mark.parametrize(
    "bits_,M,K,N,G,scheme",
    [
        (4, 100, 1000, 1000, 128, 0),  # 13 row groups, padded to 16; one scale column per strip (N % G != 0)
        (4, 72, 2048, 1024, 128, 0),  # 9 row groups -> 16
        (4, 120, 512, 384, 64, 0),
        (8, 128, 1024, 1024, 0, 0),  # C1's shape: 16 row groups
        (8, 57, 777, 515, 0, 1),  # ragged K and N
        (8, 17, 4099, 30, 0, 0),
    ],
)
def test_mid_batches_on_gemv(sgq, dev, oracle, synth, bits_, M, K, N, G, scheme):
    # Batches of 17..128 rows with little work run the GEMV in row groups of 8
    # (no workspace), not the split-K GEMM.
    assert sgq.load_library().sgq_linear_workspace_bytes(bits_, M, K, N) == 0
    y, yref = _case(sgq, dev, oracle, synth, bits_, M, K, N, G, scheme, True, 12)
    assert rel_err(y, yref) <= TOL


@pytest.mark.parametrize(
    "M,K,N,G",
    [(1, 1, 8, 8), (3, 17, 24, 8), (5, 130, 77, 7), (2, 33, 40, 24), (19, 18, 200, 40), (7, 100, 12, 8),
     (40, 61, 136, 8), (1, 4099, 24, 8), (20, 45, 13, 5)],
)
def test_ragged_int4(sgq, dev, oracle, synth, M, K, N, G):
    y, yref = _case(sgq, dev, oracle, synth, 4, M, K, N, G, 0, True, 8)
    assert rel_err(y, yref) <= TOL


@pytest.mark.parametrize("M,K,N,scheme", [(1, 1, 1, 0), (3, 17, 70, 1), (18, 130, 65, 0), (33, 7, 129, 1),
                                          (2, 4099, 3, 0), (200, 45, 300, 1)])
def test_ragged_int8(sgq, dev, oracle, synth, M, K, N, scheme):
    y, yref = _case(sgq, dev, oracle, synth, 8, M, K, N, 0, scheme, True, 9)
    assert rel_err(y, yref) <= TOL


# Small batches (2 <= M <= 16, the decode kernel's multi-row passes): K ragged
# against the 4-row chunk and the 256-row-quad iteration, long and short K,
# several group sizes.
@pytest.mark.parametrize("M", [2, 4, 6, 8, 11, 16])
@pytest.mark.parametrize("K,N,G", [(1000, 256, 128), (1001, 96, 32), (5000, 384, 64), (300, 512, 256),
                                   (4096, 128, 128)])
def test_small_batch_int4(sgq, dev, oracle, synth, M, K, N, G):
    y, yref = _case(sgq, dev, oracle, synth, 4, M, K, N, G, 0, M % 2 == 0, 10)
    assert rel_err(y, yref) <= TOL


# Five to eight INT4 rows over K <= 2048 run the GEMV as two row groups of four
# (the second reading each strip's codes again): odd and even M, K past and on
# a row-quad boundary, with and without bias.
@pytest.mark.parametrize("M", [5, 7, 8])
@pytest.mark.parametrize("K,N,G", [(2048, 2048, 128), (1023, 512, 64), (2048, 256, 32), (6, 64, 16)])
def test_two_row_groups_of_four(sgq, dev, oracle, synth, M, K, N, G):
    y, yref = _case(sgq, dev, oracle, synth, 4, M, K, N, G, 0, M % 2 == 1, 13)
    assert rel_err(y, yref) <= TOL


# Two to sixteen rows over narrow weights (fewer workgroups than compute units
# in the default grouping) run the GEMV in more, smaller row groups: two groups
# of two at three and four rows, groups of four from five (and, at five to
# eight rows, over any K <= 2048).  K past 2048, ragged K, a single-strip-group
# N, with and without bias; INT4 and INT8.
@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 9, 12, 16])
@pytest.mark.parametrize("K,N,G", [(8192, 1024, 128), (4100, 256, 128), (2048, 512, 128), (3001, 64, 32)])
def test_row_groups_on_narrow_weights(sgq, dev, oracle, synth, M, K, N, G):
    y, yref = _case(sgq, dev, oracle, synth, 4, M, K, N, G, 0, M % 2 == 0, 17)
    assert rel_err(y, yref) <= TOL


@pytest.mark.parametrize("M", [2, 4, 5, 6, 8, 12])
@pytest.mark.parametrize("K,N,scheme", [(4096, 512, 0), (2051, 300, 1), (8192, 1020, 0), (2048, 2048, 0),
                                        (1023, 500, 1)])
def test_row_groups_on_narrow_weights_int8(sgq, dev, oracle, synth, M, K, N, scheme):
    y, yref = _case(sgq, dev, oracle, synth, 8, M, K, N, 0, scheme, M % 4 == 0, 19)
    assert rel_err(y, yref) <= TOL


# INT8 strips ragged (N % 4 != 0), per-tensor and per-channel scales.
@pytest.mark.parametrize("M", [2, 7, 13, 16])
@pytest.mark.parametrize("K,N,scheme", [(1000, 70, 1), (4099, 30, 0), (333, 1000, 1), (64, 17, 0), (6000, 256, 1)])
def test_small_batch_int8(sgq, dev, oracle, synth, M, K, N, scheme):
    y, yref = _case(sgq, dev, oracle, synth, 8, M, K, N, 0, scheme, M % 2 == 1, 11)
    assert rel_err(y, yref) <= TOL


@pytest.mark.parametrize("bits_,M", [(4, 8), (8, 5), (4, 16), (8, 2)])
def test_batch_rows_are_independent(sgq, dev, synth, bits_, M):
    # Batch row r of x feeds output row r only: a NaN in x[r] poisons y[r] and
    # nothing else.
    W = _to_dev(synth.normal((4096, 256), 71, 0, 0.0, 0.02), dev)
    qw = sgq.quantize_int8(W, 1) if bits_ == 8 else sgq.quantize_int4(W, 128)
    x = _to_dev(synth.normal((M, 4096), 71, 1), dev)
    for r in sorted({0, 2 % M, M - 1}):
        xx = x.clone()
        xx[r, 1234] = float("nan")
        y = sgq.quantized_matmul(xx, qw)
        torch.cuda.synchronize()
        others = [i for i in range(M) if i != r]
        assert torch.isnan(y[r]).all(), r
        assert torch.isfinite(y[others]).all(), r


def test_small_batch_deterministic(sgq, dev, synth):
    # Lanes and wavefronts are summed in a fixed order: identical bits every call.
    W = _to_dev(synth.normal((4096, 1024), 81, 0, 0.0, 0.02), dev)
    x = _to_dev(synth.normal((8, 4096), 81, 1), dev)
    for qw in (sgq.quantize_int4(W, 128), sgq.quantize_int8(W, 0)):
        y1 = sgq.quantized_matmul(x, qw).clone()
        for _ in range(3):
            assert torch.equal(sgq.quantized_matmul(x, qw), y1)


def test_unaligned_x_pointer(sgq, dev, oracle, synth):
    # x offset by one float: the kernels must not assume 16-byte alignment.
    W = synth.normal((64, 128), 31, 0, 0.0, 0.02)
    xs = synth.normal((4 * 64 + 1,), 31, 1)
    x = _to_dev(xs, dev)[1:].view(4, 64)
    for bits_ in (8, 4):
        qw = sgq.quantize_int8(_to_dev(W, dev), 0) if bits_ == 8 else sgq.quantize_int4(_to_dev(W, dev), 32)
        y = sgq.quantized_matmul(x, qw)
        if bits_ == 8:
            q, s = oracle.quantize_int8(W, 0)
            yref = oracle.quantized_matmul_int8(xs[1:].reshape(4, 64), q, s, 0)
        else:
            q, s = oracle.quantize_int4(W, 32)
            yref = oracle.quantized_matmul_int4(xs[1:].reshape(4, 64), q, s, 32)
        assert rel_err(_np(y), yref) <= TOL


def test_empty_shapes(sgq, dev):
    qw = sgq.quantize_int4(torch.zeros((0, 16), device=dev), 8)
    b = torch.arange(16, dtype=torch.float32, device=dev)
    y = sgq.quantized_matmul_int4(torch.zeros((3, 0), device=dev), qw, b)
    assert torch.equal(y, b.expand(3, 16))  # K == 0: y = bias (matmul of zeros, then bias)
    qw8 = sgq.quantize_int8(torch.ones((8, 4), device=dev), 1)
    y0 = sgq.quantized_matmul_int8(torch.zeros((0, 8), device=dev), qw8)
    assert y0.shape == (0, 4)


def test_deterministic_and_workspace_reuse(sgq, dev, synth):
    # Lanes and wavefronts are summed in a fixed order: repeated calls give
    # identical bits, also after the workspace served other shapes.
    W = _to_dev(synth.normal((4096, 4096), 41, 0, 0.0, 0.02), dev)
    x = _to_dev(synth.normal((1, 4096), 41, 1), dev)
    qw = sgq.quantize_int4(W, 128)
    y1 = sgq.quantized_matmul_int4(x, qw).clone()
    W2 = _to_dev(synth.normal((512, 640), 42, 0, 0.0, 0.02), dev)
    qw2 = sgq.quantize_int8(W2, 1)
    for m in (1, 7, 16):
        sgq.quantized_matmul_int8(_to_dev(synth.normal((m, 512), 43, 1), dev), qw2)
    for _ in range(3):
        y2 = sgq.quantized_matmul_int4(x, qw)
        assert torch.equal(y1, y2)


def test_workspace_shared_across_shapes(sgq, dev, oracle, synth):
    # One caller-owned workspace serves calls of different shapes back to back
    # (regression: state kept in a shared workspace must not depend on the shape).
    lib = sgq.load_library()
    shapes = [(1, 4096, 4096), (1, 4096, 11008), (3, 512, 640), (1, 11008, 4096), (16, 2048, 2048),
              (128, 1024, 1024), (40, 2048, 640), (200, 640, 256)]  # the last three split K over workgroups
    nbytes = max(lib.sgq_linear_workspace_bytes(4, m, k, n) for m, k, n in shapes)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    assert lib.sgq_workspace_init(ws.data_ptr(), ws.numel(), stream) == 0
    for rep in range(2):
        for (M, K, N) in shapes:
            W = synth.normal((K, N), 61 + K + N, 0, 0.0, 0.02)
            x = synth.normal((M, K), 61 + K + N, 1)
            qw = sgq.quantize_int4(_to_dev(W, dev), 128)
            y = torch.empty((M, N), device=dev)
            xd = _to_dev(x, dev)
            rc = lib.sgq_linear_int4(xd.data_ptr(), M, K, N, qw.packed.data_ptr(), qw.scales.data_ptr(),
                                     qw.devscales.data_ptr(), 128, None, y.data_ptr(), ws.data_ptr(), ws.numel(),
                                     stream)
            assert rc == 0
            q, s = oracle.quantize_int4(W, 128)
            assert rel_err(_np(y), oracle.quantized_matmul_int4(x, q, s, 128)) <= TOL, (rep, M, K, N)


def test_nonfinite_propagates(sgq, dev):
    # A NaN activation poisons the outputs it touches, as in the reference.
    W = torch.full((32, 64), 0.01, device=dev)
    x = torch.ones((1, 32), device=dev)
    x[0, 5] = float("nan")
    for qw in (sgq.quantize_int8(W, 0), sgq.quantize_int4(W, 32)):
        y = sgq.quantized_matmul(x, qw)
        assert torch.isnan(y).all()


def _same_nonfinite(y, yref):
    """NaN where the reference has NaN, +-inf with its sign, finite entries within TOL."""
    assert np.array_equal(np.isnan(y), np.isnan(yref))
    assert np.array_equal(np.isposinf(y), np.isposinf(yref))
    assert np.array_equal(np.isneginf(y), np.isneginf(yref))
    fin = np.isfinite(yref)
    if fin.any():
        err = np.max(np.abs(y[fin].astype(np.float64) - yref[fin]))
        assert err <= TOL * max(np.max(np.abs(yref[fin])), 1e-30)


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_infinite_activation_matches_reference(sgq, dev, oracle, synth, M):
    # An infinite activation gives +-inf in every column whose code is nonzero
    # and NaN where it meets a zero code (inf * 0), as in the reference's
    # x . (q * s); a row with both signs of infinity is NaN.  The INT4 decode
    # path sums an offset form of the codes, so it must hand such rows to its
    # exact k-order fallback rather than produce inf - inf.
    K, N, G = 1024, 512, 128
    W = synth.normal((K, N), 91, 0, 0.0, 0.02)
    x = synth.normal((M, K), 91, 1)
    x[0, 17] = np.inf
    if M > 1:
        x[M - 1, 600] = -np.inf
    if M > 2:
        x[1, 3] = np.inf
        x[1, 900] = -np.inf
    q, s = oracle.quantize_int4(W, G)
    qw = sgq.quantize_int4(_to_dev(W, dev), G)
    y = _np(sgq.quantized_matmul(_to_dev(x, dev), qw))
    yref = oracle.quantized_matmul_int4(x, q, s, G)
    assert np.isinf(yref).any() and np.isnan(yref).any()
    _same_nonfinite(y, yref)


@pytest.mark.parametrize("bits_,scheme,M", [(8, 0, 40), (8, 1, 40), (4, 0, 40), (8, 0, 300), (4, 0, 150)])
def test_infinite_activation_gemm(sgq, dev, oracle, synth, bits_, scheme, M):
    # The prefill GEMM splits x * s into three bf16 terms, which turns an
    # infinite activation into inf - inf; such outputs must take the exact
    # k-order fallback (per K split when the grid splits K: M = 40 and 150
    # run split-K at this width) and land as the reference's x . (q * s).
    K, N, G = 1024, 512, 128
    W = synth.normal((K, N), 93, 0, 0.0, 0.02)
    x = synth.normal((M, K), 93, 1)
    x[0, 17] = np.inf
    x[M - 1, 600] = -np.inf
    x[1, 3] = np.inf
    x[1, 900] = -np.inf
    x[M // 2, 5] = np.nan
    if bits_ == 8:
        q, s = oracle.quantize_int8(W, scheme)
        qw = sgq.quantize_int8(_to_dev(W, dev), scheme)
        yref = oracle.quantized_matmul_int8(x, q, s, scheme)
    else:
        q, s = oracle.quantize_int4(W, G)
        qw = sgq.quantize_int4(_to_dev(W, dev), G)
        yref = oracle.quantized_matmul_int4(x, q, s, G)
    y = _np(sgq.quantized_matmul(_to_dev(x, dev), qw))
    assert np.isinf(yref).any() and np.isnan(yref).any()
    _same_nonfinite(y, yref)


@pytest.mark.parametrize("bits_,scheme,G", [(8, 0, 0), (8, 1, 0), (4, 0, 128)])
def test_gemm_accuracy_vs_fp64(sgq, dev, oracle, synth, bits_, scheme, G):
    # The prefill GEMM runs the fp32 products on bf16 matrix cores as three
    # exact terms (x * s = h + m + l, codes exact, products exact, fp32
    # sums).  Against an fp64 product with the reference's fp32 weights
    # (q * s), it must be at least as accurate as the reference's own fp32
    # dequantize-then-matmul (the oracle), not merely within the 1e-5 bar.
    M, K, N = 256, 4096, 512
    W = synth.normal((K, N), 95, 0, 0.0, 0.02)
    x = synth.normal((M, K), 95, 1)
    if bits_ == 8:
        q, s = oracle.quantize_int8(W, scheme)
        qw = sgq.quantize_int8(_to_dev(W, dev), scheme)
        yref = oracle.quantized_matmul_int8(x, q, s, scheme)
        w32 = oracle.dequantize_int8(q, s, scheme)
    else:
        q, s = oracle.quantize_int4(W, G)
        qw = sgq.quantize_int4(_to_dev(W, dev), G)
        yref = oracle.quantized_matmul_int4(x, q, s, G)
        w32 = oracle.dequantize_int4(q, s, G)
    y = _np(sgq.quantized_matmul(_to_dev(x, dev), qw))
    y64 = x.astype(np.float64) @ np.asarray(w32, np.float64).reshape(K, N)
    scale = np.max(np.abs(y64))
    e_gpu = np.max(np.abs(y - y64)) / scale
    e_ref = np.max(np.abs(yref - y64)) / scale
    print(f"    max rel err vs fp64: gpu {e_gpu:.3e}, reference fp32 path {e_ref:.3e}", flush=True)
    assert e_gpu <= TOL
    assert e_gpu <= 2.0 * e_ref


@pytest.mark.parametrize("bits_,scheme,k0", [(8, 0, 0), (8, 1, 0), (8, 1, 150), (4, 0, 0), (4, 0, 150)])
def test_gemm_split_sums_to_rounded_product(sgq, dev, bits_, scheme, k0):
    # The three bf16 planes of x * s must add up to x * s rounded once to
    # fp32, exactly.  With one nonzero activation per row (column k0) and
    # codes of 1 in weight row k0, every GEMM output is h + m + l (each sum
    # exact), so y == float32(x * s) bit for bit -- whatever the rounding of
    # the matrix cores' accumulation.  A split of the unrounded product (an
    # fma fused into the split) misses by an ulp in about a quarter of them.
    # M = 256 takes the GEMM; K = 256 splits it over four K ranges.
    M, K, N, G = 256, 256, 256, 128
    rng = np.random.default_rng(1000 + k0 + bits_)
    x = np.zeros((M, K), np.float32)
    x[:, k0] = (rng.standard_normal(M) * 10.0 ** rng.uniform(-3, 3, M)).astype(np.float32)
    lim = 127 if bits_ == 8 else 7
    q = rng.integers(-lim, lim + 1, (K, N)).astype(np.float32)
    q[k0, :] = 1.0
    if bits_ == 8:
        s = rng.uniform(1e-3, 1.0, 1 if scheme == 0 else K).astype(np.float32)
        qw = sgq.pack_int8(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), scheme)
        s_kn = np.broadcast_to(s[0] if scheme == 0 else s[k0], (N,))
    else:
        s = rng.uniform(1e-3, 1.0, K * N // G).astype(np.float32)
        qw = sgq.pack_int4(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), G)
        s_kn = s[(k0 * N + np.arange(N)) // G]
    y = _np(sgq.quantized_matmul(_to_dev(x, dev), qw))
    want = x[:, k0:k0 + 1] * s_kn[None, :].astype(np.float32)  # float32 products, one rounding
    assert want.dtype == np.float32
    assert helpers.same_bits(y, want), np.count_nonzero(y != want)


def test_dequantize_matches_reference_product(sgq, dev, oracle, synth):
    W = synth.normal((130, 72), 51, 0, 0.0, 0.02)
    qx = sgq.quantize_int8(_to_dev(W, dev), 1)
    q, s = oracle.quantize_int8(W, 1)
    assert helpers.same_value_allow_zero_sign(_np(sgq.dequantize_int8(qx)), oracle.dequantize_int8(q, s, 1))
    qx4 = sgq.quantize_int4(_to_dev(W, dev), 24)
    q4, s4 = oracle.quantize_int4(W, 24)
    assert helpers.same_value_allow_zero_sign(_np(sgq.dequantize_int4(qx4)), oracle.dequantize_int4(q4, s4, 24))


def test_plan_uses_the_device_cu_count(sgq, dev):
    # compute_units = 0 plans for the current device: the same plan as its CU
    # count given explicitly, on the first query and on the cached ones after.
    lib = sgq.load_library()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    shapes = [(4, 1, 4096, 4096, 128), (4, 16, 11008, 4096, 128), (4, 256, 4096, 4096, 128), (8, 512, 4096, 1024, 0),
              (8, 128, 1024, 1024, 0), (4, 8, 2048, 6144, 128)]
    for bits_, M, K, N, G in shapes:
        want_p, want_k = ctypes.c_int(), ctypes.c_int()
        assert lib.sgq_linear_plan(bits_, M, K, N, G, cus, ctypes.byref(want_p), ctypes.byref(want_k)) == 0
        for _ in range(3):
            p, k = ctypes.c_int(), ctypes.c_int()
            assert lib.sgq_linear_plan(bits_, M, K, N, G, 0, ctypes.byref(p), ctypes.byref(k)) == 0
            assert (p.value, k.value) == (want_p.value, want_k.value), (bits_, M, K, N, G, cus)
