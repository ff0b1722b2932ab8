"""GPU parity of the gated MLP: h = silu(x . Wg + bg) * (x . Wu + bu), the
first three lines of SwiGLU::forward (include/sovereigngrad/nn.hpp:151-154)
with quantized projections, against the golden fixtures (compiled reference)
and the oracle on the same quantized weights.

Bar: max|h - h_ref| / max|h_ref| <= 1e-5, as for the forward (the projections
accumulate in another order than the CPU, and the device expf is not libm's).
"""
import ctypes

import numpy as np
import pytest
import torch

import helpers
from helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def test_golden_swiglu(sgq, dev, golden):
    n = 0
    for c in golden:
        if c["kind"] not in ("swiglu_int8", "swiglu_int4"):
            continue
        p = c["params"]
        print(f"  case {c['kind']} {p}", flush=True)
        x = _to_dev(c["x"], dev)
        bg = _to_dev(c["bias_gate"], dev) if "bias_gate" in c else None
        bu = _to_dev(c["bias_up"], dev) if "bias_up" in c else None
        if c["kind"] == "swiglu_int8":
            wg = sgq.pack_int8(_to_dev(c["qg"], dev), _to_dev(c["sg"], dev), p["scheme"])
            wu = sgq.pack_int8(_to_dev(c["qu"], dev), _to_dev(c["su"], dev), p["scheme"])
        else:
            wg = sgq.pack_int4(_to_dev(c["qg"], dev), _to_dev(c["sg"], dev), p["group_size"])
            wu = sgq.pack_int4(_to_dev(c["qu"], dev), _to_dev(c["su"], dev), p["group_size"])
        h = sgq.quantized_swiglu(x, wg, wu, bg, bu)
        e = rel_err(_np(h), c["y"])
        assert e <= TOL, (p, e)
        n += 1
    assert n >= 6


def _weights(synth, K, N, seed):
    cs = synth.config_seed(seed)
    Wg = synth.normal((K, N), cs, synth.STREAM_W, 0.0, 0.02)
    Wu = synth.normal((K, N), cs, synth.STREAM_W2, 0.0, 0.02)
    bg = synth.normal((1, N), cs, synth.STREAM_BIAS, 0.0, 0.02)
    bu = synth.normal((1, N), cs, synth.STREAM_BIAS2, 0.0, 0.02)
    return Wg, Wu, bg, bu


def _case(sgq, dev, oracle, synth, bits_, M, K, N, G=128, scheme=0, bias=True, seed=7):
    Wg, Wu, bg, bu = _weights(synth, K, N, seed)
    x = synth.normal((M, K), synth.config_seed(seed), synth.STREAM_X, 0.0, 1.0)
    if not bias:
        bg = bu = None
    bgd = _to_dev(bg, dev) if bias else None
    bud = _to_dev(bu, dev) if bias else None
    if bits_ == 8:
        wg, wu = sgq.quantize_int8(_to_dev(Wg, dev), scheme), sgq.quantize_int8(_to_dev(Wu, dev), scheme)
        qg, sg = oracle.quantize_int8(Wg, scheme)
        qu, su = oracle.quantize_int8(Wu, scheme)
        href = oracle.swiglu_int8(x, qg, sg, qu, su, scheme, bg, bu)
    else:
        wg, wu = sgq.quantize_int4(_to_dev(Wg, dev), G), sgq.quantize_int4(_to_dev(Wu, dev), G)
        qg, sg = oracle.quantize_int4(Wg, G)
        qu, su = oracle.quantize_int4(Wu, G)
        href = oracle.swiglu_int4(x, qg, sg, qu, su, G, bg, bu)
    h = sgq.quantized_swiglu(_to_dev(x, dev), wg, wu, bgd, bud)
    return _np(h), href, (x, wg, wu, bgd, bud)


@pytest.mark.parametrize(
    "name,bits_,M,K,N,G,scheme,bias",
    [
        ("C3_gate_up_M1", 4, 1, 4096, 11008, 128, 0, False),
        ("C3_gate_up_M8", 4, 8, 4096, 11008, 128, 0, False),
        ("C5_gate_up_M8", 4, 8, 2048, 5632, 128, 0, True),
        ("C5_gate_up_M16", 4, 16, 2048, 5632, 128, 0, True),
        ("int4_gemm_M64", 4, 64, 2048, 5632, 128, 0, True),
        ("int4_gemm_splitk_M32", 4, 32, 1024, 1024, 128, 0, True),
        ("int8_pt_M1", 8, 1, 1024, 2816, 0, 0, True),
        ("int8_pc_M5", 8, 5, 1001, 1000, 0, 1, True),
        ("int8_pt_M13_ragged", 8, 13, 300, 77, 0, 0, False),
        ("int8_pc_gemm_M200", 8, 200, 640, 256, 0, 1, True),
        ("int8_pt_gemm_M128", 8, 128, 1024, 1024, 0, 0, True),
        ("int4_ragged_K1001_M3", 4, 3, 1001, 512, 128, 0, True),
        ("int4_g32_M2", 4, 2, 512, 96, 32, 0, True),
        ("int4_g64_M9", 4, 9, 256, 192, 64, 0, False),
        ("int4_g24_tiled_M6", 4, 6, 96, 40, 24, 0, True),
        ("int4_g24_tiled_M30", 4, 30, 96, 40, 24, 0, True),
        ("int4_flat_M4", 4, 4, 60, 50, 7, 0, True),
        ("int4_flat_M40", 4, 40, 64, 36, 24, 0, True),
    ],
)
def test_swiglu_vs_oracle(sgq, dev, oracle, synth, name, bits_, M, K, N, G, scheme, bias):
    print(f"  case {name}", flush=True)
    h, href, _ = _case(sgq, dev, oracle, synth, bits_, M, K, N, G, scheme, bias)
    e = rel_err(h, href)
    print(f"    rel_err={e:.3e}", flush=True)
    assert np.isfinite(h).all()
    assert e <= TOL


@pytest.mark.parametrize("M", [1, 3])
def test_swiglu_infinite_activation(sgq, dev, oracle, synth, M):
    # +-inf in x reaches the gate and up sums of the fused INT4 GEMV: NaN and
    # +-inf must land where the reference's silu(x.Wg + bg) * (x.Wu + bu) has
    # them (both weights take the exact fallback of the offset-binary decode).
    K, N, G = 1024, 384, 128
    Wg, Wu, bg, bu = _weights(synth, K, N, 13)
    x = synth.normal((M, K), 13, 1)
    x[0, 40] = np.inf
    x[M - 1, 700] = -np.inf if M > 1 else x[M - 1, 700]
    qg, sg = oracle.quantize_int4(Wg, G)
    qu, su = oracle.quantize_int4(Wu, G)
    href = oracle.swiglu_int4(x, qg, sg, qu, su, G, bg, bu)
    wg, wu = sgq.quantize_int4(_to_dev(Wg, dev), G), sgq.quantize_int4(_to_dev(Wu, dev), G)
    h = _np(sgq.quantized_swiglu(_to_dev(x, dev), wg, wu, _to_dev(bg, dev), _to_dev(bu, dev)))
    assert not np.isfinite(href).all()
    assert np.array_equal(np.isnan(h), np.isnan(href))
    assert np.array_equal(np.isposinf(h), np.isposinf(href))
    assert np.array_equal(np.isneginf(h), np.isneginf(href))
    fin = np.isfinite(href)
    if fin.any():
        assert np.max(np.abs(h[fin] - href[fin])) <= TOL * max(np.max(np.abs(href[fin])), 1e-30)


@pytest.mark.parametrize("bits_,M", [(4, 1), (4, 7), (4, 16), (8, 3), (8, 16), (4, 48), (8, 40)])
def test_swiglu_matches_two_linears(sgq, dev, oracle, synth, bits_, M):
    # The fused form and two separate library projections followed by the
    # oracle's silu and mul must agree to rounding (the GEMV's fused gate/up
    # sums run the same reduction as the single-weight kernel).
    K, N = 1536, 1040
    h, _, (x, wg, wu, bgd, bud) = _case(sgq, dev, oracle, synth, bits_, M, K, N, 128, 0, True, seed=9)
    xd = _to_dev(x, dev)
    g = _np(sgq.quantized_matmul(xd, wg, bgd))
    u = _np(sgq.quantized_matmul(xd, wu, bud))
    h2 = oracle.mul(oracle.silu(g), u)
    assert rel_err(h, h2) <= 2e-7


def test_swiglu_k_zero_is_bias_only(sgq, dev, oracle):
    lib = sgq.load_library()
    M, N = 3, 40
    bg = torch.linspace(-6.0, 6.0, N, device=dev)
    bu = torch.linspace(0.5, -2.0, N, device=dev)
    h = torch.full((M, N), float("nan"), device=dev)
    nws = lib.sgq_swiglu_workspace_bytes(8, M, 0, N, 0)
    assert nws >= M * N * 4
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    st = lib.sgq_swiglu_int8(None, M, 0, N, None, None, bg.data_ptr(), None, None, bu.data_ptr(), 0, h.data_ptr(),
                             ws.data_ptr(), nws, None)
    assert st == 0, lib.sgq_last_error()
    ref = oracle.mul(oracle.silu(np.tile(_np(bg), (M, 1))), np.tile(_np(bu), (M, 1)))
    assert rel_err(_np(h), ref) <= 1e-6
    # no biases: both projections are zero
    st = lib.sgq_swiglu_int4(None, M, 0, N, None, None, None, None, None, None, None, None, 32, h.data_ptr(),
                             ws.data_ptr(), nws, None)
    assert st == 0, lib.sgq_last_error()
    assert np.array_equal(_np(h), np.zeros((M, N), np.float32))


def test_swiglu_empty_and_errors(sgq, dev, synth):
    lib = sgq.load_library()
    # M == 0 is a no-op success without pointers
    assert lib.sgq_swiglu_int4(None, 0, 64, 64, None, None, None, None, None, None, None, None, 32, None, None, 0,
                               None) == 0
    Wg, Wu, _, _ = _weights(synth, 64, 64, 3)
    wg = sgq.quantize_int4(_to_dev(Wg, dev), 32)
    wu8 = sgq.quantize_int8(_to_dev(Wu, dev), 0)
    with pytest.raises(ValueError):
        sgq.quantized_swiglu(torch.zeros((2, 64), device=dev), wg, wu8)
    wu = sgq.quantize_int4(_to_dev(Wu, dev), 64)
    with pytest.raises(ValueError):
        sgq.quantized_swiglu(torch.zeros((2, 64), device=dev), wg, wu)


def test_swiglu_deterministic(sgq, dev, oracle, synth):
    for M in (4, 96):
        h1, _, (x, wg, wu, bgd, bud) = _case(sgq, dev, oracle, synth, 4, M, 1024, 1024, 128, 0, True, seed=11)
        h2 = _np(sgq.quantized_swiglu(_to_dev(x, dev), wg, wu, bgd, bud))
        assert helpers.same_bits(h1, h2), M
