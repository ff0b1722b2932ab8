"""GPU parity of the quantize / pack / unpack / dequantize kernels.

Codes and scales must be bit-exact with the reference (golden fixtures written
by the compiled reference, and the oracle on the benchmark shapes); packed
bytes must match the documented device layout (numpy model in helpers.py).
"""
import numpy as np
import pytest
import torch

import helpers
from helpers import same_bits, same_value_allow_zero_sign

pytestmark = pytest.mark.gpu


def _to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def test_golden_quantize_int8(sgq, dev, golden):
    n = 0
    for c in golden:
        if c["kind"] != "quantize_int8":
            continue
        p = c["params"]
        print(f"  case quantize_int8 {p}", flush=True)
        x = _to_dev(c["x"], dev)
        qx = sgq.quantize_int8(x, p["scheme"])
        assert same_bits(_np(qx.qdata), c["q"]), p
        assert same_bits(_np(qx.scales), c["s"]), p
        if c["x"].size:
            codes = c["q"].reshape(c["x"].shape[0] if c["x"].ndim == 2 else 1, -1)
            exp = helpers.model_pack_i8(codes.astype(np.int64))
            assert np.array_equal(_np(qx.packed)[: exp.size], exp), p
            assert same_value_allow_zero_sign(_np(sgq.unpack_codes(qx)).reshape(-1), c["q"].reshape(-1))
        if "deq" in c and c["x"].size:
            assert same_value_allow_zero_sign(_np(sgq.dequantize_int8(qx)), c["deq"]), p
            assert same_bits(_np(sgq.dequantize_codes(qx)), c["deq"]), p  # -0.0 included
        n += 1
    assert n >= 20


def test_golden_quantize_int4(sgq, dev, golden):
    for c in golden:
        if c["kind"] != "quantize_int4":
            continue
        p = c["params"]
        print(f"  case quantize_int4 {p}", flush=True)
        x = _to_dev(c["x"], dev)
        qx = sgq.quantize_int4(x, p["group_size"])
        assert same_bits(_np(qx.qdata), c["q"]), p
        assert same_bits(_np(qx.scales), c["s"]), p
        K, N = c["x"].shape
        g = helpers.i4_geom(K, N, p["group_size"])
        if g["tiled"]:
            exp = helpers.model_pack_i4_tiled(c["q"].astype(np.int64), p["group_size"])
            ds = helpers.model_devscales_i4(c["s"], K, N, p["group_size"])
            assert same_bits(_np(qx.devscales)[: ds.size], ds), p
        else:
            exp = helpers.model_pack_i4_flat(c["q"].astype(np.int64))
        assert np.array_equal(_np(qx.packed)[: exp.size], exp), p
        assert same_value_allow_zero_sign(_np(sgq.unpack_codes(qx)), c["q"])
        if "deq" in c:
            assert same_value_allow_zero_sign(_np(sgq.dequantize_int4(qx)), c["deq"]), p
            assert same_bits(_np(sgq.dequantize_codes(qx)), c["deq"]), p  # -0.0 included


BENCH_SHAPES_INT8 = [(1024, 1024, 0), (4096, 4096, 0), (4096, 4096, 1), (2048, 6144, 1)]
BENCH_SHAPES_INT4 = [(4096, 4096, 128), (4096, 11008, 128), (11008, 4096, 128), (2048, 6144, 128),
                     (2048, 5632, 128), (5632, 2048, 128), (2048, 2048, 32)]


@pytest.mark.parametrize("K,N,scheme", BENCH_SHAPES_INT8)
def test_bench_shapes_int8(sgq, dev, oracle, synth, K, N, scheme):
    print(f"  case int8 {K}x{N} scheme={scheme}", flush=True)
    W = synth.normal((K, N), synth.config_seed(3), synth.STREAM_W, 0.0, 0.02)
    qx = sgq.quantize_int8(_to_dev(W, dev), scheme)
    q, s = oracle.quantize_int8(W, scheme)
    assert same_bits(_np(qx.qdata), q)
    assert same_bits(_np(qx.scales), s)
    assert np.array_equal(_np(qx.packed), helpers.model_pack_i8(q.astype(np.int64)))


@pytest.mark.parametrize("K,N,G", BENCH_SHAPES_INT4)
def test_bench_shapes_int4(sgq, dev, oracle, synth, K, N, G):
    print(f"  case int4 {K}x{N} G={G}", flush=True)
    W = synth.normal((K, N), synth.config_seed(1), synth.STREAM_W, 0.0, 0.02)
    qx = sgq.quantize_int4(_to_dev(W, dev), G)
    q, s = oracle.quantize_int4(W, G)
    assert same_bits(_np(qx.qdata), q)
    assert same_bits(_np(qx.scales), s)
    assert np.array_equal(_np(qx.packed), helpers.model_pack_i4_tiled(q.astype(np.int64), G))
    ds = helpers.model_devscales_i4(s, K, N, G)
    assert same_bits(_np(qx.devscales), ds)


def test_pack_from_codes_roundtrip(sgq, dev, synth):
    W = synth.normal((96, 80), 21, 0, 0.0, 0.02)
    for bits_ in (8, 4):
        qx = sgq.quantize_int8(_to_dev(W, dev), 1) if bits_ == 8 else sgq.quantize_int4(_to_dev(W, dev), 16)
        re = sgq.pack_int8(qx.qdata, qx.scales, 1) if bits_ == 8 else sgq.pack_int4(qx.qdata, qx.scales, 16)
        assert torch.equal(re.packed, qx.packed)
        if bits_ == 4:
            assert torch.equal(re.devscales, qx.devscales)


@pytest.mark.parametrize("K,N,G", [(40, 72, 8), (17, 24, 8), (96, 80, 16), (33, 136, 136)])
def test_int4_buffer_with_koct_copy(sgq, dev, oracle, synth, K, N, G):
    """The whole INT4 strip-major buffer, from the quantizer and from codes:
    the strips, zeros up to the 256-byte boundary, and the k-octet copy, with
    K inside a 32-row k block and a half-empty last column block (N % 16 == 8)."""
    print(f"  case int4 {K}x{N} G={G}", flush=True)
    W = synth.normal((K, N), synth.config_seed(5), synth.STREAM_W, 0.0, 0.02)
    q, s = oracle.quantize_int4(W, G)
    exp = helpers.model_pack_i4_tiled(q.astype(np.int64), G)
    qx = sgq.quantize_int4(_to_dev(W, dev), G)
    assert np.array_equal(_np(qx.packed), exp)
    re = sgq.pack_int4(qx.qdata, qx.scales, G)
    assert np.array_equal(_np(re.packed), exp)


@pytest.mark.parametrize("bad", [0.5, 128.0, float("nan"), float("inf"), -129.0])
def test_pack_rejects_bad_codes_int8(sgq, dev, bad):
    q = torch.zeros((8, 8), dtype=torch.float32, device=dev)
    q[3, 5] = bad
    with pytest.raises(sgq.SGQError) as e:
        sgq.pack_int8(q, torch.ones(8, device=dev), 1)
    assert e.value.status == 5


@pytest.mark.parametrize("bad", [8.0, -9.0, 2.5])
def test_pack_rejects_bad_codes_int4(sgq, dev, bad):
    q = torch.zeros((8, 16), dtype=torch.float32, device=dev)
    q[7, 15] = bad
    with pytest.raises(sgq.SGQError):
        sgq.pack_int4(q, torch.ones(16, device=dev), 8)
    # -8 is representable and accepted
    q[7, 15] = -8.0
    sgq.pack_int4(q, torch.ones(16, device=dev), 8)


def test_rank1_and_empty(sgq, dev, oracle):
    x = np.linspace(-2, 3, 41, dtype=np.float32)
    qx = sgq.quantize_int8(_to_dev(x, dev), 1)
    q, s = oracle.quantize_int8(x, 1)
    assert qx.scales.numel() == 1 and same_bits(_np(qx.qdata), q) and same_bits(_np(qx.scales), s)
    e = sgq.quantize_int8(torch.zeros((3, 0), device=dev), 1)
    assert e.scales.numel() == 3
    assert same_bits(_np(e.scales), np.full(3, np.float32(1e-8) / np.float32(127), np.float32))
    e4 = sgq.quantize_int4(torch.zeros((0, 8), device=dev), 32)
    assert e4.scales.numel() == 0
