"""Forward calls captured into a HIP graph (how bench.py times them) give, on
every replay, the bits of the eager call.

Between replays the test runs eager work of its own: it poisons the output
and runs another forward through the same cached workspace, so a replay that
relied on state left by the capture (a memset node, stale split-K partials)
would show.  The library records no memset into a stream: its kernels
overwrite every output and partial they read.
"""
import numpy as np
import pytest
import torch

import helpers

pytestmark = pytest.mark.gpu


def _to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _weights(sgq, dev, synth, bits_, K, N, G, scheme, seed):
    W = synth.normal((K, N), seed, 0, 0.0, 0.02)
    return sgq.quantize_int8(_to_dev(W, dev), scheme) if bits_ == 8 else sgq.quantize_int4(_to_dev(W, dev), G)


@pytest.mark.parametrize(
    "name,bits_,M,K,N,G,scheme,bias",
    [
        ("gemv_int4_M1", 4, 1, 4096, 4096, 128, 0, False),
        ("gemv_int4_M8", 4, 8, 2048, 6144, 128, 0, True),
        ("gemv_int8_M5", 8, 5, 1000, 700, 0, 1, True),
        ("skinny_int8_M128", 8, 128, 1024, 1024, 0, 0, True),
        ("skinny_int8_pc_M8", 8, 8, 4096, 4096, 0, 1, False),
        ("gemm_int8_splitk_M256", 8, 256, 4096, 1024, 0, 0, True),
        ("gemm_int8_pc_M300", 8, 300, 1024, 768, 0, 1, False),
        ("gemm_int4_M256", 4, 256, 1024, 1024, 128, 0, True),
        ("gemm_int4_g32_M40", 4, 40, 512, 256, 32, 0, True),
        ("skinny_int4_M16", 4, 16, 4096, 11008, 128, 0, True),
        ("skinny_int4_two_blocks_M24", 4, 24, 2048, 6144, 128, 0, True),
        ("skinny_int4_split_k_M16", 4, 16, 11008, 4096, 128, 0, True),
    ],
)
def test_linear_graph_replays_match_eager(sgq, dev, synth, name, bits_, M, K, N, G, scheme, bias):
    print(f"  case {name}", flush=True)
    qw = _weights(sgq, dev, synth, bits_, K, N, G, scheme, 71)
    x = _to_dev(synth.normal((M, K), 72, 1), dev)
    x2 = _to_dev(synth.normal((M, K), 73, 1), dev)
    b = _to_dev(synth.normal((1, N), 74, 2, 0.0, 0.02), dev) if bias else None
    s = torch.cuda.Stream(dev)  # the workspace is cached per stream: eager calls on s share the graph's
    with torch.cuda.stream(s):
        y_eager = sgq.quantized_matmul(x, qw, b)  # also sizes that workspace outside the capture
        y2_eager = sgq.quantized_matmul(x2, qw, b)
    torch.cuda.synchronize()
    y = torch.empty_like(y_eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        sgq.quantized_matmul(x, qw, b, out=y)
    for rep in range(4):
        with torch.cuda.stream(s):
            y.fill_(float("nan"))
            y2 = sgq.quantized_matmul(x2, qw, b)  # eager, same workspace
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert helpers.same_bits(y.cpu().numpy(), y_eager.cpu().numpy()), (name, rep)
        assert helpers.same_bits(y2.cpu().numpy(), y2_eager.cpu().numpy()), (name, rep)


@pytest.mark.parametrize("bits_,M", [(4, 8), (4, 64), (8, 3), (8, 64)])
def test_swiglu_graph_replays_match_eager(sgq, dev, synth, bits_, M):
    K, N, G = 1024, 1536, 128
    wg = _weights(sgq, dev, synth, bits_, K, N, G, 0, 81)
    wu = _weights(sgq, dev, synth, bits_, K, N, G, 0, 82)
    x = _to_dev(synth.normal((M, K), 83, 1), dev)
    x2 = _to_dev(synth.normal((M, K), 84, 1), dev)
    s = torch.cuda.Stream(dev)
    with torch.cuda.stream(s):
        h_eager = sgq.quantized_swiglu(x, wg, wu)
    torch.cuda.synchronize()
    h = torch.empty_like(h_eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        sgq.quantized_swiglu(x, wg, wu, out=h)
    for rep in range(3):
        with torch.cuda.stream(s):
            h.fill_(float("nan"))
            sgq.quantized_swiglu(x2, wg, wu)  # eager, same workspace (the up projection lives there)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert helpers.same_bits(h.cpu().numpy(), h_eager.cpu().numpy()), (bits_, M, rep)
