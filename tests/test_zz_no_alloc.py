"""sgq_linear_int4_noalloc: the INT4 forward with no workspace argument, whose
split-K partials live in the library's static per-GPU scratch array.

Checked through the C ABI against sgq_linear_int4 (caller workspace) on the
same inputs -- bit for bit, the same kernels and plan -- and against the CPU
oracle within 1e-5, on consecutive calls that reuse the scratch array (the
second smaller than the first), plus a GEMV call (no scratch) and a shape whose
partials do not fit (refused before any launch).
"""
import numpy as np
import pytest
import torch

import helpers
from helpers import rel_err

pytestmark = pytest.mark.gpu

SGQ_ERR_UNSUPPORTED = 2


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _run(sgq, dev, oracle, synth, M, K, N, G, seed):
    lib = sgq.load_library()
    W = synth.normal((K, N), synth.config_seed(seed), synth.STREAM_W, 0.0, 0.02)
    x = synth.normal((M, K), synth.config_seed(seed), synth.STREAM_X, 0.0, 1.0)
    b = synth.normal((1, N), synth.config_seed(seed), synth.STREAM_BIAS, 0.0, 0.02)
    qw = sgq.quantize_int4(_t(W, dev), G)
    xd, bd = _t(x, dev), _t(b, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    need = lib.sgq_linear_workspace_bytes(4, M, K, N)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    y_ws = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    y_na = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    rc = lib.sgq_linear_int4(xd.data_ptr(), M, K, N, qw.packed.data_ptr(), qw.scales.data_ptr(),
                             qw.devscales.data_ptr(), G, bd.data_ptr(), y_ws.data_ptr(), ws.data_ptr(), ws.numel(),
                             stream)
    assert rc == 0, lib.sgq_last_error()
    rc = lib.sgq_linear_int4_noalloc(xd.data_ptr(), M, K, N, qw.packed.data_ptr(), qw.scales.data_ptr(),
                                     qw.devscales.data_ptr(), G, bd.data_ptr(), y_na.data_ptr(), stream)
    assert rc == 0, lib.sgq_last_error()
    torch.cuda.synchronize()
    a, c = y_ws.cpu().numpy(), y_na.cpu().numpy()
    assert helpers.same_bits(a, c), f"M={M} K={K} N={N}: differs from sgq_linear_int4"
    q, s = oracle.quantize_int4(W, G)
    e = rel_err(c, oracle.quantized_matmul_int4(x, q, s, G, b))
    print(f"  M={M} K={K} N={N} G={G} workspace={need} rel_err={e:.3e}", flush=True)
    assert e <= 1e-5
    return need


def test_noalloc_matches_workspace_entry_point(sgq, dev, oracle, synth):
    # Two split-K GEMM calls in a row through the one scratch array, the
    # second smaller, then a GEMV (no scratch), then the first shape again.
    n1 = _run(sgq, dev, oracle, synth, 256, 4096, 1024, 128, 60)
    n2 = _run(sgq, dev, oracle, synth, 160, 2048, 512, 128, 61)
    assert n1 > n2 > 0
    assert _run(sgq, dev, oracle, synth, 1, 4096, 4096, 128, 62) == 0
    _run(sgq, dev, oracle, synth, 256, 4096, 1024, 128, 63)


def test_noalloc_skinny_split_k(sgq, dev, oracle, synth):
    # The skinny MFMA kernel's K ranges over a narrow weight put their partial
    # sums in the same scratch: two calls in a row, the second smaller.
    n1 = _run(sgq, dev, oracle, synth, 32, 11008, 4096, 128, 64)
    n2 = _run(sgq, dev, oracle, synth, 16, 11008, 4096, 128, 65)
    assert n1 > n2 > 0


def test_noalloc_refuses_oversized_scratch(sgq, dev):
    lib = sgq.load_library()
    # The skinny kernel over K = 131072 takes 16 K ranges of 8192 rows:
    # partials of 16 x 32 x 16512 floats, 32.25 MiB.
    M, K, N = 32, 131072, 16512
    assert lib.sgq_linear_workspace_bytes(4, M, K, N) > 32 << 20
    stream = torch.cuda.current_stream(dev).cuda_stream
    # Real device buffers (far smaller than the shape): the call must refuse
    # before it launches anything, and no argument is a made-up address.
    x, packed, scales, devscales, y = (torch.zeros(64, dtype=torch.float32, device=dev) for _ in range(5))
    rc = lib.sgq_linear_int4_noalloc(x.data_ptr(), M, K, N, packed.data_ptr(), scales.data_ptr(),
                                     devscales.data_ptr(), 128, None, y.data_ptr(), stream)
    assert rc == SGQ_ERR_UNSUPPORTED and b"scratch" in lib.sgq_last_error()
    torch.cuda.synchronize()
    assert not y.any()  # nothing was written
