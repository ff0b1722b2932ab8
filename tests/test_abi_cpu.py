"""CPU tests of the C ABI: the library loads, exports every declared symbol,
answers its host-only size queries, and rejects bad arguments before any GPU
work.  Also checks the numpy models of the device layouts used by the GPU
tests.  No call here launches a kernel."""
import ctypes

import numpy as np
import pytest

import helpers


@pytest.fixture(scope="module")
def lib(sgq):
    return sgq.load_library()


def test_exports_every_declared_symbol(sgq):
    raw = ctypes.CDLL(str(sgq.LIB_PATH))
    declared = helpers.header_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(raw, name), name
    assert set(declared) == set(sgq.SIGNATURES), "binding and header disagree"


def test_abi_version(lib):
    assert lib.sgq_abi_version() == 2  # 2: INT4 strip-major buffers carry the k-octet copy
    assert lib.sgq_last_error() is not None


@pytest.mark.parametrize("K,N", [(1, 1), (16, 64), (17, 65), (1024, 1024), (4096, 11008), (11008, 4096), (3, 0)])
def test_int8_sizes(lib, K, N):
    Kpad, RQ, NS = helpers.i8_geom(K, N)
    assert lib.sgq_int8_packed_bytes(K, N) == NS * RQ * 16
    assert lib.sgq_int8_scale_count(K, N, 0) == 1
    assert lib.sgq_int8_scale_count(K, N, 1) == K


@pytest.mark.parametrize("K,N,G", [(4096, 4096, 128), (2048, 5632, 128), (16, 32, 32), (32, 16, 16), (5, 13, 7),
                                   (3, 11, 8), (16, 40, 24), (8, 24, 0), (4, 9, -5), (100, 12, 8)])
def test_int4_sizes(lib, K, N, G):
    g = helpers.i4_geom(K, N, G)
    assert lib.sgq_int4_layout(K, N, G) == (0 if g["tiled"] else 1)
    off, KB, NB = helpers.i4_koct_geom(K, N, G)
    exp_bytes = off + NB * KB * 256 if g["tiled"] else (K * N + 1) // 2
    assert helpers.i4_packed_bytes(K, N, G) == exp_bytes
    assert lib.sgq_int4_packed_bytes(K, N, G) == exp_bytes
    assert lib.sgq_int4_devscale_count(K, N, G) == (g["nsc"] * g["Kpad"] if g["tiled"] else 0)
    assert lib.sgq_int4_scale_count(K, N, G) == (K * N + g["G"] - 1) // g["G"]


def test_workspace_sizes(lib):
    # The GEMV (M <= 16, or up to 128 rows of small work) and GEMMs with at
    # least one tile per CU need no workspace; smaller GEMM grids split K and
    # keep KS * M * N fp32 partials, as does the INT4 skinny kernel over a
    # narrow weight (4 K ranges for 16 x 4096 -> 4096).
    assert lib.sgq_linear_workspace_bytes(4, 1, 4096, 4096) == 0
    assert lib.sgq_linear_workspace_bytes(4, 8, 4096, 4096) == 0
    assert lib.sgq_linear_workspace_bytes(4, 16, 4096, 4096) == 4 * 16 * 4096 * 4
    assert lib.sgq_linear_workspace_bytes(8, 16, 4096, 4096) == 0
    assert lib.sgq_linear_workspace_bytes(8, 128, 1024, 1024) == 0  # INT8 skinny kernel: whole K
    assert lib.sgq_linear_workspace_bytes(8, 2048, 4096, 4096) == 0  # 256 or 512 tiles
    ws = lib.sgq_linear_workspace_bytes(8, 256, 4096, 1024)  # GEMM of 8 or 16 tiles: split K
    assert ws > 0 and ws % (256 * 1024 * 4) == 0 and 2 <= ws // (256 * 1024 * 4) <= 16
    assert lib.sgq_linear_workspace_bytes(4, 64, 96, 512) == 0  # three 32-row stages: too short to split
    assert lib.sgq_linear_workspace_bytes(3, 1, 4, 4) == -1
    assert lib.sgq_quantize_workspace_bytes(4, 4096, 4096, 128) >= 4096 * 4096 // 128 * 4
    # Regression: K == 0 (and other degenerate shapes) must not divide by zero on the host.
    for bits_ in (4, 8):
        for (M, K, N) in [(3, 0, 16), (0, 0, 0), (1, 1, 0), (16, 0, 1), (1, 15, 1)]:
            assert lib.sgq_linear_workspace_bytes(bits_, M, K, N) >= 0


def test_swiglu_workspace_sizes(lib):
    # One-launch GEMV (tiled, M <= 16): none.  Otherwise the up projection
    # (M*N floats, 256-byte aligned) followed by the GEMM's split-K partials;
    # INT8 batches of the skinny kernel need the up projection only.
    assert lib.sgq_swiglu_workspace_bytes(4, 1, 4096, 11008, 128) == 0
    assert lib.sgq_swiglu_workspace_bytes(8, 16, 1024, 1024, 0) == 0
    assert lib.sgq_swiglu_workspace_bytes(8, 32, 1024, 1024, 0) == 0  # GEMV form, as the plain forward
    assert lib.sgq_swiglu_workspace_bytes(8, 128, 1024, 1024, 0) == 128 * 1024 * 4  # skinny kernel, twice
    assert lib.sgq_swiglu_workspace_bytes(8, 8, 4096, 4096, 0) == 8 * 4096 * 4
    assert lib.sgq_swiglu_workspace_bytes(4, 2048, 4096, 4096, 128) == 2048 * 4096 * 4
    u = 256 * 1024 * 4
    assert lib.sgq_swiglu_workspace_bytes(8, 256, 4096, 1024, 0) == u + lib.sgq_linear_workspace_bytes(8, 256, 4096, 1024)
    assert lib.sgq_swiglu_workspace_bytes(4, 3, 60, 50, 7) == 768  # flat INT4: always two projections
    assert lib.sgq_swiglu_workspace_bytes(8, 3, 0, 5, 0) == 256  # K == 0: bias-only projections
    assert lib.sgq_swiglu_workspace_bytes(8, 0, 64, 64, 0) == 0
    assert lib.sgq_swiglu_workspace_bytes(5, 1, 4, 4, 0) == -1


def test_swiglu_argument_errors_before_gpu(lib):
    # int8: bad scheme, missing pointers, misalignment, missing workspace
    assert lib.sgq_swiglu_int8(16, 1, 64, 64, 16, 16, None, 16, 16, None, 7, 16, None, 0, None) == 1
    assert lib.sgq_swiglu_int8(16, 1, 64, 64, 16, 16, None, None, 16, None, 0, 16, None, 0, None) == 1
    assert lib.sgq_swiglu_int8(16, 1, 64, 64, 16, 16, None, 24, 16, None, 0, 16, None, 0, None) == 1
    assert b"aligned" in lib.sgq_last_error()
    # 200 rows: past the GEMV form, so the up projection needs the workspace
    need = lib.sgq_swiglu_workspace_bytes(8, 200, 64, 64, 0)
    assert need >= 200 * 64 * 4
    assert lib.sgq_swiglu_int8(16, 200, 64, 64, 16, 16, None, 16, 16, None, 0, 16, None, 0, None) == 3
    assert str(need).encode() in lib.sgq_last_error()
    assert lib.sgq_swiglu_int8(16, 200, 64, 64, 16, 16, None, 16, 16, None, 0, 16, 16, need - 4, None) == 3
    # int4: tiled layout needs devscales; flat layout needs scales and a workspace even for M = 1
    assert lib.sgq_swiglu_int4(16, 1, 64, 64, 16, 16, None, None, 16, 16, 16, None, 32, 16, None, 0, None) == 1
    assert b"devscales" in lib.sgq_last_error()
    assert lib.sgq_swiglu_int4(16, 1, 60, 50, 16, 16, None, None, 16, 16, None, None, 7, 16, None, 0, None) == 3
    assert lib.sgq_swiglu_int4(16, 1, 60, 50, 16, None, None, None, 16, 16, None, None, 7, 16, 16, 256, None) == 1
    assert b"scales" in lib.sgq_last_error()
    assert lib.sgq_swiglu_int4(None, -1, 64, 64, None, None, None, None, None, None, None, None, 32, None, None, 0,
                               None) == 1


def _block_struct(D, H, G, ptr=16):
    import soverign_grad_amd.decode as dm

    st = dm.LlamaBlockInt4()
    st.D, st.H, st.group_size, st.eps, st.attn_scale = D, H, G, 1e-5, 0.125
    st.norm1 = st.norm2 = ptr
    for f in ("q", "k", "v", "o", "gate", "up", "down"):
        setattr(st, f, dm.Int4Linear(ptr, ptr, None))
    return st


def test_llama_decode_sizes_and_errors(lib, sgq):
    import ctypes

    # Workspace: normed input, q|k|v, context, h, MLP hidden, a projection
    # output, attention partials (several key chunks), split-K partials (B > 16).
    w1 = lib.sgq_llama_decode_workspace_bytes(8, 2048, 5632, 64)
    assert w1 >= 4 * (8 * 2048 * 7 + 8 * 5632 * 2)
    assert lib.sgq_llama_decode_workspace_bytes(8, 2048, 5632, 4096) > w1  # more key chunks
    assert lib.sgq_llama_decode_workspace_bytes(32, 2048, 5632, 64) > lib.sgq_llama_decode_workspace_bytes(16, 2048,
                                                                                                             5632, 64)
    assert lib.sgq_llama_decode_workspace_bytes(1, 0, 8, 1) == -1
    assert lib.sgq_llama_decode_workspace_bytes(1, 8, 8, 0) == -1
    st = _block_struct(64, 128, 32)
    need = lib.sgq_llama_decode_workspace_bytes(2, 64, 128, 4)
    call = lambda blk, B=2, mt=8, ml=4, ws=16, nws=need, kc=256: lib.sgq_llama_block_decode_int4(
        None if blk is None else ctypes.byref(blk), 16, 16, B, kc, kc, mt, 16, ml, ws, nws, None)
    assert call(None) == 1
    assert call(st, ml=9) == 1 and b"max_len" in lib.sgq_last_error()  # max_len > max_tokens
    assert call(st, ml=0) == 1
    assert call(st, ws=None) == 3 and str(need).encode() in lib.sgq_last_error()
    assert call(st, nws=need - 4) == 3
    assert call(st, kc=260) == 1 and b"aligned" in lib.sgq_last_error()
    assert call(st, B=0) == 0  # nothing to do
    assert call(_block_struct(60, 128, 32)) == 2  # D not a multiple of 8: no tiled layout
    assert call(_block_struct(64, 128, 12)) == 2  # group size not a multiple of 8
    assert call(_block_struct(16384, 128, 32)) == 2
    bad = _block_struct(64, 128, 32)
    bad.up = type(bad.up)(16, None, None)
    assert call(bad) == 1 and b"null weight" in lib.sgq_last_error()
    mis = _block_struct(64, 128, 32)
    mis.down = type(mis.down)(24, 16, None)
    assert call(mis) == 1 and b"aligned" in lib.sgq_last_error()
    assert lib.sgq_rms_norm(None, -1, 4, None, ctypes.c_float(1e-5), None, None) == 1
    assert lib.sgq_rms_norm(None, 0, 4, None, ctypes.c_float(1e-5), None, None) == 0
    assert lib.sgq_rms_norm(None, 2, 4, 16, ctypes.c_float(1e-5), 16, None) == 1
    assert lib.sgq_embedding(None, -1, None, 4, 4, None, None) == 1
    assert lib.sgq_embedding(None, 0, None, 4, 4, None, None) == 0
    assert lib.sgq_embedding(16, 3, None, 4, 4, 16, None) == 1 and b"null" in lib.sgq_last_error()


def test_argument_errors_before_gpu(lib, sgq):
    # Each of these fails validation on the host; nothing reaches the GPU.
    assert lib.sgq_quantize_int8(None, -1, 4, 0, None, None, None, None, 0, None) == 1
    assert lib.sgq_quantize_int8(None, 4, 4, 7, None, None, None, None, 0, None) == 1
    assert lib.sgq_quantize_int8(None, 0, 4, 1, None, None, None, None, 0, None) == 1
    assert b"per-channel" in lib.sgq_last_error()
    assert lib.sgq_quantize_int8(1, 4, 4, 0, None, None, None, None, 0, None) == 1
    assert lib.sgq_linear_int8(None, 1, 4, 4, None, None, 9, None, None, None, 0, None) == 1
    assert lib.sgq_linear_int4(None, -2, 4, 4, None, None, None, 32, None, None, None, 0, None) == 1
    assert lib.sgq_linear_int4(16, 1, 64, 64, 16, 16, None, 32, None, 16, None, 0, None) == 1  # no devscales
    assert lib.sgq_linear_int4(16, 1, 64, 64, 24, 16, 16, 32, None, 16, None, 0, None) == 1  # misaligned packed
    assert b"aligned" in lib.sgq_last_error()
    assert lib.sgq_linear_int8(16, 1, 64, 64, 16, 20, 1, None, 16, None, 0, None) == 1  # misaligned scales
    assert lib.sgq_quantize_int4(16, 4, 64, 32, None, 16, 24, 16, None, 0, None) == 1  # misaligned packed
    # A split-K GEMM checks its workspace before any launch.
    need = lib.sgq_linear_workspace_bytes(8, 256, 4096, 1024)
    need4 = lib.sgq_linear_workspace_bytes(4, 256, 4096, 1024)
    assert need > 0 and need4 > 0
    assert lib.sgq_linear_int8(16, 256, 4096, 1024, 16, 16, 0, None, 16, None, 0, None) == 3
    assert str(need).encode() in lib.sgq_last_error()
    assert lib.sgq_linear_int8(16, 256, 4096, 1024, 16, 16, 0, None, 16, 256, need - 4, None) == 3
    assert lib.sgq_linear_int4(16, 256, 4096, 1024, 16, 16, 16, 128, None, 16, 260, need4, None) == 3  # misaligned
    # empty outputs are a no-op success
    assert lib.sgq_linear_int8(None, 0, 4, 4, None, None, 0, None, None, None, 0, None) == 0


def test_dequantize_alignment_checked_before_gpu(lib):
    # The unpack kernels read packed codes 16 bytes at a time (tiled layouts).
    assert lib.sgq_dequantize_int8(24, 16, 0, 64, 64, 16, None) == 1
    assert b"aligned" in lib.sgq_last_error()
    assert lib.sgq_dequantize_int4(24, 16, 64, 64, 32, 16, None) == 1  # tiled: N % 8 == 0, G % 8 == 0
    assert b"aligned" in lib.sgq_last_error()


def test_forward_refuses_k_past_32bit_offsets(lib):
    """K long enough that the kernels' 32-bit buffer offsets would wrap is
    refused (SGQ_ERR_UNSUPPORTED) before any launch: past 2^22 rows for the
    MFMA GEMM (128-row tiles of x), past 2^29 rows for the GEMV."""
    big_gemm = (1 << 22) + 16  # GEMM path at M=32 (M * K * N > 2^28)
    assert lib.sgq_linear_int8(16, 32, big_gemm, 64, 16, 16, 0, None, 16, 16, 1 << 40, None) == 2
    assert b"too long" in lib.sgq_last_error()
    assert lib.sgq_linear_int4(16, 32, big_gemm, 64, 16, 16, 16, 128, None, 16, 16, 1 << 40, None) == 2
    big_gemv = (1 << 29)  # GEMV path at M=1
    assert lib.sgq_linear_int8(16, 1, big_gemv, 8, 16, 16, 0, None, 16, None, 0, None) == 2
    assert lib.sgq_linear_int4(16, 1, big_gemv, 8, 16, 16, 16, 128, None, 16, None, 0, None) == 2
    assert lib.sgq_swiglu_int8(16, 1, big_gemv, 8, 16, 16, None, 16, 16, None, 0, 16, 16, 1 << 40, None) == 2
    assert lib.sgq_swiglu_int4(16, 1, big_gemv, 8, 16, 16, 16, None, 16, 16, 16, None, 128, 16, 16, 1 << 40,
                               None) == 2


# ---- numpy layout models -------------------------------------------------

def _unpack_model_i8(buf, K, N):
    Kpad, RQ, NS = helpers.i8_geom(K, N)
    t = buf.view(np.int8).reshape(NS, RQ, 4, 4)  # j, rq, d, r
    full = t.transpose(1, 3, 0, 2).reshape(Kpad, NS * 4)
    return full[:K, :N]


def test_model_pack_i8_roundtrip():
    rng = np.random.default_rng(0)
    for K, N in [(16, 64), (17, 70), (33, 130)]:
        q = rng.integers(-127, 128, size=(K, N))
        buf = helpers.model_pack_i8(q)
        Kpad, RQ, NS = helpers.i8_geom(K, N)
        assert buf.size == NS * RQ * 16
        assert np.array_equal(_unpack_model_i8(buf, K, N), q)
        # element (k, n) sits at the documented byte
        k, n = K - 1, N - 1
        off = ((n // 4) * RQ + k // 4) * 16 + (n % 4) * 4 + k % 4
        assert buf.view(np.int8)[off] == q[k, n]


def test_model_pack_i4_positions():
    rng = np.random.default_rng(1)
    K, N = 20, 136
    q = rng.integers(-7, 8, size=(K, N))
    buf = helpers.model_pack_i4_tiled(q, 8)
    g = helpers.i4_geom(K, N, 8)
    for (k, n) in [(0, 0), (19, 135), (5, 77), (16, 128)]:
        off = ((n // 8) * g["RQ"] + k // 4) * 16 + (k % 4) * 4 + (n % 8) // 2
        nib = (int(buf[off]) >> (4 * (n % 2))) & 0xF
        assert ((nib ^ 8) - 8) == q[k, n]


def test_model_pack_i4_koct_positions():
    """The k-octet copy: each dword holds eight consecutive rows of one column
    (an MFMA B operand), blocks of 16 columns x 32 rows contiguous over K; the
    padding rows and columns are code 0."""
    rng = np.random.default_rng(2)
    K, N = 40, 24  # two k blocks (the second padded), two column blocks (the second half empty)
    q = rng.integers(-8, 8, size=(K, N))
    buf = helpers.model_pack_i4_tiled(q, 8)
    off, KB, NB = helpers.i4_koct_geom(K, N, 8)
    assert (KB, NB) == (2, 2) and off % 256 == 0 and buf.size == off + KB * NB * 256
    words = buf[off:].view(np.uint32)
    for (k, n) in [(0, 0), (39, 23), (7, 15), (8, 16), (33, 5)]:
        d = ((n // 16) * KB + k // 32) * 64 + ((k % 32) // 8) * 16 + n % 16
        nib = (int(words[d]) >> (4 * (k % 8))) & 0xF
        assert ((nib ^ 8) - 8) == q[k, n]
    # rows 40..63 of every column and columns 24..31 of every row are zeros
    dense = np.zeros((KB * 32, NB * 16), np.int64)
    for d, w in enumerate(words):
        blk, t = divmod(d, 64)
        cb, kb = divmod(blk, KB)
        for i in range(8):
            nib = (int(w) >> (4 * i)) & 0xF
            dense[32 * kb + 8 * (t // 16) + i, 16 * cb + t % 16] = (nib ^ 8) - 8
    assert np.array_equal(dense[:K, :N], q) and not dense[K:].any() and not dense[:, N:].any()
    # the strips precede it unchanged, zero-filled up to the offset
    strips = helpers.model_pack_i4_strips(q, 8)
    assert np.array_equal(buf[:strips.size], strips) and not buf[strips.size:off].any()


def test_model_devscales():
    K, N, G = 5, 24, 8
    s = np.arange(1, (K * N) // G + 1, dtype=np.float32)
    ds = helpers.model_devscales_i4(s, K, N, G).reshape(-1, 16)
    g = helpers.i4_geom(K, N, G)
    assert g["spc"] == 1
    # strip 1 of row 2 covers elements 2*24+8 .. +7 -> group (56)//8 = 7
    assert ds[1, 2] == s[7]


def _plan(lib, bits, M, K, N, G, cus):
    path, ks = ctypes.c_int(-1), ctypes.c_int(-1)
    assert lib.sgq_linear_plan(bits, M, K, N, G, cus, ctypes.byref(path), ctypes.byref(ks)) == 0
    return path.value, ks.value


def _ws_covers(lib, bits, M, K, N, G, cus):
    """The size queries cover the plan this device runs: the forward's
    workspace holds its K splits' partials, the gated MLP's those of both
    weights (one skinny launch) or the up projection plus one GEMM's."""
    path, ks = _plan(lib, bits, M, K, N, G, cus)
    assert ks >= 1
    if ks == 1:
        return path, ks
    part = ks * M * N * 4
    ws = lib.sgq_linear_workspace_bytes(bits, M, K, N)
    sw = lib.sgq_swiglu_workspace_bytes(bits, M, K, N, G)
    assert ws >= part, (bits, M, K, N, G, cus, ks)
    if path == 4:
        assert sw >= 2 * part, (bits, M, K, N, G, cus, ks)
    elif path in (1, 2):
        assert sw >= -(-M * N * 4 // 256) * 256 + part, (bits, M, K, N, G, cus, ks)
    return path, ks


def test_plan_follows_the_device_cu_count(lib):
    """The launch plan takes the CU count of the device (a partitioned MI355X
    reports fewer than 256).  Fewer CUs can mean more K splits: a weight that
    is narrow (or left to the GEMV) on 256 CUs can be wide on 32, where 17..32
    rows split a long K into ranges.  The workspace queries must cover the
    plan of every CU count from 1 to 256."""
    shapes = [(8, 128, 1024, 1024, 0), (8, 512, 4096, 4096, 0), (8, 256, 4096, 1024, 0), (4, 256, 4096, 1024, 128),
              (4, 300, 2048, 640, 32), (8, 2048, 4096, 4096, 0), (4, 64, 11008, 4096, 128), (8, 17, 8192, 512, 0),
              (4, 16, 11008, 4096, 128), (4, 32, 11008, 4096, 64), (4, 24, 16384, 11008, 128),
              (4, 20, 28672, 8192, 128), (4, 32, 8192, 3072, 32),
              # the GEMV on 256 CUs, a wide weight with two row blocks (K ranges) on a partition
              (4, 24, 16384, 640, 128), (4, 24, 8320, 1280, 128)]
    for bits, M, K, N, G in shapes:
        for cus in range(1, 257):
            _ws_covers(lib, bits, M, K, N, G, cus)
    # The two shapes above: no workspace on the full chip's plan, K ranges below it.
    assert _plan(lib, 4, 24, 16384, 640, 128, 256) == (0, 1)
    assert _plan(lib, 4, 24, 16384, 640, 128, 32) == (4, 2)
    assert _plan(lib, 4, 24, 8320, 1280, 128, 64)[0] == 4 and _plan(lib, 4, 24, 8320, 1280, 128, 64)[1] > 1
    assert lib.sgq_linear_workspace_bytes(4, 24, 16384, 640) >= 2 * 24 * 640 * 4
    assert lib.sgq_swiglu_workspace_bytes(4, 24, 16384, 640, 128) >= 2 * 2 * 24 * 640 * 4


def test_workspace_covers_every_device_sweep(lib):
    """Skinny batches (3..32 rows) over long K and narrow N, every group size
    the skinny kernel takes, on every CU count from 1 to 256: the forward's
    and the gated MLP's workspace queries hold each device's K-split partials."""
    for M in range(3, 33):
        for K in (8320, 11008, 16384, 24576):
            for N in (256, 512, 640, 1280, 2048):
                for G in (16, 32, 64, 128):
                    for cus in range(1, 257):
                        _ws_covers(lib, 4, M, K, N, G, cus)


def test_plan_examples(lib):
    # C4 fills any device without splitting K; a small GEMM splits less on a partition.
    assert _plan(lib, 8, 2048, 4096, 4096, 0, 256) == (1, 1)
    assert _plan(lib, 8, 256, 4096, 1024, 0, 256)[1] > _plan(lib, 8, 256, 4096, 1024, 0, 32)[1]
    assert _plan(lib, 4, 1, 4096, 4096, 128, 256) == (0, 1)  # decode: the GEMV
    assert _plan(lib, 4, 300, 2048, 640, 32, 256)[0] == 2  # group 32: the fp32 MFMA kernel
    assert _plan(lib, 4, 300, 2048, 644, 32, 256)[0] == 3  # N % 8 != 0: flat layout
    # A CU count above the full chip is planned as the full chip.
    assert _plan(lib, 8, 256, 4096, 1024, 0, 1024) == _plan(lib, 8, 256, 4096, 1024, 0, 256)
    assert _plan(lib, 4, 8, 4096, 11008, 128, 1024) == _plan(lib, 4, 8, 4096, 11008, 128, 256)
    assert lib.sgq_linear_plan(8, 1, 4, 4, 0, -1, ctypes.byref(ctypes.c_int()), ctypes.byref(ctypes.c_int())) == 1


def _xcd_plan(lib, bits, M, K, N, G, cus, xcds):
    rows, xlog = ctypes.c_int(-1), ctypes.c_int(-1)
    assert lib.sgq_gemm_xcd_plan(bits, M, K, N, G, cus, xcds, ctypes.byref(rows), ctypes.byref(xlog)) == 0
    return rows.value, xlog.value


def test_gemm_places_tiles_by_the_device_xcd_count(lib):
    """The GEMM's per-XCD rectangles and the workgroup permutation follow the
    device's XCD count: a full MI355X (256 CUs, 8 XCDs) and a partition of
    128 CUs on 4 XCDs.  C4's 16 x 16 tiles of 128 x 256: 8 XCDs take 4 x 8
    rectangles (4 row blocks of x, 8 column blocks of codes per L2: 16 MiB);
    4 XCDs take 64 tiles each, 4 x 16 (8 + 16 MiB, against 16 + 8 for 8 x 8,
    the first of the equal costs)."""
    assert _xcd_plan(lib, 8, 2048, 4096, 4096, 0, 256, 8) == (4, 3)
    assert _xcd_plan(lib, 8, 2048, 4096, 4096, 0, 128, 4) == (4, 2)
    # One XCD: one rectangle holds the whole grid, a single row block.
    assert _xcd_plan(lib, 8, 2048, 4096, 4096, 0, 32, 1)[1] == 0
    # A count that is not a power of two keeps the identity order.
    assert _xcd_plan(lib, 8, 2048, 4096, 4096, 0, 192, 6)[1] == 0
    # A grid that splits K has no rectangles.
    assert _xcd_plan(lib, 8, 256, 4096, 1024, 0, 256, 8)[0] == 0
    # Tiles that do not fall into one rectangle per XCD: 3 x 3 tiles on 8 XCDs.
    assert _xcd_plan(lib, 8, 384, 4096, 768, 0, 8, 8)[0] == 0
    for cus, xcds in ((256, 8), (128, 4), (64, 2)):
        rows, xlog = _xcd_plan(lib, 8, 2048, 4096, 4096, 0, cus, xcds)
        assert 1 << xlog == xcds
        per = 16 * 16 // xcds
        assert per % rows == 0 and 16 % rows == 0 and 16 % (per // rows) == 0


def test_plan_splits_fill_one_pass(lib):
    """A split-K grid never runs past the device's resident slots (one 128x256
    INT8 tile, two 128x128 INT4 or 64-row tiles, four 32-row tiles per CU):
    the split count is rounded down, so no few workgroups run as a second
    pass.  Each case below is one the previous, rounded-up plan overfilled."""
    cases = [  # bits, M, K, N, G, tiles, workgroups per CU
        (4, 128, 4096, 11008, 128, 86, 2),  # was 6 splits: 516 workgroups on 512 slots
        (4, 256, 4096, 11008, 128, 172, 2),  # was 3: 516
        (8, 128, 4096, 11008, 0, 43, 1),  # was 6: 258 on 256
        (4, 48, 4096, 11008, 128, 86, 2),  # 64-row tile, was planned at three per CU
        (8, 32, 4096, 11008, 0, 86, 4),  # 32-row tile: four per CU
    ]
    for bits, M, K, N, G, tiles, per_cu in cases:
        for cus in (256, 200, 64):
            path, ks = _plan(lib, bits, M, K, N, G, cus)
            assert path == 1, (bits, M, K, N, path)
            assert ks == max(1, min(16, per_cu * cus // tiles)), (bits, M, K, N, cus, ks)
            assert ks * tiles <= per_cu * cus or ks == 1, (bits, M, K, N, cus, ks)


def test_plan_skinny_int8(lib):
    """INT8 batches of 5..128 rows take the skinny bf16 MFMA kernel (path 4,
    no K split) once (M rounded up to 8) * K * N reaches 2^26; above 16 rows
    only while M * K * N <= 2^29.  Four rows and less work stay on the GEMV;
    larger work above 16 rows on the GEMM.  The choice does not depend on the
    CU count, and the kernel needs no workspace."""
    for cus in (256, 80, 8):
        assert _plan(lib, 8, 128, 1024, 1024, 0, cus) == (4, 1)  # C1
        assert _plan(lib, 8, 4, 4096, 4096, 0, cus) == (0, 1)
        for M in (5, 8, 16):
            assert _plan(lib, 8, M, 4096, 4096, 0, cus) == (4, 1)
            assert _plan(lib, 8, M, 11008, 4096, 0, cus) == (4, 1)
        assert _plan(lib, 8, 8, 2048, 2048, 0, cus) == (0, 1)  # 2^25
        assert _plan(lib, 8, 9, 2048, 2048, 0, cus) == (4, 1)  # 16 * 2^22 = 2^26
        assert _plan(lib, 8, 16, 1024, 1024, 0, cus) == (0, 1)
        assert _plan(lib, 8, 17, 1024, 1024, 0, cus) == (0, 1)  # 24 * 2^20 < 2^26
        assert _plan(lib, 8, 64, 1024, 1024, 0, cus) == (4, 1)
        assert _plan(lib, 8, 64, 2048, 2048, 0, cus) == (4, 1)
        assert _plan(lib, 8, 128, 2048, 2048, 0, cus) == (4, 1)  # 2^29
        assert _plan(lib, 8, 32, 4096, 4096, 0, cus) == (4, 1)  # 2^29
        assert _plan(lib, 8, 128, 2048, 2056, 0, cus)[0] == 1
        assert _plan(lib, 8, 33, 4096, 4096, 0, cus)[0] == 1
        assert _plan(lib, 8, 129, 1024, 1024, 0, cus)[0] == 1
    for M, K, N in [(128, 1024, 1024), (128, 2048, 2048), (32, 4096, 4096), (16, 11008, 4096)]:
        assert lib.sgq_linear_workspace_bytes(8, M, K, N) == 0
        assert lib.sgq_swiglu_workspace_bytes(8, M, K, N, 0) == M * N * 4  # the up projection only


def test_plan_skinny_mfma(lib):
    """Batches of 3..16 rows over a wide INT4 weight take the skinny bf16 MFMA
    kernel (path 4, whole K) when its 32- or 64-column workgroups fill at least
    5/8 of the CUs, and need 2C strips per scale column; 17..32 rows take its
    super-block form, and weights too narrow to fill the device split K
    (k_splits > 1) from 5 rows once M (rounded up to 8) * K * N reaches 2^28.
    Everything else stays on the GEMV (path 0) or the GEMM (path 1)."""
    for M in range(3, 33):
        assert _plan(lib, 4, M, 4096, 11008, 128, 256) == (4, 1)  # 172 workgroups of 64 columns
        assert _plan(lib, 4, M, 2048, 6144, 128, 256) == (4, 1)  # 192 of 32
    for M in range(1, 33):  # 128 column blocks of 16: split K from 24 rows' worth of work (2^28), else GEMV
        assert _plan(lib, 4, M, 5632, 2048, 128, 256) == ((4, 4) if M >= 17 else (0, 1))
        assert _plan(lib, 4, M, 2048, 2048, 128, 256) == (0, 1)
    for M in (1, 2):
        assert _plan(lib, 4, M, 4096, 11008, 128, 256) == (0, 1)
        assert _plan(lib, 4, M, 2048, 6144, 128, 256) == (0, 1)
    assert _plan(lib, 4, 33, 4096, 11008, 128, 256)[0] == 1  # the GEMM from 33 rows
    # Narrow weights: K split into 4 ranges of 2752 rows (64 column groups x 4
    # = 256 workgroups) from 5 rows with M (rounded up to 8) * K * N >= 2^28.
    assert _plan(lib, 4, 4, 11008, 4096, 128, 256) == (0, 1)
    for M in (5, 8, 11, 12, 16, 17, 32):
        assert _plan(lib, 4, M, 11008, 4096, 128, 256) == (4, 4)
    assert _plan(lib, 4, 8, 4096, 4096, 128, 256) == (0, 1)  # 2^27: the GEMV
    assert _plan(lib, 4, 9, 4096, 4096, 128, 256) == (4, 4)
    assert _plan(lib, 4, 32, 4096, 4096, 128, 256) == (4, 4)
    assert _plan(lib, 8, 8, 4096, 11008, 0, 256) == (4, 1)  # INT8: its own skinny kernel, no split
    assert _plan(lib, 4, 8, 2048, 6144, 8, 256) == (0, 1)  # one strip per scale column
    assert _plan(lib, 4, 8, 2048, 6144, 16, 256) == (0, 1)  # two strips: 16 columns, too narrow
    assert _plan(lib, 4, 8, 2048, 5120, 32, 256) == (4, 1)  # four strips: 160 workgroups of 32
    assert _plan(lib, 4, 8, 1024, 5120, 32, 256) == (0, 1)  # K too short
    assert _plan(lib, 4, 8, 2048, 5112, 24, 256) == (0, 1)  # three strips per scale column
    assert _plan(lib, 4, 8, 4096, 8192, 64, 256) == (4, 1)  # C = 2: 256 workgroups
    assert _plan(lib, 4, 8, 4096, 11004, 128, 256)[0] == 3  # flat layout
    # Two row blocks keep the scales of a K range in LDS: at most 8192 rows a
    # range, so a long K splits even over a wide weight.
    assert _plan(lib, 4, 24, 16384, 11008, 128, 256) == (4, 2)
    assert _plan(lib, 4, 8, 16384, 11008, 128, 256) == (4, 1)  # one row block: whole K
    # The threshold follows the device: a quarter of the CUs needs a quarter
    # of the workgroups (64 of 32 columns for N = 2048).
    assert _plan(lib, 4, 8, 5632, 2048, 128, 64) == (4, 1)
    assert _plan(lib, 4, 8, 5632, 2048, 128, 128) == (0, 1)
    assert _plan(lib, 4, 8, (1 << 24) + 16, 6144, 128, 256) == (0, 1)  # K beyond 32-bit x offsets
