"""Exact, size-independent properties of the forward at full BASELINE sizes.

These need no CPU reference, so they run at the shapes the oracle comparisons
can only sample, on every kernel the dispatcher picks (GEMV, both skinny MFMA
forms, the three-term GEMM with and without split K, the fp32 MFMA GEMM):

- power-of-two homogeneity: every product and partial sum of the forward
  scales exactly by 2^e when x does (no rounding step depends on magnitude
  while values stay normal), so y(x * 2^e) must equal y(x) * 2^e bit for bit.
  A race between workgroups, a read of uninitialised workspace or any
  nonlinear step breaks it.
- column independence: rewriting the codes of one group of columns must leave
  every other output column bit for bit unchanged (each output's summation
  order does not depend on other columns), and the rewritten columns must
  follow the new codes: negated codes give the negated output within the
  forward's tolerance.  A strip or scale-column indexing mistake breaks it.
- row permutation: each output row is formed from its own x row by the same
  operations wherever it sits in a tile or row group, so permuting the rows
  of x permutes the rows of y bit for bit.  A row-stride mistake breaks it.

Reference semantics: quantized_matmul_int8/int4 (src/quantization.cpp:189-206)
is linear in x and computes each output column from that column's codes and
scales only (src/ops.cpp:378-455).
"""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 1e-5

# (name, bits, M, K, N, group_size or scheme)
CASES = [
    ("c2_gemv", 4, 1, 4096, 4096, 128),
    ("c3_gate_m2_gemv", 4, 2, 4096, 11008, 128),
    ("c3_gate_m4_skinny", 4, 4, 4096, 11008, 128),
    ("c3_down_m4_gemv", 4, 4, 11008, 4096, 128),
    ("c3_gate_m8_skinny", 4, 8, 4096, 11008, 128),
    ("c3_down_m16_skinny_splitk", 4, 16, 11008, 4096, 128),
    ("c3_gate_m32_skinny_two_row_blocks", 4, 32, 4096, 11008, 128),
    ("c5_out_m8_gemv", 4, 8, 2048, 2048, 128),
    ("int4_prefill_gemm", 4, 256, 4096, 4096, 128),
    ("int4_g32_fp32_mfma_gemm", 4, 512, 1024, 1024, 32),
    ("c4_gemm", 8, 2048, 4096, 4096, 0),
    ("c1_skinny8", 8, 128, 1024, 1024, 0),
    ("int8_per_channel_gemm_splitk", 8, 512, 4096, 1024, 1),
]


def _plan(sgq, bits, M, K, N, g):
    lib = sgq.load_library()
    path, ks = ctypes.c_int(), ctypes.c_int()
    G = g if bits == 4 else 0
    assert lib.sgq_linear_plan(bits, M, K, N, G, 256, ctypes.byref(path), ctypes.byref(ks)) == 0
    return path.value, ks.value


def test_cases_cover_every_forward_kernel(sgq):
    plans = {name: _plan(sgq, bits, M, K, N, g) for name, bits, M, K, N, g in CASES}
    paths = {p for p, _ in plans.values()}
    assert {0, 1, 2, 4} <= paths, plans
    assert any(p == 1 and ks > 1 for p, ks in plans.values()), plans  # split-K GEMM
    assert any(p == 4 and ks > 1 for p, ks in plans.values()), plans  # skinny K ranges


def _weights(sgq, dev, bits, K, N, g, seed):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    W = torch.randn((K, N), generator=gen, device=dev) * 0.02
    qw = sgq.quantize_int4(W, g) if bits == 4 else sgq.quantize_int8(W, g)
    x_seed = seed + 1
    return qw, x_seed


def _x(dev, M, K, seed):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    return torch.randn((M, K), generator=gen, device=dev)


@pytest.mark.parametrize("name,bits,M,K,N,g", CASES, ids=[c[0] for c in CASES])
def test_power_of_two_homogeneity(sgq, dev, name, bits, M, K, N, g):
    qw, xs = _weights(sgq, dev, bits, K, N, g, 1000 + M)
    x = _x(dev, M, K, xs)
    y = sgq.quantized_matmul(x, qw).clone()
    for e in (3, -2):
        ys = sgq.quantized_matmul(x * (2.0 ** e), qw)
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
        assert torch.equal(ys, y * (2.0 ** e)), (name, e, (ys - y * 2.0 ** e).abs().max().item())


@pytest.mark.parametrize("name,bits,M,K,N,g", CASES, ids=[c[0] for c in CASES])
def test_column_independence(sgq, dev, name, bits, M, K, N, g):
    qw, xs = _weights(sgq, dev, bits, K, N, g, 2000 + M)
    x = _x(dev, M, K, xs)
    y = sgq.quantized_matmul(x, qw).clone()
    # One group of columns away from the edges (a whole INT4 scale group, so
    # the scales stay valid): its codes negated.  Symmetric quantization keeps
    # |q| <= 7 (INT4) / 127 (INT8), so the negated codes are in range.
    width = g if bits == 4 and N % g == 0 else 64
    n0 = (N // 2) // width * width
    q2 = qw.qdata.clone()
    assert q2.abs().max().item() <= (7 if bits == 4 else 127)
    q2[:, n0:n0 + width] = -q2[:, n0:n0 + width]
    qw2 = sgq.pack_int4(q2, qw.scales, g) if bits == 4 else sgq.pack_int8(q2, qw.scales, g)
    y2 = sgq.quantized_matmul(x, qw2)
    torch.cuda.synchronize()
    keep = torch.ones(N, dtype=torch.bool, device=dev)
    keep[n0:n0 + width] = False
    assert torch.equal(y2[:, keep], y[:, keep]), name
    changed, ref = y2[:, n0:n0 + width], -y[:, n0:n0 + width]
    assert ((changed - ref).abs().max() / ref.abs().max()).item() <= TOL, name


@pytest.mark.parametrize("name,bits,M,K,N,g", [c for c in CASES if c[2] > 1], ids=[c[0] for c in CASES if c[2] > 1])
def test_row_permutation(sgq, dev, name, bits, M, K, N, g):
    # Each output row is formed from its own x row by the same operations
    # wherever the row sits in a tile, row block or row group, so permuting
    # the rows of x permutes the rows of y bit for bit.
    qw, xs = _weights(sgq, dev, bits, K, N, g, 3000 + M)
    x = _x(dev, M, K, xs)
    gen = torch.Generator(device=dev)
    gen.manual_seed(M)
    perm = torch.randperm(M, generator=gen, device=dev)
    y = sgq.quantized_matmul(x, qw).clone()
    yp = sgq.quantized_matmul(x[perm].contiguous(), qw)
    torch.cuda.synchronize()
    assert torch.equal(yp, y[perm]), (name, (yp - y[perm]).abs().max().item())


# The gated MLP (silu(x . Wg) * (x . Wu)) in one library call: (name, bits, M, K, N, group or scheme).
SWIGLU_CASES = [
    ("c3_m1_gemv", 4, 1, 4096, 11008, 128),
    ("c3_m8_skinny", 4, 8, 4096, 11008, 128),
    ("c3_m32_skinny", 4, 32, 4096, 11008, 128),
    ("c5_m8_skinny", 4, 8, 2048, 5632, 128),
    ("int4_m256_gemm", 4, 256, 2048, 5632, 128),
    ("int8_m8_skinny8", 8, 8, 4096, 4096, 0),
    ("int8_m256_gemm", 8, 256, 2048, 5632, 1),
]


@pytest.mark.parametrize("name,bits,M,K,N,g", SWIGLU_CASES, ids=[c[0] for c in SWIGLU_CASES])
def test_swiglu_rows_and_columns(sgq, dev, name, bits, M, K, N, g):
    # Row permutation and column independence of the gated MLP: silu and the
    # product act elementwise on two forwards that each have both properties.
    qg, xs = _weights(sgq, dev, bits, K, N, g, 4000 + M)
    qu, _ = _weights(sgq, dev, bits, K, N, g, 5000 + M)
    x = _x(dev, M, K, xs)
    h = sgq.quantized_swiglu(x, qg, qu).clone()
    if M > 1:
        gen = torch.Generator(device=dev)
        gen.manual_seed(M)
        perm = torch.randperm(M, generator=gen, device=dev)
        hp = sgq.quantized_swiglu(x[perm].contiguous(), qg, qu)
        torch.cuda.synchronize()
        assert torch.equal(hp, h[perm]), name
    width = g if bits == 4 else 64
    n0 = (N // 2) // width * width
    q2 = qu.qdata.clone()
    q2[:, n0:n0 + width] = -q2[:, n0:n0 + width]
    qu2 = sgq.pack_int4(q2, qu.scales, g) if bits == 4 else sgq.pack_int8(q2, qu.scales, g)
    h2 = sgq.quantized_swiglu(x, qg, qu2)
    torch.cuda.synchronize()
    keep = torch.ones(N, dtype=torch.bool, device=dev)
    keep[n0:n0 + width] = False
    assert torch.equal(h2[:, keep], h[:, keep]), name
    changed, ref = h2[:, n0:n0 + width], -h[:, n0:n0 + width]
    assert ((changed - ref).abs().max() / ref.abs().max()).item() <= TOL, name


@pytest.mark.parametrize("B", [4, 8, 16])
def test_block_decode_sequence_permutation(sgq, dev, B):
    # One LLaMA block decode step at the NanoLLaMA shape with ragged cached
    # lengths: permuting the sequences (their tokens, caches and positions)
    # permutes the outputs and the appended cache rows bit for bit, since each
    # sequence's projections, attention chunks and combine do not depend on its
    # index in the batch.
    import soverign_grad_amd.decode as dm

    D, H, heads, G, T, L = 2048, 5632, 16, 128, 160, 129
    gen = torch.Generator(device=dev)
    gen.manual_seed(77 + B)
    shapes = dm.projection_shapes(D, H)
    W = {k: torch.randn(shapes[k], generator=gen, device=dev) * 0.02 for k in dm.PROJECTIONS}
    b = {k: torch.randn((shapes[k][1],), generator=gen, device=dev) * 0.02 for k in dm.PROJECTIONS}
    g1 = 1.0 + 0.1 * torch.randn((D,), generator=gen, device=dev)
    g2 = 1.0 + 0.1 * torch.randn((D,), generator=gen, device=dev)
    blk = dm.QuantizedLLaMABlock.from_float(W, b, g1, g2, heads, G)
    x = torch.randn((B, D), generator=gen, device=dev)
    kc = torch.randn((B, T, D), generator=gen, device=dev)
    vc = torch.randn((B, T, D), generator=gen, device=dev)
    pos = torch.randint(0, L - 1, (B,), generator=gen, device=dev, dtype=torch.int32)
    pos[0] = 0
    pos[-1] = L - 2
    perm = torch.randperm(B, generator=gen, device=dev)
    k1, v1 = kc.clone(), vc.clone()
    y = blk.decode(x, k1, v1, pos, L).clone()
    k2, v2 = kc[perm].contiguous(), vc[perm].contiguous()
    yp = blk.decode(x[perm].contiguous(), k2, v2, pos[perm].contiguous(), L)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert torch.equal(yp, y[perm])
    assert torch.equal(k2, k1[perm]) and torch.equal(v2, v1[perm])
