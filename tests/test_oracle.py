"""CPU tests of the oracle (the checker every GPU parity test relies on).

The oracle (oracle/sgq_oracle.c) is pinned by:
  * the golden fixtures, written by the compiled reference (bit-exact);
  * a live comparison with the compiled reference on fresh shapes, when
    oracle/_ref is built (dev container);
  * closed forms and invariants that do not restate the oracle's formulas:
    round-trip error bounds, the fp64 error bound of the dot products,
    identity weights, linearity, special values.
"""
import math

import numpy as np
import pytest

from helpers import bits, same_bits

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


# ---- golden fixtures (reference outputs) ---------------------------------

def test_golden_quantize_int8(oracle, golden):
    n = 0
    for c in golden:
        if c["kind"] != "quantize_int8":
            continue
        q, s = oracle.quantize_int8(c["x"], c["params"]["scheme"])
        assert same_bits(q, c["q"]), c["params"]
        assert same_bits(s, c["s"]), c["params"]
        if "deq" in c and c["x"].size:
            d = oracle.dequantize_int8(q, s, c["params"]["scheme"])
            assert same_bits(d, c["deq"]), c["params"]
        n += 1
    assert n >= 20


def test_golden_quantize_int4(oracle, golden):
    n = 0
    for c in golden:
        if c["kind"] != "quantize_int4":
            continue
        g = c["params"]["group_size"]
        q, s = oracle.quantize_int4(c["x"], g)
        assert same_bits(q, c["q"]), c["params"]
        assert same_bits(s, c["s"]), c["params"]
        if "deq" in c:
            d = oracle.dequantize_int4(q, s, g)
            assert same_bits(d, c["deq"]), c["params"]
        n += 1
    assert n >= 10


def test_golden_linear(oracle, golden):
    n = 0
    for c in golden:
        if c["kind"] == "linear_int8":
            y = oracle.quantized_matmul_int8(c["x"], c["q"], c["s"], c["params"]["scheme"], c.get("bias"))
        elif c["kind"] == "linear_int4":
            y = oracle.quantized_matmul_int4(c["x"], c["q"], c["s"], c["params"]["group_size"], c.get("bias"))
        else:
            continue
        # The oracle restates the reference's loop order and FMA contraction,
        # so the outputs agree to the bit.
        assert same_bits(y, c["y"]), c["params"]
        n += 1
    assert n >= 16


# ---- live comparison with the compiled reference -------------------------

@pytest.mark.parametrize("shape", [(1, 1), (9, 17), (64, 100), (257, 31), (128, 1024)])
def test_reference_live_quantize(oracle, ref, synth, shape):
    x = synth.normal(shape, 77, 0, 0.0, 0.02)
    for scheme in (0, 1):
        assert same_bits(oracle.quantize_int8(x, scheme)[0], ref.quantize_int8(x, scheme)[0])
        assert same_bits(oracle.quantize_int8(x, scheme)[1], ref.quantize_int8(x, scheme)[1])
    for g in (0, 8, 32, 128, 7, 1000):
        qo, so = oracle.quantize_int4(x, g)
        qr, sr = ref.quantize_int4(x, g)
        assert same_bits(qo, qr) and same_bits(so, sr), g


@pytest.mark.parametrize("mkn", [(1, 300, 70), (7, 129, 33), (9, 257, 131), (37, 130, 77), (8, 2048, 512)])
def test_reference_live_matmul(oracle, ref, synth, mkn):
    M, K, N = mkn
    a = synth.normal((M, K), 5, 1)
    b = synth.normal((K, N), 5, 0, 0.0, 0.02)
    assert same_bits(oracle.matmul(a, b), ref.matmul(a, b))


# ---- closed forms and special cases --------------------------------------

def test_zero_tensor_uses_floor(oracle):
    x = np.zeros((3, 4), np.float32)
    q, s = oracle.quantize_int8(x, 0)
    assert s[0] == np.float32(np.float32(1e-8) / np.float32(127.0))
    assert np.all(q == 0)
    q4, s4 = oracle.quantize_int4(x, 4)
    assert np.all(s4 == np.float32(np.float32(1e-8) / np.float32(7.0)))


def test_ties_round_away_and_negative_zero(oracle):
    # max |x| = 127 -> inv_scale = 1, so codes are round-half-away of x itself.
    x = np.array([127, 2.5, -2.5, 0.5, -0.5, -0.3, 126.5, -126.5], np.float32).reshape(2, 4)
    q, s = oracle.quantize_int8(x, 0)
    assert s[0] == 1.0
    assert q.reshape(-1).tolist() == [127, 3, -3, 1, -1, -0.0, 127, -127]
    assert bits(q.reshape(-1)[5:6])[0] == 0x80000000  # -0.0 is kept in qdata


def test_nan_and_inf(oracle):
    x = np.array([np.nan, 1.0, -2.0, 0.25], np.float32).reshape(2, 2)
    q, s = oracle.quantize_int8(x, 0)
    assert q.reshape(-1)[0] == 127  # NaN never sets max_abs and clamps to +hi
    assert s[0] == np.float32(2.0) / np.float32(127.0)
    x = np.array([np.inf, 1.0, -2.0, -0.25], np.float32).reshape(2, 2)
    q, s = oracle.quantize_int8(x, 0)
    assert math.isinf(s[0]) and q.reshape(-1)[0] == 127
    assert np.all(q.reshape(-1)[1:] == 0) and bits(q.reshape(-1)[2:3])[0] == 0x80000000
    q4, s4 = oracle.quantize_int4(np.array([np.nan, 3.0], np.float32), 2)
    assert q4.tolist() == [7.0, 7.0]


def test_group_defaults_and_partial(oracle):
    x = np.arange(1, 71, dtype=np.float32).reshape(7, 10)
    q0, s0 = oracle.quantize_int4(x, 0)
    q32, s32 = oracle.quantize_int4(x, 32)
    assert same_bits(q0, q32) and same_bits(s0, s32)
    qn, sn = oracle.quantize_int4(x, -3)
    assert same_bits(qn, q32)
    assert s32.size == 3  # ceil(70/32); the last group has 6 elements
    assert s32[2] == np.float32(70.0) / np.float32(7.0)


def test_rank1_is_per_tensor(oracle):
    x = np.linspace(-3, 5, 17, dtype=np.float32)
    q_pc, s_pc = oracle.quantize_int8(x, 1)
    q_pt, s_pt = oracle.quantize_int8(x, 0)
    assert s_pc.size == 1 and same_bits(q_pc, q_pt) and same_bits(s_pc, s_pt)


@pytest.mark.parametrize("bits_", [8, 4])
def test_roundtrip_error_bound(oracle, synth, bits_):
    # |x - q*s| <= s/2 (+ rounding of the products) for every element that is
    # not clamped; codes stay in [-hi, hi] and hit +-hi at the group maximum.
    x = synth.normal((64, 96), 9, 0)
    if bits_ == 8:
        q, s = oracle.quantize_int8(x, 1)
        sc = np.repeat(s, 96).reshape(64, 96)
        hi = 127
    else:
        q, s = oracle.quantize_int4(x, 32)
        sc = np.repeat(s, 32).reshape(64, 96)
        hi = 7
    d = q.astype(np.float64) * sc
    assert np.all(np.abs(q) <= hi) and np.all(q == np.round(q))
    err = np.abs(x.astype(np.float64) - d)
    assert np.all(err <= sc * 0.5 * (1 + 1e-5) + 1e-30)
    amax = np.abs(x.reshape(-1, 96 if bits_ == 8 else 32)).argmax(axis=1)
    qq = np.abs(q.reshape(-1, 96 if bits_ == 8 else 32))
    assert np.all(qq[np.arange(qq.shape[0]), amax] == hi)


def test_matmul_fp64_bound_identity_linearity(oracle, synth):
    K, N, M = 257, 65, 11
    a = synth.normal((M, K), 3, 1)
    b = synth.normal((K, N), 3, 0, 0.0, 0.02)
    y = oracle.matmul(a, b)
    y64, yabs = oracle.matmul_f64(a, b)
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    assert np.all(np.abs(y - y64) <= gamma * yabs + 1e-30)
    # identity weight returns x exactly
    eye = np.eye(K, dtype=np.float32)
    assert same_bits(oracle.matmul(a, eye), a)
    # linearity within rounding
    a2 = synth.normal((M, K), 4, 1)
    lhs = oracle.matmul(a + a2, b).astype(np.float64)
    rhs = oracle.matmul(a, b).astype(np.float64) + oracle.matmul(a2, b)
    assert np.max(np.abs(lhs - rhs)) <= 4 * gamma * (np.abs(a) + np.abs(a2)).sum(axis=1).max() * np.abs(b).max()


def test_per_tensor_factorisation(oracle, synth):
    # For per-tensor scales y = s * (x . q) up to rounding.
    W = synth.normal((128, 48), 11, 0, 0.0, 0.02)
    x = synth.normal((5, 128), 11, 1)
    q, s = oracle.quantize_int8(W, 0)
    y = oracle.quantized_matmul_int8(x, q, s, 0)
    yq = (x.astype(np.float64) @ q.astype(np.float64)) * float(s[0])
    assert np.max(np.abs(y - yq)) <= 1e-5 * np.max(np.abs(yq))


def test_bias_broadcast(oracle, synth):
    W = synth.normal((32, 16), 12, 0, 0.0, 0.02)
    x = synth.normal((6, 32), 12, 1)
    b = synth.normal((1, 16), 12, 2)
    q, s = oracle.quantize_int8(W, 1)
    y0 = oracle.quantized_matmul_int8(x, q, s, 1)
    y1 = oracle.quantized_matmul_int8(x, q, s, 1, b)
    assert same_bits(y1, (y0 + b).astype(np.float32))


# ---- silu and the gated MLP (SwiGLU::forward, nn.hpp:151-154) -------------

def test_golden_silu_and_swiglu(oracle, golden):
    kinds = {"silu": 0, "swiglu_int4": 0, "swiglu_int8": 0}
    for c in golden:
        k = c["kind"]
        if k == "silu":
            y = oracle.silu(c["x"])
        elif k == "swiglu_int4":
            y = oracle.swiglu_int4(c["x"], c["qg"], c["sg"], c["qu"], c["su"], c["params"]["group_size"],
                                   c.get("bias_gate"), c.get("bias_up"))
        elif k == "swiglu_int8":
            y = oracle.swiglu_int8(c["x"], c["qg"], c["sg"], c["qu"], c["su"], c["params"]["scheme"],
                                   c.get("bias_gate"), c.get("bias_up"))
        else:
            continue
        assert same_bits(y, c["y"]), (k, c["params"])  # same libm expf, same products
        kinds[k] += 1
    assert kinds["silu"] >= 1 and kinds["swiglu_int4"] >= 4 and kinds["swiglu_int8"] >= 2


def test_reference_live_silu(oracle, ref, synth):
    x = synth.normal((4096,), 91, 0, 0.0, 8.0)
    assert same_bits(oracle.silu(x), ref.silu(x))
    y = synth.normal((4096,), 92, 0)
    assert same_bits(oracle.mul(x, y), ref.mul(x, y))


def test_silu_closed_forms(oracle):
    # silu(x) - silu(-x) = x (x*s(x) + x*s(-x) = x since s(x) + s(-x) = 1),
    # saturation to x and to -0, the value at 0 and the known global minimum
    # (about -0.27846 at x about -1.27846).
    x = np.linspace(-30, 30, 6001, dtype=np.float32)
    s, sm = oracle.silu(x).astype(np.float64), oracle.silu(-x).astype(np.float64)
    assert np.all(np.abs((s - sm) - x) <= 4 * np.spacing(np.abs(x).astype(np.float32)) + 1e-7)
    big = np.array([50.0, 100.0, 1e6], np.float32)
    assert np.array_equal(oracle.silu(big), big)
    # exp(-x) overflows fp32 past x = 88.7: x / inf = -0; before that the tail is x * e^x
    tiny = oracle.silu(-big[1:])
    assert np.all(tiny == 0.0) and np.all(np.signbit(tiny))
    assert abs(float(oracle.silu(np.array([-50.0], np.float32))[0]) / (-50.0 * math.exp(-50.0)) - 1.0) < 1e-6
    assert oracle.silu(np.zeros(1, np.float32))[0] == 0.0
    grid = np.linspace(-2.0, -0.5, 150001, dtype=np.float32)
    v = oracle.silu(grid)
    i = int(np.argmin(v))
    assert abs(float(grid[i]) + 1.27846) < 1e-3 and abs(float(v[i]) + 0.278465) < 1e-5
    assert np.isnan(oracle.silu(np.array([np.nan], np.float32))[0])


def test_swiglu_is_silu_of_gate_times_up(oracle, synth):
    # The composition against the oracle's pinned pieces, with bias on both
    # projections and an odd group size.
    M, K, N, G = 6, 70, 24, 8
    x = synth.normal((M, K), 93, 1)
    Wg, Wu = synth.normal((K, N), 94, 0, 0.0, 0.05), synth.normal((K, N), 95, 0, 0.0, 0.05)
    bg, bu = synth.normal((1, N), 96, 2, 0.0, 0.5), synth.normal((1, N), 97, 2, 0.0, 0.5)
    qg, sg = oracle.quantize_int4(Wg, G)
    qu, su = oracle.quantize_int4(Wu, G)
    g = oracle.quantized_matmul_int4(x, qg, sg, G, bg)
    u = oracle.quantized_matmul_int4(x, qu, su, G, bu)
    ref = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64))) * u
    h = oracle.swiglu_int4(x, qg, sg, qu, su, G, bg, bu)
    assert np.max(np.abs(h - ref)) <= 1e-6 * max(1.0, np.max(np.abs(ref)))


# ---- rms_norm, softmax, embedding, attention, quantized LLaMA block ----------

def _block_proj(c):
    from oracle.oracle import BLOCK_PROJ

    return [(c[f"q_{n}"], c[f"s_{n}"], c.get(f"b_{n}")) for n in BLOCK_PROJ]


def test_golden_norm_softmax_embedding_block(oracle, golden):
    kinds = {"rms_norm": 0, "softmax": 0, "embedding": 0, "qllama_block_int4": 0}
    for c in golden:
        k, p = c["kind"], c["params"]
        if k == "rms_norm":
            y = oracle.rms_norm(c["x"], c["g"], p["eps"])
        elif k == "softmax":
            y = oracle.softmax_rows(c["x"])
        elif k == "embedding":
            y = oracle.embedding(c["idx"], c["w"])
        elif k == "qllama_block_int4":
            y = oracle.qllama_block_int4(c["x"], _block_proj(c), c["g1"], c["g2"], p["eps"], float(c["attn_scale"][0]),
                                         p["group_size"])
        else:
            continue
        assert same_bits(y, c["y"]), (k, p)
        kinds[k] += 1
    assert kinds["rms_norm"] >= 12 and kinds["softmax"] >= 5 and kinds["embedding"] >= 1
    assert kinds["qllama_block_int4"] >= 5


def _random_block(oracle, synth, L, D, H, G, seed, bias=True, zero_codes=False):
    from oracle.oracle import block_shapes

    proj = []
    for i, (K, N) in enumerate(block_shapes(D, H)):
        W = synth.normal((K, N), seed + i, 0, 0.0, 0.05)
        q, s = oracle.quantize_int4(W, G)
        if zero_codes:
            q = np.zeros_like(q)
        b = synth.normal((N,), seed + i, 2, 0.0, 0.3) if bias else None
        proj.append((q, s, b))
    x = synth.normal((L, D), seed, 1)
    g1 = 1.0 + synth.normal((D,), seed + 20, 2, 0.0, 0.1)
    g2 = 1.0 + synth.normal((D,), seed + 21, 2, 0.0, 0.1)
    return x, proj, g1.astype(np.float32), g2.astype(np.float32)


@pytest.mark.parametrize("L,D,H,G", [(7, 64, 96, 32), (10, 96, 128, 32), (3, 256, 512, 128)])
def test_reference_live_block(oracle, ref, synth, L, D, H, G):
    x, proj, g1, g2 = _random_block(oracle, synth, L, D, H, G, 300 + L)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D // 4)))
    assert same_bits(oracle.qllama_block_int4(x, proj, g1, g2, 1e-5, scale, G),
                     ref.qllama_block_int4(x, proj, g1, g2, 1e-5, scale, G))
    for Dn in (1, 5, 8, 13, 64, 67, 1001):
        xn = synth.normal((3, Dn), 400 + Dn, 1, 0.0, 2.0)
        gn = synth.normal((Dn,), 401 + Dn, 2)
        assert same_bits(oracle.rms_norm(xn, gn), ref.rms_norm(xn, gn)), Dn


def test_rms_norm_closed_forms(oracle, synth):
    # A constant row c gives c / sqrt(c^2 + eps) * g; the mean square of the
    # output with g = 1 is D*ss/(ss + D*eps)/D, i.e. 1 up to eps; scaling x by
    # a power of two leaves the output unchanged when eps is negligible.
    D = 64
    g = synth.normal((D,), 501, 2)
    row = np.full((1, D), 3.0, np.float32)
    out = oracle.rms_norm(row, g)
    inv = np.float32(1.0) / np.sqrt(np.float32(9.0 + 1e-5))
    assert np.array_equal(out[0], (np.float32(3.0) * inv) * g)
    x = synth.normal((4, D), 502, 1)
    y = oracle.rms_norm(x, np.ones(D, np.float32), 0.0)
    assert np.allclose((y.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-6)
    assert np.allclose(oracle.rms_norm(x * 64.0, np.ones(D, np.float32), 0.0), y, rtol=0, atol=2e-7)
    z = oracle.rms_norm(np.zeros((1, D), np.float32), g)
    assert np.all(z == 0)


def test_softmax_closed_forms(oracle, synth):
    # Rows sum to 1; a shift by an exactly representable constant leaves the
    # bits unchanged (x - max is the same); -1e9 entries get weight exactly 0;
    # equal entries get exactly 1/C when C is a power of two.
    x = np.round(synth.normal((5, 33), 503, 1, 0.0, 4.0)).astype(np.float32)
    p = oracle.softmax_rows(x)
    assert np.allclose(p.astype(np.float64).sum(axis=1), 1.0, atol=1e-6)
    assert same_bits(p, oracle.softmax_rows(x + np.float32(1000.0)))
    m = x.copy()
    m[:, 10:] = -1e9
    pm = oracle.softmax_rows(m)
    assert np.all(pm[:, 10:] == 0.0)
    assert np.array_equal(oracle.softmax_rows(np.full((1, 16), 2.5, np.float32)), np.full((1, 16), 1 / 16, np.float32))


def test_causal_attention_closed_forms(oracle, synth):
    # Row 0 attends to itself only, so it is V[0] exactly; with equal keys
    # every row r averages V[0..r]; changing later rows of Q, K, V never
    # changes earlier output rows.
    L, D = 9, 32
    q, k, v = (synth.normal((L, D), 504 + i, 1) for i in range(3))
    ctx = oracle.causal_attention(q, k, v, 0.25)
    assert same_bits(ctx[0], v[0])
    keq = np.tile(k[:1], (L, 1))
    ce = oracle.causal_attention(q, keq, v, 0.25)
    for r in range(L):
        assert np.allclose(ce[r], v[: r + 1].astype(np.float64).mean(axis=0), rtol=1e-5, atol=1e-6)
    q2, k2, v2 = q.copy(), k.copy(), v.copy()
    q2[5:], k2[5:], v2[5:] = 7.0, -3.0, 11.0
    assert same_bits(oracle.causal_attention(q2, k2, v2, 0.25)[:5], ctx[:5])


def test_block_closed_forms(oracle, synth):
    # All-zero codes leave only the biases: attention returns b_out, the MLP
    # returns b_down, so out = (x + b_out) + b_down exactly.  Causality: later
    # rows of x never change earlier output rows.  A prefix of the sequence
    # reproduces the same rows up to summation order (decode equivalence).
    L, D, H, G = 11, 64, 96, 32
    x, proj, g1, g2 = _random_block(oracle, synth, L, D, H, G, 600, zero_codes=True)
    out = oracle.qllama_block_int4(x, proj, g1, g2, 1e-5, 0.25, G)
    assert same_bits(out, (x + proj[3][2]) + proj[6][2])
    x, proj, g1, g2 = _random_block(oracle, synth, L, D, H, G, 700)
    full = oracle.qllama_block_int4(x, proj, g1, g2, 1e-5, 0.25, G)
    x2 = x.copy()
    x2[6:] = 5.0
    assert same_bits(oracle.qllama_block_int4(x2, proj, g1, g2, 1e-5, 0.25, G)[:6], full[:6])
    for t in (0, 3, 8):
        pre = oracle.qllama_block_int4(x[: t + 1], proj, g1, g2, 1e-5, 0.25, G)
        assert np.allclose(pre[t], full[t], rtol=0, atol=2e-6 * np.abs(full[t]).max()), t


def test_embedding_closed_forms(oracle, synth):
    w = synth.normal((6, 8), 505, 0)
    idx = np.array([5, 0, 2.99, -0.99, -1, 6], np.float32)
    e = oracle.embedding(idx, w)
    assert same_bits(e[0], w[5]) and same_bits(e[1], w[0]) and same_bits(e[2], w[2]) and same_bits(e[3], w[0])
    assert np.all(e[4] == 0) and np.all(e[5] == 0)
