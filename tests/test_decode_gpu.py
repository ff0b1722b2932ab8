"""GPU parity of the quantized LLaMA block decode step (sgq_llama_block_decode_int4)
and of sgq_rms_norm.

A decode step computes, for one new token per sequence, the row the
reference's LLaMABlock::forward (include/sovereigngrad/models.hpp:217-222)
gives for that position of the whole sequence.  The tests run the GPU step
token by token from an empty cache and compare every row with the reference
(golden fixtures) or the oracle's full-sequence forward, within
max|y - y_ref| / max|y_ref| <= 1e-5 per row.
"""
import numpy as np
import pytest
import torch

import helpers

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _row_err(y, yref):
    y, yref = np.asarray(y, np.float64), np.asarray(yref, np.float64)
    return float(np.max(np.abs(y - yref)) / max(np.max(np.abs(yref)), 1e-30))


def _decode_mod(sgq):
    import soverign_grad_amd.decode as d  # noqa: F401 (loaded through the package)

    return d


def _block_from_case(sgq, dev, codes, scales, biases, g1, g2, heads, G, eps=1e-5):
    dm = _decode_mod(sgq)
    return dm.QuantizedLLaMABlock.from_codes({k: _dev(v, dev) for k, v in codes.items()},
                                             {k: _dev(v, dev) for k, v in scales.items()},
                                             {k: (None if v is None else _dev(v, dev)) for k, v in biases.items()},
                                             _dev(g1, dev), _dev(g2, dev), heads, G, eps)


def _run_sequences(sgq, dev, blk, xs, max_tokens, starts=None):
    """xs[b]: [L_b, D] tokens of sequence b; sequence b joins at global step
    starts[b] and leaves after its last token (inactive sequences get pos = -1,
    whose rows come back NaN and write nothing).  Returns per-sequence outputs."""
    dm = _decode_mod(sgq)
    B, D = len(xs), xs[0].shape[1]
    starts = starts or [0] * B
    steps = max(s + x.shape[0] for s, x in zip(starts, xs))
    cache = dm.KVCache(B, max_tokens, D, dev)
    outs = [np.zeros_like(x) for x in xs]
    for t in range(steps):
        pos = np.full(B, -1, np.int32)
        xin = np.zeros((B, D), np.float32)
        for b in range(B):
            i = t - starts[b]
            if 0 <= i < xs[b].shape[0]:
                pos[b], xin[b] = i, xs[b][i]
        cache.pos.copy_(torch.from_numpy(pos))
        max_len = int(pos.max()) + 1 if pos.max() >= 0 else 1
        y = _np(blk.decode(_dev(xin, dev), cache.k[0], cache.v[0], cache.pos, max_len))
        for b in range(B):
            i = t - starts[b]
            if 0 <= i < xs[b].shape[0]:
                outs[b][i] = y[b]
            else:
                assert np.all(np.isnan(y[b])), (t, b)
    return outs


def test_rms_norm_golden(sgq, dev, golden):
    dm = _decode_mod(sgq)
    n = 0
    for c in golden:
        if c["kind"] != "rms_norm":
            continue
        y = _np(dm.rms_norm(_dev(c["x"], dev), _dev(c["g"], dev), c["params"]["eps"]))
        ref = c["y"]
        fin = np.isfinite(ref)
        assert np.array_equal(np.isnan(y), np.isnan(ref)), c["params"]
        if fin.any():
            # Elementwise relative error: the sum of squares runs in another
            # order (a workgroup tree instead of the CPU's in-order sum), so
            # inv_rms differs by a few ulp of D-term sums.
            assert np.max(np.abs(y[fin] - ref[fin]) / np.maximum(np.abs(ref[fin]), 1e-30)) <= 2e-6, c["params"]
        n += 1
    assert n >= 12


def test_block_decode_golden(sgq, dev, golden):
    from oracle.oracle import BLOCK_PROJ

    n = 0
    for c in golden:
        if c["kind"] != "qllama_block_int4":
            continue
        p = c["params"]
        print(f"  case {p}", flush=True)
        codes = {k: c[f"q_{k}"] for k in BLOCK_PROJ}
        scales = {k: c[f"s_{k}"] for k in BLOCK_PROJ}
        biases = {k: c.get(f"b_{k}") for k in BLOCK_PROJ}
        blk = _block_from_case(sgq, dev, codes, scales, biases, c["g1"], c["g2"], p["heads"], p["group_size"],
                               p["eps"])
        assert np.float32(blk.attn_scale) == c["attn_scale"][0]
        out = _run_sequences(sgq, dev, blk, [c["x"]], max_tokens=p["L"] + 3)[0]
        for t in range(p["L"]):
            assert _row_err(out[t], c["y"][t]) <= TOL, (p, t, _row_err(out[t], c["y"][t]))
        n += 1
    assert n >= 5


def _random_block(oracle, synth, D, H, G, seed, bias=True):
    from oracle.oracle import BLOCK_PROJ, block_shapes

    codes, scales, biases = {}, {}, {}
    for i, (name, (K, N)) in enumerate(zip(BLOCK_PROJ, block_shapes(D, H))):
        W = synth.normal((K, N), seed + i, synth.STREAM_W, 0.0, 0.02)
        codes[name], scales[name] = oracle.quantize_int4(W, G)
        biases[name] = synth.normal((N,), seed + i, synth.STREAM_BIAS, 0.0, 0.02) if bias else None
    g1 = (1.0 + synth.normal((D,), seed + 10, synth.STREAM_BIAS, 0.0, 0.1)).astype(np.float32)
    g2 = (1.0 + synth.normal((D,), seed + 11, synth.STREAM_BIAS, 0.0, 0.1)).astype(np.float32)
    return codes, scales, biases, g1, g2


def _oracle_rows(oracle, x, codes, scales, biases, g1, g2, scale, G):
    from oracle.oracle import BLOCK_PROJ

    proj = [(codes[k], scales[k], biases[k]) for k in BLOCK_PROJ]
    return oracle.qllama_block_int4(x, proj, g1, g2, 1e-5, scale, G)


@pytest.mark.parametrize("B,D,H,G,heads,lengths", [
    (1, 256, 512, 128, 4, [9]),
    (3, 256, 640, 64, 8, [4, 11, 7]),
    (8, 512, 1024, 128, 8, [5, 3, 12, 1, 8, 6, 2, 9]),
    (16, 128, 256, 32, 2, [3] * 16),
    (20, 128, 256, 32, 2, [2 + (b % 5) for b in range(20)]),  # 3 row groups of 8 on the GEMV (padded to 4)
    (130, 64, 128, 32, 2, [1 + (b % 3) for b in range(130)]),  # B > 128: GEMM projections
])
def test_block_decode_batched(sgq, dev, oracle, synth, B, D, H, G, heads, lengths):
    dm = _decode_mod(sgq)
    codes, scales, biases, g1, g2 = _random_block(oracle, synth, D, H, G, 900 + B)
    blk = _block_from_case(sgq, dev, codes, scales, biases, g1, g2, heads, G)
    xs = [synth.normal((L, D), 950 + b, synth.STREAM_X) for b, L in enumerate(lengths)]
    starts = [(b * 3) % 5 for b in range(B)]  # sequences join at different steps
    outs = _run_sequences(sgq, dev, blk, xs, max_tokens=max(lengths) + 4, starts=starts)
    for b in range(B):
        ref = _oracle_rows(oracle, xs[b], codes, scales, biases, g1, g2, dm.attention_scale(D, heads), G)
        for t in range(lengths[b]):
            e = _row_err(outs[b][t], ref[t])
            assert e <= TOL, (b, t, e)


def test_block_decode_nanollama_shape(sgq, dev, oracle, synth):
    # NanoLLaMA shape (d_model 2048, 16 heads, SwiGLU hidden 5632, INT4 g128),
    # batch 8 with ragged lengths, so the attention splits keys into chunks.
    dm = _decode_mod(sgq)
    D, H, G, heads = 2048, 5632, 128, 16
    codes, scales, biases, g1, g2 = _random_block(oracle, synth, D, H, G, 1000)
    blk = _block_from_case(sgq, dev, codes, scales, biases, g1, g2, heads, G)
    lengths = [6, 1, 3, 6, 2, 5, 4, 6]
    xs = [synth.normal((L, D), 1100 + b, synth.STREAM_X) for b, L in enumerate(lengths)]
    outs = _run_sequences(sgq, dev, blk, xs, max_tokens=64)
    for b in (0, 2, 7):
        ref = _oracle_rows(oracle, xs[b], codes, scales, biases, g1, g2, dm.attention_scale(D, heads), G)
        for t in range(lengths[b]):
            assert _row_err(outs[b][t], ref[t]) <= TOL, (b, t)


@pytest.mark.parametrize("B", [5, 13, 16])
def test_block_decode_skinny_batches(sgq, dev, oracle, synth, B):
    # 5..16 sequences at the NanoLLaMA shape run the norm-fused q/k/v and
    # gate/up projections on the skinny MFMA kernel (q, k and v side by
    # side); the first and last sequences are checked against the oracle.
    dm = _decode_mod(sgq)
    D, H, G, heads = 2048, 5632, 128, 16
    codes, scales, biases, g1, g2 = _random_block(oracle, synth, D, H, G, 1050 + B)
    blk = _block_from_case(sgq, dev, codes, scales, biases, g1, g2, heads, G)
    lengths = [2 + (b % 2) for b in range(B)]
    xs = [synth.normal((L, D), 1150 + b, synth.STREAM_X) for b, L in enumerate(lengths)]
    outs = _run_sequences(sgq, dev, blk, xs, max_tokens=8)
    for b in (0, B - 1):
        ref = _oracle_rows(oracle, xs[b], codes, scales, biases, g1, g2, dm.attention_scale(D, heads), G)
        for t in range(lengths[b]):
            e = _row_err(outs[b][t], ref[t])
            print(f"  case B={B} seq={b} t={t} rel_err={e:.3e}", flush=True)
            assert e <= TOL, (b, t, e)


def test_block_decode_long_context_chunks(sgq, dev, oracle, synth):
    # 70 positions with B = 2: the attention runs several key chunks and the
    # combine kernel; every row is checked.
    dm = _decode_mod(sgq)
    D, H, G, heads = 128, 256, 32, 4
    codes, scales, biases, g1, g2 = _random_block(oracle, synth, D, H, G, 1200)
    blk = _block_from_case(sgq, dev, codes, scales, biases, g1, g2, heads, G)
    xs = [synth.normal((70, D), 1300 + b, synth.STREAM_X) for b in range(2)]
    outs = _run_sequences(sgq, dev, blk, xs, max_tokens=80)
    for b in range(2):
        ref = _oracle_rows(oracle, xs[b], codes, scales, biases, g1, g2, dm.attention_scale(D, heads), G)
        errs = [_row_err(outs[b][t], ref[t]) for t in range(70)]
        assert max(errs) <= TOL, (b, int(np.argmax(errs)), max(errs))


def test_block_decode_in_place_and_deterministic(sgq, dev, oracle, synth):
    dm = _decode_mod(sgq)
    D, H, G, heads, B = 256, 512, 64, 4, 4
    codes, scales, biases, g1, g2 = _random_block(oracle, synth, D, H, G, 1400)
    blk = _block_from_case(sgq, dev, codes, scales, biases, g1, g2, heads, G)
    x = _dev(synth.normal((B, D), 1401, synth.STREAM_X), dev)
    runs = []
    for in_place in (False, True, True):
        cache = dm.KVCache(B, 8, D, dev)
        h = x.clone()
        y = blk.decode(h, cache.k[0], cache.v[0], cache.pos, 1, out=h if in_place else None)
        runs.append(_np(y))
    assert helpers.same_bits(runs[0], runs[1]) and helpers.same_bits(runs[1], runs[2])


def test_block_decode_cache_rows(sgq, dev, oracle, synth):
    # The step writes this token's key and value at row pos[b] of the cache,
    # equal to k_proj / v_proj of the normed input (within the forward's
    # tolerance), and leaves every other row alone.
    dm = _decode_mod(sgq)
    D, H, G, heads, B = 128, 256, 32, 2, 3
    codes, scales, biases, g1, g2 = _random_block(oracle, synth, D, H, G, 1500)
    blk = _block_from_case(sgq, dev, codes, scales, biases, g1, g2, heads, G)
    cache = dm.KVCache(B, 6, D, dev)
    cache.k[0].fill_(7.0)
    cache.v[0].fill_(-7.0)
    pos = np.array([0, 3, 5], np.int32)
    cache.pos.copy_(torch.from_numpy(pos))
    x = synth.normal((B, D), 1501, synth.STREAM_X)
    blk.decode(_dev(x, dev), cache.k[0], cache.v[0], cache.pos, 6)
    k, v = _np(cache.k[0]), _np(cache.v[0])
    n1 = oracle.rms_norm(x, g1)
    kref = oracle.quantized_matmul_int4(n1, codes["k"], scales["k"], G, biases["k"])
    vref = oracle.quantized_matmul_int4(n1, codes["v"], scales["v"], G, biases["v"])
    for b in range(B):
        assert _row_err(k[b, pos[b]], kref[b]) <= TOL and _row_err(v[b, pos[b]], vref[b]) <= TOL
        others = [r for r in range(6) if r != pos[b]]
        assert np.all(k[b, others] == 7.0) and np.all(v[b, others] == -7.0)


def test_block_decode_invalid_positions(sgq, dev, oracle, synth):
    # pos outside [0, min(max_len, max_tokens)) gives a NaN row and no cache
    # write; the other sequences are unaffected.
    dm = _decode_mod(sgq)
    D, H, G, heads, B = 128, 256, 32, 2, 4
    codes, scales, biases, g1, g2 = _random_block(oracle, synth, D, H, G, 1600)
    blk = _block_from_case(sgq, dev, codes, scales, biases, g1, g2, heads, G)
    cache = dm.KVCache(B, 4, D, dev)
    cache.k[0].fill_(1.0)
    cache.v[0].fill_(1.0)
    cache.pos.copy_(torch.tensor([0, -1, 4, 2], dtype=torch.int32))
    x = synth.normal((B, D), 1601, synth.STREAM_X)
    y = _np(blk.decode(_dev(x, dev), cache.k[0], cache.v[0], cache.pos, 3))
    assert np.all(np.isnan(y[1])) and np.all(np.isnan(y[2]))  # pos -1; pos 4 >= max_tokens
    assert np.all(np.isfinite(y[0])) and np.all(np.isfinite(y[3]))
    ref0 = _oracle_rows(oracle, x[:1], codes, scales, biases, g1, g2, dm.attention_scale(D, heads), G)
    assert _row_err(y[0], ref0[0]) <= TOL
    k = _np(cache.k[0])
    assert np.all(k[1] == 1.0) and np.all(k[2] == 1.0)  # no writes for the invalid sequences
    assert not np.all(k[3, 2] == 1.0) and np.all(k[3, [0, 1, 3]] == 1.0)
    # pos == max_len - 1 is the last valid position; pos == max_len is not
    cache.pos.copy_(torch.tensor([2, 3, 0, 0], dtype=torch.int32))
    y = _np(blk.decode(_dev(x, dev), cache.k[0], cache.v[0], cache.pos, 3))
    assert np.all(np.isfinite(y[0])) and np.all(np.isnan(y[1]))


def test_embedding_golden(sgq, dev, golden):
    dm = _decode_mod(sgq)
    n = 0
    for c in golden:
        if c["kind"] != "embedding":
            continue
        y = _np(dm.embedding(_dev(c["idx"], dev), _dev(c["w"], dev)))
        assert helpers.same_bits(y, c["y"])
        n += 1
    assert n >= 1


def _oracle_model_logits(oracle, ids, emb, layers, normf, lm, G, scale):
    """NanoLLaMA::forward (models.hpp:257-266) on one sequence, composed from
    the oracle's pinned pieces: embedding, quantized blocks, rms_norm, INT4 lm_head."""
    h = oracle.embedding(np.asarray(ids, np.float32), emb)
    for (codes, scales, biases, g1, g2) in layers:
        h = _oracle_rows(oracle, h, codes, scales, biases, g1, g2, scale, G)
    return oracle.quantized_matmul_int4(oracle.rms_norm(h, normf), lm[0], lm[1], G, lm[2])


def test_nanollama_generate(sgq, dev, oracle, synth):
    # A 2-layer quantized NanoLLaMA: every step's logits match the oracle's
    # full-sequence forward on the same prefix, and greedy generation picks the
    # same tokens (prompts of 3 tokens, 6 new tokens, batch 3).
    dm = _decode_mod(sgq)
    V, D, H, G, heads, nl = 50, 64, 128, 32, 4, 2
    emb = synth.normal((V, D), 1700, synth.STREAM_W, 0.0, 1.0)
    layers = [_random_block(oracle, synth, D, H, G, 1710 + 20 * i) for i in range(nl)]
    normf = (1.0 + synth.normal((D,), 1790, synth.STREAM_BIAS, 0.0, 0.1)).astype(np.float32)
    lq, ls = oracle.quantize_int4(synth.normal((D, V), 1791, synth.STREAM_W, 0.0, 0.3), G)
    lb = synth.normal((V,), 1792, synth.STREAM_BIAS, 0.0, 0.02)
    blocks = [_block_from_case(sgq, dev, *ly, heads, G) for ly in layers]
    lm = sgq.pack_int4(_dev(lq, dev), _dev(ls, dev), G)
    model = dm.QuantizedNanoLLaMA(_dev(emb, dev), blocks, _dev(normf, dev), lm, _dev(lb, dev))
    scale = dm.attention_scale(D, heads)
    prompts = [[3, 17, 42], [0, 49, 5], [7, 7, 7]]
    out = model.generate(prompts, 6)
    for b, seq in enumerate(out):
        assert seq[:3] == prompts[b]
        for t in range(3, len(seq)):
            logits = _oracle_model_logits(oracle, seq[:t], emb, layers, normf, (lq, ls, lb), G, scale)[-1]
            top = np.sort(logits)[::-1]
            if top[0] - top[1] > 1e-4 * np.abs(logits).max():  # not a near-tie
                assert seq[t] == int(np.argmax(logits)), (b, t)
    # Logits of one step against the oracle, batch of two sequences at different positions.
    cache = model.new_cache(2, 8)
    seqs = [[5, 6, 7, 8], [9, 10]]
    logits = None
    for t in range(4):
        pos = np.array([t if t < len(s) else -1 for s in seqs], np.int32)
        cache.pos.copy_(torch.from_numpy(pos))
        ids = torch.tensor([float(s[t]) if t < len(s) else 0.0 for s in seqs], device=dev)
        logits = _np(model.step(ids, cache, t + 1))
        for b, s in enumerate(seqs):
            if t < len(s):
                ref = _oracle_model_logits(oracle, s[: t + 1], emb, layers, normf, (lq, ls, lb), G, scale)[-1]
                assert _row_err(logits[b], ref) <= TOL, (b, t)
