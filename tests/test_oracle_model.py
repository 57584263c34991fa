"""The oracle's fixture-model restatement (oracle/strata_oracle_model.c,
oracle/fixture.py) against the reference's own known answers and float64
equations. CPU only.

Known answers held by the reference for its untrained fixture (createFixture(1234)):
  * decode of 2, 7, 4, 7, 4 from a fresh engine -> argmax tokens 29, 2, 15, 9, 15
    (reports/wasm.json:172-178, reports/validation.md:11-13; the run is
    tests/conformance.js:70-74);
  * after 2, 7, 4, 8, 7, 4, the step of token 8 routes layers 0-3 to experts
    [0,5], [5,3], [4,1], [4,5] (reports/wasm.json stats.routes: the last step
    of that engine, tests/conformance.js:84-91 with chunk size 5);
  * prompt 2, 7, 4 then greedy generation -> 15, 18, 3, 15
    (reports/validation.md:25, scripts/test-browser.mjs:25-26).
"""
import math
import struct

import numpy as np
import pytest

import reference_f64 as f64
from conftest import ref_compare


@pytest.fixture(scope="module")
def fx(oracle):
    from oracle import fixture
    return fixture


@pytest.fixture(scope="module")
def model(fx):
    return fx.create_fixture(1234)


def test_fixture_decode_known_tokens(fx, model):
    e = fx.OracleEngine(model)
    assert [e.step(t)[0] for t in (2, 7, 4, 7, 4)] == [29, 2, 15, 9, 15]


def test_fixture_decode_known_routes(fx, model):
    e = fx.OracleEngine(model)
    for t in (2, 7, 4, 8, 7, 4):
        e.step(t)
    e.step(8)
    assert [r["ids"] for r in e.routes] == [[0, 5], [5, 3], [4, 1], [4, 5]]


def test_fixture_prompt_then_generate(fx, model):
    e = fx.OracleEngine(model)
    for t in (2, 7, 4):
        nxt, _ = e.step(t)
    out = []
    for _ in range(4):
        out.append(nxt)
        nxt, _ = e.step(nxt)
    assert out == [15, 18, 3, 15]


def test_fixture_decode_matches_float64_engine(fx, model):
    # 16 seeded tokens uniform over the vocabulary; tests/conformance.js:73
    # compares full logits at 8e-5 under |a-e| <= tol (1 + |e|).
    rng = np.random.default_rng(20261202)
    tokens = rng.integers(0, model.config["vocab"], 16).tolist()
    e, r = fx.OracleEngine(model), f64.ReferenceEngine(model, fx.ngram_rows)
    for t in tokens:
        tok, logits = e.step(t)
        rtok, rlogits, routes = r.step(t)
        assert [x["ids"] for x in e.routes] == routes
        assert tok == rtok
        ref_compare(logits, rlogits, 8e-5)


def test_fixture_generator_values(fx, model):
    # The LCG and value rules of src/fixture.js:7-8 at their first draws: the
    # first tensor is token_embd (mode 'embedding', scale 0.4).
    state = 1234
    vals = []
    for _ in range(3):
        state = (state * 1664525 + 1013904223) % 2 ** 32
        vals.append(np.float32((state / 2 ** 32 * 2 - 1) * 0.4))
    assert np.array_equal(model.data("token_embd.weight")[:3], np.array(vals, np.float32))
    # Norm tensors are 1 + 0.05 U(-1, 1) and ssm_a is -0.1 - |U|.
    assert np.all(np.abs(model.data("output_hc_norm.weight") - 1) <= 0.05)
    assert np.all(model.data("blk.0.ssm_a") <= -0.1)
    assert model.shape("per_layer_token_embd.weight") == [8, 88]


def test_ngram_rows_ranges_and_cut(fx, model):
    c, eos = model.constants, model.config["eos"]
    for token in range(model.config["vocab"]):
        for prev in ([], [3], [5, 9], [eos, 9], [9, eos]):
            rows = fx.ngram_rows(token, prev, c, eos)
            for h, r in enumerate(rows):
                assert c["offsets"][h] <= r < c["offsets"][h] + c["vocab"][h]
    # A history cut at EOS makes every older position EOS (src/model.js:25-26):
    # [x, EOS] and [y, EOS] give the same rows, and a missing history equals EOS.
    assert fx.ngram_rows(5, [1, eos], c, eos) == fx.ngram_rows(5, [2, eos], c, eos)
    assert fx.ngram_rows(5, [], c, eos) == fx.ngram_rows(5, [eos, eos], c, eos)
    # Products wrap modulo 2^64: a token large enough to overflow.
    big = 2 ** 40
    t0 = (big * c["multipliers"][0]) % 2 ** 64
    t1 = (eos * c["multipliers"][1]) % 2 ** 64
    assert fx.ngram_rows(big, [], c, eos)[0] == (t0 ^ t1) % c["vocab"][0]


# ------------------------------------------------------------ kernels alone
def _bits(f):
    return struct.unpack("<I", struct.pack("<f", f))[0]


@pytest.mark.parametrize("fn,lo,hi", [("logf", 1.0, 5e8), ("logf", 1e-30, 1.0), ("sinf", 0.0, 4.0),
                                      ("cosf", 0.0, 4.0), ("sinf", -0.0, -4.0), ("cosf", -0.0, -4.0)])
def test_transcendentals_within_one_ulp_of_libm(oracle, fn, lo, hi):
    # Every 101st float bit pattern of the range (about 10^7 inputs).
    diff, far = oracle.math_survey(fn, _bits(lo), _bits(hi), 101)
    assert far == 0
    assert diff < 0.01 * (_bits(hi) - _bits(lo)) / 101


def test_transcendental_special_values(oracle):
    assert oracle.logf(1.0) == 0.0 and oracle.logf(2.0) == np.float32(math.log(2))
    assert np.isneginf(oracle.logf(0.0)) and np.isnan(oracle.logf(-1.0))
    assert oracle.sinf(0.0) == 0.0 and oracle.cosf(0.0) == 1.0
    assert oracle.sinf(np.float32(math.pi / 2)) == 1.0


def test_gdn_production_state(oracle):
    # tests/conformance.js:45-50: dim 128, 16 key heads, 48 value heads, 3 steps.
    dim, kh, vh = 128, 16, 48
    state = np.zeros(dim * vh * dim, np.float32)
    ref = np.zeros(dim * vh * dim)
    for step in range(3):
        i = np.arange(kh * dim)
        q = (np.sin(i + step) * 0.04).astype(np.float32)
        k = (np.cos(i * 0.3 - step) * 0.04).astype(np.float32)
        v = np.sin(np.arange(vh * dim) * 0.1 + step).astype(np.float32)
        d = (0.9 + np.arange(vh) * 0.001).astype(np.float32)
        beta = np.full(vh, 0.6, np.float32)
        want = f64.gdn(ref, q, k, v, d, beta, dim, kh, vh)
        ref_compare(oracle.gdn_step(state, q, k, v, d, beta, dim, kh, vh), want)
    ref_compare(state, ref)


def test_conv_dilated_history(oracle):
    # tests/conformance.js:51-53: 7 channels, 4 taps, dilation 3, 12 steps.
    ch, taps, dil = 7, 4, 3
    hist = np.zeros(ch * 9, np.float32)
    ref = np.zeros(ch * 9)
    w = np.cos(np.arange(ch * taps)).astype(np.float32)
    for step in range(12):
        x = np.sin(np.arange(ch) + step).astype(np.float32)
        want = f64.conv(ref, x, w, taps, dil, True)
        ref_compare(oracle.conv(hist, x, w, ch, taps, dil, 1), want)
    ref_compare(hist, ref)


@pytest.mark.parametrize("dim,count", [(8, 3), (70, 65), (256, 2048)])
def test_attention_cells(oracle, dim, count):
    # tests/conformance.js:54-61: selected cells [0, 3, 8]; 70-component tails
    # and 2048 reversed cells.
    heads, kvh = 4, 2
    if count == 3:
        q = np.sin(np.arange(32)).astype(np.float32)
        keys = np.cos(np.arange(9 * 16) * 0.13).astype(np.float32)
        vals = np.sin(np.arange(9 * 16) * 0.07).astype(np.float32)
        cells = np.array([0, 3, 8], np.int32)
    else:
        q = (np.sin(np.arange(heads * dim) * 0.13) * 0.2).astype(np.float32)
        keys = np.cos(np.arange(count * kvh * dim) * 0.07).astype(np.float32)
        vals = np.sin(np.arange(count * kvh * dim) * 0.11).astype(np.float32)
        cells = (count - 1 - np.arange(count)).astype(np.int32)
    got = oracle.attention(q, keys, vals, cells, dim, heads, kvh, len(cells), np.float32(1 / math.sqrt(dim)))
    ref_compare(got, f64.attention(q, keys, vals, cells.tolist(), dim, heads, kvh))


@pytest.mark.parametrize("dim,rotary,heads", [(8, 8, 4), (256, 64, 2)])
def test_rope_table_and_rotation(oracle, dim, rotary, heads):
    # Frequencies by the double series, the table through position 2047, and
    # the NeoX rotation against float64 pos / base^(2i/rotary) (the reference's
    # RoPE check through position 2047, reports/validation.md:17).
    base, context = 1e7, 2048
    hi, lo = oracle.rope_frequencies(rotary, base)
    ref_f = base ** (-2 * np.arange(rotary // 2) / rotary)
    assert np.all(np.abs(hi.astype(np.float64) + lo - ref_f) <= 1e-15)
    cos, sin = oracle.rope_table(hi, lo, rotary, context)
    x = np.sin(np.arange(dim * heads) * 0.37).astype(np.float32)
    for pos in (0, 1, 17, 1000, 2047):
        got = oracle.rope_position(x, cos, sin, dim, heads, rotary, pos)
        want = f64.rope(x.astype(np.float64), dim, rotary, pos, base)
        ref_compare(got, want)


def test_small_kernels_against_float64(oracle):
    rng = np.random.default_rng(7)
    W, S = 32, 2
    norm_ = rng.standard_normal(W * S).astype(np.float32)
    gate = rng.standard_normal(W * S).astype(np.float32)
    mixed = oracle.hc_mix(norm_, gate, W, S)
    ref_compare(mixed, sum(norm_[c * W:(c + 1) * W] * f64.sigmoid(gate[c * W:(c + 1) * W].astype(np.float64))
                           for c in range(S)) / S)
    res = rng.standard_normal(W * S).astype(np.float32)
    out, inj = rng.standard_normal(W).astype(np.float32), rng.standard_normal(S).astype(np.float32)
    want = res + out[np.arange(W * S) % W] * 2 * f64.sigmoid(inj[np.arange(W * S) // W] / S)
    ref_compare(oracle.hc_write(res.copy(), out, inj, W, S), want)
    key, query = rng.standard_normal(W * S).astype(np.float32), rng.standard_normal(W * S).astype(np.float32)
    g = oracle.ple_gate(key, query, W, S)
    for c in range(S):
        sc = key[c * W:(c + 1) * W].astype(np.float64) @ query[c * W:(c + 1) * W] / math.sqrt(W)
        ref_compare([g[c]], [f64.sigmoid(np.sign(sc) * math.sqrt(max(abs(sc), 1e-6)))])
    alpha, beta = rng.standard_normal(4).astype(np.float32), rng.standard_normal(4).astype(np.float32)
    a, dt = (-0.1 - rng.random(4)).astype(np.float32), rng.standard_normal(4).astype(np.float32)
    alpha[0] = 25.0  # softplus passes values above 20 through
    decay, strength = oracle.gdn_gates(alpha, beta, a, dt, 4)
    sp = np.where(alpha + dt > 20, alpha.astype(np.float64) + dt, np.log1p(np.exp(alpha.astype(np.float64) + dt)))
    ref_compare(decay, np.exp(a * sp))
    ref_compare(strength, f64.sigmoid(beta.astype(np.float64)))
    full = rng.standard_normal(2 * 4 * 8).astype(np.float32)
    att = rng.standard_normal(4 * 8).astype(np.float32)
    i = np.arange(32)
    ref_compare(oracle.attention_gate(att, full, 8, 4), att * f64.sigmoid(full[(i // 8) * 16 + 8 + i % 8]))


def test_argmax_ties_and_slice(oracle):
    logits = np.zeros(130, np.float32)
    logits[[5, 69, 100]] = 3.0
    assert oracle.argmax(logits, 130) == 5  # ties go to the lowest index
    logits[129] = 4.0
    assert oracle.argmax(logits, 130) == 129
    x = np.arange(40, dtype=np.float32)
    assert np.array_equal(oracle.slice_(x, 3, 4, 10, 2), np.array([2, 3, 4, 12, 13, 14, 22, 23, 24, 32, 33, 34],
                                                                  np.float32))


def test_embedding_formats(oracle):
    W, S = 64, 2
    vals = np.linspace(-1, 1, W).astype(np.float32)
    res = np.zeros(W * S + 3, np.float32)
    oracle.embedding(res, W, S, values=vals, output_offset=3)
    assert np.array_equal(res[3:], np.tile(vals, S))
    # bf16: the upper halves of the f32 bit patterns.
    hi = (vals.view(np.uint32) >> 16).astype(np.uint32)
    codes = (hi[0::2] | (hi[1::2] << 16)).astype(np.uint32)
    res = np.zeros(W, np.float32)
    oracle.embedding(res, W, 1, codes=codes, fmt=1)
    assert np.array_equal(res.view(np.uint32), hi << 16)
    # S4 codes with bias -8 and per-16 scales plus offsets.
    c4 = np.arange(W) % 16
    words = np.zeros(W * 4 // 32, np.uint32)
    for i, c in enumerate(c4):
        words[i * 4 // 32] |= np.uint32(c << ((i * 4) % 32))
    sc = np.array([0.5, -0.25, 2.0, 1.0], np.float32)
    off = np.array([0.0, 1.0, -1.0, 0.5], np.float32)
    res = np.zeros(W, np.float32)
    oracle.embedding(res, W, 1, codes=words, scales=sc, offsets=off, fmt=2, bits=4, group_size=16, bias=-8,
                     has_offset=1)
    want = ((c4 - 8) * sc[np.arange(W) // 16]).astype(np.float32) + off[np.arange(W) // 16]
    assert np.array_equal(res, want.astype(np.float32))


def test_bf16_projection_is_lossless_compact_f32(oracle):
    # tests/conformance.js:101-107 "Lossless compact BF16 projections": f32
    # weights whose low 16 bits are zero project bit-identically from their
    # bf16 halves.
    rng = np.random.default_rng(11)
    cols, rows, tokens = 2560, 37, 3
    w = (rng.normal(0, 0.05, rows * cols).astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)
    x = rng.normal(0, 1, tokens * cols).astype(np.float32)
    hi = (w.view(np.uint32) >> 16).astype(np.uint32)
    codes = (hi[0::2] | (hi[1::2] << 16)).astype(np.uint32)
    got = oracle.bf16_project(x, codes, cols, rows, tokens, rows + 5, 2)
    want = oracle.project(x, w, cols, rows, tokens, rows + 5, 2)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quant_gemv_kat(oracle, bits):
    # tests/conformance.js:40-44: cols 64, rows 5, group 16, bias -3, signed
    # scales (i % 7 - 3) * 0.03, offsets i * 0.001, codes (i * 13 + 7) & mask.
    cols, rows, gs, mask = 64, 5, 16, (1 << bits) - 1
    codes = np.zeros((cols * rows * bits + 31) // 32, np.uint32)
    for i in range(cols * rows):
        bit = i * bits
        codes[bit >> 5] |= np.uint32(((i * 13 + 7) & mask) << (bit & 31))
    scales = ((np.arange(cols * rows // gs) % 7 - 3) * 0.03).astype(np.float32)
    offsets = (np.arange(cols * rows // gs) * 0.001).astype(np.float32)
    x = np.sin(np.arange(cols)).astype(np.float32)
    i = np.arange(rows * cols)
    wv = (((i * 13 + 7) & mask) - 3) * scales[i // gs].astype(np.float64) + offsets[i // gs]
    ref = wv.reshape(rows, cols) @ x.astype(np.float64)
    ref_compare(oracle.quant_gemv(x, codes, scales, offsets, cols, rows, bits, gs, -3, 0, 1), ref)


def test_ple_decode_iq4nl_blocks(oracle):
    # IQ4_NL blocks (18 bytes: fp16 scale + 16 bytes of 32 nibbles, low
    # nibbles first) at unaligned 18-byte strides with signed scales.
    rng = np.random.default_rng(3)
    blocks = 37
    raw = np.zeros(blocks * 18 + 2, np.uint8)
    scales = (rng.normal(0, 0.02, blocks)).astype(np.float16)
    nib = rng.integers(0, 16, (blocks, 32))
    for b in range(blocks):
        raw[b * 18:b * 18 + 2] = np.frombuffer(scales[b].tobytes(), np.uint8)
        raw[b * 18 + 2:b * 18 + 18] = (nib[b, :16] | (nib[b, 16:] << 4)).astype(np.uint8)
    packed = np.frombuffer(raw.tobytes(), np.uint32)
    iq4 = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
    want = (scales.astype(np.float32)[:, None] * iq4[nib]).reshape(-1)
    got = oracle.ple_decode(packed, blocks * 32)
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_partial_neox_rope_kat(oracle):
    # tests/conformance.js:67-68: x = sin(i) (24 values: 3 heads of 8), rotary
    # 4, cos/sin of 13 / 10000^(i/2), against pos 13, base 10000.
    x = np.sin(np.arange(24)).astype(np.float32)
    c = np.cos(13 / 10000 ** (np.arange(2) / 2)).astype(np.float32)
    s = np.sin(13 / 10000 ** (np.arange(2) / 2)).astype(np.float32)
    ref_compare(oracle.rope(x, c, s, 8, 3, 4), f64.rope(x.astype(np.float64), 8, 4, 13, 10000))
    assert np.array_equal(oracle.embed(x[:8], 8, 3), np.tile(x[:8], 3))


def test_prompt_batches_equal_token_steps():
    """Layer-major prompt batches (src/prefill.js) do each token's arithmetic
    exactly as a decode step does, only grouped differently, so every chunk
    size must give the step path's bits: the final logits and the state the
    next step reads (KV cache, GDN state, conv and PLE histories)."""
    from oracle import fixture as fx
    rng = np.random.default_rng(11)
    tokens = [int(t) for t in rng.integers(0, 40, 19)]
    ref = fx.OracleEngine(fx.create_fixture(1234))
    ref.step(3, predict=False)
    for t in tokens[:-1]:
        ref.step(t, predict=False)
    want_tok, want = ref.step(tokens[-1])
    after_tok, after = ref.step(9)
    for chunk in (1, 3, 7, 19):
        e = fx.OracleEngine(fx.create_fixture(1234))
        e.step(3, predict=False)
        tok, logits = fx.prefill(e, tokens, chunk_size=chunk)
        assert tok == want_tok
        assert np.array_equal(np.asarray(logits, np.float32).view(np.uint32), want.view(np.uint32)), chunk
        tok, logits = e.step(9)
        assert tok == after_tok
        assert np.array_equal(np.asarray(logits, np.float32).view(np.uint32), after.view(np.uint32)), chunk
