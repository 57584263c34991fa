"""The oracle against the reference's own threaded-WASM conformance run.

reports/wasm.json holds, for each check of tests/conformance.js (and the
fused-conformance.js checks it calls), the largest |WASM f32 result - F64
expected value| the reference measured. Each test here rebuilds a check's
inputs from the same recipe, computes the f32 result with the oracle and the
expected values with the reference's float64 equations in the reference's
operation order (tests/reference_js64.py), and requires the same largest
error: to 1e-13 where the reference's was non-zero (the double functions of
this platform and V8 differ in the last bits at most, while one f32 ulp at
the largest-error element would move the figure by ~1e-8), exactly where it
was zero. So at the worst element of every check the oracle's f32 value is
the WASM artifact's.
"""
import json
import math
import os

import numpy as np
import pytest

import reference_js64 as js
from conftest import REFERENCE

REPORT = os.path.join(REFERENCE, "reports", "wasm.json")
# The reported figures (reports/wasm.json "checks"), copied here so the tests
# also run where the reference tree is absent; test_report_figures checks them.
REPORTED = {
    "Fused Q2 gate/up/SiLU with reordered input rows": 1.0239313797885674e-09,
    "Fused Q2 down with sparse destinations and untouched padding": 5.309979834305922e-10,
    "CUDA-expanded expert scales preserve fused output": 5.309979834305922e-10,
    "CUDA S2 embedding decode and stream replication": 0.0,
    "CUDA S4 embedding decode and stream replication": 0.0,
    "CUDA S8 embedding decode and stream replication": 0.0,
    "CUDA IQ4_NL PLE decode with unaligned blocks and signed scales": 0.0,
    "CUDA RoPE trigonometry at position 0": 1.084339706913795e-07,
    "CUDA RoPE trigonometry at position 17": 1.1323454840450609e-07,
    "CUDA RoPE trigonometry at position 2045": 1.8010758318087738e-07,
    "Packed Q2 gate with strided prompt output": 4.709581844508648e-07,
    "Packed Q2 up with strided prompt output": 7.806374924257398e-07,
    "Packed Q2 down with strided prompt output": 7.806374924257398e-07,
    "router ties": 1.4901161138336505e-09,
    "router spread": 6.32118379861879e-09,
    "2560-wide projection": 5.479781449435617e-08,
    "S2 signed scales and offset plane": 4.8147357989414274e-08,
    "S4 signed scales and offset plane": 4.784743088404042e-07,
    "S8 signed scales and offset plane": 2.1148506377244303e-06,
    "GDN production state step 0": 1.2652152134133565e-09,
    "GDN production state step 1": 1.7083762477582143e-09,
    "GDN production state step 2": 2.081172082108243e-09,
    "GDN persistent state": 8.077114373172822e-09,
    "PLE dilated convolution and 12 history shifts": 0.0,
    "GQA attention selected cells": 1.705779532901186e-08,
    "GQA attention 70 dimensions and 65 cells": 3.007641314473064e-08,
    "GQA attention 256 dimensions and 2048 cells": 8.306236644675669e-09,
    "Partial NeoX RoPE": 5.5643095686619404e-08,
    "4-layer GDN + QSA + PLE + HC + MoE decode, 5 tokens": 3.313240437563536e-08,
    "Checkpoint restore replays logits": 0.0,
    "Reset clears recurrent, KV and PLE state": 1.8186727630820076e-08,
    "Prompt-only state updates preserve final logits": 2.7479434658306268e-08,
    "Batched prompt chunk 1 at nonzero position": 3.797034098251828e-08,
    "Decode after prompt chunk 1": 1.751358383317303e-08,
    "Batched prompt chunk 2 at nonzero position": 3.797034098251828e-08,
    "Decode after prompt chunk 2": 1.751358383317303e-08,
    "Batched prompt chunk 5 at nonzero position": 3.797034098251828e-08,
    "Decode after prompt chunk 5": 1.751358383317303e-08,
}
TOL = 1e-13


def max_err(actual, expected):
    a = np.asarray(actual, np.float32).astype(np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape and np.all(np.isfinite(a))
    return float(np.max(np.abs(a - e))) if a.size else 0.0


def check(name, err):
    want = REPORTED[name]
    assert abs(err - want) <= (0.0 if want == 0.0 else TOL), "%s: %r versus reported %r" % (name, err, want)


def f32(v):
    return np.asarray(v, np.float64).astype(np.float32)


def half_to_float(h):
    return float(np.array([h], np.uint16).view(np.float16)[0])


@pytest.mark.skipif(not os.path.exists(REPORT), reason="reference tree not present")
def test_report_figures():
    checks = {c["name"]: c["maxAbsoluteError"] for c in json.load(open(REPORT))["checks"]}
    for name, v in REPORTED.items():
        assert checks[name] == v, name


# ------------------------------------------------------- the MoE path's kernels
def test_fused_q2_gate_up_down(oracle):
    # tests/fused-conformance.js:4-22
    width, ff, tokens = 128, 64, 3
    cb, sb = width * ff // 4, width * ff // 64 * 2
    raw = np.zeros(3 * (cb + sb), np.uint8)
    raw[:3 * cb] = [(i * 71 + 13) & 255 for i in range(3 * cb)]
    halves = np.array([0x2800 + (i % 11) * 51 + (32768 if i % 3 == 0 else 0) for i in range(3 * sb // 2)], np.uint16)
    raw[3 * cb:] = halves.view(np.uint8)
    x = f32([math.sin(i * .17) * .3 for i in range(tokens * width)])
    mapping = np.array([2, 4, 0, 1, 1, 3], np.int32)

    def weight(index, down):
        off, soff = (2 * cb if down else 0), 3 * cb + (2 * sb if down else 0)
        code = (int(raw[off + (index >> 2)]) >> ((index % 4) * 2)) & 3
        h = int(raw[soff + 2 * (index // 64)]) | (int(raw[soff + 2 * (index // 64) + 1]) << 8)
        return (code - 1) * half_to_float(h)

    xd = [float(v) for v in x]
    hidden_ref = [0.0] * (tokens * ff)
    for t in range(tokens):
        for r in range(ff):
            gate = up = 0.0
            for c in range(width):
                gate = gate + weight(2 * r * width + c, False) * xd[mapping[2 * t] * width + c]
                up = up + weight((2 * r + 1) * width + c, False) * xd[mapping[2 * t] * width + c]
            hidden_ref[t * ff + r] = gate / (1 + math.exp(-gate)) * up
    ref = [-99.0] * (5 * width + 7)
    for t in range(tokens):
        for r in range(width):
            s = 0.0
            for c in range(ff):
                s = s + weight(r * ff + c, True) * hidden_ref[t * ff + c]
            ref[7 + mapping[2 * t + 1] * width + r] = s
    blob = raw.view(np.uint32)
    hidden = oracle.q2_gate_up(x, blob, width, ff, tokens, mapping=mapping, scale_offset=3 * cb // 2)
    check("Fused Q2 gate/up/SiLU with reordered input rows", max_err(hidden, hidden_ref))
    out = oracle.q2_down(hidden, blob, np.full(len(ref), -99, np.float32), width, ff, tokens, mapping=mapping,
                         output_offset=7, code_offset=2 * cb // 4, scale_offset=(3 * cb + 2 * sb) // 2)
    check("Fused Q2 down with sparse destinations and untouched padding", max_err(out, ref))
    scales = oracle.expert_scales(blob, 3 * cb // 2, 3 * sb // 2)
    hidden = oracle.q2_gate_up(x, blob, width, ff, tokens, mapping=mapping, scales=scales)
    out = oracle.q2_down(hidden, blob, np.full(len(ref), -99, np.float32), width, ff, tokens, mapping=mapping,
                         scales=scales, output_offset=7, code_offset=2 * cb // 4, scale_offset=sb)
    check("CUDA-expanded expert scales preserve fused output", max_err(out, ref))


def test_packed_q2_projections(oracle):
    # tests/conformance.js:22-34
    cols, rows, tokens = 64, 65, 3
    cb, sb = rows * cols // 4, rows * 2
    raw = np.zeros((3 * (cb + sb) + 3) // 4 * 4, np.uint8)
    raw[:3 * cb] = [(i * 13 + 7) & 255 for i in range(3 * cb)]
    halves = np.array([0x3800 + (i % 6) * 64 + (0x8000 if i % 3 == 0 else 0) for i in range(3 * rows)], np.uint16)
    raw[3 * cb:3 * cb + 6 * rows] = halves.view(np.uint8)
    x = f32([math.sin(i * .23) for i in range(tokens * cols)])
    xd = [float(v) for v in x]
    stride, off = rows + 7, 3
    for role in ("gate", "up", "down"):
        down = role == "down"
        code_off, scale_off = (2 * cb if down else 0) // 4, (3 * cb + (2 * sb if down else 0)) // 2
        weight_row, row_stride = (1 if role == "up" else 0), (1 if down else 2)
        ref = [0.0] * (tokens * stride)
        for t in range(tokens):
            for r in range(rows):
                row = weight_row + r * row_stride
                h = int(raw[(scale_off + row) * 2]) | (int(raw[(scale_off + row) * 2 + 1]) << 8)
                scale, s = half_to_float(h), 0.0
                for c in range(cols):
                    code = ((int(raw[code_off * 4 + row * cols // 4 + (c >> 2)]) >> ((c % 4) * 2)) & 3) - 1
                    s = s + xd[t * cols + c] * code * scale
                ref[t * stride + off + r] = s
        got = oracle.q2_project(x, raw.view(np.uint32), np.zeros(tokens * stride, np.float32), cols, rows, tokens,
                                stride, off, code_off, scale_off, weight_row, row_stride)
        check("Packed Q2 %s with strided prompt output" % role, max_err(got, ref))


@pytest.mark.parametrize("style", ["ties", "spread"])
def test_router(oracle, style):
    # tests/conformance.js:35-39
    logits = f32([7.0 if style == "ties" else math.sin(i * 3.1) * 90 for i in range(512)])
    ids, w = oracle.router(logits, 512, 10)
    rids, rw = js.router([float(v) for v in logits], 10)
    assert list(ids) == rids
    check("router " + style, max_err(w, rw))


def test_projection_2560_wide(oracle):
    # tests/conformance.js:41-43
    cols, rows = 2560, 37
    x = f32([math.sin(i * .73) for i in range(cols)])
    w = f32([math.cos(i * .17) * .03 for i in range(cols * rows)])
    xd, wd = [float(v) for v in x], [float(v) for v in w]
    expected = [js.dot(xd, wd[r * cols:(r + 1) * cols]) for r in range(rows)]
    check("2560-wide projection", max_err(oracle.project(x, w, cols, rows, 1), expected))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quant_gemv(oracle, bits):
    # tests/conformance.js:44-48
    cols, rows, gs, mask = 64, 5, 16, (1 << bits) - 1
    codes = np.zeros((cols * rows * bits + 31) // 32, np.uint32)
    for i in range(cols * rows):
        codes[(i * bits) >> 5] |= np.uint32(((i * 13 + 7) & mask) << ((i * bits) & 31))
    scales = f32([(i % 7 - 3) * .03 for i in range(cols * rows // gs)])
    offsets = f32([i * .001 for i in range(cols * rows // gs)])
    x = f32([math.sin(i) for i in range(cols)])
    ref = []
    for r in range(rows):
        s = 0.0
        for c in range(cols):
            i = r * cols + c
            s = s + float(x[c]) * ((((i * 13 + 7) & mask) - 3) * float(scales[i // gs]) + float(offsets[i // gs]))
        ref.append(s)
    got = oracle.quant_gemv(x, codes, scales, offsets, cols, rows, bits, gs, -3, 0, 1)
    check("S%d signed scales and offset plane" % bits, max_err(got, ref))


# ------------------------------------------------- the fixture model's kernels
def test_embedding_and_ple_decode(oracle):
    # tests/fused-conformance.js:24-40
    for bits in (2, 4, 8):
        width, streams, gs, mask, off = 96, 3, 16, (1 << bits) - 1, 5
        codes = np.zeros(width * bits // 32, np.uint32)
        for i in range(width):
            codes[(i * bits) // 32] |= np.uint32(((i * 7 + 3) & mask) << ((i * bits) % 32))
        scales = f32([(i - 2) * .03125 for i in range(width // gs)])
        offsets = f32([i * .125 for i in range(width // gs)])
        expected = [47.0] * (width * streams + off)
        for s in range(streams):
            for i in range(width):
                expected[off + s * width + i] = (((i * 7 + 3) & mask) - 3) * float(scales[i // gs]) + float(offsets[i // gs])
        got = oracle.embedding(np.full(len(expected), 47, np.float32), width, streams, codes=codes, scales=scales,
                               offsets=offsets, output_offset=off, fmt=2, bits=bits, group_size=gs, bias=-3,
                               has_offset=1)
        check("CUDA S%d embedding decode and stream replication" % bits, max_err(got, expected))
    blocks = 19
    raw = np.zeros((blocks * 18 + 3) // 4 * 4, np.uint8)
    iq4 = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    expected = []
    for b in range(blocks):
        half = 0x2000 + b * 61 + (32768 if b % 3 == 0 else 0)
        raw[b * 18:b * 18 + 2] = np.array([half], np.uint16).view(np.uint8)
        for i in range(16):
            raw[b * 18 + 2 + i] = (i * 23 + b * 13) & 255
        for i in range(32):
            expected.append(half_to_float(half) * iq4[(int(raw[b * 18 + 2 + i % 16]) >> (0 if i < 16 else 4)) & 15])
    check("CUDA IQ4_NL PLE decode with unaligned blocks and signed scales",
          max_err(oracle.ple_decode(raw.view(np.uint32), blocks * 32), expected))


@pytest.mark.parametrize("position", [0, 17, 2045])
def test_rope_trigonometry(oracle, position):
    # tests/fused-conformance.js:42-51: frequencies and table in the kernels'
    # f64 series and float sin / cos, against float64 pos / base^(2i/rotary).
    dim, heads, tokens, base = 96, 3, 3, 10000000
    rotary = 48 if position == 17 else 64
    x = f32([math.sin(i * .1) for i in range(dim * heads * tokens)])
    ref = [float(v) for v in x]
    for t in range(tokens):
        for h in range(heads):
            for i in range(rotary // 2):
                at = (t * heads + h) * dim + i
                angle = (position + t) / base ** (2 * i / rotary)
                c, s, a, bb = math.cos(angle), math.sin(angle), float(x[at]), float(x[at + rotary // 2])
                ref[at] = a * c - bb * s
                ref[at + rotary // 2] = bb * c + a * s
    hi, lo = oracle.rope_frequencies(rotary, base)
    cos, sin = oracle.rope_table(hi, lo, rotary, position + tokens)
    got = oracle.rope_position(x, cos, sin, dim, heads, rotary, position, tokens)
    check("CUDA RoPE trigonometry at position %d" % position, max_err(got, ref))


def test_gdn_production_state(oracle):
    # tests/conformance.js:50-55
    dim, kh, vh = 128, 16, 48
    state = np.zeros(dim * vh * dim, np.float32)
    ref_state = [0.0] * (dim * vh * dim)
    for step in range(3):
        q = f32([math.sin(i + step) * .04 for i in range(kh * dim)])
        k = f32([math.cos(i * .3 - step) * .04 for i in range(kh * dim)])
        v = f32([math.sin(i * .1 + step) for i in range(vh * dim)])
        d = f32([.9 + i * .001 for i in range(vh)])
        beta = f32([.6] * vh)
        ref = js.gdn(ref_state, *[[float(a) for a in arr] for arr in (q, k, v, d, beta)], dim, kh, vh)
        check("GDN production state step %d" % step, max_err(oracle.gdn_step(state, q, k, v, d, beta, dim, kh, vh),
                                                            ref))
    check("GDN persistent state", max_err(state, ref_state))


def test_ple_conv_history(oracle):
    # tests/conformance.js:56-58
    ch, taps, dil = 7, 4, 3
    hist, ref_hist = np.zeros(ch * 9, np.float32), [0.0] * (ch * 9)
    w = f32([math.cos(i) for i in range(ch * taps)])
    for step in range(12):
        x = f32([math.sin(i + step) for i in range(ch)])
        js.conv(ref_hist, [float(v) for v in x], [float(v) for v in w], taps, dil, True)
        oracle.conv(hist, x, w, ch, taps, dil, 1)
    check("PLE dilated convolution and 12 history shifts", max_err(hist, ref_hist))


@pytest.mark.parametrize("dim,count", [(8, 3), (70, 65), (256, 2048)])
def test_gqa_attention(oracle, dim, count):
    # tests/conformance.js:59-66
    heads, kvh = 4, 2
    if count == 3:
        q = f32([math.sin(i) for i in range(32)])
        keys = f32([math.cos(i * .13) for i in range(9 * 16)])
        values = f32([math.sin(i * .07) for i in range(9 * 16)])
        cells, name = [0, 3, 8], "GQA attention selected cells"
    else:
        q = f32([math.sin(i * .13) * .2 for i in range(heads * dim)])
        keys = f32([math.cos(i * .07) for i in range(count * kvh * dim)])
        values = f32([math.sin(i * .11) for i in range(count * kvh * dim)])
        cells, name = [count - 1 - i for i in range(count)], "GQA attention %d dimensions and %d cells" % (dim, count)
    got = oracle.attention(q, keys, values, np.array(cells, np.int32), dim, heads, kvh, len(cells),
                           np.float32(1 / math.sqrt(dim)))
    ref = js.attention([float(v) for v in q], [float(v) for v in keys], [float(v) for v in values], cells, dim,
                       heads, kvh)
    check(name, max_err(got, ref))


def test_partial_neox_rope(oracle):
    # tests/conformance.js:67-68
    x = f32([math.sin(i) for i in range(24)])
    c = f32([math.cos(13 / 10000 ** (i / 2)) for i in range(2)])
    s = f32([math.sin(13 / 10000 ** (i / 2)) for i in range(2)])
    got = oracle.rope(x, c, s, 8, 3, 4)
    check("Partial NeoX RoPE", max_err(got, js.rope([float(v) for v in x], 8, 4, 13, 10000)))


# ----------------------------------------------------- the whole fixture decode
@pytest.fixture(scope="module")
def fx(oracle):
    from oracle import fixture
    return fixture


@pytest.fixture(scope="module")
def model(fx):
    return fx.create_fixture(1234)


def test_fixture_decode_checks(fx, model):
    # tests/conformance.js:70-80
    e, r = fx.OracleEngine(model), js.ReferenceEngine(model, fx.ngram_rows)
    worst = 0.0
    for t in (2, 7, 4, 7, 4):
        tok, logits = e.step(t)
        rtok, rlogits = r.step(t)
        assert tok == rtok
        worst = max(worst, max_err(logits, rlogits))
    check("4-layer GDN + QSA + PLE + HC + MoE decode, 5 tokens", worst)
    state = {k: (v.copy() if hasattr(v, "copy") else v) for k, v in vars(e).items()}
    import copy
    snap = copy.deepcopy(e)
    _, first = e.step(8)
    _, replay = snap.step(8)
    check("Checkpoint restore replays logits", max_err(replay, first.astype(np.float64)))
    del state
    e = fx.OracleEngine(model)  # reset clears every persistent buffer
    _, again = e.step(2)
    check("Reset clears recurrent, KV and PLE state", max_err(again, js.ReferenceEngine(model, fx.ngram_rows).step(2)[1]))
    e, r = fx.OracleEngine(model), js.ReferenceEngine(model, fx.ngram_rows)
    for t in (2, 7):
        e.step(t, predict=False)
        r.step(t)
    tok, logits = e.step(4)
    rtok, rlogits = r.step(4)
    assert tok == rtok
    check("Prompt-only state updates preserve final logits", max_err(logits, rlogits))


@pytest.mark.parametrize("chunk", [1, 2, 5])
def test_fixture_prompt_chunks(fx, model, chunk):
    # tests/conformance.js:83-91: a batched prompt at a nonzero position, then
    # the next decode step, against token-by-token float64 decoding.
    e, r = fx.OracleEngine(model), js.ReferenceEngine(model, fx.ngram_rows)
    e.step(2, predict=False)
    r.step(2)
    for t in (7, 4, 8, 7, 4):
        wanted = r.step(t)
    _, logits = fx.prefill(e, [7, 4, 8, 7, 4], chunk_size=chunk)
    check("Batched prompt chunk %d at nonzero position" % chunk, max_err(logits, wanted[1]))
    _, nxt = e.step(8)
    check("Decode after prompt chunk %d" % chunk, max_err(nxt, r.step(8)[1]))
