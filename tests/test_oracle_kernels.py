"""The oracle's kernel restatements against the reference's known-answer
recipes (tests/conformance.js, tests/fused-conformance.js, tests/model.test.mjs,
scripts/test-upstream.mjs), float64 equations (tests/reference.mjs) and brute
force. CPU only; every case finishes in well under a second."""
import os

import numpy as np
import pytest

import reference_f64 as f64
from conftest import ROOT, ref_compare, tol_ok


def q2_matrix(oracle, blob_u32, cols, rows, code_offset, scale_offset, weight_row=0, row_stride=1):
    """Dequantised rows extracted through strata_q2_project with one-hot inputs
    (adding exact zeros leaves each weight unchanged)."""
    X = np.eye(cols, dtype=np.float32).reshape(-1)
    Y = np.zeros(cols * rows, np.float32)
    oracle.q2_project(X, blob_u32, Y, cols, rows, cols, rows, 0, code_offset, scale_offset, weight_row, row_stride)
    return Y.reshape(cols, rows).T  # [rows, cols]


def test_q2_decode_matches_reference_dequantizer(oracle):
    # 256 Q2_0 blocks of the upstream KAT recipe (scripts/test-upstream.mjs:20),
    # laid out as 256 rows of 64 weights; compared bit for bit with the
    # reference's dequantize_q2_0 (dequant.hpp:68-78) output.
    golden = np.load(os.path.join(ROOT, "tests", "golden", "ref_dequant.npz"))["q2"]
    codes = np.zeros((256, 16), np.uint8)
    halves = np.zeros(256, np.uint16)
    for b in range(256):
        halves[b] = ((b % 16) + 8) * 1024 + (b * 7) % 1024 + (32768 if b % 2 else 0)
        codes[b] = [(i * 19 + b * 73) & 255 for i in range(16)]
    raw = np.concatenate([codes.reshape(-1), halves.view(np.uint8)])
    blob = np.frombuffer(raw.tobytes(), np.uint32).copy()
    M = q2_matrix(oracle, blob, 64, 256, 0, codes.size // 2)
    golden = golden.astype(np.float32)
    # Extraction by a dot product turns -0 into +0 (0 + -0 = +0); all other
    # values must match bit for bit.
    assert np.array_equal(M, golden)
    nz = golden != 0
    assert np.array_equal(M[nz].view(np.uint32), golden[nz].view(np.uint32))


def test_q2_gate_up_interleave_kat(oracle):
    # tests/model.test.mjs:32-50: gate/up codes bytes 0xe4, down 0x1b, scales 1.0.
    rows = cols = 64
    cb, sb = rows * cols // 4, rows * cols // 64 * 2
    raw = np.zeros(3 * (cb + sb), np.uint8)
    raw[:2 * cb] = 0xE4
    raw[2 * cb:3 * cb] = 0x1B
    raw[3 * cb:].view(np.uint16)[:] = 0x3C00
    blob = raw.view(np.uint32)
    gate = q2_matrix(oracle, blob, cols, 1, 0, 3 * cb // 2, weight_row=2 * 3, row_stride=2)
    up = q2_matrix(oracle, blob, cols, 1, 0, 3 * cb // 2, weight_row=2 * 3 + 1, row_stride=2)
    down = q2_matrix(oracle, blob, cols, 1, 2 * cb // 4, (3 * cb + 2 * sb) // 2, weight_row=3)
    assert list(gate[0, :8]) == [-1, 0, 1, 2, -1, 0, 1, 2]
    assert list(up[0, :8]) == [-1, 0, 1, 2, -1, 0, 1, 2]
    assert list(down[0, :4]) == [2, 1, 0, -1]


def fused_recipe():
    # tests/fused-conformance.js:3-18
    width, ff, tokens = 128, 64, 3
    cb, sb = width * ff // 4, width * ff // 64 * 2
    raw = np.zeros(3 * (cb + sb), np.uint8)
    raw[:3 * cb] = (np.arange(3 * cb) * 71 + 13) & 255
    i = np.arange(3 * sb // 2)
    raw[3 * cb:].view(np.uint16)[:] = 0x2800 + (i % 11) * 51 + np.where(i % 3 == 0, 32768, 0)
    x = (np.sin(np.arange(tokens * width) * .17) * .3).astype(np.float32)
    mapping = np.array([2, 4, 0, 1, 1, 3], np.int32)
    return width, ff, tokens, cb, sb, raw, x, mapping


def fused_expected(width, ff, tokens, cb, sb, raw, x, mapping):
    scales = f64.half_to_float(raw[3 * cb:].view(np.uint16))
    codes = f64.unpack_codes(raw[:3 * cb])

    def weight(index, down):
        off, soff = (2 * cb * 4 if down else 0), (2 * sb // 2 if down else 0)
        return (codes[off + index] - 1) * scales[soff + index // 64]

    hidden = np.zeros(tokens * ff)
    for t in range(tokens):
        xr = x[mapping[2 * t] * width:(mapping[2 * t] + 1) * width].astype(np.float64)
        for r in range(ff):
            g = sum(weight(2 * r * width + c, False) * xr[c] for c in range(width))
            u = sum(weight((2 * r + 1) * width + c, False) * xr[c] for c in range(width))
            hidden[t * ff + r] = g / (1 + np.exp(-g)) * u
    out = np.full(5 * width + 7, -99.0)
    for t in range(tokens):
        for r in range(width):
            out[7 + mapping[2 * t + 1] * width + r] = sum(weight(r * ff + c, True) * hidden[t * ff + c]
                                                          for c in range(ff))
    return hidden, out


def test_fused_q2_gate_up_down_kat(oracle):
    width, ff, tokens, cb, sb, raw, x, mapping = fused_recipe()
    hidden_ref, out_ref = fused_expected(width, ff, tokens, cb, sb, raw, x, mapping)
    blob = raw.view(np.uint32)
    hidden = oracle.q2_gate_up(x, blob, width, ff, tokens, mapping=mapping, scale_offset=3 * cb // 2)
    ref_compare(hidden, hidden_ref, 2e-5)
    out = np.full(out_ref.size, -99, np.float32)
    oracle.q2_down(hidden, blob, out, width, ff, tokens, mapping=mapping, output_offset=7, code_offset=2 * cb // 4,
                   scale_offset=(3 * cb + 2 * sb) // 2)
    ref_compare(out, out_ref, 2e-5)  # includes the untouched -99 padding
    # Expanded (f32) scales give bit-identical results (fused-conformance.js:19-22).
    scales = oracle.expert_scales(blob, 3 * cb // 2, 3 * sb // 2)
    hidden2 = oracle.q2_gate_up(x, blob, width, ff, tokens, mapping=mapping, scales=scales)
    assert np.array_equal(hidden.view(np.uint32), hidden2.view(np.uint32))
    out2 = np.full(out_ref.size, -99, np.float32)
    oracle.q2_down(hidden2, blob, out2, width, ff, tokens, mapping=mapping, scales=scales, output_offset=7,
                   code_offset=2 * cb // 4, scale_offset=sb)
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))


def test_q2_project_strided_kat(oracle):
    # tests/conformance.js:24-34: rows 65, cols 64, 3 tokens, signed scales,
    # output stride rows+7, offset 3.
    cols, rows, tokens = 64, 65, 3
    cb, sb = rows * cols // 4, rows * 2
    raw = np.zeros((3 * (cb + sb) + 3) // 4 * 4, np.uint8)
    raw[:3 * cb] = (np.arange(3 * cb) * 13 + 7) & 255
    i = np.arange(3 * rows)
    raw[3 * cb:3 * cb + 6 * rows].view(np.uint16)[:] = 0x3800 + (i % 6) * 64 + np.where(i % 3 == 0, 0x8000, 0)
    x = np.sin(np.arange(tokens * cols) * .23).astype(np.float32)
    blob = raw.view(np.uint32)
    codes = f64.unpack_codes(raw[:3 * cb])
    halves = f64.half_to_float(raw[3 * cb:3 * cb + 6 * rows].view(np.uint16))
    stride, off = rows + 7, 3
    for role in ("gate", "up", "down"):
        down = role == "down"
        code_offset, scale_offset = (2 * cb if down else 0) // 4, (3 * cb + (2 * sb if down else 0)) // 2
        weight_row, row_stride = (1 if role == "up" else 0), (1 if down else 2)
        ref = np.zeros(tokens * stride)
        for t in range(tokens):
            for r in range(rows):
                row = weight_row + r * row_stride
                scale = halves[scale_offset - 3 * cb // 2 + row]
                w = (codes[code_offset * 16 + row * cols:code_offset * 16 + (row + 1) * cols] - 1) * scale
                ref[t * stride + off + r] = w @ x[t * cols:(t + 1) * cols]
        out = np.zeros(tokens * stride, np.float32)
        oracle.q2_project(x, blob, out, cols, rows, tokens, stride, off, code_offset, scale_offset, weight_row,
                          row_stride)
        ref_compare(out, ref, 2e-5)


def test_router_ties_and_spread_kats(oracle):
    # tests/conformance.js:35-39 against the F64 router (tests/reference.mjs:173-177)
    for style in ("ties", "spread"):
        logits = np.full(512, 7, np.float32) if style == "ties" else (np.sin(np.arange(512) * 3.1) * 90).astype(
            np.float32)
        ids, w = oracle.router(logits, 512, 10)
        rids, rw, _ = f64.router(logits, 10)
        assert list(ids) == list(rids)
        ref_compare(w, rw, 2e-5)
        if style == "ties":
            assert list(ids) == list(range(10)) and np.allclose(w, 0.1)


def test_router_random_vs_f64_and_small_expert_counts(oracle):
    rng = np.random.default_rng(3)
    for experts, k in [(512, 10), (6, 2), (64, 32), (100, 7), (1, 1), (33, 33)]:
        for _ in range(20):
            logits = rng.normal(0, 1, experts).astype(np.float32)
            ids, w = oracle.router(logits, experts, k)
            rids, rw, p = f64.router(logits, k)
            srt = np.sort(p)[::-1]
            if k < experts and np.min(np.abs(np.diff(srt[:k + 1]))) < 1e-6:
                continue  # near tie: the f32 order is decided below F64 resolution
            assert list(ids) == list(rids)
            ref_compare(w, rw, 2e-5)
            assert len(set(ids)) == k and ids.min() >= 0 and ids.max() < experts


def test_project_2560_wide_kat(oracle):
    # tests/conformance.js:40-43 (strata_gemv)
    cols, rows = 2560, 37
    x = np.sin(np.arange(cols) * .73).astype(np.float32)
    w = (np.cos(np.arange(cols * rows) * .17) * .03).astype(np.float32)
    y = oracle.project(x, w, cols, rows, 1)
    ref_compare(y, w.astype(np.float64).reshape(rows, cols) @ x.astype(np.float64))


def test_quant_project_s248_kat(oracle):
    # tests/conformance.js:44-49
    for bits in (2, 4, 8):
        cols, rows, gs, mask = 64, 5, 16, (1 << bits) - 1
        codes = np.zeros((cols * rows * bits + 31) // 32, np.uint32)
        for i in range(cols * rows):
            codes[(i * bits) >> 5] |= np.uint32(((i * 13 + 7) & mask) << ((i * bits) & 31))
        scales = ((np.arange(cols * rows // gs) % 7 - 3) * .03).astype(np.float32)
        offsets = (np.arange(scales.size) * .001).astype(np.float32)
        x = np.sin(np.arange(cols)).astype(np.float32)
        ref = np.array([sum(x[c] * ((((r * cols + c) * 13 + 7) & mask) - 3) * scales[(r * cols + c) // gs] +
                            x[c] * offsets[(r * cols + c) // gs] for c in range(cols)) for r in range(rows)])
        out = np.zeros(rows, np.float32)
        oracle.quant_project(x, codes, scales, offsets, out, cols, rows, 1, rows, 0, bits, gs, -3, 0, 1)
        ref_compare(out, ref)


def test_norm_elementwise_combine_vs_f64(oracle):
    rng = np.random.default_rng(5)
    X = rng.normal(0, 2, 3 * 130).astype(np.float32)
    Wn = rng.normal(1, 0.1, 130).astype(np.float32)
    y = oracle.norm(X, Wn, 130, 3, 1, 0)
    Xd = X.astype(np.float64).reshape(3, 130)
    ref = Xd / np.sqrt((Xd ** 2).mean(axis=1, keepdims=True) + 1e-6) * Wn
    ref_compare(y, ref.reshape(-1))
    y1 = oracle.norm(X, Wn, 130, 3, 1, 1, scale=0.5)
    ref1 = Xd * 0.5 / np.sqrt((Xd ** 2).sum(axis=1, keepdims=True) + 1e-6)
    ref_compare(y1, ref1.reshape(-1))
    A, B = rng.normal(0, 3, 257).astype(np.float32), rng.normal(0, 3, 257).astype(np.float32)
    a, b = A.astype(np.float64) * 1.5, B.astype(np.float64)
    for mode, ref in [(0, a), (1, f64.silu(a)), (2, f64.sigmoid(a)), (3, f64.silu(a) * b), (4, a * f64.sigmoid(b)),
                      (5, a + b)]:
        ref_compare(oracle.elementwise(A, B, mode, 1.5), ref)
    T, K, Wd = 3, 4, 50
    parts = rng.normal(0, 1, T * K * Wd).astype(np.float32)
    wts = rng.random(T * K).astype(np.float32)
    shared = rng.normal(0, 1, T * Wd).astype(np.float32)
    gate = rng.normal(0, 1, T).astype(np.float32)
    y = oracle.moe_combine(parts, wts, shared, gate, Wd, K, T)
    ref = shared.reshape(T, Wd) * f64.sigmoid(gate.astype(np.float64))[:, None] + np.einsum(
        "tkd,tk->td", parts.reshape(T, K, Wd).astype(np.float64), wts.reshape(T, K).astype(np.float64))
    ref_compare(y, ref.reshape(-1))


def test_gather_scatter_rows(oracle):
    X = np.arange(5 * 8, dtype=np.float32)
    idx = np.array([4, 0, 2], np.int32)
    g = oracle.gather_rows(X, idx, 8, 3)
    assert np.array_equal(g.reshape(3, 8), X.reshape(5, 8)[idx])
    Y = np.full(5 * 8, -1, np.float32)
    oracle.scatter_rows(g, idx, Y, 8, 3)
    assert np.array_equal(Y.reshape(5, 8)[idx], X.reshape(5, 8)[idx]) and np.all(Y.reshape(5, 8)[[1, 3]] == -1)


def reference_grouping(ids, tokens, topk):
    """src/prefill.js:56-61: Map in first-appearance order over (t, k); each
    expert's jobs in ascending token order with part = t*topK + k."""
    groups = {}
    for t in range(tokens):
        for k in range(topk):
            groups.setdefault(int(ids[t * topk + k]), []).append((t, t * topk + k))
    return groups


@pytest.mark.parametrize("tokens,topk,experts", [(1, 10, 512), (5, 2, 6), (64, 10, 512), (65, 10, 512),
                                                 (300, 4, 16), (2048, 10, 512)])
def test_dispatch_vs_reference_grouping(oracle, tokens, topk, experts):
    rng = np.random.default_rng(tokens)
    p = rng.zipf(1.5, experts * 4).astype(np.float64)
    ids = np.stack([rng.choice(experts, topk, replace=False, p=None if t % 2 else np.bincount(
        np.minimum(p.astype(np.int64), experts) - 1, minlength=experts) / len(p)) for t in range(tokens)]).reshape(-1)
    offsets, rows, parts, where = oracle.dispatch(ids.astype(np.int32), tokens, topk, experts)
    groups = reference_grouping(ids, tokens, topk)
    assert offsets[-1] == tokens * topk
    for e in range(experts):
        seg = list(zip(rows[offsets[e]:offsets[e + 1]], parts[offsets[e]:offsets[e + 1]]))
        assert seg == groups.get(e, [])
    assert np.array_equal(np.sort(parts), np.arange(tokens * topk))
    assert np.array_equal(parts[where], np.arange(tokens * topk))


def small_layer(oracle, width=128, ff=64, experts=16, seed=11):
    from stratacuda_amd import workload as wl
    return wl.host_layer(oracle, 0, width=width, ff=ff, experts=experts, base_seed=seed)


@pytest.mark.parametrize("tokens,topk,bias", [(1, 4, False), (5, 4, False), (9, 3, True)])
def test_moe_layer_vs_f64(oracle, tokens, topk, bias):
    W, F, E = 128, 64, 16
    h = small_layer(oracle, W, F, E)
    X = oracle.synth_normal(tokens * W, h["seed"], 4, 1.0)
    b = (np.linspace(-1, 1, E) * 0.5).astype(np.float32) if bias else None
    Y, ids, w = oracle.moe_layer(X, tokens, h["Wr"], h["arena"], h["stride"], h["shared"], h["Wsg"], W, F, E, topk,
                                 bias=b)
    rY, rids, rw, gaps = f64.moe_layer(X, tokens, h["Wr"], h["arena"], h["stride"], h["shared"], h["Wsg"], W, F, E,
                                       topk, bias=b)
    assert np.all(gaps > 1e-6)
    assert np.array_equal(ids, rids)
    ref_compare(w, rw, 2e-5)
    assert tol_ok(Y, rY, 1e-5, 1e-5)


def test_moe_block_norm_residual(oracle):
    W, F, E, K, T = 128, 64, 16, 4, 3
    h = small_layer(oracle, W, F, E, seed=21)
    H = oracle.synth_normal(T * W, 99, 4, 1.0)
    Hout, ids, w = oracle.moe_block(H, T, h["gamma"], h["Wr"], h["arena"], h["stride"], h["shared"], h["Wsg"], W, F,
                                    E, K)
    Hd = H.astype(np.float64).reshape(T, W)
    xn = Hd / np.sqrt((Hd ** 2).mean(axis=1, keepdims=True) + 1e-6) * h["gamma"]
    rY, rids, _, _ = f64.moe_layer(xn.reshape(-1), T, h["Wr"], h["arena"], h["stride"], h["shared"], h["Wsg"], W, F,
                                   E, K)
    assert np.array_equal(ids, rids)
    assert tol_ok(Hout, Hd.reshape(-1) + rY, 1e-5, 1e-5)
