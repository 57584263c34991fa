"""The fixture model's kernels outside the MoE path on the GPU (sm_run through
the C ABI) against the CPU oracle on identical inputs, bit for bit: every
kernel keeps the reference's f32 (and, for RoPE, f64) operation order and the
device logf / sin / cos are the oracle's. Inputs follow the reference's own
recipes (tests/conformance.js:45-69) at production sizes where it has them.
Invalid layouts are rejected before any launch."""
import math

import numpy as np
import pytest

import stratacuda_amd as sm

pytestmark = pytest.mark.gpu


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    assert a.shape == b.shape
    nan = np.isnan(b)
    assert np.array_equal(np.isnan(a), nan)
    assert np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan]), \
        "max |diff| %g" % np.max(np.abs(a.astype(np.float64) - b))


def grid(n):
    return [(n + 63) // 64, 1, 1]


def test_gdn_production_state_three_steps(backend, oracle):
    dim, kh, vh = 128, 16, 48
    state = np.zeros(dim * vh * dim, np.float32)
    sbuf = backend.alloc(state)
    y = backend.alloc(vh * dim)
    for step in range(3):
        i = np.arange(kh * dim)
        q = (np.sin(i + step) * 0.04).astype(np.float32)
        k = (np.cos(i * 0.3 - step) * 0.04).astype(np.float32)
        v = np.sin(np.arange(vh * dim) * 0.1 + step).astype(np.float32)
        d = (0.9 + np.arange(vh) * 0.001).astype(np.float32)
        beta = np.full(vh, 0.6, np.float32)
        backend.run("strata_gdn_step", {"State": sbuf, "Q": backend.alloc(q), "K": backend.alloc(k),
                                        "V": backend.alloc(v), "Decay": backend.alloc(d), "Beta": backend.alloc(beta),
                                        "Y": y, "dim": dim, "keyHeads": kh, "valueHeads": vh}, grid(vh * dim))
        same(backend.read(y), oracle.gdn_step(state, q, k, v, d, beta, dim, kh, vh))
    same(backend.read(sbuf), state)


def test_gdn_gates_and_conv(backend, oracle):
    rng = np.random.default_rng(3)
    heads = 48
    alpha, beta = rng.normal(0, 3, heads).astype(np.float32), rng.normal(0, 1, heads).astype(np.float32)
    alpha[:4] = [25.0, 19.9, -30.0, 0.0]  # both softplus branches and a large negative input
    a, dt = (-0.1 - rng.random(heads)).astype(np.float32), rng.normal(0, 1, heads).astype(np.float32)
    decay, strength = backend.alloc(heads), backend.alloc(heads)
    backend.run("strata_gdn_gates", {"Alpha": backend.alloc(alpha), "Beta": backend.alloc(beta),
                                     "A": backend.alloc(a), "Dt": backend.alloc(dt), "Decay": decay,
                                     "Strength": strength, "heads": heads}, grid(heads))
    want_d, want_s = oracle.gdn_gates(alpha, beta, a, dt, heads)
    same(backend.read(decay), want_d)
    same(backend.read(strength), want_s)
    # tests/conformance.js:51-53 and the fixture's GDN shape (4 taps, dilation 1).
    for ch, taps, dil in [(7, 4, 3), (64, 4, 1), (300, 4, 3)]:
        hist = np.zeros(ch * (taps - 1) * dil, np.float32)
        hb, wv = backend.alloc(hist), np.cos(np.arange(ch * taps)).astype(np.float32)
        wb, yb = backend.alloc(wv), backend.alloc(ch)
        for step in range(12):
            x = np.sin(np.arange(ch) + step).astype(np.float32)
            backend.run("strata_conv", {"History": hb, "X": backend.alloc(x), "W": wb, "Y": yb, "channels": ch,
                                        "taps": taps, "dilation": dil, "activation": step % 2}, grid(ch))
            same(backend.read(yb), oracle.conv(hist, x, wv, ch, taps, dil, step % 2))
        same(backend.read(hb), hist)


@pytest.mark.parametrize("dim,count,heads,kvh", [(8, 3, 4, 2), (70, 65, 4, 2), (256, 2048, 4, 2), (8, 32, 4, 2),
                                                 (128, 700, 24, 2)])
def test_attention(backend, oracle, dim, count, heads, kvh):
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
    scale = np.float32(1 / math.sqrt(dim))
    y = backend.alloc(np.full(heads * dim, -5, np.float32))
    backend.run("strata_attention", {"Q": backend.alloc(q), "Keys": backend.alloc(keys), "Values": backend.alloc(vals),
                                     "Cells": backend.alloc(cells, "i32"), "Y": y, "dim": dim, "heads": heads,
                                     "kvHeads": kvh, "count": len(cells), "scale": float(scale)},
                [heads, (dim + 63) // 64, 1])
    same(backend.read(y), oracle.attention(q, keys, vals, cells, dim, heads, kvh, len(cells), scale))


def test_attention_gate_ple_and_hc(backend, oracle):
    rng = np.random.default_rng(5)
    dim, heads = 8, 4
    att, full = rng.normal(0, 1, dim * heads).astype(np.float32), rng.normal(0, 2, 2 * dim * heads).astype(np.float32)
    y = backend.alloc(dim * heads)
    backend.run("strata_attention_gate", {"Attention": backend.alloc(att), "FullQ": backend.alloc(full), "Y": y,
                                          "dim": dim, "heads": heads}, grid(dim * heads))
    same(backend.read(y), oracle.attention_gate(att, full, dim, heads))
    for W, S in [(32, 2), (2560, 4)]:
        key, query = rng.normal(0, 1, W * S).astype(np.float32), rng.normal(0, 1, W * S).astype(np.float32)
        query[:W] = 0  # a zero dot product takes the sign-0 branch
        gate = backend.alloc(S)
        backend.run("strata_ple_gate", {"Key": backend.alloc(key), "Query": backend.alloc(query), "Gate": gate,
                                        "width": W, "streams": S}, [S, 1, 1])
        want_gate = oracle.ple_gate(key, query, W, S)
        same(backend.read(gate), want_gate)
        value = rng.normal(0, 1, W).astype(np.float32)
        out = backend.alloc(W * S)
        backend.run("strata_ple_broadcast", {"Value": backend.alloc(value), "Gate": gate, "Y": out, "width": W,
                                             "streams": S}, grid(W * S))
        same(backend.read(out), oracle.ple_broadcast(value, want_gate, W, S))
        res, conv = rng.normal(0, 1, W * S).astype(np.float32), rng.normal(0, 1, W * S).astype(np.float32)
        rb = backend.alloc(res)
        backend.run("strata_ple_add", {"Residual": rb, "Gated": out, "Conv": backend.alloc(conv), "n": W * S},
                    grid(W * S))
        same(backend.read(rb), oracle.ple_add(res.copy(), oracle.ple_broadcast(value, want_gate, W, S), conv, W * S))
        norm, g = rng.normal(0, 1, W * S).astype(np.float32), rng.normal(0, 3, W * S).astype(np.float32)
        mixed = backend.alloc(W)
        backend.run("strata_hc_mix", {"Norm": backend.alloc(norm), "Gate": backend.alloc(g), "Mixed": mixed,
                                      "width": W, "streams": S}, grid(W))
        same(backend.read(mixed), oracle.hc_mix(norm, g, W, S))
        inj = rng.normal(0, 1, S).astype(np.float32)
        rb = backend.alloc(res)
        backend.run("strata_hc_write", {"Residual": rb, "Output": mixed, "Inject": backend.alloc(inj), "width": W,
                                        "streams": S}, grid(W * S))
        same(backend.read(rb), oracle.hc_write(res.copy(), oracle.hc_mix(norm, g, W, S), inj, W, S))


@pytest.mark.parametrize("dim,rotary,heads,tokens", [(8, 8, 4, 1), (256, 64, 24, 1), (256, 64, 2, 3)])
def test_rope_tables_and_rotation(backend, oracle, dim, rotary, heads, tokens):
    base, context = 1e7, 2048
    hi, lo = backend.alloc(rotary // 2), backend.alloc(rotary // 2)
    backend.run("strata_rope_frequencies", {"High": hi, "Low": lo, "rotary": rotary, "base": base},
                grid(rotary // 2))
    whi, wlo = oracle.rope_frequencies(rotary, base)
    same(backend.read(hi), whi)
    same(backend.read(lo), wlo)
    n = context * rotary // 2
    cos, sin = backend.alloc(n), backend.alloc(n)
    backend.run("strata_rope_table", {"High": hi, "Low": lo, "Cos": cos, "Sin": sin, "rotary": rotary,
                                      "context": context}, grid(n))
    wcos, wsin = oracle.rope_table(whi, wlo, rotary, context)
    same(backend.read(cos), wcos)
    same(backend.read(sin), wsin)
    x = np.sin(np.arange(dim * heads * tokens) * 0.37).astype(np.float32)
    xb, y = backend.alloc(x), backend.alloc(dim * heads * tokens)
    for pos in (0, 1, 31, 1000, 2048 - tokens):
        backend.run("strata_rope_position", {"X": xb, "Cos": cos, "Sin": sin, "Y": y, "dim": dim, "heads": heads,
                                             "rotary": rotary, "position": pos, "tokens": tokens},
                    grid(dim * heads * tokens))
        same(backend.read(y), oracle.rope_position(x, wcos, wsin, dim, heads, rotary, pos, tokens))


def test_embedding_slice_kv_and_argmax(backend, oracle):
    rng = np.random.default_rng(9)
    W, S = 64, 2
    vals = rng.normal(0, 1, W).astype(np.float32)
    res = backend.alloc(np.zeros(W * S + 5, np.float32))
    dummy = backend.alloc(1)
    common = {"Codes": dummy, "Scales": dummy, "Offsets": dummy, "width": W, "streams": S, "outputOffset": 5,
              "bits": 0, "groupSize": 1, "bias": 0, "codebook": 0, "hasOffset": 0}
    backend.run("strata_embedding", dict(common, Values=backend.alloc(vals), Residual=res, format=0), grid(W))
    same(backend.read(res), oracle.embedding(np.zeros(W * S + 5, np.float32), W, S, values=vals, output_offset=5))
    # IQ4_NL codebook with offsets (format 2, codebook 1).
    codes = rng.integers(0, 2 ** 32, W * 4 // 32, dtype=np.uint64).astype(np.uint32)
    sc, off = rng.normal(0, 0.01, W // 16).astype(np.float32), rng.normal(0, 1, W // 16).astype(np.float32)
    res2 = backend.alloc(W)
    backend.run("strata_embedding", {"Values": dummy, "Codes": backend.alloc(codes, "u32"), "Scales": backend.alloc(sc),
                                     "Offsets": backend.alloc(off), "Residual": res2, "width": W, "streams": 1,
                                     "outputOffset": 0, "format": 2, "bits": 4, "groupSize": 16, "bias": 0,
                                     "codebook": 1, "hasOffset": 1}, grid(W))
    same(backend.read(res2), oracle.embedding(np.zeros(W, np.float32), W, 1, codes=codes, scales=sc, offsets=off,
                                              fmt=2, bits=4, group_size=16, codebook=1, has_offset=1))
    x = np.arange(100, dtype=np.float32)
    y = backend.alloc(12)
    backend.run("strata_slice", {"X": backend.alloc(x), "Y": y, "width": 3, "rows": 4, "stride": 10, "offset": 2},
                grid(12))
    same(backend.read(y), oracle.slice_(x, 3, 4, 10, 2))
    k, v = rng.normal(0, 1, 16).astype(np.float32), rng.normal(0, 1, 16).astype(np.float32)
    keys, values = backend.alloc(32 * 16), backend.alloc(32 * 16)
    backend.run("strata_kv_append", {"K": backend.alloc(k), "V": backend.alloc(v), "Keys": keys, "Values": values,
                                     "width": 16, "position": 31}, grid(16))
    same(backend.read(keys)[31 * 16:], k)
    same(backend.read(values)[31 * 16:], v)
    for count, ties in [(40, [3, 17]), (130, [5, 69, 100]), (248320, [7, 200000])]:
        logits = rng.normal(0, 1, count).astype(np.float32)
        logits[ties] = 50.0
        tok = backend.alloc(1, "i32")
        backend.run("strata_argmax", {"Logits": backend.alloc(logits), "Token": tok, "count": count}, [1, 1, 1])
        assert int(backend.read(tok)[0]) == oracle.argmax(logits, count) == ties[0]


def test_invalid_layouts_are_rejected(backend):
    cos, sin, x = backend.alloc(16), backend.alloc(16), backend.alloc(32)
    with pytest.raises(sm.StrataError) as e:  # rotary wider than the head
        backend.run("strata_rope_position", {"X": x, "Cos": cos, "Sin": sin, "Y": backend.alloc(32), "dim": 8,
                                             "heads": 4, "rotary": 10, "position": 0, "tokens": 1}, [1, 1, 1])
    assert e.value.code == -2
    with pytest.raises(sm.StrataError) as e:  # table too short for the position
        backend.run("strata_rope_position", {"X": x, "Cos": cos, "Sin": sin, "Y": backend.alloc(32), "dim": 8,
                                             "heads": 4, "rotary": 8, "position": 4, "tokens": 1}, [1, 1, 1])
    assert e.value.code == -2
    q, kv = backend.alloc(32), backend.alloc(3 * 16)
    with pytest.raises(sm.StrataError) as e:  # heads not a multiple of kvHeads
        backend.run("strata_attention", {"Q": q, "Keys": kv, "Values": kv, "Cells": backend.alloc(np.zeros(1, np.int32), "i32"),
                                         "Y": backend.alloc(32), "dim": 8, "heads": 3, "kvHeads": 2, "count": 1,
                                         "scale": 1.0}, [3, 1, 1])
    assert e.value.code == -2
    with pytest.raises(sm.StrataError) as e:  # a cell beyond the three cached positions
        backend.run("strata_attention", {"Q": q, "Keys": kv, "Values": kv,
                                         "Cells": backend.alloc(np.array([0, 3], np.int32), "i32"),
                                         "Y": backend.alloc(32), "dim": 8, "heads": 4, "kvHeads": 2, "count": 2,
                                         "scale": 1.0}, [4, 1, 1])
    assert e.value.code == -3
    with pytest.raises(sm.StrataError) as e:  # residual too short for the streams
        d = backend.alloc(1)
        backend.run("strata_embedding", {"Values": backend.alloc(64), "Codes": d, "Scales": d, "Offsets": d,
                                         "Residual": backend.alloc(100), "width": 64, "streams": 2, "outputOffset": 0,
                                         "format": 0, "bits": 0, "groupSize": 1, "bias": 0, "codebook": 0,
                                         "hasOffset": 0}, [1, 1, 1])
    assert e.value.code == -2
    with pytest.raises(sm.StrataError) as e:  # history shorter than channels x span
        backend.run("strata_conv", {"History": backend.alloc(10), "X": backend.alloc(7), "W": backend.alloc(28),
                                    "Y": backend.alloc(7), "channels": 7, "taps": 4, "dilation": 3, "activation": 1},
                    [1, 1, 1])
    assert e.value.code == -3


def test_bf16_project_quant_gemv_ple_decode_embed_rope(backend, oracle):
    rng = np.random.default_rng(21)
    # bf16 projection with a strided, offset batch output
    cols, rows, tokens, stride, off = 2560, 37, 3, 45, 4
    w = rng.normal(0, 0.05, rows * cols).astype(np.float32)
    hi = (w.view(np.uint32) >> 16).astype(np.uint32)
    codes = (hi[0::2] | (hi[1::2] << 16)).astype(np.uint32)
    x = rng.normal(0, 1, tokens * cols).astype(np.float32)
    y = backend.alloc(np.full(tokens * stride, -3, np.float32))
    backend.run("strata_bf16_project", {"X": backend.alloc(x), "Codes": backend.alloc(codes, "u32"), "Y": y,
                                        "cols": cols, "rows": rows, "tokens": tokens, "outputStride": stride,
                                        "outputOffset": off}, [rows, tokens, 1])
    same(backend.read(y), oracle.bf16_project(x, codes, cols, rows, tokens, stride, off,
                                              Y=np.full(tokens * stride, -3, np.float32)))
    # S2 / S4 / S8 GEMV (tests/conformance.js:40-44 recipe)
    for bits in (2, 4, 8):
        cols, rows, gs, mask = 64, 5, 16, (1 << bits) - 1
        cw = np.zeros((cols * rows * bits + 31) // 32, np.uint32)
        for i in range(cols * rows):
            cw[(i * bits) >> 5] |= np.uint32(((i * 13 + 7) & mask) << ((i * bits) & 31))
        sc = ((np.arange(cols * rows // gs) % 7 - 3) * 0.03).astype(np.float32)
        of = (np.arange(cols * rows // gs) * 0.001).astype(np.float32)
        xv = np.sin(np.arange(cols)).astype(np.float32)
        out = backend.alloc(rows)
        backend.run("strata_quant_gemv", {"X": backend.alloc(xv), "Codes": backend.alloc(cw, "u32"),
                                          "Scales": backend.alloc(sc), "Offsets": backend.alloc(of), "Y": out,
                                          "cols": cols, "rows": rows, "bits": bits, "groupSize": gs, "bias": -3,
                                          "codebook": 0, "hasOffset": 1}, [rows, 1, 1])
        same(backend.read(out), oracle.quant_gemv(xv, cw, sc, of, cols, rows, bits, gs, -3, 0, 1))
    # IQ4_NL PLE rows: 2560 values (80 blocks of 18 bytes)
    raw = rng.integers(0, 256, 80 * 18, dtype=np.uint8)
    for b in range(80):
        raw[b * 18:b * 18 + 2] = np.frombuffer(np.float16(rng.normal(0, 0.02)).tobytes(), np.uint8)
    packed = np.frombuffer(raw.tobytes(), np.uint32).copy()
    vals = backend.alloc(2560)
    backend.run("strata_ple_decode", {"Packed": backend.alloc(packed, "u32"), "Values": vals, "count": 2560},
                grid(2560))
    same(backend.read(vals), oracle.ple_decode(packed, 2560))
    # row broadcast and rotation with supplied cos / sin
    row = rng.normal(0, 1, 64).astype(np.float32)
    res = backend.alloc(256)
    backend.run("strata_embed", {"Row": backend.alloc(row), "Residual": res, "width": 64, "streams": 4}, grid(256))
    same(backend.read(res), oracle.embed(row, 64, 4))
    xr = np.sin(np.arange(24)).astype(np.float32)
    c = np.cos(13 / 10000 ** (np.arange(2) / 2)).astype(np.float32)
    s = np.sin(13 / 10000 ** (np.arange(2) / 2)).astype(np.float32)
    yr = backend.alloc(24)
    backend.run("strata_rope", {"X": backend.alloc(xr), "Cos": backend.alloc(c), "Sin": backend.alloc(s), "Y": yr,
                                "dim": 8, "heads": 3, "rotary": 4}, [1, 1, 1])
    same(backend.read(yr), oracle.rope(xr, c, s, 8, 3, 4))
    with pytest.raises(sm.StrataError):  # count not a whole number of blocks
        backend.run("strata_ple_decode", {"Packed": backend.alloc(packed, "u32"), "Values": vals, "count": 100},
                    grid(100))


@pytest.mark.parametrize("cols,rows,tokens", [(512, 9, 1), (4096, 5, 2), (300, 7, 2), (4608, 3, 1), (2560, 70, 1),
                                               (4096, 17, 1)])
def test_bf16_project_shapes(backend, oracle, cols, rows, tokens):
    """Row widths that are and are not whole 512-value (eight-load) batches,
    one and two tokens, rows staged in LDS (one token, cols % 64 == 0, up
    to 4096) and not: the reference's bits in every case."""
    rng = np.random.default_rng(cols)
    w = rng.normal(0, 0.05, rows * cols + 1).astype(np.float32)
    hi = (w.view(np.uint32) >> 16).astype(np.uint32)
    codes = (hi[0:-1:2] | (hi[1::2] << 16)).astype(np.uint32)
    x = rng.normal(0, 1, tokens * cols).astype(np.float32)
    y = backend.alloc(tokens * rows)
    backend.run("strata_bf16_project", {"X": backend.alloc(x), "Codes": backend.alloc(codes, "u32"), "Y": y,
                                        "cols": cols, "rows": rows, "tokens": tokens, "outputStride": rows,
                                        "outputOffset": 0}, [rows, tokens, 1])
    same(backend.read(y), oracle.bf16_project(x, codes, cols, rows, tokens, rows, 0,
                                              Y=np.zeros(tokens * rows, np.float32)))


@pytest.mark.parametrize("cols,bits,gs,has_offset,codebook,rows",
                         [(2560, 4, 32, 1, 0, 11), (2560, 8, 64, 0, 0, 11), (4096, 8, 16, 1, 0, 11),
                          (96, 2, 32, 1, 0, 11), (4096, 2, 8, 0, 0, 11), (336, 4, 48, 1, 0, 11),
                          (2560, 2, 128, 1, 0, 37), (1024, 4, 64, 1, 1, 53), (2560, 4, 32, 0, 1, 16)])
def test_quant_gemv_shapes(backend, oracle, cols, bits, gs, has_offset, codebook, rows):
    """S2 / S4 / S8 rows of 96 to 4096 values, groups of 8 to 128, with and
    without offsets, the IQ4 codebook, rows staged in LDS (cols % 64 == 0,
    whole 16-byte code chunks, power-of-two groups, at most 256 per row) and
    not: the reference's bits in every case."""
    rng = np.random.default_rng(cols * bits + gs)
    cw = rng.integers(0, 2 ** 32, (cols * rows * bits + 31) // 32, dtype=np.uint64).astype(np.uint32)
    sc = rng.normal(0, 0.03, cols * rows // gs).astype(np.float32)
    of = rng.normal(0, 0.01, cols * rows // gs).astype(np.float32)
    xv = rng.normal(0, 1, cols).astype(np.float32)
    out = backend.alloc(rows)
    bias = -(1 << (bits - 1))
    backend.run("strata_quant_gemv", {"X": backend.alloc(xv), "Codes": backend.alloc(cw, "u32"),
                                      "Scales": backend.alloc(sc), "Offsets": backend.alloc(of), "Y": out,
                                      "cols": cols, "rows": rows, "bits": bits, "groupSize": gs, "bias": bias,
                                      "codebook": codebook, "hasOffset": has_offset}, [rows, 1, 1])
    same(backend.read(out), oracle.quant_gemv(xv, cw, sc, of, cols, rows, bits, gs, bias, codebook, has_offset))
