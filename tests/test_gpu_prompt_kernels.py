"""The prompt (layer-major batch) kernels of kernels/strata.cu on the GPU (sm_run
through the C ABI) against the CPU oracle on identical inputs, bit for bit:
each batch kernel runs tokens x the single-token work in token order, so the
recurrent state (conv history, GDN state), the KV cache and the outputs must
equal the oracle's restatement of the reference's loops exactly. Sizes cover
the fixture model and the production shapes (GDN 128 x 16/48 heads, attention
over 2048 cells, HC over 4 streams of 2048)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    assert a.shape == b.shape
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
        "max |diff| %g" % np.max(np.abs(a.astype(np.float64) - b))


def grid(n):
    return [(n + 63) // 64, 1, 1]


@pytest.mark.parametrize("width,streams,tokens", [(32, 4, 5), (2048, 4, 16)])
def test_embed_hc_and_ple_broadcast(backend, oracle, width, streams, tokens):
    rng = np.random.default_rng(width + tokens)
    hc = width * streams
    rows = rng.normal(0, 1, width * tokens).astype(np.float32)
    res = backend.alloc(hc * tokens)
    backend.run("strata_embed_batch", {"Rows": backend.alloc(rows), "Residual": res, "width": width,
                                       "streams": streams, "tokens": tokens}, grid(hc * tokens))
    same(backend.read(res), oracle.embed_batch(rows, width, streams, tokens))
    norm = rng.normal(0, 1, hc * tokens).astype(np.float32)
    gate = rng.normal(0, 2, hc * tokens).astype(np.float32)
    mixed = backend.alloc(width * tokens)
    backend.run("strata_hc_mix_batch", {"Norm": backend.alloc(norm), "Gate": backend.alloc(gate), "Mixed": mixed,
                                        "width": width, "streams": streams, "tokens": tokens}, grid(width * tokens))
    same(backend.read(mixed), oracle.hc_mix_batch(norm, gate, width, streams, tokens))
    residual = rng.normal(0, 1, hc * tokens).astype(np.float32)
    output = rng.normal(0, 1, width * tokens).astype(np.float32)
    inject = rng.normal(0, 3, streams * tokens).astype(np.float32)
    rb = backend.alloc(residual)
    backend.run("strata_hc_write_batch", {"Residual": rb, "Output": backend.alloc(output),
                                          "Inject": backend.alloc(inject), "width": width, "streams": streams,
                                          "tokens": tokens}, grid(hc * tokens))
    same(backend.read(rb), oracle.hc_write_batch(residual.copy(), output, inject, width, streams, tokens))
    value = rng.normal(0, 1, width * tokens).astype(np.float32)
    g = rng.random(streams * tokens).astype(np.float32)
    y = backend.alloc(hc * tokens)
    backend.run("strata_ple_broadcast_batch", {"Value": backend.alloc(value), "Gate": backend.alloc(g), "Y": y,
                                               "width": width, "streams": streams, "tokens": tokens},
                grid(hc * tokens))
    same(backend.read(y), oracle.ple_broadcast_batch(value, g, width, streams, tokens))


@pytest.mark.parametrize("channels,taps,dilation,tokens", [(7, 4, 3, 5), (64, 4, 1, 2), (8192, 4, 1, 16),
                                                           (300, 4, 3, 9), (12, 1, 1, 3)])
def test_conv_batch_state_across_chunks(backend, oracle, channels, taps, dilation, tokens):
    """Two chunks in a row: the history the first leaves is the second's."""
    span = (taps - 1) * dilation
    hist = np.zeros(max(channels * span, 1), np.float32)
    hb = backend.alloc(hist)
    w = np.cos(np.arange(channels * taps) * 0.7).astype(np.float32)
    wb, yb = backend.alloc(w), backend.alloc(channels * tokens)
    for chunk in range(2):
        x = np.sin(np.arange(channels * tokens) * 0.37 + chunk).astype(np.float32)
        act = chunk % 2
        backend.run("strata_conv_batch", {"History": hb, "X": backend.alloc(x), "W": wb, "Y": yb,
                                          "channels": channels, "taps": taps, "dilation": dilation,
                                          "activation": act, "tokens": tokens}, grid(channels))
        same(backend.read(yb), oracle.conv_batch(hist, x, w, channels, taps, dilation, act, tokens))
        same(backend.read(hb), hist)


@pytest.mark.parametrize("dim,kh,vh,tokens", [(8, 2, 4, 5), (128, 16, 48, 4), (128, 16, 48, 21), (64, 2, 6, 3)])
def test_gdn_gates_and_gdn_batch(backend, oracle, dim, kh, vh, tokens):
    rng = np.random.default_rng(dim * tokens)
    alpha = rng.normal(0, 3, vh * tokens).astype(np.float32)
    alpha[:3] = [25.0, -30.0, 0.0]
    beta_in = rng.normal(0, 1, vh * tokens).astype(np.float32)
    a = (-0.1 - rng.random(vh)).astype(np.float32)
    dt = rng.normal(0, 1, vh).astype(np.float32)
    decay, strength = backend.alloc(vh * tokens), backend.alloc(vh * tokens)
    backend.run("strata_gdn_gates_batch", {"Alpha": backend.alloc(alpha), "Beta": backend.alloc(beta_in),
                                           "A": backend.alloc(a), "Dt": backend.alloc(dt), "Decay": decay,
                                           "Strength": strength, "heads": vh, "tokens": tokens}, grid(vh * tokens))
    want_d, want_s = oracle.gdn_gates_batch(alpha, beta_in, a, dt, vh, tokens)
    same(backend.read(decay), want_d)
    same(backend.read(strength), want_s)
    state = (rng.normal(0, 0.1, dim * vh * dim)).astype(np.float32)
    sb, y = backend.alloc(state), backend.alloc(vh * dim * tokens)
    for chunk in range(2):
        q = (rng.normal(0, 1, kh * dim * tokens) / np.sqrt(dim)).astype(np.float32)
        k = (rng.normal(0, 1, kh * dim * tokens) / np.sqrt(dim)).astype(np.float32)
        v = rng.normal(0, 1, vh * dim * tokens).astype(np.float32)
        backend.run("strata_gdn_batch", {"State": sb, "Q": backend.alloc(q), "K": backend.alloc(k),
                                         "V": backend.alloc(v), "Decay": decay, "Beta": strength, "Y": y,
                                         "dim": dim, "keyHeads": kh, "valueHeads": vh, "tokens": tokens},
                    grid(vh * dim))
        same(backend.read(y), oracle.gdn_batch(state, q, k, v, want_d, want_s, dim, kh, vh, tokens))
        same(backend.read(sb), state)


@pytest.mark.parametrize("dim,kh,vh,tokens,alias", [(160, 2, 4, 3, False), (16, 2, 4, 3, True),
                                                    (160, 2, 3, 5, True)])
def test_gdn_batch_general_kernel(backend, oracle, dim, kh, vh, tokens, alias):
    # The kernel for a state column longer than 128 values, or a State that
    # another argument aliases (here Y: each thread's token outputs overwrite
    # rows of its own column, as in the reference's loop), bit-exact with the
    # oracle over two chunks.
    rng = np.random.default_rng(dim + 7 * tokens + alias)
    decay = (0.9 + 0.1 * rng.random(vh * tokens)).astype(np.float32)
    strength = rng.random(vh * tokens).astype(np.float32)
    state = rng.normal(0, 0.1, dim * vh * dim).astype(np.float32)
    sb = backend.alloc(state)
    y = sb if alias else backend.alloc(vh * dim * tokens)
    db, stb = backend.alloc(decay), backend.alloc(strength)
    for chunk in range(2):
        q = (rng.normal(0, 1, kh * dim * tokens) / np.sqrt(dim)).astype(np.float32)
        k = (rng.normal(0, 1, kh * dim * tokens) / np.sqrt(dim)).astype(np.float32)
        v = rng.normal(0, 1, vh * dim * tokens).astype(np.float32)
        backend.run("strata_gdn_batch", {"State": sb, "Q": backend.alloc(q), "K": backend.alloc(k),
                                         "V": backend.alloc(v), "Decay": db, "Beta": stb, "Y": y,
                                         "dim": dim, "keyHeads": kh, "valueHeads": vh, "tokens": tokens},
                    grid(vh * dim))
        if alias:
            # the oracle's loop with Y = State, as the GPU call had it
            oracle.lib().or_gdn_batch(state, q, k, v, decay, strength, state, dim, kh, vh, tokens)
        else:
            same(backend.read(y), oracle.gdn_batch(state, q, k, v, decay, strength, dim, kh, vh, tokens))
        same(backend.read(sb), state)


@pytest.mark.parametrize("dim,rotary,heads,tokens", [(8, 8, 4, 3), (256, 64, 24, 5)])
def test_rope_batch(backend, oracle, dim, rotary, heads, tokens):
    rng = np.random.default_rng(dim)
    x = rng.normal(0, 1, dim * heads * tokens).astype(np.float32)
    ang = np.arange(tokens * rotary // 2, dtype=np.float64) * 0.173
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = backend.alloc(x.size)
    backend.run("strata_rope_batch", {"X": backend.alloc(x), "Cos": backend.alloc(cos), "Sin": backend.alloc(sin),
                                      "Y": y, "dim": dim, "heads": heads, "rotary": rotary, "tokens": tokens},
                grid(x.size))
    same(backend.read(y), oracle.rope_batch(x, cos, sin, dim, heads, rotary, tokens))


@pytest.mark.parametrize("dim,heads,kvh,position,tokens", [(8, 4, 2, 1, 5), (70, 4, 2, 60, 7), (256, 24, 2, 0, 16),
                                                           (256, 24, 2, 2032, 16), (128, 4, 4, 100, 64),
                                                           (64, 12, 2, 500, 20)])
def test_kv_append_attention_and_gate_batch(backend, oracle, dim, heads, kvh, position, tokens):
    rng = np.random.default_rng(position + tokens)
    width, cells = kvh * dim, position + tokens
    keys = np.zeros(cells * width, np.float32)
    values = np.zeros(cells * width, np.float32)
    keys[:position * width] = rng.normal(0, 1, position * width)
    values[:position * width] = rng.normal(0, 1, position * width)
    kb, vb = backend.alloc(keys), backend.alloc(values)
    k = rng.normal(0, 1, width * tokens).astype(np.float32)
    v = rng.normal(0, 1, width * tokens).astype(np.float32)
    backend.run("strata_kv_append_batch", {"K": backend.alloc(k), "V": backend.alloc(v), "Keys": kb, "Values": vb,
                                           "width": width, "position": position, "tokens": tokens},
                grid(width * tokens))
    oracle.kv_append_batch(k, v, keys, values, width, position, tokens)
    same(backend.read(kb), keys)
    same(backend.read(vb), values)
    q = rng.normal(0, 1, heads * dim * tokens).astype(np.float32)
    scale = 1 / np.sqrt(dim)
    att = backend.alloc(q.size)
    backend.run("strata_attention_batch", {"Q": backend.alloc(q), "Keys": kb, "Values": vb, "Y": att, "dim": dim,
                                           "heads": heads, "kvHeads": kvh, "position": position, "scale": scale},
                [heads, (dim + 63) // 64, tokens])
    want = oracle.attention_batch(q, keys, values, dim, heads, kvh, position, scale, tokens)
    same(backend.read(att), want)
    full = rng.normal(0, 2, 2 * heads * dim * tokens).astype(np.float32)
    gated = backend.alloc(q.size)
    backend.run("strata_attention_gate_batch", {"Attention": att, "FullQ": backend.alloc(full), "Y": gated,
                                                "dim": dim, "heads": heads, "tokens": tokens}, grid(q.size))
    same(backend.read(gated), oracle.attention_gate_batch(want, full, dim, heads, tokens))


def test_batch_attention_rejects_overflowing_prompt(backend):
    dim, heads, kvh = 8, 4, 2
    kb, vb = backend.alloc(2048 * kvh * dim), backend.alloc(2048 * kvh * dim)
    q, y = backend.alloc(3 * heads * dim), backend.alloc(3 * heads * dim)
    with pytest.raises(Exception, match="2048 cells"):
        backend.run("strata_attention_batch", {"Q": q, "Keys": kb, "Values": vb, "Y": y, "dim": dim, "heads": heads,
                                               "kvHeads": kvh, "position": 2046, "scale": 0.3}, [heads, 1, 3])
    with pytest.raises(Exception, match="tokens"):
        backend.run("strata_conv_batch", {"History": kb, "X": q, "W": kb, "Y": y, "channels": 4, "taps": 4,
                                          "dilation": 1, "activation": 1, "tokens": 0}, [1, 1, 1])
