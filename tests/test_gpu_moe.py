"""The fused MoE path on the GPU (sm_moe_route / sm_moe_dispatch /
sm_moe_layer through the C ABI) against the CPU oracle on identical seeded
inputs: routed expert IDs, their order and the dispatch permutation
bit-exact; layer outputs within |a - e| <= 1e-4 + 1e-3 |e|.

Full-size cases (2048 hidden, 512 experts, top-10 + shared, Q2) compare every
token's routing and every token's output. Batches of 512 tokens or more
route with the certified router (approximate logits on MFMA with an error
bound, exact logits near the top-k boundary): their IDs and order are
bit-exact and their routing weights within 1e-6 relative; smaller batches
use the exact router, whose weights are bit-exact too."""
import numpy as np
import pytest

import stratacuda_amd as sm
from conftest import CERTIFIED_MIN_TOKENS, tol_ok, weights_close, weights_ok
from stratacuda_amd import workload as wl

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def full_layer(backend):
    layer = wl.DeviceLayer(backend, layer=0)
    yield layer
    layer.free()


@pytest.fixture(scope="module")
def small(backend, oracle):
    W, F, E = 128, 64, 16
    layer = wl.DeviceLayer(backend, layer=0, width=W, ff=F, experts=E, base_seed=11)
    host = wl.host_layer(oracle, 0, width=W, ff=F, experts=E, base_seed=11)
    yield layer, host
    layer.free()


def test_synth_matches_oracle(backend, oracle, small, full_layer):
    layer, host = small
    assert np.array_equal(backend.read_bytes(layer.arena), host["arena"])
    assert np.array_equal(backend.read_bytes(layer.shared), host["shared"])
    assert same_bits(backend.read(layer.Wr), host["Wr"])
    assert same_bits(backend.read(layer.Wsg), host["Wsg"])
    assert same_bits(backend.read(layer.gamma), host["gamma"])
    e = 417
    got = backend.read_bytes(full_layer.arena, wl.blob_bytes(), e * full_layer.stride)
    assert np.array_equal(got, oracle.synth_blob(wl.WIDTH, wl.FF, full_layer.seed, wl.STREAM_BLOB0 + e, 0.05))


def device_inputs(backend, tokens, width, seed, normalise):
    X = backend.alloc(tokens * width, "f32", zero=False)
    backend.synth_normal(X, tokens * width, seed, wl.STREAM_INPUT, 1.0)
    if not normalise:
        return X
    Xn = backend.alloc(tokens * width, "f32", zero=False)
    ones = backend.alloc(np.ones(width, np.float32))
    backend.run("strata_norm", {"X": X, "W": ones, "Y": Xn, "cols": width, "rows": tokens, "weightRows": 1,
                                "mode": 0, "epsilon": 1e-6, "scale": 1.0}, [tokens, 1, 1])
    return Xn


@pytest.mark.parametrize("tokens,bias", [(1, False), (8, False), (9, False), (37, False), (128, True),
                                         (129, False), (512, False), (2048, True)])
def test_route_bit_exact(backend, oracle, full_layer, tokens, bias):
    W, E, K = wl.WIDTH, wl.EXPERTS, wl.TOPK
    X = device_inputs(backend, tokens, W, full_layer.seed + tokens, tokens == 1)
    b = wl.zipf_bias(E, full_layer.seed) if bias else None
    B = backend.alloc(b) if bias else None
    logits, ids, w = backend.alloc(tokens * E), backend.alloc(tokens * K, "i32"), backend.alloc(tokens * K)
    backend.moe_route(X, tokens, W, full_layer.Wr, E, K, ids, w, logits=logits, bias=B)
    xh, Wr = backend.read(X), backend.read(full_layer.Wr)
    ref_logits = oracle.project(xh, Wr, W, E, tokens)
    if bias:
        ref_logits = (ref_logits.reshape(tokens, E) * np.float32(1.0) + b).reshape(-1)
    assert same_bits(backend.read(logits), ref_logits)
    rids, rw = oracle.router(ref_logits, E, K, tokens)
    assert np.array_equal(backend.read(ids), rids)
    assert same_bits(backend.read(w), rw)
    if bias:  # the Zipf prior concentrates assignments: ~20 experts take > 50 %
        counts = np.sort(np.bincount(rids, minlength=E))[::-1]
        assert counts[:20].sum() > 0.5 * rids.size


@pytest.mark.parametrize("tokens,topk,experts,zipf", [(1, 10, 512, False), (63, 10, 512, False),
                                                      (65, 3, 16, False), (300, 4, 40, True),
                                                      (512, 10, 512, False), (513, 10, 512, True),
                                                      (2048, 10, 512, True)])
def test_dispatch_bit_exact(backend, oracle, tokens, topk, experts, zipf):
    rng = np.random.default_rng(tokens + experts)
    p = None
    if zipf:
        p = 1.0 / np.arange(1, experts + 1) ** 1.1
        p = rng.permutation(p / p.sum())
    ids = np.stack([rng.choice(experts, topk, replace=False, p=p) for _ in range(tokens)]).reshape(-1).astype(np.int32)
    n = tokens * topk
    bufs = dict(offsets=backend.alloc(experts + 2, "i32"), rows=backend.alloc(n, "i32"),
                parts=backend.alloc(n, "i32"), where=backend.alloc(n, "i32"))
    ws = backend.alloc_bytes(1 << 20)
    backend.moe_dispatch(backend.alloc(ids, "i32"), tokens, topk, experts, bufs["offsets"], bufs["rows"],
                         bufs["parts"], bufs["where"], ws)
    ro, rr, rp, rw = oracle.dispatch(ids, tokens, topk, experts)
    assert np.array_equal(backend.read(bufs["offsets"])[:experts + 1], ro)
    assert np.array_equal(backend.read(bufs["rows"]), rr)
    assert np.array_equal(backend.read(bufs["parts"]), rp)
    assert np.array_equal(backend.read(bufs["where"]), rw)


def test_dispatch_rejects_invalid_ids_safely(backend):
    # An out-of-range or repeated ID never reaches memory (src/engine.js:138):
    # it is left out of the permutation and flagged.
    ids = np.array([0, 1, 99, 2, 3, 3], np.int32)  # token 1: out of range; token 2: repeated
    bufs = [backend.alloc(8, "i32") for _ in range(4)]
    ws = backend.alloc_bytes(1 << 16)
    backend.moe_dispatch(backend.alloc(ids, "i32"), 3, 2, 4, *bufs, ws)
    where = backend.read(bufs[3])[:6]
    assert where[2] == -1
    status = backend.read_bytes(ws, 4).view(np.uint32)[0]
    assert status & 1 and status & 2


@pytest.mark.parametrize("tokens,topk", [(1, 4), (5, 4), (37, 3), (130, 4)])
def test_layer_small_geometry(backend, oracle, small, tokens, topk):
    layer, host = small
    W, F, E = 128, 64, 16
    X = device_inputs(backend, tokens, W, 5 + tokens, False)
    Y, ids, w = backend.alloc(tokens * W), backend.alloc(tokens * topk, "i32"), backend.alloc(tokens * topk)
    ws = backend.alloc_bytes(backend.moe_workspace_bytes(tokens, W, F, E, topk))
    backend.moe_layer(X, tokens, layer.Wr, layer.arena, layer.stride, layer.shared, layer.Wsg, W, F, E, topk, Y, ids,
                      w, ws)
    eY, eids, ew = oracle.moe_layer(backend.read(X), tokens, host["Wr"], host["arena"], host["stride"],
                                    host["shared"], host["Wsg"], W, F, E, topk)
    assert np.array_equal(backend.read(ids), eids)
    assert weights_ok(tokens, backend.read(w), ew)
    assert tol_ok(backend.read(Y), eY)


def check_route_stats(backend, ws, tokens, W, F, E, K):
    """The certified router's records for a batch of random inputs: the
    exact logits it formed are a few more than top-k per token, and hardly
    any token fell back to the exact path (only exponentials of two of a
    token's top-k + 1 experts within 2^-21 of each other force it: a few
    tokens in ten thousand on random logits)."""
    st = backend.route_stats(ws, tokens, W, F, E, K)
    if tokens < CERTIFIED_MIN_TOKENS:
        assert st is None
        return None
    cand, fallbacks = st
    assert fallbacks <= max(1, tokens // 200), st
    assert K * tokens <= cand <= 3 * K * tokens, st
    return cand / tokens


def check_full_layer(backend, oracle, layer, tokens, bias, input_seed=0):
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    X = device_inputs(backend, tokens, W, layer.seed + 1000 + tokens + input_seed, tokens == 1)
    b = wl.zipf_bias(E, layer.seed) if bias else None
    Y, ids, w = backend.alloc(tokens * W), backend.alloc(tokens * K, "i32"), backend.alloc(tokens * K)
    ws = backend.alloc_bytes(backend.moe_workspace_bytes(tokens, W, F, E, K))
    backend.moe_layer(X, tokens, layer.Wr, layer.arena, layer.stride, layer.shared, layer.Wsg, W, F, E, K, Y, ids, w,
                      ws, bias=backend.alloc(b) if bias else None)
    got_y, got_ids, got_w, xh = backend.read(Y), backend.read(ids), backend.read(w), backend.read(X)
    assert np.all(np.isfinite(got_y))
    # routing of every token, bit-exact
    logits = oracle.project(xh, backend.read(layer.Wr), W, E, tokens)
    if bias:
        logits = (logits.reshape(tokens, E) + b).reshape(-1)
    rids, rw = oracle.router(logits, E, K, tokens)
    assert np.array_equal(got_ids, rids)
    assert weights_ok(tokens, got_w, rw)
    check_route_stats(backend, ws, tokens, W, F, E, K)
    # every token's output (the oracle's experts: those the tokens routed to)
    host = wl.host_layer(oracle, 0, expert_ids=got_ids)
    eY, eids, _ = oracle.moe_layer(xh, tokens, host["Wr"], host["arena"], host["stride"], host["shared"],
                                   host["Wsg"], W, F, E, K, bias=b)
    assert np.array_equal(eids, got_ids)
    err = np.abs(got_y - eY)
    assert tol_ok(got_y, eY), "max abs err %g at token %d" % (err.max(), int(np.argmax(err)) // W)
    return err.max()


@pytest.mark.parametrize("input_seed", [0, 1, 2])
def test_layer_decode_full(backend, oracle, full_layer, input_seed):
    check_full_layer(backend, oracle, full_layer, 1, False, input_seed)


def test_layer_prefill_512_full(backend, oracle, full_layer):
    check_full_layer(backend, oracle, full_layer, 512, False)


def test_layer_prefill_2048_zipf_full(backend, oracle, full_layer):
    check_full_layer(backend, oracle, full_layer, 2048, True)


@pytest.mark.parametrize("tokens,bias", [(700, True), (1023, False)])
def test_layer_prefill_one_grid_full(backend, oracle, full_layer, tokens, bias):
    # Past the one-block dispatch (512 tokens) and below 1,024 tokens: the
    # masks / scan / place dispatch with every segment in 16-row tiles, the
    # Zipf-biased router's hot experts (hundreds of rows) and the shared
    # expert's segment (one row per token) included.
    check_full_layer(backend, oracle, full_layer, tokens, bias)


def routing_styles(E):
    x = np.arange(E)
    styles = {"ties": np.full(E, 7, np.float32),
              "spread": (np.sin(x * 3.1) * 90).astype(np.float32),  # most probabilities underflow to 0
              "pairs": np.repeat(np.random.default_rng(3).normal(0, 1, E // 2), 2).astype(np.float32)}
    v = np.random.default_rng(5).normal(0, 1, E).astype(np.float32)
    styles["nan_one"] = v.copy()
    styles["nan_one"][3] = np.nan
    styles["neg_inf_tail"] = v.copy()
    styles["neg_inf_tail"][5:] = -np.inf
    styles["pos_inf"] = v.copy()
    styles["pos_inf"][100] = np.inf
    styles["one_finite"] = np.full(E, -np.inf, np.float32)
    styles["one_finite"][7] = 0.0
    # adjacent floats, the larger at the higher ID: their exponentials round
    # to the same probability, so the reference takes the lower ID (smaller
    # logit) first, against the logits' own order
    u = (np.random.default_rng(11).normal(0, 1, E // 2) * 0.05).astype(np.float32)
    styles["ulp_pairs"] = np.empty(E, np.float32)
    styles["ulp_pairs"][0::2] = u
    styles["ulp_pairs"][1::2] = np.nextafter(u, np.float32(np.inf))
    return styles


@pytest.mark.parametrize("tokens", [1, 3, 6, 8, 20, 30, CERTIFIED_MIN_TOKENS])
def test_layer_routing_edge_logits(backend, oracle, full_layer, tokens):
    # W_r = 0 makes every logit exactly the per-expert bias, so the layer's
    # routing (the in-block top-k up to 4 tokens, the top-k kernel up to 6,
    # the exact prefill router up to 511, the certified router from 512 on)
    # sees ties, underflow to 0, NaN and +-inf. (With W_r = 0 the certified
    # router's approximate logits are exact, so its weights are too.)
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    Wr0 = backend.alloc(np.zeros(E * W, np.float32))
    X = device_inputs(backend, tokens, W, 77 + tokens, False)
    Y, ids, w = backend.alloc(tokens * W), backend.alloc(tokens * K, "i32"), backend.alloc(tokens * K)
    ws = backend.alloc_bytes(backend.moe_workspace_bytes(tokens, W, F, E, K))
    for name, b in routing_styles(E).items():
        backend.moe_layer(X, tokens, Wr0, full_layer.arena, full_layer.stride, full_layer.shared, full_layer.Wsg, W,
                          F, E, K, Y, ids, w, ws, bias=backend.alloc(b))
        rids, rw = oracle.router(np.tile(b, tokens), E, K, tokens)
        assert np.array_equal(backend.read(ids), rids), name
        assert same_bits(backend.read(w), rw), name


@pytest.mark.parametrize("tokens", [5, 6, 7, 16, 17, 24, 25, 40, 64, 65])
def test_layer_small_batch_full(backend, oracle, full_layer, tokens):
    # 5 and 6 tokens: the decode kernels with a token dimension (one top-k
    # kernel for the batch); 7..64: 16-row tiles of 128 weight rows over every
    # segment; 65: the first batch with 256 weight rows per 16-row tile.
    check_full_layer(backend, oracle, full_layer, tokens, False)


@pytest.mark.parametrize("W,F,E,topk,tokens", [(512, 512, 24, 4, 40), (2048, 2048, 8, 2, 33),
                                               (512, 2048, 12, 3, 100), (2048, 512, 20, 4, 48),
                                               # the real model's widths: 40 and 10 groups
                                               (2560, 640, 20, 4, 70), (2048, 640, 16, 3, 48),
                                               (2560, 512, 16, 3, 40),
                                               # 1,024 tokens and more: 64-row tiles for 8, 10, 32
                                               # and 40 groups beside the 16-row grid
                                               (512, 2048, 12, 3, 1024), (2560, 640, 20, 4, 1024)])
def test_layer_stream_geometries(backend, oracle, W, F, E, topk, tokens):
    # Every (width, ff) pair of the streaming kernels, with and without the
    # K split, against the oracle on all tokens.
    layer = wl.DeviceLayer(backend, layer=0, width=W, ff=F, experts=E, base_seed=23)
    host = wl.host_layer(oracle, 0, width=W, ff=F, experts=E, base_seed=23)
    X = device_inputs(backend, tokens, W, 31 + tokens, False)
    Y, ids, w = backend.alloc(tokens * W), backend.alloc(tokens * topk, "i32"), backend.alloc(tokens * topk)
    ws = backend.alloc_bytes(backend.moe_workspace_bytes(tokens, W, F, E, topk))
    backend.moe_layer(X, tokens, layer.Wr, layer.arena, layer.stride, layer.shared, layer.Wsg, W, F, E, topk, Y, ids,
                      w, ws)
    eY, eids, ew = oracle.moe_layer(backend.read(X), tokens, host["Wr"], host["arena"], host["stride"],
                                    host["shared"], host["Wsg"], W, F, E, topk)
    layer.free()
    assert np.array_equal(backend.read(ids), eids)
    assert weights_ok(tokens, backend.read(w), ew)
    got = backend.read(Y)
    assert tol_ok(got, eY), "max abs err %g" % np.abs(got - eY).max()


def test_layer_rejects_bad_arguments(backend, small):
    layer, _ = small
    W, F, E, K = 128, 64, 16, 4
    X, Y = backend.alloc(W), backend.alloc(W)
    ids, w = backend.alloc(K, "i32"), backend.alloc(K)
    tiny = backend.alloc_bytes(64)
    with pytest.raises(sm.ArgumentError, match="workspace"):
        backend.moe_layer(X, 1, layer.Wr, layer.arena, layer.stride, layer.shared, layer.Wsg, W, F, E, K, Y, ids, w,
                          tiny)
    ws = backend.alloc_bytes(backend.moe_workspace_bytes(1, W, F, E, K))
    with pytest.raises(sm.ArgumentError, match="stride"):
        backend.moe_layer(X, 1, layer.Wr, layer.arena, layer.stride + 4, layer.shared, layer.Wsg, W, F, E, K, Y, ids,
                          w, ws)
    with pytest.raises(sm.ArgumentError):
        backend.moe_layer(X, 1, layer.Wr, layer.arena, layer.stride, layer.shared, layer.Wsg, W, F, 17, K, Y, ids, w,
                          ws)  # arena holds 16 experts
    with pytest.raises(sm.ArgumentError, match="Router supports"):
        backend.moe_layer(X, 1, layer.Wr, layer.arena, layer.stride, layer.shared, layer.Wsg, W, F, E, 33, Y, ids, w,
                          ws)


@pytest.mark.parametrize("tokens,style", [(512, "normal"), (640, "normed"), (600, "scaled_up"), (512, "tiny_router"),
                                          (1024, "zipf"), (2048, "normal")])
def test_certified_router_matches_exact(backend, full_layer, tokens, style):
    # The layer's certified routing against the exact router on the same
    # inputs (sm_moe_route with logits: every logit in the reference's order,
    # bit-exact with the oracle in test_route_bit_exact): IDs and order
    # bit-exact, weights within 1e-6. "scaled_up" (x * 300) spreads the
    # logits so that most exponentials underflow; "tiny_router" (W_r * 2^-20)
    # leaves every logit within the error bound of the others, so each token
    # takes the exact fallback.
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    X = device_inputs(backend, tokens, W, 4242 + tokens, style == "normed")
    Wr = full_layer.Wr
    if style == "scaled_up":
        backend.write(X, backend.read(X) * np.float32(300.0))
    if style == "tiny_router":
        Wr = backend.alloc(backend.read(full_layer.Wr) * np.float32(2.0 ** -20))
    bias = backend.alloc(wl.zipf_bias(E, full_layer.seed)) if style == "zipf" else None
    Y, ids, w = backend.alloc(tokens * W), backend.alloc(tokens * K, "i32"), backend.alloc(tokens * K)
    ws = backend.alloc_bytes(backend.moe_workspace_bytes(tokens, W, F, E, K))
    backend.moe_layer(X, tokens, Wr, full_layer.arena, full_layer.stride, full_layer.shared, full_layer.Wsg, W, F, E,
                      K, Y, ids, w, ws, bias=bias)
    cand, fallbacks = backend.route_stats(ws, tokens, W, F, E, K)
    logits, rids, rw = backend.alloc(tokens * E), backend.alloc(tokens * K, "i32"), backend.alloc(tokens * K)
    backend.moe_route(X, tokens, W, Wr, E, K, rids, rw, logits=logits, bias=bias)
    assert np.array_equal(backend.read(ids), backend.read(rids))
    assert weights_close(backend.read(w), backend.read(rw))
    if style != "scaled_up":
        # (x * 300 makes the hidden values pass fp16's range, which the
        # prefill GEMMs' hi/lo activations need: routing only, there)
        assert np.all(np.isfinite(backend.read(Y)))
    print("%s T=%d: %.2f exact logits per token, %d fallbacks" % (style, tokens, cand / tokens, fallbacks))
    if style == "tiny_router":
        assert fallbacks == tokens
    elif style in ("normal", "normed", "zipf"):
        assert fallbacks <= max(1, tokens // 200) and cand <= 3 * K * tokens


def test_certified_router_partial_fallback(backend, full_layer):
    # Tokens whose logits tie (zero rows: every logit is the bias, all equal)
    # take the exact path inside the same launch; the others stay certified.
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    tokens = CERTIFIED_MIN_TOKENS
    xh = np.random.default_rng(8).normal(0, 1, (tokens, W)).astype(np.float32)
    zero_rows = [0, 5, 63, 64, tokens - 1]
    xh[zero_rows] = 0.0
    X = backend.alloc(xh.reshape(-1))
    bias = backend.alloc(np.full(E, 0.25, np.float32))
    Y, ids, w = backend.alloc(tokens * W), backend.alloc(tokens * K, "i32"), backend.alloc(tokens * K)
    ws = backend.alloc_bytes(backend.moe_workspace_bytes(tokens, W, F, E, K))
    backend.moe_layer(X, tokens, full_layer.Wr, full_layer.arena, full_layer.stride, full_layer.shared,
                      full_layer.Wsg, W, F, E, K, Y, ids, w, ws, bias=bias)
    cand, fallbacks = backend.route_stats(ws, tokens, W, F, E, K)
    assert len(zero_rows) <= fallbacks <= len(zero_rows) + 1  # (+ a rare near-tie among the random rows)
    logits, rids, rw = backend.alloc(tokens * E), backend.alloc(tokens * K, "i32"), backend.alloc(tokens * K)
    backend.moe_route(X, tokens, W, full_layer.Wr, E, K, rids, rw, logits=logits, bias=bias)
    got, exp = backend.read(ids).reshape(tokens, K), backend.read(rids).reshape(tokens, K)
    assert np.array_equal(got, exp)
    assert np.array_equal(got[0], np.arange(K))  # all tied: the lowest IDs, in order
    gw, ew = backend.read(w).reshape(tokens, K), backend.read(rw).reshape(tokens, K)
    assert same_bits(gw[zero_rows], ew[zero_rows])  # the fallback is the exact path
    assert weights_close(gw, ew)
