"""Reference-named kernels on the GPU (sm_run through the C ABI) against the
CPU oracle on identical inputs. These kernels keep the reference's f32
operation order, so results must match bit for bit; the reference's own
known-answer recipes supply the inputs."""
import numpy as np
import pytest

import stratacuda_amd as sm
from test_oracle_kernels import fused_recipe

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    assert a.shape == b.shape
    nan = np.isnan(b)
    assert np.array_equal(np.isnan(a), nan)
    assert np.array_equal(bits(a)[~nan], bits(b)[~nan])


def test_unpack_half_all_patterns(backend, oracle):
    h = np.arange(65536, dtype=np.uint32)
    packed = (h[0::2] | (h[1::2] << 16)).astype(np.uint32)
    out = backend.alloc(65536)
    backend.run("strata_unpack_half", {"Packed": backend.alloc(packed, "u32"), "Values": out, "count": 65536},
                [1024, 1, 1])
    assert np.array_equal(backend.read(out).view(np.uint32), oracle.unpack_half(packed, 65536).view(np.uint32))


def test_project_kat_and_ragged(backend, oracle):
    cols, rows = 2560, 37
    x = np.sin(np.arange(cols) * .73).astype(np.float32)
    w = (np.cos(np.arange(cols * rows) * .17) * .03).astype(np.float32)
    y = backend.alloc(rows)
    backend.run("strata_gemv", {"X": backend.alloc(x), "W": backend.alloc(w), "Y": y, "cols": cols, "rows": rows,
                                "tokens": 1}, [rows, 1, 1])
    same(backend.read(y), oracle.project(x, w, cols, rows, 1))
    rng = np.random.default_rng(0)
    for cols, rows, tokens, stride, off in [(130, 9, 3, 12, 2), (64, 1, 5, 1, 0), (2048, 513, 2, 600, 40), (7, 3, 1, 3, 0)]:
        X = rng.normal(0, 1, tokens * cols).astype(np.float32)
        W = rng.normal(0, .05, rows * cols).astype(np.float32)
        Y = backend.alloc(np.full(tokens * stride, -7, np.float32))
        backend.run("strata_project", {"X": backend.alloc(X), "W": backend.alloc(W), "Y": Y, "cols": cols,
                                       "rows": rows, "tokens": tokens, "outputStride": stride, "outputOffset": off},
                    [rows, tokens, 1])
        ref = oracle.project(X, W, cols, rows, tokens, stride, off, Y=np.full(tokens * stride, -7, np.float32))
        same(backend.read(Y), ref)


def test_fused_q2_gate_up_down_kat(backend, oracle):
    width, ff, tokens, cb, sb, raw, x, mapping = fused_recipe()
    blob_u32 = raw.view(np.uint32)
    b = {"blob": backend.alloc(blob_u32, "u32"), "map": backend.alloc(mapping, "i32"), "x": backend.alloc(x),
         "hidden": backend.alloc(tokens * ff), "dummy": backend.alloc(1)}
    out = backend.alloc(np.full(5 * width + 7, -99, np.float32))
    backend.run("strata_q2_gate_up", {"X": b["x"], "Blob": b["blob"], "Scales": b["dummy"], "Mapping": b["map"],
                                      "Hidden": b["hidden"], "width": width, "ff": ff, "tokens": tokens, "mapped": 1,
                                      "expanded": 0, "codeOffset": 0, "scaleOffset": 3 * cb // 2}, [ff, tokens, 1])
    hid = oracle.q2_gate_up(x, blob_u32, width, ff, tokens, mapping=mapping, scale_offset=3 * cb // 2)
    same(backend.read(b["hidden"]), hid)
    backend.run("strata_q2_down", {"Hidden": b["hidden"], "Blob": b["blob"], "Scales": b["dummy"], "Mapping": b["map"],
                                   "Y": out, "width": width, "ff": ff, "tokens": tokens, "mapped": 1, "expanded": 0,
                                   "outputOffset": 7, "codeOffset": 2 * cb // 4,
                                   "scaleOffset": (3 * cb + 2 * sb) // 2}, [width, tokens, 1])
    ref = oracle.q2_down(hid, blob_u32, np.full(5 * width + 7, -99, np.float32), width, ff, tokens, mapping=mapping,
                         output_offset=7, code_offset=2 * cb // 4, scale_offset=(3 * cb + 2 * sb) // 2)
    same(backend.read(out), ref)
    # expanded scales (strata_expert_scales) path
    scales = backend.alloc(3 * sb // 2)
    backend.run("strata_expert_scales", {"Blob": b["blob"], "Scales": scales, "offset": 3 * cb // 2,
                                         "count": 3 * sb // 2}, [(3 * sb // 2 + 63) // 64, 1, 1])
    same(backend.read(scales), oracle.expert_scales(blob_u32, 3 * cb // 2, 3 * sb // 2))
    backend.run("strata_q2_gate_up", {"X": b["x"], "Blob": b["blob"], "Scales": scales, "Mapping": b["map"],
                                      "Hidden": b["hidden"], "width": width, "ff": ff, "tokens": tokens, "mapped": 1,
                                      "expanded": 1, "codeOffset": 0, "scaleOffset": 0}, [ff, tokens, 1])
    same(backend.read(b["hidden"]), hid)


def test_q2_project_and_quant_project(backend, oracle):
    cols, rows, tokens = 64, 65, 3
    cb, sb = rows * cols // 4, rows * 2
    raw = np.zeros((3 * (cb + sb) + 3) // 4 * 4, np.uint8)
    raw[:3 * cb] = (np.arange(3 * cb) * 13 + 7) & 255
    i = np.arange(3 * rows)
    raw[3 * cb:3 * cb + 6 * rows].view(np.uint16)[:] = 0x3800 + (i % 6) * 64 + np.where(i % 3 == 0, 0x8000, 0)
    x = np.sin(np.arange(tokens * cols) * .23).astype(np.float32)
    blob, X = backend.alloc(raw.view(np.uint32), "u32"), backend.alloc(x)
    stride, off = rows + 7, 3
    for role in ("gate", "up", "down"):
        down = role == "down"
        args = dict(cols=cols, rows=rows, tokens=tokens, outputStride=stride, outputOffset=off,
                    codeOffset=(2 * cb if down else 0) // 4, scaleOffset=(3 * cb + (2 * sb if down else 0)) // 2,
                    weightRow=1 if role == "up" else 0, rowStride=1 if down else 2)
        Y = backend.alloc(tokens * stride)
        backend.run("strata_q2_project", dict(X=X, Blob=blob, Y=Y, **args), [rows, tokens, 1])
        ref = oracle.q2_project(x, raw.view(np.uint32), np.zeros(tokens * stride, np.float32), cols, rows, tokens,
                                stride, off, args["codeOffset"], args["scaleOffset"], args["weightRow"],
                                args["rowStride"])
        same(backend.read(Y), ref)
    for nbits in (2, 4, 8):
        cols, rows, gs, mask = 64, 5, 16, (1 << nbits) - 1
        codes = np.zeros((cols * rows * nbits + 31) // 32, np.uint32)
        for k in range(cols * rows):
            codes[(k * nbits) >> 5] |= np.uint32(((k * 13 + 7) & mask) << ((k * nbits) & 31))
        scales = ((np.arange(cols * rows // gs) % 7 - 3) * .03).astype(np.float32)
        offsets = (np.arange(scales.size) * .001).astype(np.float32)
        xx = np.sin(np.arange(cols)).astype(np.float32)
        Y = backend.alloc(rows)
        backend.run("strata_quant_project", {"X": backend.alloc(xx), "Codes": backend.alloc(codes, "u32"),
                                             "Scales": backend.alloc(scales), "Offsets": backend.alloc(offsets),
                                             "Y": Y, "cols": cols, "rows": rows, "tokens": 1, "outputStride": rows,
                                             "outputOffset": 0, "bits": nbits, "groupSize": gs, "bias": -3,
                                             "codebook": 0, "hasOffset": 1}, [rows, 1, 1])
        ref = oracle.quant_project(xx, codes, scales, offsets, np.zeros(rows, np.float32), cols, rows, 1, rows, 0,
                                   nbits, gs, -3, 0, 1)
        same(backend.read(Y), ref)


def test_norm_and_elementwise(backend, oracle):
    rng = np.random.default_rng(2)
    X = rng.normal(0, 2, 3 * 2048).astype(np.float32)
    Wn = rng.normal(1, .1, 2048).astype(np.float32)
    for mode, scale in ((0, 1.0), (1, 0.25)):
        Y = backend.alloc(3 * 2048)
        backend.run("strata_norm", {"X": backend.alloc(X), "W": backend.alloc(Wn), "Y": Y, "cols": 2048, "rows": 3,
                                    "weightRows": 1, "mode": mode, "epsilon": 1e-6, "scale": scale}, [3, 1, 1])
        same(backend.read(Y), oracle.norm(X, Wn, 2048, 3, 1, mode, 1e-6, scale))
    A = rng.normal(0, 4, 1000).astype(np.float32)
    B = rng.normal(0, 4, 1000).astype(np.float32)
    for mode in range(6):
        Y = backend.alloc(1000)
        backend.run("strata_elementwise", {"A": backend.alloc(A), "B": backend.alloc(B), "Y": Y, "n": 1000,
                                           "mode": mode, "scale": 1.25}, [16, 1, 1])
        same(backend.read(Y), oracle.elementwise(A, B, mode, 1.25))


@pytest.mark.parametrize("style", ["ties", "spread", "random", "small", "nonfinite"])
def test_router_and_batch(backend, oracle, style):
    rng = np.random.default_rng(4)
    experts, k, tokens = (6, 2, 5) if style == "small" else (512, 10, 37)
    if style == "ties":
        logits = np.full(tokens * experts, 7, np.float32)
    elif style == "spread":
        logits = np.tile((np.sin(np.arange(experts) * 3.1) * 90).astype(np.float32), tokens)
    else:
        logits = rng.normal(0, 1, tokens * experts).astype(np.float32)
    if style == "nonfinite":
        # NaN anywhere makes every probability NaN (ID `experts` each round);
        # -inf logits give probability 0, so the last rounds break ties at 0
        # by the lower ID; +inf makes the max inf and every probability NaN.
        t = logits.reshape(tokens, experts)
        t[0, 3] = np.nan
        t[1, :] = np.nan
        t[2, 5:] = -np.inf
        t[3, 100] = np.inf
        t[4, ::2] = -np.inf
        t[5, :] = -np.inf
        t[5, 7] = 0.0
    L = backend.alloc(logits)
    ids, w = backend.alloc(tokens * k, "i32"), backend.alloc(tokens * k)
    backend.run("strata_router_batch", {"Logits": L, "Ids": ids, "Weights": w, "experts": experts, "topK": k},
                [tokens, 1, 1])
    rids, rw = oracle.router(logits, experts, k, tokens)
    assert np.array_equal(backend.read(ids), rids)
    same(backend.read(w), rw)
    ids1, w1 = backend.alloc(k, "i32"), backend.alloc(k)
    backend.run("strata_router", {"Logits": L, "Ids": ids1, "Weights": w1, "experts": experts, "topK": k}, [1, 1, 1])
    assert np.array_equal(backend.read(ids1), rids[:k])
    same(backend.read(w1), rw[:k])


def test_combine_gather_scatter(backend, oracle):
    rng = np.random.default_rng(6)
    T, K, Wd = 4, 10, 2048
    parts = rng.normal(0, 1, T * K * Wd).astype(np.float32)
    wts = rng.random(T * K).astype(np.float32)
    shared = rng.normal(0, 1, T * Wd).astype(np.float32)
    gate = rng.normal(0, 1, T).astype(np.float32)
    Y = backend.alloc(T * Wd)
    backend.run("strata_moe_combine_batch", {"Parts": backend.alloc(parts), "Weights": backend.alloc(wts),
                                             "Shared": backend.alloc(shared), "SharedGate": backend.alloc(gate),
                                             "Y": Y, "width": Wd, "count": K, "tokens": T}, [T * Wd // 64, 1, 1])
    same(backend.read(Y), oracle.moe_combine(parts, wts, shared, gate, Wd, K, T))
    Y1 = backend.alloc(Wd)
    backend.run("strata_moe_combine", {"Parts": backend.alloc(parts), "Weights": backend.alloc(wts),
                                       "Shared": backend.alloc(shared), "SharedGate": backend.alloc(gate), "Y": Y1,
                                       "width": Wd, "count": K}, [Wd // 64, 1, 1])
    same(backend.read(Y1), oracle.moe_combine(parts[:K * Wd], wts[:K], shared[:Wd], gate[:1], Wd, K, 1))
    X = np.arange(5 * 8, dtype=np.float32)
    idx = np.array([4, 0, 2], np.int32)
    G = backend.alloc(24)
    backend.run("strata_gather_rows", {"X": backend.alloc(X), "Indices": backend.alloc(idx, "i32"), "Y": G,
                                       "width": 8, "rows": 3}, [1, 1, 1])
    same(backend.read(G), oracle.gather_rows(X, idx, 8, 3))
    S = backend.alloc(np.full(40, -1, np.float32))
    backend.run("strata_scatter_rows", {"X": G, "Indices": backend.alloc(idx, "i32"), "Y": S, "width": 8, "rows": 3},
                [1, 1, 1])
    same(backend.read(S), oracle.scatter_rows(oracle.gather_rows(X, idx, 8, 3), idx, np.full(40, -1, np.float32), 8, 3))


def test_validation_rejects_before_launch(backend):
    # src/backend.js:10-56 conventions, plus host-side bounds checks.
    L, ids, w = backend.alloc(513), backend.alloc(10, "i32"), backend.alloc(10)
    with pytest.raises(sm.ArgumentError, match="Router supports"):
        backend.run("strata_router", {"Logits": L, "Ids": ids, "Weights": w, "experts": 513, "topK": 10}, [1, 1, 1])
    with pytest.raises(sm.ArgumentError, match="Router supports"):
        backend.run("strata_router", {"Logits": L, "Ids": ids, "Weights": w, "experts": 6, "topK": 7}, [1, 1, 1])
    X, Y = backend.alloc(64), backend.alloc(64)
    with pytest.raises(sm.ArgumentError, match="complete groups"):
        backend.run("strata_q2_gate_up", {"X": X, "Blob": backend.alloc(64, "u32"), "Scales": X, "Mapping": ids,
                                          "Hidden": Y, "width": 96, "ff": 64, "tokens": 1, "mapped": 0, "expanded": 0,
                                          "codeOffset": 0, "scaleOffset": 0}, [64, 1, 1])
    with pytest.raises(sm.ArgumentError, match="Projection batch"):
        backend.run("strata_project", {"X": X, "W": X, "Y": Y, "cols": 64, "rows": 2, "tokens": 1, "outputStride": 2,
                                       "outputOffset": 1}, [2, 1, 1])
    with pytest.raises(sm.ArgumentError):
        backend.run("strata_project", {"X": X, "W": X, "Y": Y, "cols": 64, "rows": 4, "tokens": 1, "outputStride": 4,
                                       "outputOffset": 0}, [4, 1, 1])  # W holds one row only
    bad_idx = backend.alloc(np.array([0, 9], np.int32), "i32")
    with pytest.raises(sm.ArgumentError, match="outside"):
        backend.run("strata_gather_rows", {"X": X, "Indices": bad_idx, "Y": Y, "width": 8, "rows": 2}, [1, 1, 1])
    with pytest.raises(sm.StrataError, match="Unknown kernel"):
        backend.run("strata_nope", {}, [1, 1, 1])
    with pytest.raises(sm.ArgumentError, match="Invalid dispatch"):
        backend.run("strata_elementwise", {"A": X, "B": X, "Y": Y, "n": 64, "mode": 0, "scale": 1.0}, [0, 1, 1])
