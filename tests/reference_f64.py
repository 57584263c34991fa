"""Independent float64 restatement of the MoE layer for tests (numpy), in the
style of the reference's tests/reference.mjs: plain equations, no kernel
operation order. Used to bound the oracle's and the GPU's f32 results."""
import numpy as np


def half_to_float(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float64)


def unpack_codes(raw):
    """2-bit codes, 4 per byte, LSB first (dequant.hpp:72-76)."""
    raw = np.asarray(raw, np.uint8)
    return np.stack([(raw >> (2 * s)) & 3 for s in range(4)], axis=-1).reshape(-1).astype(np.int64)


def blob_matrices(blob, width, ff):
    """(gate_up [2ff x width] interleaved rows, down [width x ff]) in float64."""
    blob = np.asarray(blob, np.uint8)
    cgu, cd = 2 * ff * width // 4, width * ff // 4
    sgu, sd = 2 * ff * width // 64, width * ff // 64
    codes_gu = unpack_codes(blob[:cgu]).reshape(2 * ff, width)
    codes_d = unpack_codes(blob[cgu:cgu + cd]).reshape(width, ff)
    s_gu = half_to_float(blob[cgu + cd:cgu + cd + 2 * sgu].view(np.uint16)).reshape(2 * ff, width // 64)
    s_d = half_to_float(blob[cgu + cd + 2 * sgu:cgu + cd + 2 * sgu + 2 * sd].view(np.uint16)).reshape(width, ff // 64)
    gu = (codes_gu - 1) * np.repeat(s_gu, 64, axis=1)
    d = (codes_d - 1) * np.repeat(s_d, 64, axis=1)
    return gu, d


def silu(x):
    return x / (1 + np.exp(-x))


def sigmoid(x):
    return 1 / (1 + np.exp(-x))


def router(logits, k):
    """tests/reference.mjs:173-177: softmax, sort by probability (desc) then
    id (asc), renormalise by max(sum, 2^-14)."""
    logits = np.asarray(logits, np.float64)
    p = np.exp(logits - logits.max())
    p /= p.sum()
    ids = sorted(range(len(p)), key=lambda i: (-p[i], i))[:k]
    denom = max(sum(p[i] for i in ids), 2.0 ** -14)
    return np.array(ids), np.array([p[i] / denom for i in ids]), p


def expert(blob, x, width, ff):
    gu, d = blob_matrices(blob, width, ff)
    g, u = gu[0::2] @ x, gu[1::2] @ x
    return d @ (silu(g) * u)


def moe_layer(X, tokens, Wr, arena, stride, shared, Wsg, width, ff, experts, topk, bias=None):
    X = np.asarray(X, np.float64).reshape(tokens, width)
    Wr = np.asarray(Wr, np.float64).reshape(experts, width)
    Y = np.zeros((tokens, width))
    ids_all, w_all, gaps = [], [], []
    for t in range(tokens):
        logits = Wr @ X[t] + (0 if bias is None else np.asarray(bias, np.float64))
        ids, w, p = router(logits, topk)
        srt = np.sort(p)[::-1]
        gaps.append(np.min(np.abs(np.diff(srt[:topk + 1]))))
        y = expert(shared, X[t], width, ff) * sigmoid(np.asarray(Wsg, np.float64) @ X[t])
        for e, wk in zip(ids, w):
            y = y + wk * expert(arena[e * stride:e * stride + len(shared)], X[t], width, ff)
        Y[t] = y
        ids_all.append(ids)
        w_all.append(w)
    return Y.reshape(-1), np.concatenate(ids_all), np.concatenate(w_all), np.array(gaps)
