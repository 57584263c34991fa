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


# ----------------------------------------------------------------------------
# The fixture model's other operations and its whole decode step, restating the
# float64 equations of the reference's tests/reference.mjs:2-46 (mat, norm,
# conv, gdn, rope, attention) and ReferenceEngine.step (:48-95).
def mat(weights, x):
    x = np.asarray(x, np.float64)
    return np.asarray(weights, np.float64).reshape(-1, len(x)) @ x


def norm(x, weights, width, l2=False, scale=1.0):
    x = np.asarray(x, np.float64)
    y = np.zeros_like(x)
    for r in range(len(x) // width):
        row = x[r * width:(r + 1) * width]
        inv = scale / np.sqrt(row @ row / (1 if l2 else width) + 1e-6)
        w = 1.0 if l2 else np.asarray(weights, np.float64)[(r * width + np.arange(width)) % len(weights)]
        y[r * width:(r + 1) * width] = row * inv * w
    return y


def conv(history, x, weights, taps, dilation, activate):
    """history: float64 array updated in place (tests/reference.mjs:19-27)."""
    span = (taps - 1) * dilation
    x = np.asarray(x, np.float64)
    w = np.asarray(weights, np.float64)
    y = np.zeros(len(x))
    for c in range(len(x)):
        v = x[c] * w[c * taps + taps - 1]
        for tap in range(taps - 1):
            v += history[c * span + tap * dilation] * w[c * taps + tap]
        y[c] = silu(v) if activate else v
        if span:
            history[c * span:(c + 1) * span - 1] = history[c * span + 1:(c + 1) * span].copy()
            history[(c + 1) * span - 1] = x[c]
    return y


def gdn(state, q, k, v, decay, beta, dim, key_heads, value_heads):
    """state: float64 [dim x value_heads x dim] updated in place (tests/reference.mjs:28-36)."""
    out = np.zeros(len(v))
    for h in range(value_heads):
        src = h % key_heads
        kk, qq = np.asarray(k[src * dim:(src + 1) * dim], np.float64), np.asarray(q[src * dim:(src + 1) * dim], np.float64)
        for j in range(dim):
            ix = (np.arange(dim) * value_heads + h) * dim + j
            state[ix] *= decay[h]
            pred = state[ix] @ kk
            upd = beta[h] * (v[h * dim + j] - pred)
            state[ix] += kk * upd
            out[h * dim + j] = state[ix] @ qq
    return out


def rope(x, dim, rotary, pos, base):
    y = np.asarray(x, np.float64).copy()
    half = rotary // 2
    for h in range(len(y) // dim):
        for i in range(half):
            a, b = x[h * dim + i], x[h * dim + half + i]
            ang = pos / base ** (2 * i / rotary)
            y[h * dim + i] = a * np.cos(ang) - b * np.sin(ang)
            y[h * dim + half + i] = a * np.sin(ang) + b * np.cos(ang)
    return y


def attention(q, keys, values, cells, dim, heads, kv_heads):
    y = np.zeros(heads * dim)
    q, keys, values = (np.asarray(a, np.float64) for a in (q, keys, values))
    for h in range(heads):
        kh = h // (heads // kv_heads)
        sc = np.array([q[h * dim:(h + 1) * dim] @ keys[(t * kv_heads + kh) * dim:(t * kv_heads + kh + 1) * dim]
                       for t in cells]) / np.sqrt(dim)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        for i, t in enumerate(cells):
            y[h * dim:(h + 1) * dim] += p[i] * values[(t * kv_heads + kh) * dim:(t * kv_heads + kh + 1) * dim]
    return y


class ReferenceEngine:
    """tests/reference.mjs:48-95 in float64 over a fixture (oracle.fixture.Fixture)."""

    def __init__(self, fixture, ngram_rows):
        self.f, self.g, self.ngram_rows = fixture, fixture.config, ngram_rows
        g = self.g
        self.position, self.previous = 0, []
        c = (2 * g["keyHeads"] + g["valueHeads"]) * g["ssmDim"]
        self.states = [dict(state=np.zeros(g["ssmDim"] * g["valueHeads"] * g["ssmDim"]), conv=np.zeros(c * 3),
                            keys=np.zeros(g["context"] * g["kvHeads"] * g["headDim"]),
                            values=np.zeros(g["context"] * g["kvHeads"] * g["headDim"]))
                       for _ in range(g["layers"])]
        self.history = np.zeros((g["pleTaps"] - 1) * g["pleDilation"] * g["width"] * g["streams"])

    def w(self, name):
        return self.f.data(name).astype(np.float64)

    def project(self, name, x):
        return mat(self.w(name), x)

    def hc(self, prefix):
        g = self.g
        x = norm(self.r, self.w(prefix + "norm.weight"), g["width"])
        lo = silu(self.project(prefix + "down.weight", x) / g["streams"])
        gate = self.project(prefix + "up.weight", lo)
        W = g["width"]
        mixed = sum(x[c * W:(c + 1) * W] * sigmoid(gate[c * W:(c + 1) * W]) for c in range(g["streams"])) / g["streams"]
        return x, mixed

    def write(self, y, inject):
        W = self.g["width"]
        idx = np.arange(len(self.r))
        self.r = self.r + y[idx % W] * 2 * sigmoid(inject[idx // W] / self.g["streams"])

    def expert(self, p, x, shared=False):
        name = (lambda r: p + "ffn_" + r + "_shexp.weight") if shared else (lambda r: p + r)
        return self.project(name("down"), silu(self.project(name("gate"), x)) * self.project(name("up"), x))

    def step(self, token):
        g = self.g
        W, hcn = g["width"], g["width"] * g["streams"]
        row = self.w("token_embd.weight")[token * W:(token + 1) * W]
        self.r = row[np.arange(hcn) % W].copy()
        routes = []
        for l in range(g["layers"]):
            p, s = "blk.%d." % l, self.states[l]
            if l == g["pleLayer"]:
                pr = p + "ple_"
                rows = self.ngram_rows(token, self.previous, self.f.constants, g["eos"])
                tab, hd = self.w("per_layer_token_embd.weight"), g["pleHeadDim"]
                emb = np.concatenate([tab[r * hd:(r + 1) * hd] for r in rows])
                key = norm(self.project(pr + "key.weight", emb), self.w(pr + "norm_key.weight"), W)
                query = norm(self.r, self.w(pr + "norm_query.weight"), W)
                value = self.project(pr + "value.weight", emb)
                gated = np.zeros(hcn)
                for c in range(g["streams"]):
                    sc = key[c * W:(c + 1) * W] @ query[c * W:(c + 1) * W] / np.sqrt(W)
                    gate = sigmoid(np.sign(sc) * np.sqrt(max(abs(sc), 1e-6)))
                    gated[c * W:(c + 1) * W] = value * gate
                n = norm(gated, self.w(pr + "norm_conv.weight"), W)
                cv = conv(self.history, n, self.w(pr + "conv1d.weight"), g["pleTaps"], g["pleDilation"], True)
                self.r = self.r + gated + cv
            ax, x = self.hc(p + "hc_attn_")
            if l % g["qsaInterval"] == g["qsaInterval"] - 1:
                hd = g["headDim"]
                full = self.project(p + "attn_q.weight", x)
                qraw = np.array([full[(i // hd) * 2 * hd + i % hd] for i in range(g["heads"] * hd)])
                q = rope(norm(qraw, self.w(p + "attn_q_norm.weight"), hd), hd, g["rotary"], self.position,
                         g["ropeBase"])
                k = rope(norm(self.project(p + "attn_k.weight", x), self.w(p + "attn_k_norm.weight"), hd), hd,
                         g["rotary"], self.position, g["ropeBase"])
                v = self.project(p + "attn_v.weight", x)
                n = g["kvHeads"] * hd
                s["keys"][self.position * n:(self.position + 1) * n] = k
                s["values"][self.position * n:(self.position + 1) * n] = v
                att = attention(q, s["keys"], s["values"], list(range(self.position + 1)), hd, g["heads"],
                                g["kvHeads"])
                gate = np.array([full[(i // hd) * hd * 2 + hd + i % hd] for i in range(len(att))])
                y = self.project(p + "attn_output.weight", att * sigmoid(gate))
            else:
                cc = conv(s["conv"], self.project(p + "attn_qkv.weight", x), self.w(p + "ssm_conv1d.weight"), 4, 1,
                          True)
                qk = g["ssmDim"] * g["keyHeads"]
                q = norm(cc[:qk], None, g["ssmDim"], l2=True, scale=1 / np.sqrt(g["ssmDim"]))
                k = norm(cc[qk:2 * qk], None, g["ssmDim"], l2=True)
                alpha = self.project(p + "ssm_alpha.weight", x)
                beta = sigmoid(self.project(p + "ssm_beta.weight", x))
                decay = np.exp(self.w(p + "ssm_a") * np.log1p(np.exp(alpha + self.w(p + "ssm_dt.bias"))))
                out = gdn(s["state"], q, k, cc[2 * qk:], decay, beta, g["ssmDim"], g["keyHeads"], g["valueHeads"])
                z = self.project(p + "attn_gate.weight", x)
                n = norm(out, self.w(p + "ssm_norm.weight"), g["ssmDim"])
                y = self.project(p + "ssm_out.weight", n * sigmoid(z))
            self.write(y, self.project(p + "hc_attn_inject.weight", ax))
            fx_, fm = self.hc(p + "hc_ffn_")
            ids, weights, _ = router(self.project(p + "ffn_gate_inp.weight", fm), g["topK"])
            routes.append([int(i) for i in ids])
            output = self.expert(p, fm, True) * sigmoid(self.project(p + "ffn_gate_inp_shexp.weight", fm)[0])
            for e, wk in zip(ids, weights):
                output = output + self.expert(p + "expert.%d." % e, fm) * wk
            self.write(output, self.project(p + "hc_ffn_inject.weight", fx_))
        _, head = self.hc("output_hc_")
        logits = self.project("output.weight", head)
        self.position += 1
        self.previous.append(token)
        if len(self.previous) > 2:
            self.previous.pop(0)
        return int(np.argmax(logits)), logits, routes
