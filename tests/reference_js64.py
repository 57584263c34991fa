"""The reference's float64 test equations (tests/reference.mjs and the
expected-value loops of tests/conformance.js / tests/fused-conformance.js),
restated in plain Python floats with the same operation order as the
JavaScript (sequential reductions, left-to-right products), so that
max |f32 result - expected| comes out as the reference's own conformance run
computed it. Math.exp / sin / cos / pow are the platform's double functions
(within an ulp of V8's), so these expected values can differ from the
reference's in the last bits only.
"""
import math


def sigmoid(x):
    return 1 / (1 + math.exp(-x))


def silu(x):
    return x * sigmoid(x)


def dot(a, b):
    s = 0.0
    for x, y in zip(a, b):
        s = s + x * y
    return s


def mat(weights, x):
    n = len(x)
    return [dot(weights[r * n:(r + 1) * n], x) for r in range(len(weights) // n)]


def norm(x, weights, width, l2=False, scale=1.0):
    y = [0.0] * len(x)
    for r in range(len(x) // width):
        row = x[r * width:(r + 1) * width]
        inverse = scale / math.sqrt(dot(row, row) / (1 if l2 else width) + 1e-6)
        for i in range(width):
            y[r * width + i] = row[i] * inverse * (1 if l2 else weights[(r * width + i) % len(weights)])
    return y


def router(logits, k):
    mx = max(logits)
    p = [math.exp(x - mx) for x in logits]
    total = 0.0
    for v in p:
        total = total + v
    prob = [v / total for v in p]
    ids = sorted(range(len(logits)), key=lambda i: (-prob[i], i))[:k]
    denom = 0.0
    for i in ids:
        denom = denom + prob[i]
    denom = max(denom, 2.0 ** -14)
    return ids, [prob[i] / denom for i in ids]


def conv(history, x, weights, taps, dilation, activate):
    """tests/reference.mjs:19-27; history (a list of floats) is updated in place."""
    span = (taps - 1) * dilation
    y = [0.0] * len(x)
    for c in range(len(x)):
        value = x[c] * weights[c * taps + taps - 1]
        for tap in range(taps - 1):
            value = value + history[c * span + tap * dilation] * weights[c * taps + tap]
        y[c] = silu(value) if activate else value
        if span:
            history[c * span:(c + 1) * span - 1] = history[c * span + 1:(c + 1) * span]
            history[(c + 1) * span - 1] = x[c]
    return y


def gdn(state, q, k, v, decay, beta, dim, key_heads, value_heads):
    """tests/reference.mjs:28-36; state (a list) is updated in place."""
    out = [0.0] * len(v)
    for h in range(value_heads):
        for j in range(dim):
            offset, source = h * dim + j, h % key_heads
            predicted = 0.0
            for i in range(dim):
                ix = (i * value_heads + h) * dim + j
                state[ix] = state[ix] * decay[h]
                predicted = predicted + state[ix] * k[source * dim + i]
            update = beta[h] * (v[offset] - predicted)
            for i in range(dim):
                ix = (i * value_heads + h) * dim + j
                state[ix] = state[ix] + k[source * dim + i] * update
                out[offset] = out[offset] + state[ix] * q[source * dim + i]
    return out


def rope(x, dim, rotary, pos, base):
    y = list(x)
    half = rotary // 2
    for h in range(len(x) // dim):
        for i in range(half):
            a, b = x[h * dim + i], x[h * dim + half + i]
            angle = pos / base ** (2 * i / rotary)
            y[h * dim + i] = a * math.cos(angle) - b * math.sin(angle)
            y[h * dim + half + i] = a * math.sin(angle) + b * math.cos(angle)
    return y


def attention(q, keys, values, cells, dim, heads, kv_heads):
    y = [0.0] * (heads * dim)
    for h in range(heads):
        kh = h // (heads // kv_heads)
        scores = [dot(q[h * dim:(h + 1) * dim], keys[(t * kv_heads + kh) * dim:(t * kv_heads + kh + 1) * dim]) /
                  math.sqrt(dim) for t in cells]
        mx = max(scores)
        probs = [math.exp(s - mx) for s in scores]
        total = 0.0
        for p in probs:
            total = total + p
        for d in range(dim):
            for ti, t in enumerate(cells):
                y[h * dim + d] = y[h * dim + d] + probs[ti] / total * values[(t * kv_heads + kh) * dim + d]
    return y


class ReferenceEngine:
    """tests/reference.mjs:48-95 (ReferenceEngine.step) over an oracle Fixture."""

    def __init__(self, fixture, ngram_rows):
        self.f, self.g, self.ngram_rows = fixture, fixture.config, ngram_rows
        g = self.g
        self.position, self.previous = 0, []
        c = (2 * g["keyHeads"] + g["valueHeads"]) * g["ssmDim"]
        self.states = [dict(state=[0.0] * (g["ssmDim"] * g["valueHeads"] * g["ssmDim"]), conv=[0.0] * (c * 3),
                            keys=[0.0] * (g["context"] * g["kvHeads"] * g["headDim"]),
                            values=[0.0] * (g["context"] * g["kvHeads"] * g["headDim"]))
                       for _ in range(g["layers"])]
        self.history = [0.0] * ((g["pleTaps"] - 1) * g["pleDilation"] * g["width"] * g["streams"])
        self.w = {name: [float(v) for v in self.f.data(name)] for name in self.f.tensors}

    def project(self, name, x):
        return mat(self.w[name], x)

    def hc(self, prefix):
        g = self.g
        W, S = g["width"], g["streams"]
        x = norm(self.r, self.w[prefix + "norm.weight"], W)
        lo = [silu(v / S) for v in self.project(prefix + "down.weight", x)]
        gate = self.project(prefix + "up.weight", lo)
        mixed = []
        for d in range(W):
            s = 0.0
            for c in range(S):
                s = s + x[c * W + d] * sigmoid(gate[c * W + d])
            mixed.append(s / S)
        return x, mixed

    def write(self, y, inject):
        W, S = self.g["width"], self.g["streams"]
        for i in range(len(self.r)):
            self.r[i] = self.r[i] + y[i % W] * 2 * sigmoid(inject[i // W] / S)

    def expert(self, p, x, shared=False):
        name = (lambda r: p + "ffn_" + r + "_shexp.weight") if shared else (lambda r: p + r)
        gate, up = self.project(name("gate"), x), self.project(name("up"), x)
        return self.project(name("down"), [silu(v) * up[i] for i, v in enumerate(gate)])

    def step(self, token):
        g = self.g
        W, hc = g["width"], g["width"] * g["streams"]
        row = self.w["token_embd.weight"][token * W:(token + 1) * W]
        self.r = [row[i % W] for i in range(hc)]
        for l in range(g["layers"]):
            p, s = "blk.%d." % l, self.states[l]
            if l == g["pleLayer"]:
                pr = p + "ple_"
                rows = self.ngram_rows(token, self.previous, self.f.constants, g["eos"])
                tab, hd = self.w["per_layer_token_embd.weight"], g["pleHeadDim"]
                emb = [v for r in rows for v in tab[r * hd:(r + 1) * hd]]
                key = norm(self.project(pr + "key.weight", emb), self.w[pr + "norm_key.weight"], W)
                query = norm(self.r, self.w[pr + "norm_query.weight"], W)
                value = self.project(pr + "value.weight", emb)
                gated = [0.0] * hc
                for c in range(g["streams"]):
                    score = dot(key[c * W:(c + 1) * W], query[c * W:(c + 1) * W]) / math.sqrt(W)
                    sign = 1.0 if score > 0 else (-1.0 if score < 0 else 0.0)
                    gate = sigmoid(sign * math.sqrt(max(abs(score), 1e-6)))
                    for i in range(W):
                        gated[c * W + i] = value[i] * gate
                n = norm(gated, self.w[pr + "norm_conv.weight"], W)
                cv = conv(self.history, n, self.w[pr + "conv1d.weight"], g["pleTaps"], g["pleDilation"], True)
                self.r = [v + gated[i] + cv[i] for i, v in enumerate(self.r)]
            ax, x = self.hc(p + "hc_attn_")
            if l % g["qsaInterval"] == g["qsaInterval"] - 1:
                hd = g["headDim"]
                full = self.project(p + "attn_q.weight", x)
                qraw = [full[(i // hd) * 2 * hd + i % hd] for i in range(g["heads"] * hd)]
                q = rope(norm(qraw, self.w[p + "attn_q_norm.weight"], hd), hd, g["rotary"], self.position,
                         g["ropeBase"])
                k = rope(norm(self.project(p + "attn_k.weight", x), self.w[p + "attn_k_norm.weight"], hd), hd,
                         g["rotary"], self.position, g["ropeBase"])
                v = self.project(p + "attn_v.weight", x)
                n = g["kvHeads"] * hd
                s["keys"][self.position * n:(self.position + 1) * n] = k
                s["values"][self.position * n:(self.position + 1) * n] = v
                att = attention(q, s["keys"], s["values"], list(range(self.position + 1)), hd, g["heads"],
                                g["kvHeads"])
                y = self.project(p + "attn_output.weight",
                                 [a * sigmoid(full[(i // hd) * hd * 2 + hd + i % hd]) for i, a in enumerate(att)])
            else:
                cc = conv(s["conv"], self.project(p + "attn_qkv.weight", x), self.w[p + "ssm_conv1d.weight"], 4, 1,
                          True)
                qk = g["ssmDim"] * g["keyHeads"]
                q = norm(cc[:qk], None, g["ssmDim"], l2=True, scale=1 / math.sqrt(g["ssmDim"]))
                k = norm(cc[qk:2 * qk], None, g["ssmDim"], l2=True)
                alpha = self.project(p + "ssm_alpha.weight", x)
                beta = [sigmoid(v) for v in self.project(p + "ssm_beta.weight", x)]
                wa, dt = self.w[p + "ssm_a"], self.w[p + "ssm_dt.bias"]
                decay = [math.exp(wa[i] * math.log1p(math.exp(a + dt[i]))) for i, a in enumerate(alpha)]
                out = gdn(s["state"], q, k, cc[2 * qk:], decay, beta, g["ssmDim"], g["keyHeads"], g["valueHeads"])
                z = self.project(p + "attn_gate.weight", x)
                n = norm(out, self.w[p + "ssm_norm.weight"], g["ssmDim"])
                y = self.project(p + "ssm_out.weight", [v * sigmoid(z[i]) for i, v in enumerate(n)])
            self.write(y, self.project(p + "hc_attn_inject.weight", ax))
            fx_, fm = self.hc(p + "hc_ffn_")
            ids, weights = router(self.project(p + "ffn_gate_inp.weight", fm), g["topK"])
            sg = sigmoid(self.project(p + "ffn_gate_inp_shexp.weight", fm)[0])
            output = [v * sg for v in self.expert(p, fm, True)]
            for e, wk in zip(ids, weights):
                part = self.expert(p + "expert.%d." % e, fm)
                for d in range(g["width"]):
                    output[d] = output[d] + part[d] * wk
            self.write(output, self.project(p + "hc_ffn_inject.weight", fx_))
        _, head = self.hc("output_hc_")
        logits = self.project("output.weight", head)
        self.position += 1
        self.previous.append(token)
        if len(self.previous) > 2:
            self.previous.pop(0)
        return logits.index(max(logits)), logits
