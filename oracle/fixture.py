"""The reference's untrained fixture model and a CPU restatement of its decode.

TEST INFRASTRUCTURE ONLY (the oracle): imported by tests/ as the checker.

``create_fixture(seed)`` restates ``createFixture`` (src/fixture.js:3-33): the
same geometry, the same LCG (``state = state * 1664525 + 1013904223 mod 2^32``,
``rnd = state / 2^32 * 2 - 1`` in double), the same tensor creation order and
value rules, each value rounded once to float32.

``OracleEngine`` restates ``StrataEngine.step`` (src/engine.js:76-196) for the
single-backend case: the same kernel sequence, arguments and host logic (the
PLE n-gram rows of src/model.js:22-32, the routing check of
src/engine.js:137-138), with every kernel evaluated by the oracle's C
restatements. Its results are pinned by the reference's own known answers
(reports/wasm.json:172-178, reports/validation.md:25) and by the float64
equations of tests/reference.mjs (tests/reference_f64.py).
"""
import math

import numpy as np

from . import (argmax, attention, attention_batch, attention_gate, attention_gate_batch, conv, conv_batch, elementwise,
               embedding, gather_rows, gdn_batch, gdn_gates, gdn_gates_batch, gdn_step, hc_mix, hc_mix_batch, hc_write,
               hc_write_batch, kv_append, kv_append_batch, moe_combine, norm, ple_add, ple_broadcast,
               ple_broadcast_batch, ple_gate, project, rope_frequencies, rope_position, rope_table, router,
               scatter_rows, slice_)

# src/fixture.js:4-6
GEOMETRY = dict(width=32, streams=2, rank=8, layers=4, qsaInterval=4, ssmDim=8, keyHeads=2, valueHeads=4, heads=4,
                kvHeads=2, headDim=8, rotary=8, experts=6, topK=2, ff=24, vocab=40, context=32, pleLayer=1,
                pleHeads=4, pleHeadDim=8, pleTaps=4, pleDilation=3, ropeBase=1e7, eos=39)
# src/fixture.js:31
PLE_CONSTANTS = dict(multipliers=[23703573157769, 20109073645365, 8052911324071], vocab=[17, 19, 23, 29],
                     offsets=[0, 17, 36, 59])


class Fixture:
    """Tensors by name (float32, flat, shape as created) plus geometry."""

    def __init__(self, config, tensors, constants):
        self.config, self.tensors, self.constants = config, tensors, constants

    def shape(self, name):
        return self.tensors[name][0]

    def data(self, name):
        return self.tensors[name][1]


def create_fixture(seed=1234):
    g = dict(GEOMETRY)
    state = seed & 0xFFFFFFFF
    tensors = {}

    def rnd():
        nonlocal state
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        return state / 4294967296 * 2 - 1

    def add(name, shape, mode="weight"):
        n = int(np.prod(shape))
        vals = np.empty(n, np.float64)
        scale = 0.4 if mode == "embedding" else 0.3 / math.sqrt(shape[0])
        for i in range(n):
            if mode == "norm":
                vals[i] = 1 + rnd() * 0.05
            elif mode == "negative":
                vals[i] = -0.1 - abs(rnd())
            else:
                vals[i] = rnd() * scale
        tensors[name] = (list(shape), vals.astype(np.float32))

    hc = g["width"] * g["streams"]

    def gr(prefix):
        add(prefix + "norm.weight", [hc], "norm")
        add(prefix + "down.weight", [hc, g["rank"]])
        add(prefix + "up.weight", [g["rank"], hc])
        add(prefix + "inject.weight", [hc, g["streams"]])

    add("token_embd.weight", [g["width"], g["vocab"]], "embedding")
    gr("output_hc_")
    add("output.weight", [g["width"], g["vocab"]])
    for l in range(g["layers"]):
        p = "blk.%d." % l
        gr(p + "hc_attn_")
        gr(p + "hc_ffn_")
        add(p + "ffn_gate_inp.weight", [g["width"], g["experts"]])
        add(p + "ffn_gate_inp_shexp.weight", [g["width"], 1])
        for role in ("gate", "up", "down"):
            add(p + "ffn_" + role + "_shexp.weight", [g["ff"], g["width"]] if role == "down" else [g["width"], g["ff"]])
        for e in range(g["experts"]):
            for role in ("gate", "up", "down"):
                add(p + "expert.%d.%s" % (e, role), [g["ff"], g["width"]] if role == "down" else [g["width"], g["ff"]])
        if l % g["qsaInterval"] == g["qsaInterval"] - 1:
            add(p + "attn_q.weight", [g["width"], 2 * g["heads"] * g["headDim"]])
            add(p + "attn_k.weight", [g["width"], g["kvHeads"] * g["headDim"]])
            add(p + "attn_v.weight", [g["width"], g["kvHeads"] * g["headDim"]])
            add(p + "attn_output.weight", [g["heads"] * g["headDim"], g["width"]])
            add(p + "attn_q_norm.weight", [g["headDim"]], "norm")
            add(p + "attn_k_norm.weight", [g["headDim"]], "norm")
        else:
            c = (2 * g["keyHeads"] + g["valueHeads"]) * g["ssmDim"]
            add(p + "attn_qkv.weight", [g["width"], c])
            add(p + "attn_gate.weight", [g["width"], g["ssmDim"] * g["valueHeads"]])
            add(p + "ssm_out.weight", [g["ssmDim"] * g["valueHeads"], g["width"]])
            add(p + "ssm_alpha.weight", [g["width"], g["valueHeads"]])
            add(p + "ssm_beta.weight", [g["width"], g["valueHeads"]])
            add(p + "ssm_conv1d.weight", [4, c])
            add(p + "ssm_norm.weight", [g["ssmDim"]], "norm")
            add(p + "ssm_dt.bias", [g["valueHeads"]])
            add(p + "ssm_a", [g["valueHeads"]], "negative")
    p = "blk.%d.ple_" % g["pleLayer"]
    add(p + "key.weight", [g["width"], hc])
    add(p + "value.weight", [g["width"], g["width"]])
    for n in ("norm_key", "norm_query", "norm_conv"):
        add(p + n + ".weight", [hc], "norm")
    add(p + "conv1d.weight", [g["pleTaps"], hc])
    add("per_layer_token_embd.weight", [g["pleHeadDim"], 88], "embedding")
    return Fixture(g, tensors, dict(PLE_CONSTANTS))


def ngram_rows(token, previous, constants, eos):
    """src/model.js:22-32: the PLE row of each head from the token and up to
    two previous tokens (EOS once the history is cut), 64-bit products."""
    ctx = [token]
    cut = False
    for back in (1, 2):
        t = previous[-back] if back <= len(previous) else -1
        cut = cut or t < 0 or t == eos
        ctx.append(eos if cut else t)
    vocab, offsets, mult = constants["vocab"], constants["offsets"], constants["multipliers"]
    n = len(vocab)
    if n % 2 or len(offsets) != n:
        raise ValueError("Invalid n-gram constants")
    terms = [(t * int(mult[i])) & 0xFFFFFFFFFFFFFFFF for i, t in enumerate(ctx)]
    out = []
    for i, v in enumerate(vocab):
        mixed = terms[0] ^ terms[1] if i < n // 2 else terms[0] ^ terms[1] ^ terms[2]
        out.append(mixed % v + offsets[i])
    return out


class OracleEngine:
    """StrataEngine.step on the oracle's kernels (src/engine.js:54-196)."""

    def __init__(self, fixture):
        self.f = fixture
        g = self.g = fixture.config
        self.position = 0
        self.previous = []
        c = (2 * g["keyHeads"] + g["valueHeads"]) * g["ssmDim"]
        self.residual = np.zeros(g["width"] * g["streams"], np.float32)
        self.ple_history = np.zeros((g["pleTaps"] - 1) * g["pleDilation"] * g["width"] * g["streams"], np.float32)
        self.states = []
        for l in range(g["layers"]):
            if l % g["qsaInterval"] == g["qsaInterval"] - 1:
                n = g["context"] * g["kvHeads"] * g["headDim"]
                self.states.append({"keys": np.zeros(n, np.float32), "values": np.zeros(n, np.float32)})
            else:
                self.states.append({"state": np.zeros(g["ssmDim"] * g["valueHeads"] * g["ssmDim"], np.float32),
                                    "conv": np.zeros(c * 3, np.float32)})
        self.rope = None
        self.routes = []

    # Ops (src/ops.js): mat is one strata_project over all rows (the fixture's
    # tiles hold every row), vector the tensor itself.
    def mat(self, name, x):
        shape = self.f.shape(name)
        cols, rows = shape[0], int(np.prod(shape[1:]))
        if len(x) != cols:
            raise ValueError("%s: expected %d inputs, got %d" % (name, cols, len(x)))
        return project(x, self.f.data(name), cols, rows, 1)

    def vec(self, name):
        return self.f.data(name)

    def hc(self, prefix, inject=True):
        g = self.g
        n = norm(self.residual, self.vec(prefix + "norm.weight"), g["width"], g["streams"], g["streams"])
        down = self.mat(prefix + "down.weight", n)
        lo = elementwise(down, down, 1, np.float32(1 / g["streams"]))
        gate = self.mat(prefix + "up.weight", lo)
        mixed = hc_mix(n, gate, g["width"], g["streams"])
        return mixed, (self.mat(prefix + "inject.weight", n) if inject else None)

    def hc_write(self, output, inject):
        hc_write(self.residual, output, inject, self.g["width"], self.g["streams"])

    def ple(self, token):
        g, p = self.g, "blk.%d.ple_" % self.g["pleLayer"]
        rows = ngram_rows(token, self.previous, self.f.constants, g["eos"])
        table, hd = self.f.data("per_layer_token_embd.weight"), g["pleHeadDim"]
        emb = np.concatenate([table[r * hd:(r + 1) * hd] for r in rows]).astype(np.float32)
        key = norm(self.mat(p + "key.weight", emb), self.vec(p + "norm_key.weight"), g["width"], g["streams"],
                   g["streams"])
        query = norm(self.residual, self.vec(p + "norm_query.weight"), g["width"], g["streams"], g["streams"])
        value = self.mat(p + "value.weight", emb)
        gate = ple_gate(key, query, g["width"], g["streams"])
        gated = ple_broadcast(value, gate, g["width"], g["streams"])
        n = norm(gated, self.vec(p + "norm_conv.weight"), g["width"], g["streams"], g["streams"])
        cv = conv(self.ple_history, n, self.vec(p + "conv1d.weight"), g["width"] * g["streams"], g["pleTaps"],
                  g["pleDilation"], 1)
        ple_add(self.residual, gated, cv, g["width"] * g["streams"])

    def gdn(self, layer, x):
        g, p, st = self.g, "blk.%d." % layer, self.states[layer]
        qk, vn = g["ssmDim"] * g["keyHeads"], g["ssmDim"] * g["valueHeads"]
        c = 2 * qk + vn
        qkv = self.mat(p + "attn_qkv.weight", x)
        cv = conv(st["conv"], qkv, self.vec(p + "ssm_conv1d.weight"), c, 4, 1, 1)
        qr, kr, v = slice_(cv, qk), slice_(cv, qk, 1, qk, qk), slice_(cv, vn, 1, vn, 2 * qk)
        q = norm(qr, qr, g["ssmDim"], g["keyHeads"], 1, 1, 1e-6, np.float32(1 / math.sqrt(g["ssmDim"])))
        k = norm(kr, kr, g["ssmDim"], g["keyHeads"], 1, 1)
        alpha, beta = self.mat(p + "ssm_alpha.weight", x), self.mat(p + "ssm_beta.weight", x)
        decay, strength = gdn_gates(alpha, beta, self.vec(p + "ssm_a"), self.vec(p + "ssm_dt.bias"), g["valueHeads"])
        y = gdn_step(st["state"], q, k, v, decay, strength, g["ssmDim"], g["keyHeads"], g["valueHeads"])
        z = self.mat(p + "attn_gate.weight", x)
        n = norm(y, self.vec(p + "ssm_norm.weight"), g["ssmDim"], g["valueHeads"])
        return self.mat(p + "ssm_out.weight", elementwise(n, z, 4))

    def rotate(self, x, heads):
        g = self.g
        if self.rope is None:
            hi, lo = rope_frequencies(g["rotary"], g["ropeBase"])
            self.rope = rope_table(hi, lo, g["rotary"], g["context"])
        return rope_position(x, self.rope[0], self.rope[1], g["headDim"], heads, g["rotary"], self.position)

    def qsa(self, layer, x):
        g, p, st = self.g, "blk.%d." % layer, self.states[layer]
        hd = g["headDim"]
        full = self.mat(p + "attn_q.weight", x)
        qr = slice_(full, hd, g["heads"], hd * 2)
        q = self.rotate(norm(qr, self.vec(p + "attn_q_norm.weight"), hd, g["heads"]), g["heads"])
        kr = self.mat(p + "attn_k.weight", x)
        k = self.rotate(norm(kr, self.vec(p + "attn_k_norm.weight"), hd, g["kvHeads"]), g["kvHeads"])
        v = self.mat(p + "attn_v.weight", x)
        kv_append(k, v, st["keys"], st["values"], g["kvHeads"] * hd, self.position)
        cells = np.arange(self.position + 1, dtype=np.int32)
        attn = attention(q, st["keys"], st["values"], cells, hd, g["heads"], g["kvHeads"], self.position + 1,
                         np.float32(1 / math.sqrt(hd)))
        return self.mat(p + "attn_output.weight", attention_gate(attn, full, hd, g["heads"]))

    def expert(self, prefix, x, shared=False):
        name = (lambda r: prefix + "ffn_" + r + "_shexp.weight") if shared else (lambda r: prefix + r)
        gate, up = self.mat(name("gate"), x), self.mat(name("up"), x)
        return self.mat(name("down"), elementwise(gate, up, 3))

    def moe(self, layer, x):
        g, p = self.g, "blk.%d." % layer
        logits = self.mat(p + "ffn_gate_inp.weight", x)
        ids, weights = router(logits, g["experts"], g["topK"])
        if any(i < 0 or i >= g["experts"] for i in ids) or len(set(ids.tolist())) != g["topK"]:
            raise RuntimeError("Invalid expert routing result")
        self.routes.append({"layer": layer, "ids": [int(i) for i in ids]})
        parts = np.concatenate([self.expert(p + "expert.%d." % e, x) for e in ids]).astype(np.float32)
        shared = self.expert(p, x, True)
        shared_gate = self.mat(p + "ffn_gate_inp_shexp.weight", x)
        return moe_combine(parts, weights, shared, shared_gate, g["width"], g["topK"])

    def step(self, token, predict=True):
        """One decode step; returns (argmax token or None, logits or None)."""
        g = self.g
        if not (0 <= token < g["vocab"]):
            raise ValueError("token must be an integer in [0, %d]" % (g["vocab"] - 1))
        if self.position >= g["context"]:
            raise RuntimeError("Context capacity reached")
        self.routes = []
        w = g["width"]
        embedding(self.residual, w, g["streams"], values=self.f.data("token_embd.weight")[token * w:(token + 1) * w])
        for l in range(g["layers"]):
            if l == g["pleLayer"]:
                self.ple(token)
            mixed, inject = self.hc("blk.%d.hc_attn_" % l)
            out = self.qsa(l, mixed) if l % g["qsaInterval"] == g["qsaInterval"] - 1 else self.gdn(l, mixed)
            self.hc_write(out, inject)
            mixed, inject = self.hc("blk.%d.hc_ffn_" % l)
            self.hc_write(self.moe(l, mixed), inject)
        token_out = logits = None
        if predict:
            head, _ = self.hc("output_hc_", False)
            logits = self.mat("output.weight", head)
            token_out = argmax(logits, g["vocab"])
        self.previous.append(token)
        if len(self.previous) > 2:
            self.previous.pop(0)
        self.position += 1
        return token_out, logits


class OraclePromptBatch:
    """PromptBatch (src/prefill.js:5-97): one chunk of prompt tokens through
    every layer, layer-major, with the batched kernels and per-expert row
    groups, on an OracleEngine's state."""

    def __init__(self, engine, tokens):
        self.e, self.g, self.tokens, self.n = engine, engine.g, list(tokens), len(tokens)
        self.position = engine.position

    def mat(self, name, x):
        shape = self.e.f.shape(name)
        cols, rows = shape[0], int(np.prod(shape[1:]))
        return project(x, self.e.f.data(name), cols, rows, self.n)

    def hc(self, prefix, inject=True):
        g, n = self.g, self.n
        nm = norm(self.residual, self.e.vec(prefix + "norm.weight"), g["width"], n * g["streams"], g["streams"])
        down = self.mat(prefix + "down.weight", nm)
        lo = elementwise(down, down, 1, np.float32(1 / g["streams"]))
        gate = self.mat(prefix + "up.weight", lo)
        mixed = hc_mix_batch(nm, gate, g["width"], g["streams"], n)
        return mixed, (self.mat(prefix + "inject.weight", nm) if inject else None)

    def write(self, output, inject):
        hc_write_batch(self.residual, output, inject, self.g["width"], self.g["streams"], self.n)

    def ple(self):
        g, n, e = self.g, self.n, self.e
        p, hc = "blk.%d.ple_" % g["pleLayer"], g["width"] * g["streams"]
        previous, rows = list(e.previous), []
        table, hd = e.f.data("per_layer_token_embd.weight"), g["pleHeadDim"]
        for t in self.tokens:
            r = ngram_rows(t, previous, e.f.constants, g["eos"])
            rows.append(np.concatenate([table[i * hd:(i + 1) * hd] for i in r]))
            previous.append(t)
            if len(previous) > 2:
                previous.pop(0)
        emb = np.concatenate(rows).astype(np.float32)
        key = norm(self.mat(p + "key.weight", emb), e.vec(p + "norm_key.weight"), g["width"], n * g["streams"],
                   g["streams"])
        query = norm(self.residual, e.vec(p + "norm_query.weight"), g["width"], n * g["streams"], g["streams"])
        value = self.mat(p + "value.weight", emb)
        gate = ple_gate(key, query, g["width"], n * g["streams"])
        gated = ple_broadcast_batch(value, gate, g["width"], g["streams"], n)
        nm = norm(gated, e.vec(p + "norm_conv.weight"), g["width"], n * g["streams"], g["streams"])
        cv = conv_batch(e.ple_history, nm, e.vec(p + "conv1d.weight"), hc, g["pleTaps"], g["pleDilation"], 1, n)
        ple_add(self.residual, gated, cv, n * hc)

    def gdn(self, layer, x):
        g, n, e = self.g, self.n, self.e
        p, st = "blk.%d." % layer, e.states[layer]
        qk, vn = g["ssmDim"] * g["keyHeads"], g["ssmDim"] * g["valueHeads"]
        c = 2 * qk + vn
        qkv = self.mat(p + "attn_qkv.weight", x)
        cv = conv_batch(st["conv"], qkv, e.vec(p + "ssm_conv1d.weight"), c, 4, 1, 1, n)
        qr, kr, v = slice_(cv, qk, n, c), slice_(cv, qk, n, c, qk), slice_(cv, vn, n, c, 2 * qk)
        q = norm(qr, qr, g["ssmDim"], n * g["keyHeads"], 1, 1, 1e-6, np.float32(1 / math.sqrt(g["ssmDim"])))
        k = norm(kr, kr, g["ssmDim"], n * g["keyHeads"], 1, 1)
        alpha, beta = self.mat(p + "ssm_alpha.weight", x), self.mat(p + "ssm_beta.weight", x)
        decay, strength = gdn_gates_batch(alpha, beta, e.vec(p + "ssm_a"), e.vec(p + "ssm_dt.bias"), g["valueHeads"], n)
        y = gdn_batch(st["state"], q, k, v, decay, strength, g["ssmDim"], g["keyHeads"], g["valueHeads"], n)
        z = self.mat(p + "attn_gate.weight", x)
        nm = norm(y, e.vec(p + "ssm_norm.weight"), g["ssmDim"], n * g["valueHeads"])
        return self.mat(p + "ssm_out.weight", elementwise(nm, z, 4))

    def rotate(self, x, heads):
        g, e = self.g, self.e
        if e.rope is None:
            hi, lo = rope_frequencies(g["rotary"], g["ropeBase"])
            e.rope = rope_table(hi, lo, g["rotary"], g["context"])
        return rope_position(x, e.rope[0], e.rope[1], g["headDim"], heads, g["rotary"], self.position, self.n)

    def qsa(self, layer, x):
        g, n, e = self.g, self.n, self.e
        p, st, hd = "blk.%d." % layer, e.states[layer], g["headDim"]
        full = self.mat(p + "attn_q.weight", x)
        qr = slice_(full, hd, n * g["heads"], hd * 2)
        q = self.rotate(norm(qr, e.vec(p + "attn_q_norm.weight"), hd, n * g["heads"]), g["heads"])
        kr = self.mat(p + "attn_k.weight", x)
        k = self.rotate(norm(kr, e.vec(p + "attn_k_norm.weight"), hd, n * g["kvHeads"]), g["kvHeads"])
        v = self.mat(p + "attn_v.weight", x)
        kv_append_batch(k, v, st["keys"], st["values"], g["kvHeads"] * hd, self.position, n)
        attn = attention_batch(q, st["keys"], st["values"], hd, g["heads"], g["kvHeads"], self.position,
                               np.float32(1 / math.sqrt(hd)), n)
        return self.mat(p + "attn_output.weight", attention_gate_batch(attn, full, hd, g["heads"], n))

    def expert(self, prefix, x, tokens, shared=False):
        name = (lambda r: prefix + "ffn_" + r + "_shexp.weight") if shared else (lambda r: prefix + r)

        def m(nm, v):
            shape = self.e.f.shape(nm)
            return project(v, self.e.f.data(nm), shape[0], int(np.prod(shape[1:])), tokens)
        return m(name("down"), elementwise(m(name("gate"), x), m(name("up"), x), 3))

    def moe(self, layer, x):
        g, n, e = self.g, self.n, self.e
        p, K, W = "blk.%d." % layer, g["topK"], g["width"]
        logits = self.mat(p + "ffn_gate_inp.weight", x)
        ids, weights = router(logits, g["experts"], K, n)
        groups = {}
        for t in range(n):
            row = [int(i) for i in ids[t * K:(t + 1) * K]]
            if any(i < 0 or i >= g["experts"] for i in row) or len(set(row)) != K:
                raise RuntimeError("Invalid prompt expert routing")
            e.routes.append({"position": self.position + t, "layer": layer, "ids": row})
            for k, i in enumerate(row):
                groups.setdefault(i, []).append((t, t * K + k))
        parts = np.zeros(n * K * W, np.float32)
        for i, jobs in groups.items():
            inp = gather_rows(x, np.array([j[0] for j in jobs], np.int32), W, len(jobs))
            out = self.expert(p + "expert.%d." % i, inp, len(jobs))
            scatter_rows(out, np.array([j[1] for j in jobs], np.int32), parts, W, len(jobs))
        shared = self.expert(p, x, n, True)
        shared_gate = self.mat(p + "ffn_gate_inp_shexp.weight", x)
        return moe_combine(parts, weights, shared, shared_gate, W, K, n)

    def run(self):
        g, n, e = self.g, self.n, self.e
        hc = g["width"] * g["streams"]
        self.residual = np.zeros(n * hc, np.float32)
        emb, w = e.f.data("token_embd.weight"), g["width"]
        for t, tok in enumerate(self.tokens):
            self.residual[t * hc:(t + 1) * hc] = np.tile(emb[tok * w:(tok + 1) * w], g["streams"])
        for l in range(g["layers"]):
            if l == g["pleLayer"]:
                self.ple()
            mixed, inject = self.hc("blk.%d.hc_attn_" % l)
            out = self.qsa(l, mixed) if l % g["qsaInterval"] == g["qsaInterval"] - 1 else self.gdn(l, mixed)
            self.write(out, inject)
            mixed, inject = self.hc("blk.%d.hc_ffn_" % l)
            self.write(self.moe(l, mixed), inject)
        e.residual[:] = self.residual[(n - 1) * hc:]
        e.position += n
        e.previous = (e.previous + self.tokens)[-2:]


def prefill(engine, tokens, chunk_size=16, predict=True):
    """prefillChunks (src/prefill.js:99-111): chunks of the prompt through
    OraclePromptBatch, then the head on the last token's residual."""
    engine.routes = []
    tokens = list(tokens)
    for off in range(0, len(tokens), chunk_size):
        OraclePromptBatch(engine, tokens[off:off + chunk_size]).run()
    if not predict:
        return None, None
    head, _ = engine.hc("output_hc_", False)
    logits = engine.mat("output.weight", head)
    return argmax(logits, engine.g["vocab"]), logits
