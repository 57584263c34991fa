// StrataEngine: the reference's decode driver (src/engine.js:7-223) on one
// MI355X through HipBackend. Token step, layer loop, hyper-connection
// mix/write-back, gated-delta-rule and attention layers, PLE, the MoE stage,
// output head and greedy argmax run in the reference's kernel order with the
// reference's kernel names and arguments; the session API (step, reset,
// checkpoint, restore, dispose) and its error conventions are the same.
//
// Differences, all from the one-GPU, all-resident design: there is no CPU
// expert lane or hot-expert promotion (src/engine.js:21-29,147-153), every
// model tensor is resident in HBM from initialize() on (ModelResidency), and
// the MoE stage of a Q2-packed store uses the resident blobs. Written for
// Node 12 (no `?.`, `??`, or private fields).
import crypto from 'crypto';
import {performance} from 'perf_hooks';
import {Ops, grid} from './ops.js';
import {validateGeometry} from './model.js';
import {ModelResidency} from './residency.js';
import {prefillChunks} from './prefill.js';

const shapeKey = shape => {
    const s = Array.from(shape);
    while (s.length > 1 && s[s.length - 1] === 1) s.pop();
    return String(s);
};

export class StrataEngine {
    static async create(store, backend, options) {
        const engine = new StrataEngine(store, backend, options);
        try { await engine.initialize(); return engine; } catch (error) { await engine.dispose(); throw error; }
    }
    constructor(store, backend) {
        this.store = store; this.g = validateGeometry(store.config); this.b = backend;
        this.ops = new Ops(backend, store);
        this.position = 0; this.previous = []; this.states = []; this.persistent = [];
        this.busy = false; this.failed = false; this.disposed = false;
        this.checkpointOwner = crypto.randomBytes(16).toString('hex');
        this.stats = {tokens: 0, gpuExperts: 0, cpuExperts: 0, promotions: 0, routes: [], lastMs: 0};
    }
    keep(n) { const b = this.b.alloc(n, 'f32', {zero: true}); this.persistent.push(b); return b; }
    assertIdle(message) { if (this.disposed) throw Error('Session is disposed'); if (this.busy) throw Error(message); }
    // src/engine.js:31-53: every tensor the step reads, with its shape.
    expectedShapes() {
        const g = this.g, hc = g.width * g.streams, c = (2 * g.keyHeads + g.valueHeads) * g.ssmDim, specs = [];
        const add = (name, shape) => specs.push([name, shape]);
        const gr = (prefix, inject) => {
            add(prefix + 'norm.weight', [hc]); add(prefix + 'down.weight', [hc, g.rank]); add(prefix + 'up.weight', [g.rank, hc]);
            if (inject !== false) add(prefix + 'inject.weight', [hc, g.streams]);
        };
        add('token_embd.weight', [g.width, g.vocab]); add('output.weight', [g.width, g.vocab]); gr('output_hc_', false);
        for (let l = 0; l < g.layers; l++) {
            const p = 'blk.' + l + '.';
            gr(p + 'hc_attn_'); gr(p + 'hc_ffn_');
            add(p + 'ffn_gate_inp.weight', [g.width, g.experts]); add(p + 'ffn_gate_inp_shexp.weight', [g.width]);
            for (const role of ['gate', 'up', 'down'])
                add(p + 'ffn_' + role + '_shexp.weight', role === 'down' ? [g.ff, g.width] : [g.width, g.ff]);
            for (let e = 0; e < g.experts; e++)
                for (const role of ['gate', 'up', 'down'])
                    add(p + 'expert.' + e + '.' + role, role === 'down' ? [g.ff, g.width] : [g.width, g.ff]);
            if (l % g.qsaInterval === g.qsaInterval - 1) {
                add(p + 'attn_q.weight', [g.width, 2 * g.heads * g.headDim]); add(p + 'attn_k.weight', [g.width, g.kvHeads * g.headDim]);
                add(p + 'attn_v.weight', [g.width, g.kvHeads * g.headDim]); add(p + 'attn_output.weight', [g.heads * g.headDim, g.width]);
                add(p + 'attn_q_norm.weight', [g.headDim]); add(p + 'attn_k_norm.weight', [g.headDim]);
            } else {
                add(p + 'attn_qkv.weight', [g.width, c]); add(p + 'attn_gate.weight', [g.width, g.valueHeads * g.ssmDim]);
                add(p + 'ssm_out.weight', [g.valueHeads * g.ssmDim, g.width]); add(p + 'ssm_conv1d.weight', [4, c]);
                add(p + 'ssm_alpha.weight', [g.width, g.valueHeads]); add(p + 'ssm_beta.weight', [g.width, g.valueHeads]);
                add(p + 'ssm_a', [g.valueHeads]); add(p + 'ssm_dt.bias', [g.valueHeads]); add(p + 'ssm_norm.weight', [g.ssmDim]);
            }
        }
        const p = 'blk.' + g.pleLayer + '.ple_';
        add(p + 'key.weight', [g.width, hc]); add(p + 'value.weight', [g.width, g.width]);
        for (const suffix of ['norm_key', 'norm_query', 'norm_conv']) add(p + suffix + '.weight', [hc]);
        add(p + 'conv1d.weight', [g.pleTaps, hc]);
        return specs;
    }
    // src/engine.js:54-75: shape gates before any allocation, then the
    // resident weights and the persistent recurrent, KV and PLE state.
    async initialize() {
        for (const [name, expected] of this.expectedShapes()) {
            const shape = this.store.describe(name).shape;
            if (shapeKey(shape) !== shapeKey(expected))
                throw Error(name + ': expected [' + expected + '], found [' + shape + ']');
        }
        const g = this.g, c = (2 * g.keyHeads + g.valueHeads) * g.ssmDim;
        await new ModelResidency(this.ops).loadAll();
        this.residual = this.keep(g.width * g.streams);
        this.pleHistory = this.keep((g.pleTaps - 1) * g.pleDilation * g.width * g.streams);
        for (let l = 0; l < g.layers; l++) {
            this.states.push(l % g.qsaInterval === g.qsaInterval - 1
                ? {keys: this.keep(g.context * g.kvHeads * g.headDim), values: this.keep(g.context * g.kvHeads * g.headDim)}
                : {state: this.keep(g.ssmDim * g.valueHeads * g.ssmDim), conv: this.keep(c * 3)});
        }
    }
    // src/engine.js:76-83: RMSNorm of each stream, low-rank gate, stream mix.
    async hc(prefix, inject) {
        const g = this.g, o = this.ops;
        const norm = await o.norm(this.residual, await o.vector(prefix + 'norm.weight'), g.width, g.streams, g.streams);
        const down = await o.mat(prefix + 'down.weight', norm), lo = await o.elem(down, down, 1, 1 / g.streams);
        const gate = await o.mat(prefix + 'up.weight', lo), mixed = await o.alloc(g.width);
        await this.b.run('strata_hc_mix', {Norm: norm, Gate: gate, Mixed: mixed, width: g.width, streams: g.streams},
            grid(g.width));
        return {mixed, inject: inject !== false ? await o.mat(prefix + 'inject.weight', norm) : null};
    }
    async hcWrite(output, inject) {
        const g = this.g;
        await this.b.run('strata_hc_write', {Residual: this.residual, Output: output, Inject: inject, width: g.width,
            streams: g.streams}, grid(g.width * g.streams));
    }
    // src/engine.js:86-96: per-layer embedding gate, convolution and add.
    async ple(token) {
        const g = this.g, o = this.ops, b = this.b, p = 'blk.' + g.pleLayer + '.ple_', hc = g.width * g.streams;
        const emb = await o.ple(token, this.previous);
        const rawKey = await o.mat(p + 'key.weight', emb);
        const key = await o.norm(rawKey, await o.vector(p + 'norm_key.weight'), g.width, g.streams, g.streams);
        const query = await o.norm(this.residual, await o.vector(p + 'norm_query.weight'), g.width, g.streams, g.streams);
        const value = await o.mat(p + 'value.weight', emb), gate = await o.alloc(g.streams), gated = await o.alloc(hc);
        await b.run('strata_ple_gate', {Key: key, Query: query, Gate: gate, width: g.width, streams: g.streams},
            [g.streams, 1, 1]);
        await b.run('strata_ple_broadcast', {Value: value, Gate: gate, Y: gated, width: g.width, streams: g.streams},
            grid(hc));
        const norm = await o.norm(gated, await o.vector(p + 'norm_conv.weight'), g.width, g.streams, g.streams);
        const conv = await o.alloc(hc);
        await b.run('strata_conv', {History: this.pleHistory, X: norm, W: await o.vector(p + 'conv1d.weight'), Y: conv,
            channels: hc, taps: g.pleTaps, dilation: g.pleDilation, activation: 1}, grid(hc));
        await b.run('strata_ple_add', {Residual: this.residual, Gated: gated, Conv: conv, n: hc}, grid(hc));
    }
    // src/engine.js:97-111: gated delta-rule layer.
    async gdn(layer, x) {
        const g = this.g, o = this.ops, b = this.b, p = 'blk.' + layer + '.', st = this.states[layer];
        const qk = g.ssmDim * g.keyHeads, vn = g.ssmDim * g.valueHeads, c = 2 * qk + vn;
        const qkv = await o.mat(p + 'attn_qkv.weight', x), convolved = await o.alloc(c);
        await b.run('strata_conv', {History: st.conv, X: qkv, W: await o.vector(p + 'ssm_conv1d.weight'), Y: convolved,
            channels: c, taps: 4, dilation: 1, activation: 1}, grid(c));
        const qr = await o.slice(convolved, qk), kr = await o.slice(convolved, qk, 1, qk, qk);
        const v = await o.slice(convolved, vn, 1, vn, 2 * qk);
        const q = await o.norm(qr, qr, g.ssmDim, g.keyHeads, 1, 1, 1 / Math.sqrt(g.ssmDim));
        const k = await o.norm(kr, kr, g.ssmDim, g.keyHeads, 1, 1);
        const alpha = await o.mat(p + 'ssm_alpha.weight', x), beta = await o.mat(p + 'ssm_beta.weight', x);
        const decay = await o.alloc(g.valueHeads), strength = await o.alloc(g.valueHeads);
        await b.run('strata_gdn_gates', {Alpha: alpha, Beta: beta, A: await o.vector(p + 'ssm_a'),
            Dt: await o.vector(p + 'ssm_dt.bias'), Decay: decay, Strength: strength, heads: g.valueHeads}, grid(g.valueHeads));
        const y = await o.alloc(vn);
        await b.run('strata_gdn_step', {State: st.state, Q: q, K: k, V: v, Decay: decay, Beta: strength, Y: y,
            dim: g.ssmDim, keyHeads: g.keyHeads, valueHeads: g.valueHeads}, grid(vn));
        const z = await o.mat(p + 'attn_gate.weight', x);
        const norm = await o.norm(y, await o.vector(p + 'ssm_norm.weight'), g.ssmDim, g.valueHeads);
        return o.mat(p + 'ssm_out.weight', await o.elem(norm, z, 4));
    }
    async rotate(x, heads) { return this.ops.rotate(x, heads, this.position); }
    // src/engine.js:115-124: attention layer over every cached position.
    async qsa(layer, x) {
        const g = this.g, o = this.ops, b = this.b, p = 'blk.' + layer + '.', st = this.states[layer];
        const full = await o.mat(p + 'attn_q.weight', x), qr = await o.slice(full, g.headDim, g.heads, g.headDim * 2);
        const q = await this.rotate(await o.norm(qr, await o.vector(p + 'attn_q_norm.weight'), g.headDim, g.heads), g.heads);
        const kr = await o.mat(p + 'attn_k.weight', x);
        const k = await this.rotate(await o.norm(kr, await o.vector(p + 'attn_k_norm.weight'), g.headDim, g.kvHeads), g.kvHeads);
        const v = await o.mat(p + 'attn_v.weight', x);
        await b.run('strata_kv_append', {K: k, V: v, Keys: st.keys, Values: st.values, width: g.kvHeads * g.headDim,
            position: this.position}, grid(g.kvHeads * g.headDim));
        const cells = await o.alloc(Int32Array.from({length: this.position + 1}, (_, i) => i), 'i32');
        const attn = await o.alloc(g.heads * g.headDim), gated = await o.alloc(g.heads * g.headDim);
        await b.run('strata_attention', {Q: q, Keys: st.keys, Values: st.values, Cells: cells, Y: attn, dim: g.headDim,
            heads: g.heads, kvHeads: g.kvHeads, count: this.position + 1, scale: 1 / Math.sqrt(g.headDim)},
        [g.heads, Math.ceil(g.headDim / 64), 1]);
        await b.run('strata_attention_gate', {Attention: attn, FullQ: full, Y: gated, dim: g.headDim, heads: g.heads},
            grid(g.heads * g.headDim));
        return o.mat(p + 'attn_output.weight', gated);
    }
    // src/engine.js:125-132: one expert; f32 experts run as three projections
    // and the SiLU(gate)*up elementwise pass, Q2-packed ones from their blob.
    async expert(prefix, x, shared, tokens) {
        tokens = tokens || 1;
        const o = this.ops, manifest = this.store.manifest;
        if (!shared && manifest && manifest.experts && manifest.experts.source_type === 'Q2_0') {
            const m = /^blk\.(\d+)\.expert\.(\d+)\.$/.exec(prefix);
            return o.packedExpert(Number(m[1]), Number(m[2]), x, tokens);
        }
        const name = role => shared ? prefix + 'ffn_' + role + '_shexp.weight' : prefix + role;
        const gate = await o.mat(name('gate'), x, tokens), up = await o.mat(name('up'), x, tokens);
        const activation = await o.elem(gate, up, 3);
        return o.mat(name('down'), activation, tokens);
    }
    // src/engine.js:133-156: router, routing check, routed experts into their
    // slots, shared expert and gate, combine.
    async moe(layer, x) {
        const g = this.g, o = this.ops, b = this.b, p = 'blk.' + layer + '.';
        const logits = await o.mat(p + 'ffn_gate_inp.weight', x), ids = await o.alloc(g.topK, 'i32');
        const weights = await o.alloc(g.topK);
        await b.run('strata_router', {Logits: logits, Ids: ids, Weights: weights, experts: g.experts, topK: g.topK},
            [1, 1, 1]);
        const selected = await b.read(ids, 'i32');
        if (selected.some(id => id < 0 || id >= g.experts) || new Set(selected).size !== g.topK)
            throw Error('Invalid expert routing result');
        const resident = o.residency;
        for (const id of selected) resident.note(layer + ':' + id);
        this.stats.routes.push({layer, ids: Array.from(selected), devices: Array.from(selected, () => b.kind)});
        const parts = await o.alloc(g.width * g.topK);
        for (let index = 0; index < g.topK; index++) {
            await resident.admit(layer + ':' + selected[index]);
            const result = await this.expert(p + 'expert.' + selected[index] + '.', x);
            b.copy(result, parts, g.width, 0, index * g.width);
            this.stats.gpuExperts++;
        }
        const shared = await this.expert(p, x, true), sharedGate = await o.mat(p + 'ffn_gate_inp_shexp.weight', x);
        const y = await o.alloc(g.width);
        await b.run('strata_moe_combine', {Parts: parts, Weights: weights, Shared: shared, SharedGate: sharedGate, Y: y,
            width: g.width, count: g.topK}, grid(g.width));
        return y;
    }
    residencyInfo() { return this.ops.residency.info(); }
    // src/engine.js:158-165: the prompt in layer-major chunks (src/prefill.js).
    async prefill(tokens, options) {
        const o = options || {};
        this.assertIdle('A session operation is already running');
        if (this.failed) throw Error('Session failed; reset it before continuing');
        tokens = Array.from(tokens);
        if (!tokens.length) throw Error('Prompt is empty');
        for (const t of tokens)
            if (!Number.isSafeInteger(t) || t < 0 || t > this.g.vocab - 1)
                throw new RangeError('token must be an integer in [0, ' + (this.g.vocab - 1) + ']');
        if (this.position + tokens.length > this.g.context) throw Error('Context capacity reached');
        const chunk = o.chunkSize === undefined ? 16 : o.chunkSize;
        if (!Number.isSafeInteger(chunk) || chunk < 1 || chunk > 64)
            throw new RangeError('prompt chunk size must be an integer in [1, 64]');
        if (o.logits && o.predict === false) throw Error('Logits require prediction');
        this.busy = true;
        try { return await prefillChunks(this, tokens, o); } catch (error) { this.failed = true; throw error; }
        finally { this.busy = false; }
    }
    // src/engine.js:166-196.
    async step(token, options) {
        const opts = options || {}, logits = !!opts.logits, predict = opts.predict !== false;
        this.assertIdle('A session operation is already running');
        if (this.failed) throw Error('Session failed; reset it before continuing');
        if (logits && !predict) throw Error('Logits require prediction');
        if (!Number.isSafeInteger(token) || token < 0 || token > this.g.vocab - 1)
            throw new RangeError('token must be an integer in [0, ' + (this.g.vocab - 1) + ']');
        if (this.position >= this.g.context) throw Error('Context capacity reached; reset or create a larger session');
        this.busy = true;
        const start = performance.now();
        this.stats.routes = [];
        try {
            const g = this.g, o = this.ops, b = this.b;
            await o.embedding(token, this.residual);
            for (let l = 0; l < g.layers; l++) {
                if (l === g.pleLayer) await this.ple(token);
                const attn = await this.hc('blk.' + l + '.hc_attn_');
                const mixed = l % g.qsaInterval === g.qsaInterval - 1 ? await this.qsa(l, attn.mixed) : await this.gdn(l, attn.mixed);
                await this.hcWrite(mixed, attn.inject);
                const ffn = await this.hc('blk.' + l + '.hc_ffn_');
                await this.hcWrite(await this.moe(l, ffn.mixed), ffn.inject);
                await o.clearTemporary();
                if (opts.onProgress) opts.onProgress(l + 1, g.layers);
            }
            const result = {position: this.position};
            if (predict) {
                const head = await this.hc('output_hc_', false), values = await o.mat('output.weight', head.mixed);
                const next = await o.alloc(1, 'i32');
                await b.run('strata_argmax', {Logits: values, Token: next, count: g.vocab}, [1, 1, 1]);
                result.token = (await b.read(next, 'i32'))[0];
                if (!Number.isSafeInteger(result.token) || result.token < 0 || result.token >= g.vocab)
                    throw new RangeError('generated token must be an integer in [0, ' + (g.vocab - 1) + ']');
                if (logits) result.logits = await b.read(values);
                if (result.logits && result.logits.some(v => !Number.isFinite(v))) throw Error('Non-finite logits');
            }
            await o.clearTemporary();
            this.previous.push(token);
            if (this.previous.length > 2) this.previous.shift();
            this.position++; this.stats.tokens++; this.stats.lastMs = performance.now() - start;
            return result;
        } catch (error) { this.failed = true; throw error; } finally { this.busy = false; }
    }
    // src/engine.js:197-203: zeroes the persistent state.
    async reset() {
        this.assertIdle('Cannot reset during a decode step or state operation');
        this.busy = true;
        try {
            await this.ops.clearTemporary();
            for (const buffer of this.persistent) this.b.zero(buffer);
            this.position = 0; this.previous = []; this.failed = false;
        } catch (error) { this.failed = true; throw error; } finally { this.busy = false; }
    }
    // src/engine.js:204-217: host copies of every persistent buffer.
    async checkpoint() {
        this.assertIdle('Checkpoint requires an idle session');
        if (this.failed) throw Error('Checkpoint requires a healthy session');
        this.busy = true;
        try {
            const buffers = [];
            for (const b of this.persistent) buffers.push(await this.b.read(b));
            return {owner: this.checkpointOwner, geometry: JSON.stringify(this.g), position: this.position,
                previous: this.previous.slice(), buffers};
        } finally { this.busy = false; }
    }
    async restore(state) {
        this.assertIdle('Cannot restore during decode or state operation');
        const g = this.g;
        if (state.owner !== this.checkpointOwner || state.geometry !== JSON.stringify(g) ||
            state.buffers.length !== this.persistent.length ||
            state.buffers.some((a, i) => !(a instanceof Float32Array) || a.length !== this.persistent[i].length ||
                a.some(x => !Number.isFinite(x))) ||
            !Number.isInteger(state.position) || state.position < 0 || state.position > g.context ||
            state.previous.length !== Math.min(state.position, 2) ||
            state.previous.some(x => !Number.isInteger(x) || x < 0 || x >= g.vocab))
            throw Error('Checkpoint does not match this model/session geometry');
        this.busy = true;
        try {
            await this.ops.clearTemporary();
            for (let i = 0; i < this.persistent.length; i++) this.b.write(this.persistent[i], state.buffers[i]);
            this.position = state.position; this.previous = state.previous.slice(); this.failed = false;
        } catch (error) { this.failed = true; throw error; } finally { this.busy = false; }
    }
    async dispose() {
        if (this.disposed) return;
        this.assertIdle('Cannot dispose during a decode step or state operation');
        this.busy = true;
        try {
            await this.ops.dispose();
            for (const b of this.persistent) this.b.free(b);
            this.persistent = []; this.disposed = true;
        } catch (error) { this.failed = true; throw error; } finally { this.busy = false; }
    }
}
