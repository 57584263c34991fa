// Ops: kernel orchestration for the MoE path with the reference's op
// signatures (src/ops.js:5-127: alloc / release / clearTemporary / mat /
// vector / norm / elem / packedExpert / embedding / ple / rotate / slice /
// dispose), over a backend with the reference interface (HipBackend here). Weights come from the resident
// WeightResidency; there is no streaming tile cache (everything is resident).
// moe() is the fused stage for kind 'hip': one sm_moe_layer call per layer.
import {requireInteger} from './backend.js';

export const grid = n => [Math.ceil(n / 64), 1, 1];

export class Ops {
    constructor(backend, store) {
        this.b = backend; this.store = store; this.residency = null;
        this.temporary = new Set(); this.dummy = null; this.workspace = null; this.rope = null;
    }
    // Temporaries are completely written by their producing kernel (src/ops.js:13-16).
    async alloc(dataOrLength, type) {
        const b = this.b.alloc(dataOrLength, type || 'f32', {zero: false});
        this.temporary.add(b); return b;
    }
    async release(...buffers) { for (const b of buffers) if (this.temporary.delete(b)) this.b.free(b); }
    async clearTemporary() {
        this.b.flush();
        for (const b of this.temporary) this.b.free(b);
        this.temporary.clear();
    }
    // mat(name, x, tokens): y[t, r] = W[r, :] . x[t, :] with W resident f32
    // (src/ops.js:95-112, strata_project), shape [cols, rows].
    async mat(name, x, tokens) {
        tokens = tokens || 1;
        const shape = this.store.describe(name).shape, cols = shape[0], rows = shape.slice(1).reduce((a, b) => a * b, 1);
        if (x.length !== cols * tokens) throw Error(name + ': expected ' + cols * tokens + ' inputs, got ' + x.length);
        const w = this.residency ? await this.residency.get(name, 0, rows) : null;
        if (!w) throw Error(name + ' is not resident');
        const y = await this.alloc(rows * tokens);
        await this.b.run('strata_project', {X: x, W: w.data, Y: y, cols, rows, tokens, outputStride: rows,
            outputOffset: 0}, [rows, tokens, 1]);
        return y;
    }
    async vector(name) { return this.residency.vector(name); }
    async norm(x, w, cols, rows, weightRows, mode, scale) {
        rows = rows || 1; weightRows = weightRows || 1; mode = mode || 0; scale = scale === undefined ? 1 : scale;
        const y = await this.alloc(cols * rows);
        await this.b.run('strata_norm', {X: x, W: w, Y: y, cols, rows, weightRows, mode, epsilon: 1e-6, scale}, [rows, 1, 1]);
        return y;
    }
    async elem(a, b, mode, scale) {
        b = b || a; mode = mode || 0; scale = scale === undefined ? 1 : scale;
        if (a.length !== b.length) throw Error('Elementwise input shapes disagree');
        const y = await this.alloc(a.length);
        await this.b.run('strata_elementwise', {A: a, B: b, Y: y, n: a.length, mode, scale}, grid(a.length));
        return y;
    }
    // packedExpert(layer, id, x, tokens, {output, mapping, outputOffset})
    // (src/ops.js:56-72): SiLU(gate . x) * (up . x) then down, from the
    // resident blob of expert `id` (or the shared expert for id 'shared').
    // The blob sits at id * stride in the layer's arena, so the code and
    // scale offsets of the reference kernels carry that base.
    async packedExpert(layer, id, x, tokens, options) {
        tokens = tokens || 1;
        const o = options || {}, g = this.store.config, ex = this.store.manifest.experts;
        const entry = this.residency.layer(layer), shared = id === 'shared';
        if (!shared) requireInteger(id, 'expert id', 0, g.experts - 1);
        const blob = shared ? entry.shared : entry.arena, base = shared ? 0 : id * ex.stride;
        if (this.dummy === null) this.dummy = this.b.alloc(new Int32Array(1), 'i32');
        const map = o.mapping ? await this.alloc(o.mapping, 'i32') : this.dummy;
        const hidden = await this.alloc(g.ff * tokens), result = o.output || await this.alloc(g.width * tokens);
        const common = {Blob: blob, Scales: this.dummy, Mapping: map, width: g.width, ff: g.ff, tokens,
            mapped: o.mapping ? 1 : 0, expanded: 0};
        await this.b.run('strata_q2_gate_up', Object.assign({X: x, Hidden: hidden,
            codeOffset: (base + ex.offsets.gate_up_codes) / 4, scaleOffset: (base + ex.offsets.gate_up_scales) / 2}, common),
        [g.ff, tokens, 1]);
        await this.b.run('strata_q2_down', Object.assign({Hidden: hidden, Y: result, outputOffset: o.outputOffset || 0,
            codeOffset: (base + ex.offsets.down_codes) / 4, scaleOffset: (base + ex.offsets.down_scales) / 2}, common),
        [g.width, tokens, 1]);
        await this.release(hidden);
        if (o.mapping) await this.release(map);
        return result;
    }
    // embedding(token, output, outputOffset) (src/ops.js:73-78): row `token`
    // of the resident f32 embedding, replicated over the HC streams.
    async embedding(token, output, outputOffset) {
        const g = this.store.config, table = this.residency.tensor('token_embd.weight');
        requireInteger(token, 'token', 0, table.length / g.width - 1);
        if (this.dummy === null) this.dummy = this.b.alloc(new Int32Array(1), 'i32');
        const row = await this.alloc(g.width);
        this.b.copy(table, row, g.width, token * g.width, 0);
        await this.b.run('strata_embedding', {Values: row, Codes: this.dummy, Scales: this.dummy, Offsets: this.dummy,
            Residual: output, width: g.width, streams: g.streams, outputOffset: outputOffset || 0, format: 0, bits: 0,
            groupSize: 1, bias: 0, codebook: 0, hasOffset: 0}, grid(g.width));
        await this.release(row);
    }
    // ple(token, previous) (src/ops.js:79-83): the f32 PLE rows of an
    // in-memory store, gathered on the host by the n-gram hash.
    async ple(token, previous) { return this.alloc(await this.store.pleRows(token, previous)); }
    // rotate(x, heads, position, tokens) (src/ops.js:84-94): RoPE tables made
    // once on the device (strata_rope_frequencies, strata_rope_table), then
    // strata_rope_position.
    async rotate(x, heads, position, tokens) {
        tokens = tokens || 1;
        const g = this.store.config, y = await this.alloc(x.length);
        if (!this.rope) {
            const rope = {cos: this.b.alloc(g.context * g.rotary / 2), sin: this.b.alloc(g.context * g.rotary / 2)};
            const hi = await this.alloc(g.rotary / 2), lo = await this.alloc(g.rotary / 2);
            await this.b.run('strata_rope_frequencies', {High: hi, Low: lo, rotary: g.rotary, base: g.ropeBase},
                grid(g.rotary / 2));
            await this.b.run('strata_rope_table', {High: hi, Low: lo, Cos: rope.cos, Sin: rope.sin, rotary: g.rotary,
                context: g.context}, grid(g.context * g.rotary / 2));
            await this.release(hi, lo);
            this.rope = rope;
        }
        await this.b.run('strata_rope_position', {X: x, Cos: this.rope.cos, Sin: this.rope.sin, Y: y, dim: g.headDim,
            heads, rotary: g.rotary, position, tokens}, grid(x.length));
        return y;
    }
    // slice(x, width, rows, stride, offset) (src/ops.js:122-126).
    async slice(x, width, rows, stride, offset) {
        rows = rows === undefined ? 1 : rows; stride = stride === undefined ? width : stride; offset = offset || 0;
        requireInteger(width, 'slice width'); requireInteger(rows, 'slice rows');
        if (offset < 0 || (rows - 1) * stride + offset + width > x.length) throw Error('Slice exceeds buffer');
        const y = await this.alloc(width * rows);
        await this.b.run('strata_slice', {X: x, Y: y, width, rows, stride, offset}, grid(width * rows));
        return y;
    }
    // The fused MoE stage (kind 'hip'): y, plus the routed ids and weights
    // [tokens x topK] in the reference's selection order.
    async moe(layer, x, tokens, options) {
        tokens = tokens || 1;
        const o = options || {}, g = this.store.config, entry = this.residency.layer(layer);
        if (x.length !== tokens * g.width) throw Error('MoE input must hold tokens x width values');
        const bytes = this.b.moeWorkspaceBytes(tokens, g.width, g.ff, g.experts, g.topK);
        if (!this.workspace || this.workspace.byteLength < bytes) {
            if (this.workspace) this.b.free(this.workspace);
            this.workspace = this.b.allocBytes(Math.ceil(bytes / 4) * 4, 'u32', {zero: false});
        }
        const y = await this.alloc(tokens * g.width), ids = await this.alloc(tokens * g.topK, 'i32');
        const weights = await this.alloc(tokens * g.topK);
        this.b.moeLayer({X: x, tokens, Wr: entry.Wr, bias: o.bias || null, arena: entry.arena, stride: this.store.stride,
            shared: entry.shared, Wsg: entry.Wsg, width: g.width, ff: g.ff, experts: g.experts, topK: g.topK, Y: y, ids,
            weights, workspace: this.workspace});
        return {y, ids, weights};
    }
    // One stacked-decoder block on the device (kind 'hip'): h + MoE(RMSNorm(h;
    // the layer's ffn_norm gamma, eps 1e-6)) in one call, with the routed ids
    // and weights. The same bits as norm(), moe() and elem(.., 5) in turn.
    async moeBlock(layer, h, tokens, options) {
        tokens = tokens || 1;
        const o = options || {}, g = this.store.config, entry = this.residency.layer(layer);
        if (h.length !== tokens * g.width) throw Error('MoE input must hold tokens x width values');
        const bytes = this.b.moeBlockWorkspaceBytes(tokens, g.width, g.ff, g.experts, g.topK);
        if (!this.workspace || this.workspace.byteLength < bytes) {
            if (this.workspace) this.b.free(this.workspace);
            this.workspace = this.b.allocBytes(Math.ceil(bytes / 4) * 4, 'u32', {zero: false});
        }
        const out = o.output || await this.alloc(tokens * g.width), ids = await this.alloc(tokens * g.topK, 'i32');
        const weights = await this.alloc(tokens * g.topK);
        this.b.moeBlock({H: h, tokens, gamma: entry.gamma, eps: 1e-6, Wr: entry.Wr, bias: o.bias || null,
            arena: entry.arena, stride: this.store.stride, shared: entry.shared, Wsg: entry.Wsg, width: g.width, ff: g.ff,
            experts: g.experts, topK: g.topK, Hout: out, ids, weights, workspace: this.workspace});
        return {h: out, ids, weights};
    }
    async dispose() {
        await this.clearTemporary();
        if (this.residency) await this.residency.dispose();
        if (this.rope) { this.b.free(this.rope.cos); this.b.free(this.rope.sin); this.rope = null; }
        if (this.dummy) this.b.free(this.dummy);
        if (this.workspace) this.b.free(this.workspace);
        this.dummy = null; this.workspace = null;
    }
}
