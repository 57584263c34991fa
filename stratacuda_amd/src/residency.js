// WeightResidency with the all-resident policy of an MI355X: every expert
// blob of every layer lives in HBM for the life of the session (48 layers x
// 512 experts x 884,736 B = 21.7 GB of the 288 GB), so there is no budgeted
// admission and no eviction. The interface and info() fields are those of
// src/residency.js:14-80 (admit / hasExpert / note / get / vector / info /
// dispose); admit always succeeds and hasExpert is true for a loaded layer.
//
// Layout in HBM, per layer: one arena buffer holding expert e's blob at
// e * stride (stride = blob size rounded up to 256 B, so every plane starts
// 16-byte aligned), the shared expert's blob, the router matrix W_r
// [experts x width] f32, the shared-gate vector and the RMSNorm gamma.
import {requireInteger} from './backend.js';

const product = shape => shape.reduce((a, b) => a * b, 1);
// 'blk.L.expert.E.role' -> 'L:E' (src/residency.js:4).
export const expertKey = name => {
    const m = /^blk\.(\d+)\.expert\.(\d+)\./.exec(name);
    return m ? m[1] + ':' + m[2] : null;
};

export class WeightResidency {
    // (ops, denseNames, budgetBytes) as in the reference; the budget must
    // cover every layer's resident bytes.
    constructor(ops, denseNames, budgetBytes) {
        this.ops = ops; this.b = ops.b; this.store = ops.store;
        this.budgetBytes = requireInteger(budgetBytes, 'GPU weight budget', 1, Number.MAX_SAFE_INTEGER);
        this.denseNames = new Set(denseNames || []);
        this.layers = new Map(); this.frequency = new Map();
        this.hits = 0; this.misses = 0; this.evictions = 0; this.denseUsed = 0; this.expertUsed = 0;
        this.tiles = new Map();
        ops.residency = this;
    }
    layerBytes() {
        const g = this.store.config, stride = this.store.stride;
        return stride * (g.experts + 1) + 4 * (g.experts * g.width + 2 * g.width);
    }
    // Makes layer `layer` resident (allocation plus generation on the device).
    async loadLayer(layer) {
        if (this.layers.has(layer)) return this.layers.get(layer);
        const g = this.store.config, b = this.b, stride = this.store.stride;
        if (this.denseUsed + this.expertUsed + this.layerBytes() > this.budgetBytes)
            throw Error('Resident weights need ' + ((this.denseUsed + this.expertUsed + this.layerBytes()) / 1024 ** 3)
                .toFixed(2) + ' GiB; choose a larger GPU budget.');
        const entry = {
            arena: b.allocBytes(stride * g.experts, 'u32', {zero: false}),
            shared: b.allocBytes(stride, 'u32', {zero: false}),
            Wr: b.alloc(g.experts * g.width, 'f32', {zero: false}),
            Wsg: b.alloc(g.width, 'f32', {zero: false}),
            gamma: b.alloc(g.width, 'f32', {zero: false}),
        };
        this.store.generate(b, layer, entry);
        this.layers.set(layer, entry);
        this.expertUsed += stride * (g.experts + 1);
        this.denseUsed += 4 * (g.experts * g.width + 2 * g.width);
        this.misses++;
        return entry;
    }
    layer(layer) {
        const entry = this.layers.get(layer);
        if (!entry) throw Error('Layer ' + layer + ' is not resident');
        return entry;
    }
    hasExpert(key) { return this.layers.has(Number(String(key).split(':')[0])); }
    note(key, count) { this.frequency.set(key, (this.frequency.get(key) || 0) + (count === undefined ? 1 : count)); }
    async admit(key) { if (this.hasExpert(key)) { this.hits++; return true; } return false; }
    // Dense tiles: the resident f32 router matrix / shared-gate row of a layer.
    async get(name, start, rows) {
        const t = this.store.describe(name), entry = this.layer(t.layer);
        const rest = name.slice(name.indexOf('.', 4) + 1);
        const data = rest === 'ffn_gate_inp.weight' ? entry.Wr : rest === 'ffn_gate_inp_shexp.weight' ? entry.Wsg : null;
        if (!data || t.format !== 'f32') return null;
        if (start !== 0 || rows !== product(t.shape) / t.shape[0]) return null;
        this.hits++;
        return {format: 'f32', data, buffers: [], bytes: data.byteLength};
    }
    async vector(name) {
        const t = this.store.describe(name), entry = this.layer(t.layer);
        if (/ffn_norm\.weight$/.test(name)) { this.hits++; return entry.gamma; }
        if (/ffn_gate_inp_shexp\.weight$/.test(name)) { this.hits++; return entry.Wsg; }
        throw Error('No resident vector ' + name);
    }
    info() {
        return {budgetBytes: this.budgetBytes, densePlannedBytes: this.denseUsed, denseResidentBytes: this.denseUsed,
            expertResidentBytes: this.expertUsed, residentExperts: this.layers.size * this.store.config.experts,
            hits: this.hits, misses: this.misses, evictions: this.evictions};
    }
    async dispose() {
        for (const entry of this.layers.values()) for (const k of Object.keys(entry)) this.b.free(entry[k]);
        this.layers.clear(); this.expertUsed = 0; this.denseUsed = 0;
    }
}

// The all-resident policy for a whole-model f32 store (the fixture's
// MemoryStore): every tensor is uploaded once when the engine initialises and
// stays in HBM until dispose, experts included, so nothing is streamed or
// evicted. get / vector / hasExpert / admit / note / info as above.
export class ModelResidency {
    constructor(ops) {
        this.ops = ops; this.b = ops.b; this.store = ops.store;
        this.tensors = new Map(); this.frequency = new Map();
        this.hits = 0; this.misses = 0; this.evictions = 0; this.denseUsed = 0; this.expertUsed = 0;
        ops.residency = this;
    }
    async loadAll() {
        for (const [name, t] of this.store.tensors) {
            if (this.tensors.has(name)) continue;
            if (t.format !== 'f32') throw Error('Resident model tensors must be F32: ' + name);
            this.tensors.set(name, this.b.alloc(t.data, 'f32'));
            if (expertKey(name)) this.expertUsed += t.data.byteLength; else this.denseUsed += t.data.byteLength;
            this.misses++;
        }
    }
    tensor(name) {
        const buffer = this.tensors.get(name);
        if (!buffer) throw Error(name + ' is not resident');
        this.hits++;
        return buffer;
    }
    // Whole tensors only: Ops.mat asks for every row of a projection.
    async get(name, start, rows) {
        const t = this.store.describe(name);
        if (start !== 0 || rows !== product(t.shape) / t.shape[0]) return null;
        const data = this.tensor(name);
        return {format: 'f32', data, buffers: [], bytes: data.byteLength};
    }
    async vector(name) { return this.tensor(name); }
    hasExpert(key) { return true; }
    note(key, count) { this.frequency.set(key, (this.frequency.get(key) || 0) + (count === undefined ? 1 : count)); }
    async admit(key) { this.hits++; return true; }
    info() {
        return {budgetBytes: this.denseUsed + this.expertUsed, densePlannedBytes: this.denseUsed,
            denseResidentBytes: this.denseUsed, expertResidentBytes: this.expertUsed,
            residentExperts: Array.from(this.tensors.keys()).filter(n => /\.expert\.\d+\.gate$/.test(n)).length,
            hits: this.hits, misses: this.misses, evictions: this.evictions};
    }
    async dispose() {
        for (const buffer of this.tensors.values()) this.b.free(buffer);
        this.tensors.clear(); this.denseUsed = 0; this.expertUsed = 0;
    }
}
