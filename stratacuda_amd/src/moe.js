// The routed-expert stage of one layer for n tokens (the MoE of
// src/engine.js:133-156 and src/prefill.js:52-78), in one routine for a
// decode step (n = 1, one-token kernels) and a prompt chunk (*_batch
// kernels).
//
// Two ways to run it:
//   - fused (kind 'hip', Q2 store): one device call (Ops.moe) does router
//     projection, top-k, dispatch, expert products, shared expert, shared gate
//     and combine, with no host readback of the routed IDs;
//   - host-driven: the router kernel, a readback and check of the IDs, each
//     distinct expert once over the rows routed to it, the shared expert over
//     all rows, the shared-gate projection and the combine kernel. Experts are
//     f32 tensors (three projections and the SiLU(gate) * up pass) or the
//     layer's Q2 blobs (strata_q2_gate_up / strata_q2_down); f32 experts
//     serving several rows read them through a gather and write them back
//     through a scatter, Q2 experts address rows through a mapping.
// Both return {y, ids, weights} (device buffers) and record the routes in
// `stats` ({layer, position, ids, devices}; ids null when fused).
import {grid} from './ops.js';
import {KERNELS} from './plan.js';

export class MoeStage {
    constructor(ops, options) {
        const o = options || {}, manifest = ops.store.manifest;
        this.ops = ops; this.b = ops.b; this.g = ops.store.config;
        this.packed = !!(manifest && manifest.experts && manifest.experts.source_type === 'Q2_0');
        this.fused = (o.fused === undefined ? true : !!o.fused) && this.b.kind === 'hip' && this.packed;
        this.stats = o.stats || {routes: [], gpuExperts: 0};
    }
    async decode(layer, x) { return this.run(layer, x, 1, {batched: false, position: 0}); }
    async prompt(layer, x, n) { return this.run(layer, x, n, {batched: true, position: 0}); }

    async run(layer, x, n, where) {
        const w = where || {}, batched = !!w.batched, position = w.position || 0;
        if (this.fused) {
            const r = await this.ops.moe(layer, x, n);
            this.stats.routes.push({layer, position, tokens: n, ids: null, devices: [this.b.kind]});
            return r;
        }
        const g = this.g, o = this.ops, b = this.b, p = 'blk.' + layer + '.';
        const logits = await o.mat(p + 'ffn_gate_inp.weight', x, n);
        const ids = await o.alloc(n * g.topK, 'i32'), weights = await o.alloc(n * g.topK);
        await b.run(KERNELS.router[batched ? 1 : 0], {Logits: logits, Ids: ids, Weights: weights, experts: g.experts,
            topK: g.topK}, [n, 1, 1]);
        const parts = await o.alloc(n * g.topK * g.width);
        for (const [id, rows] of this.groups(layer, await b.read(ids, 'i32'), n, position)) {
            const key = layer + ':' + id;
            if (o.residency) { o.residency.note(key, rows.length); await o.residency.admit(key); }
            await this.expertRows(layer, id, x, n, rows, parts);
            this.stats.gpuExperts += rows.length;
        }
        const shared = await this.sharedExpert(layer, x, n);
        const sharedGate = await o.mat(p + 'ffn_gate_inp_shexp.weight', x, n), y = await o.alloc(n * g.width);
        const args = {Parts: parts, Weights: weights, Shared: shared, SharedGate: sharedGate, Y: y, width: g.width,
            count: g.topK};
        if (batched) args.tokens = n;
        await b.run(KERNELS.combine[batched ? 1 : 0], args, grid(n * g.width));
        await o.release(logits, parts, shared, sharedGate);
        return {y, ids, weights};
    }

    // Routed IDs [n x topK] -> distinct expert -> [{token, part}] in the
    // order the experts first appear; every token's row is checked (IDs in
    // range, no repeats) and recorded.
    groups(layer, selected, n, position) {
        const g = this.g, byExpert = new Map();
        for (let t = 0; t < n; t++) {
            const row = Array.from(selected.subarray(t * g.topK, (t + 1) * g.topK));
            if (row.some(id => !(id >= 0 && id < g.experts)) || new Set(row).size !== g.topK)
                throw Error(n === 1 ? 'Invalid expert routing result' : 'Invalid prompt expert routing');
            this.stats.routes.push({layer, position: position + t, ids: row, devices: row.map(() => this.b.kind)});
            row.forEach((id, k) => {
                if (!byExpert.has(id)) byExpert.set(id, []);
                byExpert.get(id).push({token: t, part: t * g.topK + k});
            });
        }
        return byExpert;
    }

    // Expert `id` over its rows of x, written to their slots of `parts`.
    async expertRows(layer, id, x, n, rows, parts) {
        const g = this.g, o = this.ops, b = this.b;
        if (this.packed) {
            if (n === 1) await o.packedExpert(layer, id, x, 1, {output: parts, outputOffset: rows[0].part * g.width});
            else await o.packedExpert(layer, id, x, rows.length, {output: parts,
                mapping: Int32Array.from([].concat.apply([], rows.map(r => [r.token, r.part])))});
            return;
        }
        const prefix = 'blk.' + layer + '.expert.' + id + '.';
        if (n === 1) {
            const out = await this.denseExpert(role => prefix + role, x, 1);
            b.copy(out, parts, g.width, 0, rows[0].part * g.width);
            await o.release(out);
            return;
        }
        const from = await o.alloc(Int32Array.from(rows, r => r.token), 'i32'), input = await o.alloc(rows.length * g.width);
        await b.run('strata_gather_rows', {X: x, Indices: from, Y: input, width: g.width, rows: rows.length},
            grid(input.length));
        const out = await this.denseExpert(role => prefix + role, input, rows.length);
        const to = await o.alloc(Int32Array.from(rows, r => r.part), 'i32');
        await b.run('strata_scatter_rows', {X: out, Indices: to, Y: parts, width: g.width, rows: rows.length},
            grid(out.length));
        await o.release(from, input, out, to);
    }

    // down . (SiLU(gate . x) * (up . x)) from f32 tensors [width x ff] and
    // [ff x width], for `tokens` rows of x.
    async denseExpert(name, x, tokens) {
        const o = this.ops;
        const gate = await o.mat(name('gate'), x, tokens), up = await o.mat(name('up'), x, tokens);
        const act = await o.elem(gate, up, 3), out = await o.mat(name('down'), act, tokens);
        await o.release(gate, up, act);
        return out;
    }

    async sharedExpert(layer, x, n) {
        if (this.packed) return this.ops.packedExpert(layer, 'shared', x, n);
        const p = 'blk.' + layer + '.ffn_';
        return this.denseExpert(role => p + role + '_shexp.weight', x, n);
    }
}
