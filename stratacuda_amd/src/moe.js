// The MoE stage of one layer, as the reference's drivers run it:
//   decode (one token)   StrataEngine.moe, src/engine.js:133-156
//   prompt (n tokens)    PromptBatch.moe, src/prefill.js:52-78
// For kind 'hip' the whole stage is one fused device call (Ops.moe): router
// projection, top-k, device dispatch, expert products, shared expert, shared
// gate and combine, with no host readback of the routed IDs. With
// {fused: false} the stage runs the reference's host-driven sequence on the
// same backend, kernel by kernel (strata_project, strata_router[_batch], an ID
// readback and check, strata_q2_gate_up / strata_q2_down per expert, the
// shared expert, the shared-gate projection, strata_moe_combine[_batch]).
// Both return {y, ids, weights} (device buffers) and record the routes.

function checkRoute(row, experts, topK, message) {
    const seen = new Set();
    for (const id of row) { if (id < 0 || id >= experts) throw Error(message); seen.add(id); }
    if (seen.size !== topK) throw Error(message);
}

export class MoeStage {
    constructor(ops, {fused = true} = {}) {
        this.ops = ops; this.b = ops.b; this.g = ops.store.config;
        this.fused = fused && this.b.kind === 'hip';
        this.stats = {routes: [], gpuExperts: 0};
    }
    // src/engine.js:133-156 (decode, x = [width]).
    async decode(layer, x) {
        const {g, ops: o, b} = this, p = 'blk.' + layer + '.';
        if (this.fused) {
            const r = await o.moe(layer, x, 1);
            this.stats.routes.push({layer, ids: null, devices: [b.kind]});
            return r;
        }
        const logits = await o.mat(p + 'ffn_gate_inp.weight', x), ids = await o.alloc(g.topK, 'i32');
        const weights = await o.alloc(g.topK);
        await b.run('strata_router', {Logits: logits, Ids: ids, Weights: weights, experts: g.experts, topK: g.topK},
            [1, 1, 1]);
        const selected = await b.read(ids, 'i32');
        checkRoute(selected, g.experts, g.topK, 'Invalid expert routing result');
        if (o.residency) for (const id of selected) o.residency.note(layer + ':' + id);
        this.stats.routes.push({layer, ids: Array.from(selected), devices: Array.from(selected, () => b.kind)});
        const parts = await o.alloc(g.width * g.topK);
        for (let index = 0; index < g.topK; index++) {
            await o.residency.admit(layer + ':' + selected[index]);
            await o.packedExpert(layer, selected[index], x, 1, {output: parts, outputOffset: index * g.width});
            this.stats.gpuExperts++;
        }
        const shared = await o.packedExpert(layer, 'shared', x, 1);
        const sharedGate = await o.mat(p + 'ffn_gate_inp_shexp.weight', x), y = await o.alloc(g.width);
        await b.run('strata_moe_combine', {Parts: parts, Weights: weights, Shared: shared, SharedGate: sharedGate, Y: y,
            width: g.width, count: g.topK}, [Math.ceil(g.width / 64), 1, 1]);
        await o.release(logits, parts, shared, sharedGate);
        return {y, ids, weights};
    }
    // src/prefill.js:52-78 (prompt, x = [n x width]).
    async prompt(layer, x, n) {
        const {g, ops: o, b} = this, p = 'blk.' + layer + '.';
        if (this.fused) {
            const r = await o.moe(layer, x, n);
            this.stats.routes.push({layer, tokens: n, ids: null, devices: [b.kind]});
            return r;
        }
        const logits = await o.mat(p + 'ffn_gate_inp.weight', x, n), ids = await o.alloc(n * g.topK, 'i32');
        const weights = await o.alloc(n * g.topK);
        await b.run('strata_router_batch', {Logits: logits, Ids: ids, Weights: weights, experts: g.experts,
            topK: g.topK}, [n, 1, 1]);
        const selected = await b.read(ids, 'i32'), groups = new Map(), parts = await o.alloc(n * g.topK * g.width);
        for (let t = 0; t < n; t++) {
            const row = Array.from(selected.subarray(t * g.topK, (t + 1) * g.topK));
            checkRoute(row, g.experts, g.topK, 'Invalid prompt expert routing');
            this.stats.routes.push({layer, position: t, ids: row, devices: row.map(() => b.kind)});
            for (let k = 0; k < g.topK; k++) {
                const id = row[k];
                if (!groups.has(id)) groups.set(id, []);
                groups.get(id).push({token: t, part: t * g.topK + k});
            }
        }
        for (const [id, jobs] of groups) {
            if (o.residency) o.residency.note(layer + ':' + id, jobs.length);
            await o.residency.admit(layer + ':' + id);
            const mapping = Int32Array.from([].concat.apply([], jobs.map(j => [j.token, j.part])));
            await o.packedExpert(layer, id, x, jobs.length, {output: parts, mapping});
            this.stats.gpuExperts += jobs.length;
        }
        const shared = await o.packedExpert(layer, 'shared', x, n);
        const sharedGate = await o.mat(p + 'ffn_gate_inp_shexp.weight', x, n), y = await o.alloc(n * g.width);
        await b.run('strata_moe_combine_batch', {Parts: parts, Weights: weights, Shared: shared,
            SharedGate: sharedGate, Y: y, width: g.width, count: g.topK, tokens: n}, [Math.ceil(n * g.width / 64), 1, 1]);
        await o.release(logits, parts, shared, sharedGate);
        return {y, ids, weights};
    }
}
