// A stand-in for the Node-API addon that keeps buffers in host memory and
// records every launch, for host-side tests without a GPU. Kernel
// signatures and workspace sizes come from the real addon (pure functions of
// the C ABI). With `emulate`, the two launches whose results the host reads
// back produce values: strata_router[_batch] writes distinct IDs per token
// ((5 t + 2 k + 1) mod experts, or `routes(t, k, experts)`), strata_argmax
// writes token 3.
export function fakeAddon(real, options) {
    const o = options || {}, mem = new Map(), calls = [];
    let next = 4096;
    const routes = o.routes || ((t, k, experts) => (t * 5 + k * 2 + 1) % experts);
    return {
        calls, mem, real,
        init: () => ({ctx: true}),
        shutdown: () => {},
        info: () => JSON.stringify({device: 'stand-in'}),
        alloc: (ctx, bytes) => { const h = next; next += Math.max(256, Math.ceil(bytes / 256) * 256); mem.set(h, new Uint8Array(bytes)); return h; },
        free: (ctx, h) => { if (!mem.delete(h)) throw Error('double free'); },
        write: (ctx, h, off, data) => {
            const src = ArrayBuffer.isView(data) ? new Uint8Array(data.buffer, data.byteOffset, data.byteLength) : new Uint8Array(data);
            mem.get(h).set(src, off);
        },
        read: (ctx, h, off, n) => mem.get(h).slice(off, off + n).buffer,
        copy: (ctx, s, so, d, dof, n) => { mem.get(d).set(mem.get(s).subarray(so, so + n), dof); calls.push({name: 'copy', slots: [s, so, d, dof, n]}); },
        zero: (ctx, h, off, n) => { mem.get(h).fill(0, off, off + n); calls.push({name: 'zero', slots: [h, off, n]}); },
        sync: () => {},
        signature: name => real.signature(name),
        kernels: () => real.kernels(),
        run: (ctx, name, groups, slots) => {
            calls.push({name, groups, slots});
            if (!o.emulate) return;
            if (name === 'strata_router' || name === 'strata_router_batch') {
                const ids = new Int32Array(mem.get(slots[1]).buffer), experts = slots[3], topK = slots[4];
                for (let t = 0; t < groups[0]; t++)
                    for (let k = 0; k < topK; k++) ids[t * topK + k] = routes(t, k, experts);
            }
            if (name === 'strata_argmax') new Int32Array(mem.get(slots[1]).buffer)[0] = 3;
        },
        moeWorkspace: (...a) => real.moeWorkspace(...a),
        moeLayer: (ctx, ...args) => calls.push({name: 'moeLayer', args}),
        moeBlockWorkspace: (...a) => real.moeBlockWorkspace(...a),
        moeBlock: (ctx, ...args) => calls.push({name: 'moeBlock', args}),
        synthBlobs: (ctx, ...args) => calls.push({name: 'synthBlobs', args}),
        synthNormal: (ctx, ...args) => calls.push({name: 'synthNormal', args}),
        synthUniformPm: (ctx, ...args) => calls.push({name: 'synthUniformPm', args}),
    };
}
