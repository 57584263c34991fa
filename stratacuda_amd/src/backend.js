// HipBackend: the reference's backend interface (src/backend.js:58-122 of
// SamG-Coder/StrataCuda: alloc / write / zero / read / copy / run / free /
// flush / idle / info / dispose) on an MI355X through libstrata_mi355x.so and
// its Node-API addon. Written for the Node 12 runtime of this image (no `?.`,
// `??`, private fields or top-level await).
//
// Semantics kept from the reference:
//   - buffers are handles with `.length` in 4-byte words and `.type`;
//   - run(name, args, groups) takes named buffers and scalars, groups are
//     workgroups of 64 lanes (scripts/build.mjs:10), and validateDispatch
//     throws RangeError / Error synchronously, before any launch;
//   - later failures surface from read() / idle() (rejected promise).
// Differences: work is issued in order on one HIP stream (flush is a no-op,
// there is no 128-dispatch batch), a device fault of an asynchronous launch
// is reported by the next synchronising call, and the fused MoE entries
// (moeLayer / moeRoute / moeDispatch) replace the host-driven stage of
// src/engine.js:133-156 and src/prefill.js:52-78 for kind 'hip'.
import {createRequire} from 'module';
import {fileURLToPath} from 'url';
import path from 'path';

const require = createRequire(import.meta.url);
const HERE = path.dirname(fileURLToPath(import.meta.url));

export const typed = {f32: Float32Array, i32: Int32Array, u32: Uint32Array};

// src/backend.js:6-9: an integer in [min, max] or a RangeError naming it.
export function requireInteger(n, label, min = 1, max = 0x7fffffff) {
    if (!Number.isSafeInteger(n) || n < min || n > max)
        throw new RangeError(label + ' must be an integer in [' + min + ', ' + max + ']');
    return n;
}

// Argument checks run before any launch, with the reference's conditions and
// messages (src/backend.js:10-56) for the kernels this library provides.
const PROJECTIONS = ['strata_project', 'strata_quant_project', 'strata_bf16_project', 'strata_q2_project'];
export function validateDispatch(name, args) {
    const get = k => requireInteger(args[k], name + '.' + k);
    if (name === 'strata_router' || name === 'strata_router_batch') {
        if (get('experts') > 512 || get('topK') > Math.min(args.experts, 32))
            throw new RangeError('Router supports 1–512 experts and topK <= min(experts,32)');
    }
    if (name === 'strata_quant_gemv' || name === 'strata_quant_project') {
        if ([2, 4, 8].indexOf(args.bits) < 0) throw new RangeError('Canonical code width must be 2, 4 or 8');
        if (get('cols') % get('groupSize') || args.cols * args.rows * args.bits > 0x7fffffff)
            throw new RangeError('Quantized rows must contain whole groups and fit 31-bit indexing');
    }
    if (PROJECTIONS.indexOf(name) >= 0) {
        get('tokens'); get('rows'); get('cols'); get('outputStride');
        requireInteger(args.outputOffset, 'projection output offset', 0);
        if (args.outputOffset + args.rows > args.outputStride || args.tokens * args.outputStride > args.Y.length ||
            args.tokens * args.cols > args.X.length)
            throw Error('Projection batch exceeds buffer layout');
    }
    if (name === 'strata_q2_project') {
        if (args.cols % 64) throw Error('Q2 expert columns must contain complete groups');
        for (const key of ['codeOffset', 'scaleOffset', 'weightRow']) requireInteger(args[key], key, 0);
        requireInteger(args.rowStride, 'expert row stride', 1, 2);
    }
    if (name === 'strata_q2_gate_up' || name === 'strata_q2_down') {
        if (get('width') % 64 || get('ff') % 64) throw Error('Packed expert dimensions must contain complete groups');
        const tokens = get('tokens');
        if (args.Hidden.length < tokens * args.ff || (args.mapped && args.Mapping.length < tokens * 2))
            throw Error('Packed expert batch exceeds buffer layout');
        if (name === 'strata_q2_down') requireInteger(args.outputOffset, 'expert output offset', 0);
    }
    if (name === 'strata_embedding') {
        const count = get('width') * get('streams');
        requireInteger(args.outputOffset, 'embedding output offset', 0);
        if (args.outputOffset + count > args.Residual.length || [0, 1, 2].indexOf(args.format) < 0)
            throw Error('Embedding exceeds buffer layout');
        if (args.format === 2 && ([2, 4, 8].indexOf(args.bits) < 0 || args.width % get('groupSize')))
            throw Error('Invalid packed embedding layout');
    }
    if (name === 'strata_rope_position') {
        requireInteger(args.position, 'RoPE position', 0, 2047);
        if (get('rotary') % 2 || args.rotary > get('dim') || args.position + get('tokens') > 2048 ||
            args.Cos.length < (args.position + args.tokens) * args.rotary / 2 || args.Sin.length !== args.Cos.length ||
            args.X.length !== args.dim * get('heads') * args.tokens || args.Y.length !== args.X.length)
            throw Error('Invalid RoPE layout');
    }
    if (name === 'strata_rope_frequencies' && (!Number.isFinite(args.base) || args.base <= 1 || get('rotary') % 2))
        throw Error('Invalid RoPE frequencies');
    if (name === 'strata_ple_decode' && (get('count') % 32 || Math.ceil(args.count / 32 * 18 / 4) > args.Packed.length ||
        args.count > args.Values.length))
        throw Error('Invalid packed PLE layout');
    if (name === 'strata_rope' && (get('rotary') % 2 || args.rotary > get('dim')))
        throw new RangeError('Rotary width must be even and <= head dimension');
    if (name === 'strata_attention') {
        if (get('heads') % get('kvHeads')) throw new RangeError('Attention heads must be divisible by KV heads');
        requireInteger(args.count, 'attention selected cells', 1, 2048);
    }
    if (name === 'strata_norm' && get('rows') % get('weightRows'))
        throw new RangeError('Normalization weight rows must divide input rows');
}

// Loads the addon built next to this file (stratacuda_amd/src/strata_addon.node).
export function loadAddon(file) {
    return require(file || path.join(HERE, 'strata_addon.node'));
}

function parseSignature(sig) {
    return sig.split(',').map(p => {
        const at = p.indexOf(':');
        return {name: p.slice(0, at), type: p.slice(at + 1)};
    });
}
const f32bits = new Float32Array(1), u32bits = new Uint32Array(f32bits.buffer);

export class HipBackend {
    // create({device, addon}): addon defaults to the built strata_addon.node;
    // tests pass a stand-in with the same functions.
    static async create(options) {
        const o = options || {};
        const addon = o.addon || loadAddon();
        return new HipBackend(addon, addon.init(o.device || 0));
    }
    constructor(addon, ctx) {
        this.addon = addon; this.ctx = ctx; this.kind = 'hip';
        this.buffers = new Set(); this.signatures = new Map(); this.dispatches = 0; this.failure = null;
        this.bytesAllocated = 0;
    }
    assertAlive() {
        if (!this.ctx) throw Error('HIP backend is disposed');
        if (this.failure) throw this.failure;
    }
    // alloc(dataOrLength, type, {zero}): a length counts 4-byte words
    // (src/backend.js:84-92). New buffers are zero-filled unless zero:false.
    alloc(dataOrLength, type, options) {
        type = type || 'f32';
        const zero = !options || options.zero !== false;
        if (!typed[type]) throw Error('Unsupported buffer type ' + type);
        this.assertAlive();
        const bytes = typeof dataOrLength === 'number' ? requireInteger(dataOrLength, 'allocation') * 4
            : dataOrLength.byteLength;
        const id = this.addon.alloc(this.ctx, bytes, typeof dataOrLength === 'number' ? zero : false);
        const handle = {id, type, length: bytes / 4, byteLength: bytes};
        this.buffers.add(handle); this.bytesAllocated += bytes;
        if (typeof dataOrLength !== 'number') this.addon.write(this.ctx, id, 0, dataOrLength);
        return handle;
    }
    // A buffer sized in bytes (expert arenas exceed the 2^31-word limit of
    // alloc); .length stays in words.
    allocBytes(bytes, type, options) {
        requireInteger(bytes, 'allocation bytes', 4, Number.MAX_SAFE_INTEGER);
        if (bytes % 4) throw new RangeError('allocation bytes must be a multiple of 4');
        this.assertAlive();
        const zero = !options || options.zero !== false;
        const id = this.addon.alloc(this.ctx, bytes, zero);
        const handle = {id, type: type || 'u32', length: bytes / 4, byteLength: bytes};
        this.buffers.add(handle); this.bytesAllocated += bytes;
        return handle;
    }
    owned(buffer, what) {
        if (!buffer || !this.buffers.has(buffer)) throw Error('Invalid HIP ' + what);
        return buffer.id;
    }
    // write(buffer, typed, offsetWords) (src/backend.js:93).
    write(buffer, data, offset) {
        offset = offset || 0;
        const id = this.owned(buffer, 'write');
        if (offset < 0 || offset * 4 + data.byteLength > buffer.byteLength) throw Error('Invalid HIP write');
        this.assertAlive();
        this.addon.write(this.ctx, id, offset * 4, data);
    }
    zero(buffer) { this.assertAlive(); this.addon.zero(this.ctx, this.owned(buffer, 'zero'), 0, buffer.byteLength); }
    // async read(buffer, type): a fresh typed array (src/backend.js:95).
    async read(buffer, type) {
        type = type || buffer.type;
        const id = this.owned(buffer, 'read');
        this.assertAlive();
        if (!typed[type]) throw Error('Unsupported buffer type ' + type);
        let bytes;
        try { bytes = this.addon.read(this.ctx, id, 0, buffer.byteLength); } catch (error) {
            // a wait of the single-launch decode layer gave up: the backend
            // fails like a lost device until resetFusedDecode()
            if (error.code === 'SM_E_FAULT') this.failure = error;
            throw error;
        }
        return new typed[type](bytes);
    }
    // Clears the single-launch decode layer's fault (after SM_E_FAULT from
    // read() or idle()); later launches compute again.
    resetFusedDecode() {
        if (!this.ctx) throw Error('HIP backend is disposed');
        this.addon.fusedReset(this.ctx);
        if (this.failure && this.failure.code === 'SM_E_FAULT') this.failure = null;
    }
    // The router matrix (rows x width f32) of the layer after the next one:
    // the next single-launch decode layer pulls it into L2 (a hint for that
    // one layer call; null clears it).
    prefetchRouter(buffer, rows, width) {
        this.assertAlive();
        if (buffer === null) return this.addon.prefetchRouter(this.ctx, 0, 0, 0);
        this.addon.prefetchRouter(this.ctx, this.owned(buffer, 'prefetch'), rows, width);
    }
    // Bytes [offset, offset + bytes) of a buffer as an ArrayBuffer.
    async readBytes(buffer, offset, bytes) {
        this.assertAlive();
        return this.addon.read(this.ctx, this.owned(buffer, 'read'), offset, bytes);
    }
    // copy(source, destination, countWords, sourceOffset, destinationOffset) (src/backend.js:96-100).
    copy(source, destination, count, sourceOffset, destinationOffset) {
        count = count === undefined ? source.length : count;
        sourceOffset = sourceOffset || 0; destinationOffset = destinationOffset || 0;
        const s = this.owned(source, 'copy'), d = this.owned(destination, 'copy');
        if (count < 0 || sourceOffset < 0 || destinationOffset < 0 || count + sourceOffset > source.length ||
            count + destinationOffset > destination.length)
            throw Error('Invalid HIP copy');
        this.assertAlive();
        this.addon.copy(this.ctx, s, sourceOffset * 4, d, destinationOffset * 4, count * 4);
    }
    signature(name) {
        let sig = this.signatures.get(name);
        if (!sig) {
            const text = this.addon.signature(name);
            if (text === null || text === undefined) throw Error('Unknown kernel ' + name);
            sig = parseSignature(text); this.signatures.set(name, sig);
        }
        return sig;
    }
    // run(name, args, groups) (src/backend.js:101-113): named buffers and
    // scalars, in any order; the library receives them in parameter order.
    run(name, args, groups) {
        validateDispatch(name, args);
        const sig = this.signature(name);
        const slots = sig.map(p => {
            const v = args[p.name];
            if (v === undefined) throw Error('Missing ' + name + '.' + p.name);
            if (p.type.charAt(p.type.length - 1) === '*') {
                if (typeof v === 'number') throw Error(name + '.' + p.name + ' must be a buffer');
                return this.owned(v, 'buffer ' + name + '.' + p.name);
            }
            if (typeof v !== 'number') throw Error(name + '.' + p.name + ' must be a number');
            if (p.type === 'f32') { f32bits[0] = v; return u32bits[0]; }
            if (!Number.isInteger(v) || v < -0x80000000 || v > 0x7fffffff)
                throw new RangeError(name + '.' + p.name + ' must be a 32-bit integer');
            return v >>> 0;
        });
        this.assertAlive();
        this.addon.run(this.ctx, name, [groups[0], groups[1], groups[2]], slots);
        this.dispatches++;
    }
    free(buffer) {
        if (!this.buffers.delete(buffer)) return;
        this.bytesAllocated -= buffer.byteLength;
        if (this.ctx) this.addon.free(this.ctx, buffer.id);
    }
    flush() {}
    async idle() {
        this.assertAlive();
        try { this.addon.sync(this.ctx); } catch (error) { this.failure = error; throw error; }
    }
    info() {
        const device = this.ctx ? JSON.parse(this.addon.info(this.ctx)) : {};
        return Object.assign({backend: this.kind}, device,
            {dispatches: this.dispatches, liveBuffers: this.buffers.size, allocatedBytes: this.bytesAllocated});
    }
    async dispose() {
        if (!this.ctx) return;
        try { this.addon.sync(this.ctx); } catch (error) { /* the context is released below either way */ }
        finally {
            for (const b of this.buffers) this.addon.free(this.ctx, b.id);
            this.buffers.clear(); this.bytesAllocated = 0;
            this.addon.shutdown(this.ctx); this.ctx = null;
        }
    }

    // ------------------------------------------------ fused MoE (kind 'hip')
    // loadExperts(path, fileOffset, blobBytes, count, arena, stride,
    // scalesOffset, dstOffset): `count` blobs stored back to back in a pack's
    // experts.bin streamed into the arena (blob i at dstOffset + i * stride),
    // every fp16 scale checked finite (PackStore.readExpertBlob,
    // src/model.js:160-167). Synchronous.
    loadExperts(path, fileOffset, blobBytes, count, arena, stride, scalesOffset, dstOffset) {
        this.assertAlive();
        this.addon.loadExperts(this.ctx, String(path), fileOffset, blobBytes, count, this.owned(arena, 'arena'),
            dstOffset || 0, stride, scalesOffset);
    }
    moeWorkspaceBytes(tokens, width, ff, experts, topK) {
        return this.addon.moeWorkspace(tokens, width, ff, experts, topK);
    }
    // One MoE layer on the device: router projection (+ optional bias), top-k,
    // dispatch, expert products, shared expert, shared gate and combine.
    moeLayer(a) {
        this.assertAlive();
        const ws = this.owned(a.workspace, 'workspace');
        this.addon.moeLayer(this.ctx, this.owned(a.X, 'X'), a.tokens, this.owned(a.Wr, 'Wr'),
            a.bias ? this.owned(a.bias, 'bias') : 0, this.owned(a.arena, 'arena'), a.stride,
            this.owned(a.shared, 'shared'), this.owned(a.Wsg, 'Wsg'), a.width, a.ff, a.experts, a.topK,
            this.owned(a.Y, 'Y'), this.owned(a.ids, 'ids'), this.owned(a.weights, 'weights'), ws,
            a.workspace.byteLength);
        this.dispatches++;
    }
    moeBlockWorkspaceBytes(tokens, width, ff, experts, topK) {
        return this.addon.moeBlockWorkspace(tokens, width, ff, experts, topK);
    }
    // One block of a stacked decoder around the MoE stage (strata_norm mode 0,
    // the stage, strata_elementwise mode 5): Hout = H + MoE(RMSNorm(H; gamma)).
    // Hout may be H itself. Bit-identical to the three steps run separately.
    moeBlock(a) {
        this.assertAlive();
        const ws = this.owned(a.workspace, 'workspace');
        this.addon.moeBlock(this.ctx, this.owned(a.H, 'H'), a.tokens, this.owned(a.gamma, 'gamma'), a.eps,
            this.owned(a.Wr, 'Wr'), a.bias ? this.owned(a.bias, 'bias') : 0, this.owned(a.arena, 'arena'), a.stride,
            this.owned(a.shared, 'shared'), this.owned(a.Wsg, 'Wsg'), a.width, a.ff, a.experts, a.topK,
            this.owned(a.Hout, 'Hout'), this.owned(a.ids, 'ids'), this.owned(a.weights, 'weights'), ws,
            a.workspace.byteLength);
        this.dispatches++;
    }
    moeRoute(a) {
        this.assertAlive();
        this.addon.moeRoute(this.ctx, this.owned(a.X, 'X'), a.tokens, a.width, this.owned(a.Wr, 'Wr'),
            a.bias ? this.owned(a.bias, 'bias') : 0, a.experts, a.topK, a.logits ? this.owned(a.logits, 'logits') : 0,
            this.owned(a.ids, 'ids'), this.owned(a.weights, 'weights'));
        this.dispatches++;
    }
    moeDispatch(a) {
        this.assertAlive();
        this.addon.moeDispatch(this.ctx, this.owned(a.ids, 'ids'), a.tokens, a.topK, a.experts,
            this.owned(a.offsets, 'offsets'), this.owned(a.rows, 'rows'), this.owned(a.parts, 'parts'),
            this.owned(a.where, 'where'), this.owned(a.workspace, 'workspace'), a.workspace.byteLength);
        this.dispatches++;
    }
    // Seeded synthetic data, bit-identical to the CPU oracle's generator.
    synthNormal(buffer, n, seed, stream, sigma, offsetBytes) {
        this.addon.synthNormal(this.ctx, this.owned(buffer, 'synth'), offsetBytes || 0, n, seed, stream, sigma);
    }
    synthUniformPm(buffer, n, seed, stream, amp, offsetBytes) {
        this.addon.synthUniformPm(this.ctx, this.owned(buffer, 'synth'), offsetBytes || 0, n, seed, stream, amp);
    }
    synthBlobs(buffer, stride, count, width, ff, seed, firstStream, sigma, offsetBytes) {
        this.addon.synthBlobs(this.ctx, this.owned(buffer, 'synth'), offsetBytes || 0, stride, count, width, ff, seed,
            firstStream, sigma);
    }
}
