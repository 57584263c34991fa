// StrataEngine: a decoding session over one MI355X (HipBackend), with the
// reference's session API (src/engine.js:7-223): create, step, prefill,
// reset, checkpoint, restore, dispose, residencyInfo, and the same argument
// checks and error messages.
//
// Structure: the model is a program (plan.js) built once from the geometry;
// an Interpreter (interpreter.js) executes its instruction lists for a Frame
// of tokens. A decode step is a one-token frame over the persistent residual,
// a prompt chunk an n-token frame over a chunk residual whose last row is
// kept; both run the same lists, then the head list predicts from the
// persistent residual. DecoderState owns everything that persists between
// tokens. Every model tensor is resident in HBM from create() on
// (ModelResidency); there is no CPU expert lane. Written for Node 12.
import crypto from 'crypto';
import {performance} from 'perf_hooks';
import {Ops} from './ops.js';
import {validateGeometry} from './model.js';
import {requireInteger} from './backend.js';
import {ModelResidency} from './residency.js';
import {buildProgram, weightShapes, layerStateShapes} from './plan.js';
import {Frame, Interpreter} from './interpreter.js';
import {MoeStage} from './moe.js';

// The persistent buffers of a session: the residual streams of the last
// token, the PLE convolution history and each layer's recurrent state.
class DecoderState {
    constructor(backend, g) {
        this.b = backend; this.buffers = [];
        const keep = n => { const buf = backend.alloc(n, 'f32', {zero: true}); this.buffers.push(buf); return buf; };
        this.residual = keep(g.width * g.streams);
        this.pleHistory = keep((g.pleTaps - 1) * g.pleDilation * g.width * g.streams);
        this.layers = [];
        for (let l = 0; l < g.layers; l++) {
            const shapes = layerStateShapes(g, l), entry = {};
            for (const key of Object.keys(shapes)) entry[key] = keep(shapes[key]);
            this.layers.push(entry);
        }
    }
    zero() { for (const buf of this.buffers) this.b.zero(buf); }
    async snapshot() {
        const out = [];
        for (const buf of this.buffers) out.push(await this.b.read(buf));
        return out;
    }
    load(arrays) { this.buffers.forEach((buf, i) => this.b.write(buf, arrays[i])); }
    free() { for (const buf of this.buffers) this.b.free(buf); this.buffers = []; }
}

// Per operation: the message when another operation holds the session,
// the message when the session has failed (null: allowed), whether an error
// inside marks the session failed and whether success clears a failure.
const RULES = {
    step: {busy: 'A session operation is already running', unhealthy: 'Session failed; reset it before continuing',
        failsOnError: true, heals: false},
    reset: {busy: 'Cannot reset during a decode step or state operation', unhealthy: null, failsOnError: true,
        heals: true},
    checkpoint: {busy: 'Checkpoint requires an idle session', unhealthy: 'Checkpoint requires a healthy session',
        failsOnError: false, heals: false},
    restore: {busy: 'Cannot restore during decode or state operation', unhealthy: null, failsOnError: true,
        heals: true},
    dispose: {busy: 'Cannot dispose during a decode step or state operation', unhealthy: null, failsOnError: true,
        heals: false},
};

const trimmedShape = shape => {
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
        this.ops = new Ops(backend, store); this.program = buildProgram(this.g);
        this.state = null; this.interpreter = null;
        this.position = 0; this.previous = [];
        this.busy = false; this.failed = false; this.disposed = false;
        this.checkpointOwner = crypto.randomBytes(16).toString('hex');
        this.stats = {tokens: 0, gpuExperts: 0, cpuExperts: 0, promotions: 0, routes: [], lastMs: 0};
    }
    // Shape gate first (every tensor the program reads), then the resident
    // weights and the persistent state.
    async initialize() {
        for (const [name, expected] of weightShapes(this.program)) {
            const found = this.store.describe(name).shape;
            if (trimmedShape(found) !== trimmedShape(expected))
                throw Error(name + ': expected [' + expected + '], found [' + trimmedShape(found) + ']');
        }
        await new ModelResidency(this.ops).loadAll();
        this.state = new DecoderState(this.b, this.g);
        this.interpreter = new Interpreter(this.ops, this.g, this.state,
            new MoeStage(this.ops, {fused: false, stats: this.stats}));
    }
    residencyInfo() { return this.ops.residency.info(); }

    // Runs `body` holding the session under `kind`'s rules; `check` runs
    // after the session-state checks and before the session is taken.
    async exclusive(kind, check, body) {
        const rule = RULES[kind];
        if (this.disposed) throw Error('Session is disposed');
        if (this.busy) throw Error(rule.busy);
        if (rule.unhealthy && this.failed) throw Error(rule.unhealthy);
        if (check) check();
        this.busy = true;
        try {
            const result = await body();
            if (rule.heals) this.failed = false;
            return result;
        } catch (error) {
            if (rule.failsOnError) this.failed = true;
            throw error;
        } finally { this.busy = false; }
    }

    // The embedding and every layer for the tokens of `frame`.
    async forward(frame, onProgress) {
        const it = this.interpreter, g = this.g;
        await it.run(this.program.embed, frame, -1);
        for (const layer of this.program.layers) {
            await it.run(layer.list, frame, layer.index);
            await this.ops.clearTemporary();
            if (onProgress) onProgress(layer.index + 1, g.layers);
        }
    }
    // The head on the persistent residual: the argmax token and, on request,
    // the logits.
    async predict(withLogits) {
        const g = this.g, frame = new Frame({tokens: [0], position: this.position, previous: this.previous,
            residual: this.state.residual, batched: false});
        const regs = await this.interpreter.run(this.program.head, frame, -1), out = {};
        out.token = (await this.b.read(regs.get('next'), 'i32'))[0];
        requireInteger(out.token, 'generated token', 0, g.vocab - 1);
        if (withLogits) {
            out.logits = await this.b.read(regs.get('logits'));
            if (out.logits.some(v => !Number.isFinite(v))) throw Error('Non-finite logits');
        }
        return out;
    }
    advance(tokens) {
        this.previous = this.previous.concat(tokens).slice(-2);
        this.position += tokens.length; this.stats.tokens += tokens.length;
    }

    async step(token, options) {
        const o = options || {}, predict = o.predict !== false;
        return this.exclusive('step', () => {
            if (o.logits && !predict) throw Error('Logits require prediction');
            requireInteger(token, 'token', 0, this.g.vocab - 1);
            if (this.position >= this.g.context) throw Error('Context capacity reached; reset or create a larger session');
        }, async () => {
            const start = performance.now();
            this.stats.routes = [];
            await this.forward(new Frame({tokens: [token], position: this.position, previous: this.previous,
                residual: this.state.residual, batched: false}), o.onProgress);
            const result = {position: this.position};
            if (predict) Object.assign(result, await this.predict(!!o.logits));
            await this.ops.clearTemporary();
            this.advance([token]);
            this.stats.lastMs = performance.now() - start;
            return result;
        });
    }

    // The prompt in chunks of `chunkSize` tokens (default 16), each chunk
    // layer-major through the batch kernels; then, unless predict is false,
    // the head on the last prompt token.
    async prefill(tokens, options) {
        const o = options || {}, list = Array.from(tokens);
        const chunkSize = o.chunkSize === undefined ? 16 : o.chunkSize;
        return this.exclusive('step', () => {
            if (!list.length) throw Error('Prompt is empty');
            for (const t of list) requireInteger(t, 'token', 0, this.g.vocab - 1);
            if (this.position + list.length > this.g.context) throw Error('Context capacity reached');
            requireInteger(chunkSize, 'prompt chunk size', 1, 64);
            if (o.logits && o.predict === false) throw Error('Logits require prediction');
        }, async () => {
            const start = performance.now(), hc = this.g.width * this.g.streams;
            this.stats.routes = [];
            for (let offset = 0; offset < list.length; offset += chunkSize) {
                const chunk = list.slice(offset, offset + chunkSize), residual = this.b.alloc(chunk.length * hc);
                try {
                    await this.forward(new Frame({tokens: chunk, position: this.position, previous: this.previous,
                        residual, batched: true}), o.onProgress ? (l, n) => o.onProgress(l, n, offset, chunk.length) : null);
                    this.b.copy(residual, this.state.residual, hc, (chunk.length - 1) * hc, 0);
                    this.advance(chunk);
                } finally { this.b.free(residual); }
            }
            const result = {position: this.position - 1};
            if (o.predict !== false) Object.assign(result, await this.predict(!!o.logits));
            await this.ops.clearTemporary();
            this.stats.lastMs = performance.now() - start;
            return result;
        });
    }

    async reset() {
        return this.exclusive('reset', null, async () => {
            await this.ops.clearTemporary();
            this.state.zero();
            this.position = 0; this.previous = [];
        });
    }
    async checkpoint() {
        return this.exclusive('checkpoint', null, async () => ({owner: this.checkpointOwner,
            geometry: JSON.stringify(this.g), position: this.position, previous: this.previous.slice(),
            buffers: await this.state.snapshot()}));
    }
    // Whether `cp` is a checkpoint of this session with well-formed contents.
    matches(cp) {
        const g = this.g, mine = this.state.buffers;
        if (!cp || cp.owner !== this.checkpointOwner || cp.geometry !== JSON.stringify(g)) return false;
        if (!Array.isArray(cp.buffers) || cp.buffers.length !== mine.length) return false;
        for (let i = 0; i < mine.length; i++) {
            const a = cp.buffers[i];
            if (!(a instanceof Float32Array) || a.length !== mine[i].length || !a.every(Number.isFinite)) return false;
        }
        if (!Number.isInteger(cp.position) || cp.position < 0 || cp.position > g.context) return false;
        if (!Array.isArray(cp.previous) || cp.previous.length !== Math.min(cp.position, 2)) return false;
        return cp.previous.every(t => Number.isInteger(t) && t >= 0 && t < g.vocab);
    }
    async restore(cp) {
        return this.exclusive('restore', () => {
            if (!this.matches(cp)) throw Error('Checkpoint does not match this model/session geometry');
        }, async () => {
            await this.ops.clearTemporary();
            this.state.load(cp.buffers);
            this.position = cp.position; this.previous = cp.previous.slice();
        });
    }
    async dispose() {
        if (this.disposed) return;
        return this.exclusive('dispose', null, async () => {
            await this.ops.dispose();
            if (this.state) this.state.free();
            this.disposed = true;
        });
    }
}
