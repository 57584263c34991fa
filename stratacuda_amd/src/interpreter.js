// Executes the instruction lists of plan.js on a backend. A Frame describes
// the tokens in flight: how many (n), whether they run through the one-token
// kernels (a decode step) or the *_batch kernels (a prompt chunk), their
// first position, their token IDs, the two tokens before them (for the PLE
// n-gram rows) and the residual buffer they live in. Registers are the
// Ops temporaries of the current list; clearTemporary() ends their life.
import {grid} from './ops.js';
import {KERNELS, RESIDUAL} from './plan.js';
import {MoeStage} from './moe.js';

export class Frame {
    constructor({tokens, position, previous, residual, batched}) {
        this.tokens = tokens; this.n = tokens.length; this.position = position;
        this.previous = previous; this.residual = residual; this.batched = batched;
    }
}

export class Interpreter {
    // state: the session's DecoderState (per-layer recurrent buffers and the
    // PLE history); moe: the MoeStage that runs `moe` instructions.
    constructor(ops, geometry, state, moe) {
        this.ops = ops; this.b = ops.b; this.g = geometry; this.state = state;
        this.moe = moe || new MoeStage(ops, {fused: false});
        this.registers = new Map(); this.frame = null; this.layer = -1;
    }
    reg(name) {
        if (name === RESIDUAL) return this.frame.residual;
        const buffer = this.registers.get(name);
        if (!buffer) throw Error('instruction reads register ' + name + ' before it is written');
        return buffer;
    }
    set(name, buffer) { this.registers.set(name, buffer); return buffer; }
    kernel(op) { return KERNELS[op][this.frame.batched ? 1 : 0]; }
    // Batched kernels take the token count; one-token kernels do not.
    withTokens(args) { if (this.frame.batched) args.tokens = this.frame.n; return args; }
    async vector(ins, role) { return this.ops.vector(ins.weights[role][0]); }

    // Runs `list` for `frame` with layer `layer`'s state (-1: none).
    async run(list, frame, layer) {
        this.frame = frame; this.layer = layer; this.registers.clear();
        for (const ins of list) {
            const handler = HANDLERS[ins.op];
            if (!handler) throw Error('unknown instruction ' + ins.op);
            await handler.call(this, ins);
        }
        return this.registers;
    }
    layerState(key) {
        const s = key === 'pleHistory' ? this.state.pleHistory : this.state.layers[this.layer][key];
        if (!s) throw Error('layer ' + this.layer + ' keeps no ' + key + ' state');
        return s;
    }
}

// One handler per instruction kind; `this` is the Interpreter.
const HANDLERS = {
    async embed(ins) {
        const f = this.frame, hc = this.g.width * this.g.streams;
        for (let t = 0; t < f.n; t++) await this.ops.embedding(f.tokens[t], f.residual, t * hc);
    },
    async project(ins) {
        this.set(ins.y, await this.ops.mat(ins.weights.W[0], this.reg(ins.x), this.frame.n));
    },
    async norm(ins) {
        const x = this.reg(ins.x), w = ins.weights ? await this.vector(ins, 'W') : x;
        this.set(ins.y, await this.ops.norm(x, w, ins.cols, ins.rows * this.frame.n, ins.weightRows, ins.mode || 0,
            ins.scale === undefined ? 1 : ins.scale));
    },
    async elementwise(ins) {
        this.set(ins.y, await this.ops.elem(this.reg(ins.a), this.reg(ins.b), ins.mode, ins.scale));
    },
    async slice(ins) {
        this.set(ins.y, await this.ops.slice(this.reg(ins.x), ins.width, ins.rows * this.frame.n, ins.stride, ins.offset));
    },
    async rope(ins) {
        this.set(ins.y, await this.ops.rotate(this.reg(ins.x), ins.heads, this.frame.position, this.frame.n));
    },
    async hcMix(ins) {
        const g = this.g, n = this.frame.n, y = this.set(ins.y, await this.ops.alloc(n * g.width));
        await this.b.run(this.kernel('hcMix'), this.withTokens({Norm: this.reg(ins.norm), Gate: this.reg(ins.gate),
            Mixed: y, width: g.width, streams: g.streams}), grid(n * g.width));
    },
    async hcWrite(ins) {
        const g = this.g, n = this.frame.n;
        await this.b.run(this.kernel('hcWrite'), this.withTokens({Residual: this.frame.residual, Output: this.reg(ins.x),
            Inject: this.reg(ins.inject), width: g.width, streams: g.streams}), grid(n * g.width * g.streams));
    },
    // Causal depthwise convolution whose last taps live in the layer state
    // (one-token kernel: one position; batch kernel: n positions in order).
    async conv(ins) {
        const y = this.set(ins.y, await this.ops.alloc(this.frame.n * ins.channels));
        await this.b.run(this.kernel('conv'), this.withTokens({History: this.layerState(ins.history), X: this.reg(ins.x),
            W: await this.vector(ins, 'W'), Y: y, channels: ins.channels, taps: ins.taps, dilation: ins.dilation,
            activation: 1}), grid(ins.channels));
    },
    async gdnGates(ins) {
        const heads = this.g.valueHeads, n = this.frame.n;
        const decay = this.set(ins.decay, await this.ops.alloc(n * heads));
        const strength = this.set(ins.strength, await this.ops.alloc(n * heads));
        await this.b.run(this.kernel('gdnGates'), this.withTokens({Alpha: this.reg(ins.alpha), Beta: this.reg(ins.beta),
            A: await this.vector(ins, 'A'), Dt: await this.vector(ins, 'Dt'), Decay: decay, Strength: strength, heads}),
        grid(n * heads));
    },
    async gdnScan(ins) {
        const g = this.g, vn = g.ssmDim * g.valueHeads, y = this.set(ins.y, await this.ops.alloc(this.frame.n * vn));
        await this.b.run(this.kernel('gdnScan'), this.withTokens({State: this.layerState('ssm'), Q: this.reg(ins.q),
            K: this.reg(ins.k), V: this.reg(ins.v), Decay: this.reg(ins.decay), Beta: this.reg(ins.strength), Y: y,
            dim: g.ssmDim, keyHeads: g.keyHeads, valueHeads: g.valueHeads}), grid(vn));
    },
    async kvAppend(ins) {
        const n = this.frame.n;
        await this.b.run(this.kernel('kvAppend'), this.withTokens({K: this.reg(ins.k), V: this.reg(ins.v),
            Keys: this.layerState('keys'), Values: this.layerState('values'), width: ins.width,
            position: this.frame.position}), grid(n * ins.width));
    },
    // One-token attention reads the cached positions through a cell list
    // (0..position); the batch kernel masks causally from `position` on.
    async attention(ins) {
        const g = this.g, f = this.frame, y = this.set(ins.y, await this.ops.alloc(f.n * g.heads * g.headDim));
        const args = {Q: this.reg(ins.q), Keys: this.layerState('keys'), Values: this.layerState('values'), Y: y,
            dim: g.headDim, heads: g.heads, kvHeads: g.kvHeads, scale: 1 / Math.sqrt(g.headDim)};
        const columns = Math.ceil(g.headDim / 64);
        if (f.batched) {
            args.position = f.position;
            await this.b.run(this.kernel('attention'), args, [g.heads, columns, f.n]);
        } else {
            args.Cells = await this.ops.alloc(Int32Array.from({length: f.position + 1}, (_, i) => i), 'i32');
            args.count = f.position + 1;
            await this.b.run(this.kernel('attention'), args, [g.heads, columns, 1]);
        }
    },
    async attentionGate(ins) {
        const g = this.g, size = this.frame.n * g.heads * g.headDim, y = this.set(ins.y, await this.ops.alloc(size));
        await this.b.run(this.kernel('attentionGate'), this.withTokens({Attention: this.reg(ins.attention),
            FullQ: this.reg(ins.full), Y: y, dim: g.headDim, heads: g.heads}), grid(size));
    },
    // The PLE n-gram rows of the tokens in flight, each from the two tokens
    // before it (host lookup of the in-memory store).
    async pleRows(ins) {
        const f = this.frame, o = this.ops, width = this.g.width, previous = f.previous.slice();
        if (f.n === 1) { this.set(ins.y, await o.ple(f.tokens[0], previous)); return; }
        const rows = this.set(ins.y, await o.alloc(f.n * width));
        for (let t = 0; t < f.n; t++) {
            const row = await o.ple(f.tokens[t], previous);
            this.b.copy(row, rows, width, 0, t * width);
            await o.release(row);
            previous.push(f.tokens[t]);
            if (previous.length > 2) previous.shift();
        }
    },
    async pleGate(ins) {
        const g = this.g, lanes = this.frame.n * g.streams, y = this.set(ins.y, await this.ops.alloc(lanes));
        await this.b.run('strata_ple_gate', {Key: this.reg(ins.key), Query: this.reg(ins.query), Gate: y, width: g.width,
            streams: lanes}, [lanes, 1, 1]);
    },
    async pleBroadcast(ins) {
        const g = this.g, size = this.frame.n * g.width * g.streams, y = this.set(ins.y, await this.ops.alloc(size));
        await this.b.run(this.kernel('pleBroadcast'), this.withTokens({Value: this.reg(ins.value), Gate: this.reg(ins.gate),
            Y: y, width: g.width, streams: g.streams}), grid(size));
    },
    async pleAdd(ins) {
        const size = this.frame.n * this.g.width * this.g.streams;
        await this.b.run('strata_ple_add', {Residual: this.frame.residual, Gated: this.reg(ins.gated),
            Conv: this.reg(ins.conv), n: size}, grid(size));
    },
    async moe(ins) {
        const f = this.frame;
        const r = await this.moe.run(ins.layer, this.reg(ins.x), f.n, {batched: f.batched, position: f.position});
        this.set(ins.y, r.y);
    },
    async argmax(ins) {
        const next = this.set(ins.y, await this.ops.alloc(1, 'i32'));
        await this.b.run('strata_argmax', {Logits: this.reg(ins.x), Token: next, count: this.g.vocab}, [1, 1, 1]);
    },
};
