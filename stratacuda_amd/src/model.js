// Model-store pieces of the whole-model decode (the reference's src/model.js):
// geometry validation (src/model.js:11-20), the PLE n-gram rows
// (src/model.js:22-32) and MemoryStore (src/model.js:57-68), the in-memory
// f32 store that createFixture fills. Written for Node 12.
import {requireInteger} from './backend.js';

const product = a => a.reduce((x, y) => x * y, 1);

// The real model's PLE hash constants (src/model.js:7-9); stores of other
// geometries (the fixture) carry their own.
export const PLE_CONSTANTS = {
    multipliers: ['23703573157769', '20109073645365', '8052911324071'],
    vocab: [20000003, 20000023, 20000033, 20000047, 20000059, 20000063, 20000069, 20000077, 20000081, 20000093,
        20000107, 20000147, 20000153, 20000159, 20000161, 20000171],
    offsets: [0, 20000003, 40000026, 60000059, 80000106, 100000165, 120000228, 140000297, 160000374, 180000455,
        200000548, 220000655, 240000802, 260000955, 280001114, 300001275],
};

const GEOMETRY_KEYS = ['width', 'streams', 'rank', 'layers', 'qsaInterval', 'ssmDim', 'keyHeads', 'valueHeads', 'heads',
    'kvHeads', 'headDim', 'rotary', 'experts', 'topK', 'ff', 'vocab', 'context', 'pleHeads', 'pleHeadDim', 'pleTaps',
    'pleDilation'];

// src/model.js:11-20: the same checks and messages.
export function validateGeometry(g) {
    for (const key of GEOMETRY_KEYS) requireInteger(g[key], key);
    if (g.context > 2048)
        throw Error('Portable decode currently supports at most 2048 context cells; sparse QSA selection is not enabled');
    if (g.experts > 512 || g.topK > Math.min(32, g.experts) || g.heads % g.kvHeads || g.valueHeads % g.keyHeads)
        throw Error('Invalid attention or expert geometry');
    if (g.rotary % 2 || g.rotary > g.headDim || g.pleHeads % 2 || g.pleHeads * g.pleHeadDim !== g.width)
        throw Error('Invalid rotary or PLE geometry');
    if (!Number.isFinite(g.ropeBase) || g.ropeBase <= 1) throw Error('Invalid RoPE base');
    if (!Number.isInteger(g.pleLayer) || g.pleLayer < 0 || g.pleLayer >= g.layers) throw Error('PLE layer is outside model');
    requireInteger(g.eos, 'PLE EOS token', 0);
    return g;
}

// src/model.js:22-32: the row of each PLE head from the token and up to two
// previous tokens. Once a previous token is missing or EOS, it and every
// older one count as EOS. Products wrap modulo 2^64; the first half of the
// heads hashes two tokens, the second half three.
export function ngramRows(token, previous, constants, eos) {
    constants = constants || PLE_CONSTANTS;
    eos = eos === undefined ? 248044 : eos;
    requireInteger(token, 'token', 0);
    const ctx = [BigInt(token)];
    let cut = false;
    for (let back = 1; back < 3; back++) {
        const t = previous.length >= back ? previous[previous.length - back] : -1;
        cut = cut || t < 0 || t === eos;
        ctx.push(BigInt(cut ? eos : t));
    }
    const n = constants.vocab.length;
    if (n % 2 || constants.offsets.length !== n) throw Error('Invalid n-gram constants');
    const terms = ctx.map((t, i) => BigInt.asUintN(64, t * BigInt(constants.multipliers[i])));
    return Uint32Array.from(constants.vocab, (v, i) => {
        const mixed = i < n / 2 ? terms[0] ^ terms[1] : terms[0] ^ terms[1] ^ terms[2];
        return Number(mixed % BigInt(v) + BigInt(constants.offsets[i]));
    });
}

// src/model.js:57-68: f32 tensors by name, rows of shape[0] values.
export class MemoryStore {
    constructor(config, tensors, constants) {
        this.config = validateGeometry(config); this.tensors = tensors; this.constants = constants || PLE_CONSTANTS;
        this.label = 'Untrained deterministic fixture';
    }
    describe(name) {
        const t = this.tensors.get(name);
        if (!t) throw Error('Missing tensor ' + name);
        return t;
    }
    async readRows(name, start, rows) {
        const t = this.describe(name), cols = t.shape[0], total = product(t.shape) / cols;
        if (!Number.isInteger(start) || start < 0 || !Number.isInteger(rows) || rows < 1 || start + rows > total)
            throw Error('Tensor row range invalid: ' + name);
        if (t.format !== 'f32') throw Error('Memory fixture expects F32');
        return {format: 'f32', shape: [cols, rows], data: t.data.slice(start * cols, (start + rows) * cols)};
    }
    async readValues(name, start, count) {
        const t = this.describe(name);
        if (!Number.isSafeInteger(start) || !Number.isSafeInteger(count) || start < 0 || count < 1 ||
            start + count > t.data.length)
            throw Error('Tensor value range invalid');
        return t.data.slice(start, start + count);
    }
    async pleRows(token, previous) {
        const g = this.config, rows = ngramRows(token, previous, this.constants, g.eos);
        const out = new Float32Array(g.width);
        for (let h = 0; h < rows.length; h++)
            out.set(await this.readValues('per_layer_token_embd.weight', rows[h] * g.pleHeadDim, g.pleHeadDim),
                h * g.pleHeadDim);
        return out;
    }
}
