// SyntheticStore: the model source the Ops / WeightResidency pair reads from,
// with the names, shapes and expert manifest of the reference's PackStore
// (src/model.js) for the tensors on the MoE path, filled from the seeded
// counter-based generator instead of a pack file. The same (seed, stream)
// definitions feed the CPU oracle (stratacuda_amd/workload.py), so a layer
// made here is bit-identical to the oracle's copy:
//   blk.L.ffn_gate_inp.weight       [width, experts] f32  stream 1, sigma 0.02
//   blk.L.ffn_gate_inp_shexp.weight [width]          f32  stream 2, sigma 0.02
//   blk.L.ffn_norm.weight           [width]          f32  stream 3, 1 + 0.05 U(-1,1)
//   blk.L.expert.E.{gate,up,down}   Q2 blob of expert E  stream 16 + E
//   shared expert                   Q2 blob               stream 16 + experts
// Layer L's seed is baseSeed + 7919 L.

export const STREAM_ROUTER = 1, STREAM_SHARED_GATE = 2, STREAM_GAMMA = 3, STREAM_INPUT = 4, STREAM_BLOB0 = 16;
export const BASE_SEED = 20260101;

// Blob layout of one expert (vendor/strata/tools/pack_layer.py:54-65): byte
// offsets of the four planes and the blob size.
export function blobLayout(width, ff) {
    const gateUpCodes = 0, downCodes = 2 * ff * width / 4, gateUpScales = downCodes + width * ff / 4;
    const downScales = gateUpScales + 2 * ff * (width / 64) * 2, bytes = downScales + width * (ff / 64) * 2;
    return {blob_bytes: bytes, offsets: {gate_up_codes: gateUpCodes, down_codes: downCodes,
        gate_up_scales: gateUpScales, down_scales: downScales}};
}

export function layerSeed(layer, base) { return (base === undefined ? BASE_SEED : base) + 7919 * layer; }

export class SyntheticStore {
    constructor({width = 2048, ff = 512, experts = 512, topK = 10, layers = 1, baseSeed = BASE_SEED} = {}) {
        if (width % 64 || ff % 64) throw new RangeError('width and ff must be multiples of 64');
        this.config = {width, ff, experts, topK, layers};
        this.baseSeed = baseSeed;
        const layout = blobLayout(width, ff);
        this.stride = Math.ceil(layout.blob_bytes / 256) * 256;
        this.manifest = {experts: Object.assign({source_type: 'Q2_0', stride: this.stride}, layout)};
    }
    seed(layer) { return layerSeed(layer, this.baseSeed); }
    describe(name) {
        const g = this.config, m = /^blk\.(\d+)\.(.+)$/.exec(name);
        if (!m || Number(m[1]) >= g.layers) throw Error('Unknown tensor ' + name);
        const layer = Number(m[1]), rest = m[2];
        if (rest === 'ffn_gate_inp.weight') return {shape: [g.width, g.experts], format: 'f32', layer};
        if (rest === 'ffn_gate_inp_shexp.weight') return {shape: [g.width, 1], format: 'f32', layer};
        if (rest === 'ffn_norm.weight') return {shape: [g.width], format: 'f32', layer};
        const e = /^expert\.(\d+)\.(gate|up|down)$/.exec(rest);
        if (e && Number(e[1]) < g.experts) {
            const role = e[2];
            return {shape: role === 'down' ? [g.ff, g.width] : [g.width, g.ff], format: 'q2blob', layer,
                expert: {layer, id: Number(e[1]), role}};
        }
        throw Error('Unknown tensor ' + name);
    }
    // Fills the device buffers of one layer (see the table above).
    generate(backend, layer, {arena, shared, Wr, Wsg, gamma}) {
        const g = this.config, seed = this.seed(layer);
        backend.synthBlobs(arena, this.stride, g.experts, g.width, g.ff, seed, STREAM_BLOB0, 0.05);
        backend.synthBlobs(shared, this.stride, 1, g.width, g.ff, seed, STREAM_BLOB0 + g.experts, 0.05);
        backend.synthNormal(Wr, g.experts * g.width, seed, STREAM_ROUTER, 0.02);
        backend.synthNormal(Wsg, g.width, seed, STREAM_SHARED_GATE, 0.02);
        backend.synthUniformPm(gamma, g.width, seed, STREAM_GAMMA, 0.05);
    }
}
