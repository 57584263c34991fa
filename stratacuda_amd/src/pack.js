// PackStore: the model source for a pack directory on disk in the reference's
// strata-pack layout (src/model.js:82-167; written by vendor/strata/tools/
// strata_pack.py and pack_layer.py): manifest.json, experts.bin (each layer's
// Q2 expert blobs back to back from the layer's manifest offset) and dense
// files of f32 value planes. It is the store WeightResidency.loadLayer fills a
// resident layer from: generate() streams the layer's 512 blobs into the HBM
// arena with one backend.loadExperts call (every fp16 scale checked finite on
// the device, as readExpertBlob does at src/model.js:164-165) and writes the
// router, shared-gate and norm vectors. One extension for workloads whose
// shared expert is a Q2 blob: manifest.experts.shared lists each layer's
// shared blob in experts.bin. Node 12: synchronous fs reads, no `?.`.
import fs from 'fs';
import path from 'path';
import {requireInteger} from './backend.js';
import {blobLayout} from './store.js';

const product = a => a.reduce((x, y) => x * y, 1);

export class PackStore {
    // open(dir): reads and validates manifest.json with PackStore's checks
    // (src/model.js:82-103) for what the MoE path reads.
    static open(dir) {
        const manifest = JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
        return new PackStore(dir, manifest);
    }
    constructor(dir, manifest) {
        this.dir = dir; this.manifest = manifest;
        if (manifest.format !== 'strata-pack') throw Error('Expected a Strata canonical pack or strata-webcuda-v1 manifest');
        const ex = manifest.experts;
        if (!ex || ex.source_type !== 'Q2_0')
            throw Error('Canonical expert import currently requires Q2_0; IQ expert packs are not supported');
        const c = manifest.config || {};
        this.config = {width: requireInteger(c.width, 'width'), ff: requireInteger(c.ff, 'ff'),
            experts: requireInteger(c.experts, 'experts', 1, 512), topK: requireInteger(c.topK, 'topK', 1, 32),
            layers: requireInteger(c.layers, 'layers')};
        if (this.config.width % 64 || this.config.ff % 64) throw Error('Packed expert dimensions must contain complete groups');
        const layout = blobLayout(this.config.width, this.config.ff);
        if (ex.blob_bytes !== layout.blob_bytes || JSON.stringify(ex.offsets) !== JSON.stringify(layout.offsets))
            throw Error('Expert blob layout does not match the geometry');
        for (const name of Object.keys(manifest.files || {}))
            if (fs.statSync(path.join(dir, name)).size !== manifest.files[name]) throw Error(name + ' size differs from manifest');
        for (const name of Object.keys(manifest.tensors)) {
            const t = manifest.tensors[name], p = t.values;
            if (!Array.isArray(t.shape) || !t.shape.length || t.shape.some(x => !Number.isSafeInteger(x) || x < 1))
                throw Error('Invalid tensor shape: ' + name);
            if (['P32', 'f32'].indexOf(t.form || t.format) < 0) throw Error('Unsupported tensor format: ' + name);
            if (!p || !Number.isSafeInteger(p.offset) || p.offset < 0 || p.offset + p.bytes > fs.statSync(path.join(dir, t.file)).size)
                throw Error('Invalid plane ' + name + '.values');
            if (p.bytes !== product(t.shape) * 4) throw Error('Invalid value plane size: ' + name);
        }
        // Blobs sit at stride multiples of 256 B in the resident arena.
        this.stride = Math.ceil(layout.blob_bytes / 256) * 256;
        this.manifest = Object.assign({}, manifest, {experts: Object.assign({}, ex, {stride: this.stride})});
        this.label = manifest.name || 'Local Strata pack';
    }
    describe(name) {
        const direct = this.manifest.tensors[name], g = this.config, m = /^blk\.(\d+)\./.exec(name);
        const layer = m ? Number(m[1]) : -1;
        if (direct) return {shape: direct.shape, format: 'f32', layer};
        const e = /^blk\.(\d+)\.expert\.(\d+)\.(gate|up|down)$/.exec(name);
        if (!e) throw Error('Missing tensor ' + name);
        if (layer >= g.layers || Number(e[2]) >= g.experts) throw Error('Expert out of range');
        return {shape: e[3] === 'down' ? [g.ff, g.width] : [g.width, g.ff], format: 'q2blob', layer,
            expert: {layer, id: Number(e[2]), role: e[3]}};
    }
    // The f32 values of a dense tensor, rejected when any is non-finite
    // (src/model.js:44, floats()).
    values(name) {
        const t = this.manifest.tensors[name];
        if (!t) throw Error('Missing tensor ' + name);
        const fd = fs.openSync(path.join(this.dir, t.file), 'r'), buf = Buffer.alloc(t.values.bytes);
        try { fs.readSync(fd, buf, 0, buf.length, t.values.offset); } finally { fs.closeSync(fd); }
        const data = new Float32Array(buf.buffer, buf.byteOffset, buf.length / 4).slice();
        if (data.some(v => !Number.isFinite(v))) throw Error('Non-finite model weights');
        return data;
    }
    // WeightResidency.loadLayer's fill: the layer's routed blobs and its
    // shared blob streamed from experts.bin, the dense vectors written.
    generate(backend, layer, {arena, shared, Wr, Wsg, gamma}) {
        const ex = this.manifest.experts, g = this.config, file = path.join(this.dir, 'experts.bin');
        const info = ex.layers.filter(l => l.layer === layer)[0], sh = (ex.shared || []).filter(l => l.layer === layer)[0];
        if (!info || !sh) throw Error('Expert out of range');
        backend.loadExperts(file, info.offset, ex.blob_bytes, g.experts, arena, this.stride, ex.offsets.gate_up_scales);
        backend.loadExperts(file, sh.offset, ex.blob_bytes, 1, shared, this.stride, ex.offsets.gate_up_scales);
        const p = 'blk.' + layer + '.';
        backend.write(Wr, this.values(p + 'ffn_gate_inp.weight'));
        backend.write(Wsg, this.values(p + 'ffn_gate_inp_shexp.weight'));
        backend.write(gamma, this.values(p + 'ffn_norm.weight'));
    }
}
