// PackStore (stratacuda_amd/src/pack.js) over a pack directory written by
// tests/test_js_host.py. argv: dir, mode ('cpu' | 'gpu'). CPU: manifest
// checks with the reference's messages (src/model.js:82-103). GPU: a layer
// made resident from the pack through WeightResidency.loadLayer and run by
// the fused MoE stage and the host-driven one; routed IDs must equal the
// oracle's (ids.bin), outputs within |a - e| <= 1e-4 + 1e-3 |e| (y.bin).
import assert from 'assert';
import fs from 'fs';
import os from 'os';
import path from 'path';
import {test, run} from './harness.js';
import {PackStore} from '../../stratacuda_amd/src/pack.js';

const dir = process.argv[2], mode = process.argv[3] || 'cpu';
const manifest = () => JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
function edited(fn) {
    const copy = fs.mkdtempSync(path.join(os.tmpdir(), 'pack-'));
    for (const f of fs.readdirSync(dir)) fs.copyFileSync(path.join(dir, f), path.join(copy, f));
    const m = manifest();
    fn(m, copy);
    fs.writeFileSync(path.join(copy, 'manifest.json'), JSON.stringify(m));
    return copy;
}

test('the pack opens with the geometry of its manifest', async () => {
    const s = PackStore.open(dir);
    assert.deepStrictEqual(s.config, {width: 128, ff: 64, experts: 16, topK: 4, layers: 2});
    assert.strictEqual(s.describe('blk.1.expert.3.down').expert.id, 3);
    assert.deepStrictEqual(s.describe('blk.0.ffn_gate_inp.weight').shape, [128, 16]);
    assert.strictEqual(s.values('blk.1.ffn_norm.weight').length, 128);
});

test('manifest checks reject what PackStore rejects', async () => {
    const cases = [
        [m => { m.format = 'other'; }, /Expected a Strata canonical pack/],
        [m => { m.experts.source_type = 'IQ4_NL'; }, /requires Q2_0/],
        [m => { m.experts.blob_bytes += 16; }, /layout does not match/],
        [m => { m.files['experts.bin'] += 1; }, /experts.bin size differs from manifest/],
        [m => { m.tensors['blk.0.ffn_norm.weight'].values.offset = 1e9; }, /Invalid plane/],
        [m => { m.tensors['blk.0.ffn_norm.weight'].form = 'S4'; }, /Unsupported tensor format/],
    ];
    for (const [fn, re] of cases) assert.throws(() => PackStore.open(edited(fn)), re);
    const bad = edited((m, copy) => {
        const t = m.tensors['blk.0.ffn_norm.weight'], fd = fs.openSync(path.join(copy, t.file), 'r+');
        fs.writeSync(fd, Buffer.from(new Float32Array([NaN]).buffer), 0, 4, t.values.offset + 4);
        fs.closeSync(fd);
    });
    assert.throws(() => PackStore.open(bad).values('blk.0.ffn_norm.weight'), /Non-finite model weights/);
});

if (mode === 'gpu') {
    test('a resident layer loaded from the pack matches the oracle', async () => {
        const {HipBackend} = await import('../../stratacuda_amd/src/backend.js');
        const {Ops} = await import('../../stratacuda_amd/src/ops.js');
        const {WeightResidency} = await import('../../stratacuda_amd/src/residency.js');
        const {MoeStage} = await import('../../stratacuda_amd/src/moe.js');
        const b = await HipBackend.create({device: 0}), store = PackStore.open(dir);
        try {
            const ops = new Ops(b, store), res = new WeightResidency(ops, [], 1024 ** 3);
            await res.loadLayer(1);
            const raw = n => { const buf = fs.readFileSync(path.join(dir, n)); return buf.buffer.slice(buf.byteOffset, buf.byteOffset + buf.length); };
            const x = new Float32Array(raw('x.bin')), ids = new Int32Array(raw('ids.bin')), y = new Float32Array(raw('y.bin'));
            const tokens = x.length / 128, xb = b.alloc(x);
            for (const fused of [true, false]) {
                const stage = new MoeStage(ops, {fused});
                const r = tokens === 1 ? await stage.decode(1, xb) : await stage.prompt(1, xb, tokens);
                assert.deepStrictEqual(Array.from(await b.read(r.ids, 'i32')), Array.from(ids));
                const got = await b.read(r.y);
                for (let i = 0; i < y.length; i++)
                    if (!(Math.abs(got[i] - y[i]) <= 1e-4 + 1e-3 * Math.abs(y[i]))) throw Error('y[' + i + '] ' + got[i] + ' vs ' + y[i]);
                await ops.clearTemporary();
            }
            await ops.dispose();
        } finally { await b.dispose(); }
    });
}

run();
