// The JavaScript host on the GPU, through the real Node-API addon: the MoE
// stage of one layer run fused (kind 'hip', one device call) and host-driven
// (the reference's kernel sequence, src/engine.js:133-156 and
// src/prefill.js:52-78), both against the CPU oracle's results, which
// tests/test_js_host.py computes for the same seeded layers and inputs and
// passes in the directory named by argv[2] (manifest.json + raw arrays).
// Routed IDs must match bit for bit, routing weights to the bit (within
// 1e-6 relative for a fused prompt of 512 tokens or more, whose certified
// router forms the sum of exponentials from approximate logits away from the
// top-k boundary), layer outputs within |a - e| <= 1e-4 + 1e-3 |e|.
import assert from 'assert';
import fs from 'fs';
import path from 'path';
import {test, run} from './harness.js';
import {HipBackend} from '../../stratacuda_amd/src/backend.js';
import {Ops} from '../../stratacuda_amd/src/ops.js';
import {WeightResidency} from '../../stratacuda_amd/src/residency.js';
import {SyntheticStore, STREAM_INPUT} from '../../stratacuda_amd/src/store.js';
import {MoeStage} from '../../stratacuda_amd/src/moe.js';

const dir = process.argv[2];
const manifest = JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
const load = (name, T) => { const b = fs.readFileSync(path.join(dir, name)); return new T(b.buffer, b.byteOffset, b.byteLength / 4); };

function close(actual, expected, label) {
    let worst = 0;
    for (let i = 0; i < expected.length; i++) {
        const a = actual[i], e = expected[i], err = Math.abs(a - e);
        if (!Number.isFinite(a) || err > 1e-4 + 1e-3 * Math.abs(e))
            throw Error(label + ': element ' + i + ' is ' + a + ', expected ' + e);
        worst = Math.max(worst, err);
    }
    return worst;
}
const bits = a => Array.from(new Uint32Array(a.buffer, a.byteOffset, a.length));

let backend = null;
async function session(c) {
    if (!backend) backend = await HipBackend.create({device: 0});
    const store = new SyntheticStore({width: c.width, ff: c.ff, experts: c.experts, topK: c.topK, baseSeed: c.baseSeed});
    const ops = new Ops(backend, store), res = new WeightResidency(ops, [], 64 * 1024 ** 3);
    await res.loadLayer(0);
    const x = backend.alloc(c.tokens * c.width, 'f32', {zero: false});
    backend.synthNormal(x, c.tokens * c.width, c.inputSeed, STREAM_INPUT, 1.0);
    return {ops, x};
}

for (const c of manifest.cases) {
    for (const fused of [true, false]) {
        if (!fused && !c.hostDriven) continue;
        test(c.name + (fused ? ' fused' : ' host-driven') + ' vs the oracle', async () => {
            const {ops, x} = await session(c), stage = new MoeStage(ops, {fused});
            assert.strictEqual(stage.fused, fused);
            const r = c.tokens === 1 ? await stage.decode(0, x) : await stage.prompt(0, x, c.tokens);
            await backend.idle();
            const ids = await backend.read(r.ids), w = await backend.read(r.weights), y = await backend.read(r.y);
            assert.deepStrictEqual(Array.from(ids), Array.from(load(c.name + '_ids.bin', Int32Array)));
            const ew = load(c.name + '_w.bin', Float32Array);
            if (fused && c.tokens >= 512) {
                for (let i = 0; i < ew.length; i++)
                    if (!(Math.abs(w[i] - ew[i]) <= 1e-6 * Math.abs(ew[i])))
                        throw Error(c.name + ': weight ' + i + ' is ' + w[i] + ', expected ' + ew[i]);
            } else assert.deepStrictEqual(bits(w), bits(ew));
            const ey = load(c.name + '_y.bin', Float32Array), rows = c.checkRows || [];
            let worst;
            if (rows.length) {
                // outputs of the tokens the oracle computed (the layer is per-token independent)
                const picked = new Float32Array(rows.length * c.width);
                rows.forEach((t, i) => picked.set(y.subarray(t * c.width, (t + 1) * c.width), i * c.width));
                worst = close(picked, ey, c.name);
            } else worst = close(y, ey, c.name);
            console.log('     max |err| ' + worst.toExponential(2));
            await ops.dispose();
        });
    }
}

// The block entry (one device call per stacked-decoder layer) against the
// three host steps it replaces: strata_norm mode 0, the fused stage and
// strata_elementwise mode 5, bit for bit.
const full = manifest.cases.find(c => c.name === 'full_decode');
for (const T of [1, 20]) {
    test('moeBlock equals norm, moe and residual, ' + T + ' token(s)', async () => {
        const c = Object.assign({}, full, {tokens: T, inputSeed: 300 + T});
        const {ops, x} = await session(c);
        const gamma = ops.residency.layer(0).gamma;
        const xn = await ops.norm(x, gamma, c.width, T);
        const r = await ops.moe(0, xn, T);
        const ref = await ops.elem(x, r.y, 5);
        const b = await ops.moeBlock(0, x, T);
        await backend.idle();
        assert.deepStrictEqual(bits(await backend.read(b.h)), bits(await backend.read(ref)));
        assert.deepStrictEqual(Array.from(await backend.read(b.ids)), Array.from(await backend.read(r.ids)));
        assert.deepStrictEqual(bits(await backend.read(b.weights)), bits(await backend.read(r.weights)));
        await ops.dispose();
    });
}

test('errors surface as exceptions, not faults', async () => {
    if (!backend) backend = await HipBackend.create({device: 0});
    const L = backend.alloc(513), ids = backend.alloc(10, 'i32'), w = backend.alloc(10);
    assert.throws(() => backend.run('strata_router', {Logits: L, Ids: ids, Weights: w, experts: 513, topK: 10}, [1, 1, 1]),
        RangeError);
    const small = backend.alloc(4);
    assert.throws(() => backend.run('strata_elementwise', {A: small, B: small, Y: small, n: 1000, mode: 0, scale: 1},
        [16, 1, 1]), err => err.code === 'SM_E_BOUNDS');
    await backend.idle();
});

test('dispose releases every buffer', async () => {
    if (!backend) backend = await HipBackend.create({device: 0});
    await backend.dispose();
    assert.strictEqual(backend.buffers.size, 0);
});

run();
