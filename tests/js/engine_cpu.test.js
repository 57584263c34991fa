// StrataEngine on the CPU over the stand-in addon (fake_addon.js, with the
// router and argmax emulated): the program's shape gate, the launch
// structure of a decode step and of prompt chunks (one-token kernels vs
// *_batch kernels, state carried in order), route bookkeeping, and the
// session rules (busy, failed, healed, disposed, checkpoint matching). The
// numerics of the same launches are checked on the GPU against the oracle
// (fixture_gpu.test.js).
import assert from 'assert';
import {test, run} from './harness.js';
import {HipBackend, loadAddon} from '../../stratacuda_amd/src/backend.js';
import {StrataEngine} from '../../stratacuda_amd/src/engine.js';
import {createFixture} from '../../stratacuda_amd/src/fixture.js';
import {buildProgram, weightShapes, KERNELS} from '../../stratacuda_amd/src/plan.js';
import {fakeAddon} from './fake_addon.js';

const real = loadAddon();

async function session(options) {
    const addon = fakeAddon(real, Object.assign({emulate: true}, options)), b = await HipBackend.create({addon});
    const store = createFixture(1234), e = await StrataEngine.create(store, b);
    addon.calls.length = 0;
    return {addon, b, e, g: store.config};
}
const launches = addon => addon.calls.filter(c => c.slots && c.name.startsWith('strata_')).map(c => c.name);
const count = (names, name) => names.filter(n => n === name).length;

test('the shape gate is the set of tensors the program reads', async () => {
    const store = createFixture(1234), reads = weightShapes(buildProgram(store.config));
    const names = new Set(reads.map(r => r[0]));
    // everything but the unused head inject and the host-side PLE table
    assert.deepStrictEqual(Array.from(store.tensors.keys()).filter(n => !names.has(n)),
        ['output_hc_inject.weight', 'per_layer_token_embd.weight']);
    assert.strictEqual(reads.length, 168);
    for (const [name, shape] of reads) assert.strictEqual(String(store.describe(name).shape).replace(/,1$/, ''),
        String(shape).replace(/,1$/, ''), name);
    const addon = fakeAddon(real), b = await HipBackend.create({addon});
    const bad = createFixture(1234), t = bad.tensors.get('blk.3.attn_k.weight');
    t.shape = [t.shape[0] / 2, t.shape[1] * 2];
    await assert.rejects(StrataEngine.create(bad, b), /^Error: blk\.3\.attn_k\.weight: expected \[32,16\], found \[16,32\]/);
    assert.strictEqual(addon.mem.size, 0);
});

test('a decode step: one-token kernels, layer state of each mixer, routes per layer', async () => {
    const {addon, e, g} = await session();
    const r = await e.step(2);
    const names = launches(addon);
    for (const pair of Object.values(KERNELS)) assert.strictEqual(count(names, pair[1]), 0, pair[1]);
    assert.strictEqual(count(names, 'strata_router'), g.layers);
    assert.strictEqual(count(names, 'strata_gdn_step'), 3);
    assert.strictEqual(count(names, 'strata_attention'), 1);
    assert.strictEqual(count(names, 'strata_hc_write'), 2 * g.layers);
    assert.strictEqual(count(names, 'strata_argmax'), 1);
    assert.strictEqual(count(names, 'strata_ple_add'), 1);
    assert.deepStrictEqual(r, {position: 0, token: 3});
    assert.deepStrictEqual(e.stats.routes.map(x => [x.layer, x.position, x.ids]),
        [[0, 0, [1, 3]], [1, 0, [1, 3]], [2, 0, [1, 3]], [3, 0, [1, 3]]]);
    assert.strictEqual(e.stats.gpuExperts, g.layers * g.topK);
    // attention reads positions 0..position through its cell list
    addon.calls.length = 0;
    await e.step(7, {predict: false});
    const att = addon.calls.find(c => c.name === 'strata_attention');
    assert.strictEqual(att.slots[8], 2);  // count = position + 1
    assert.strictEqual(count(launches(addon), 'strata_argmax'), 0);
    assert.strictEqual(e.position, 2);
    assert.deepStrictEqual(e.previous, [2, 7]);
});

test('prompt chunks: batch kernels, ragged last chunk, absolute route positions, last row kept', async () => {
    const {addon, b, e, g} = await session();
    await e.step(2, {predict: false});
    addon.calls.length = 0;
    const progress = [];
    const r = await e.prefill([7, 4, 8, 7, 4], {chunkSize: 2, logits: true,
        onProgress: (l, n, offset, size) => progress.push([l, offset, size])});
    const names = launches(addon);
    assert.strictEqual(count(names, 'strata_router_batch'), 3 * g.layers);
    assert.strictEqual(count(names, 'strata_router'), 0);
    assert.strictEqual(count(names, 'strata_attention_batch'), 3);
    assert.strictEqual(count(names, 'strata_argmax'), 1);
    const att = addon.calls.filter(c => c.name === 'strata_attention_batch');
    assert.deepStrictEqual(att.map(c => c.groups[2]), [2, 2, 1]);
    assert.deepStrictEqual(progress.filter(p => p[0] === g.layers), [[4, 0, 2], [4, 2, 2], [4, 4, 1]]);
    assert.strictEqual(r.position, 5); assert.strictEqual(r.token, 3); assert.strictEqual(r.logits.length, g.vocab);
    assert.strictEqual(e.position, 6); assert.deepStrictEqual(e.previous, [7, 4]);
    const positions = Array.from(new Set(e.stats.routes.map(x => x.position)));
    assert.deepStrictEqual(positions, [1, 2, 3, 4, 5]);
    assert.strictEqual(e.stats.routes.length, 5 * g.layers);
    // the last prompt row of each chunk's residual becomes the session residual
    const hc = g.width * g.streams, copies = addon.calls.filter(c => c.name === 'copy' && c.slots[2] === e.state.residual.id);
    assert.deepStrictEqual(copies.map(c => c.slots[1] / 4 / hc), [1, 1, 0]);
    // no chunk residual or temporary outlives the call: state, weights, the
    // one-word dummy operand and the two RoPE tables
    assert.strictEqual(b.info().liveBuffers, e.state.buffers.length + e.ops.residency.tensors.size + 3);
});

test('argument checks run before the session is taken, with the reference messages', async () => {
    const {e, g} = await session();
    await assert.rejects(e.step(g.vocab), RangeError);
    await assert.rejects(e.step(1.5), RangeError);
    await assert.rejects(e.step(1, {logits: true, predict: false}), /Logits require prediction/);
    await assert.rejects(e.prefill([]), /Prompt is empty/);
    await assert.rejects(e.prefill([1, 2], {chunkSize: 0}), RangeError);
    await assert.rejects(e.prefill([1, 2], {chunkSize: 65}), RangeError);
    await assert.rejects(e.prefill([1, g.vocab]), RangeError);
    await assert.rejects(e.prefill([1], {logits: true, predict: false}), /Logits require prediction/);
    await assert.rejects(e.prefill(new Array(g.context + 1).fill(1)), /Context capacity reached/);
    assert.strictEqual(e.failed, false);
    for (let i = 0; i < g.context; i++) await e.step(i % g.vocab, {predict: false});
    await assert.rejects(e.step(1), /Context capacity reached; reset or create a larger session/);
    await assert.rejects(e.prefill([1]), /Context capacity reached/);
    assert.strictEqual(e.failed, false);
});

test('busy, failed, healed and disposed sessions', async () => {
    let bad = false;
    const {e, addon} = await session({routes: (t, k, experts) => bad ? 0 : (k * 2 + 1) % experts});
    const first = e.step(2), second = e.step(3);
    await assert.rejects(second, /A session operation is already running/);
    await assert.rejects(e.reset(), /Cannot reset during a decode step or state operation/);
    await assert.rejects(e.checkpoint(), /Checkpoint requires an idle session/);
    await assert.rejects(e.dispose(), /Cannot dispose during a decode step or state operation/);
    await first;
    bad = true;  // every token routed to expert 0 twice
    await assert.rejects(e.step(4), /Invalid expert routing result/);
    assert.strictEqual(e.failed, true);
    await assert.rejects(e.step(4), /Session failed; reset it before continuing/);
    await assert.rejects(e.prefill([4]), /Session failed; reset it before continuing/);
    await assert.rejects(e.checkpoint(), /Checkpoint requires a healthy session/);
    bad = false;
    await e.reset();
    assert.strictEqual(e.failed, false); assert.strictEqual(e.position, 0); assert.deepStrictEqual(e.previous, []);
    bad = true;
    await assert.rejects(e.prefill([4, 5], {chunkSize: 2}), /Invalid prompt expert routing/);
    assert.strictEqual(e.failed, true);
    bad = false;
    await e.reset();
    await e.step(4);
    await e.dispose();
    await e.dispose();
    await assert.rejects(e.step(1), /Session is disposed/);
    await assert.rejects(e.reset(), /Session is disposed/);
    assert.strictEqual(addon.mem.size, 0);
});

test('checkpoint and restore: state contents, owner and form checks', async () => {
    const {e, b, g} = await session();
    for (const t of [2, 7, 4]) await e.step(t, {predict: false});
    // mark the state so a restore is visible
    const marks = e.state.buffers.map((buf, i) => Float32Array.from({length: buf.length}, (_, j) => i + j / 1024));
    e.state.load(marks);
    const cp = await e.checkpoint();
    assert.strictEqual(cp.position, 3); assert.deepStrictEqual(cp.previous, [7, 4]);
    assert.strictEqual(cp.buffers.length, 2 + g.layers * 2);
    await e.step(8, {predict: false});
    const mutate = fn => { const c = Object.assign({}, cp, {buffers: cp.buffers.slice(), previous: cp.previous.slice()}); fn(c); return c; };
    for (const broken of [
        mutate(c => { c.owner = 'other'; }),
        mutate(c => { c.geometry = '{}'; }),
        mutate(c => { c.buffers.pop(); }),
        mutate(c => { c.buffers[1] = new Float32Array(3); }),
        mutate(c => { c.buffers[0] = cp.buffers[0].slice(); c.buffers[0][5] = NaN; }),
        mutate(c => { c.buffers[2] = Array.from(cp.buffers[2]); }),
        mutate(c => { c.position = g.context + 1; }),
        mutate(c => { c.previous = [7]; }),
        mutate(c => { c.previous = [7, g.vocab]; }),
    ]) await assert.rejects(e.restore(broken), /Checkpoint does not match this model\/session geometry/);
    assert.strictEqual(e.failed, false);
    await e.restore(cp);
    assert.strictEqual(e.position, 3); assert.deepStrictEqual(e.previous, [7, 4]);
    for (let i = 0; i < marks.length; i++) assert.deepStrictEqual(await b.read(e.state.buffers[i]), marks[i]);
    await e.reset();
    for (const buf of e.state.buffers) assert.ok((await b.read(buf)).every(v => v === 0));
    await e.dispose();
});

run();
