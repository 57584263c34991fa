// The JavaScript host on the CPU: HipBackend, Ops, WeightResidency and the
// MoE stage over a stand-in addon that keeps buffers in host memory and
// records launches. The stand-in takes kernel signatures, workspace sizes and
// argument validation from the real addon (pure functions of the C ABI that
// need no GPU), so what is checked here is the host side: the reference's
// validation and error conventions (src/backend.js:6-56), argument packing
// in parameter order, buffer bookkeeping, the resident layer layout and the
// offsets the ops hand to the kernels.
import assert from 'assert';
import {test, run} from './harness.js';
import {HipBackend, validateDispatch, requireInteger, loadAddon} from '../../stratacuda_amd/src/backend.js';
import {Ops} from '../../stratacuda_amd/src/ops.js';
import {WeightResidency, expertKey} from '../../stratacuda_amd/src/residency.js';
import {SyntheticStore, blobLayout} from '../../stratacuda_amd/src/store.js';
import {MoeStage} from '../../stratacuda_amd/src/moe.js';
import {fakeAddon as makeFakeAddon} from './fake_addon.js';

const real = loadAddon();

const fakeAddon = () => makeFakeAddon(real);

test('the addon exports every entry of the C ABI it wraps', () => {
    for (const f of ['init', 'shutdown', 'lastError', 'info', 'alloc', 'free', 'size', 'write', 'read', 'copy', 'zero',
        'sync', 'kernels', 'signature', 'run', 'moeWorkspace', 'moeLayer', 'moeBlockWorkspace', 'moeBlock', 'moeRoute',
        'moeDispatch', 'synthNormal',
        'synthUniformPm', 'synthBlobs', 'eventRecord', 'eventElapsed', 'graphBegin', 'graphEnd', 'graphLaunch',
        'graphFree', 'fusedReset', 'prefetchRouter'])
        assert.strictEqual(typeof real[f], 'function', f);
    assert.ok(real.kernels().indexOf('strata_router') >= 0);
    assert.strictEqual(real.signature('strata_router'), 'Logits:f32*,Ids:i32*,Weights:f32*,experts:i32,topK:i32');
    assert.strictEqual(real.signature('no_such_kernel'), null);
    assert.throws(() => real.moeWorkspace(1, 2048, 512, 513, 10), RangeError);
});

test('requireInteger and validateDispatch follow the reference conventions', () => {
    assert.strictEqual(requireInteger(5, 'n'), 5);
    assert.throws(() => requireInteger(0, 'allocation'), {name: 'RangeError', message: 'allocation must be an integer in [1, 2147483647]'});
    assert.throws(() => requireInteger(1.5, 'n'), RangeError);
    const L = {length: 513}, I = {length: 10};
    assert.throws(() => validateDispatch('strata_router', {Logits: L, Ids: I, Weights: I, experts: 513, topK: 10}),
        {name: 'RangeError', message: 'Router supports 1–512 experts and topK <= min(experts,32)'});
    assert.throws(() => validateDispatch('strata_router', {experts: 6, topK: 7}), RangeError);
    assert.throws(() => validateDispatch('strata_router_batch', {experts: 512, topK: 33}), RangeError);
    validateDispatch('strata_router', {experts: 512, topK: 10});
    assert.throws(() => validateDispatch('strata_norm', {rows: 3, weightRows: 2}),
        {name: 'RangeError', message: 'Normalization weight rows must divide input rows'});
    assert.throws(() => validateDispatch('strata_q2_gate_up', {width: 100, ff: 64, tokens: 1, Hidden: {length: 64}}),
        {message: 'Packed expert dimensions must contain complete groups'});
    assert.throws(() => validateDispatch('strata_q2_down', {width: 128, ff: 64, tokens: 2, Hidden: {length: 64}, mapped: 0}),
        {message: 'Packed expert batch exceeds buffer layout'});
    assert.throws(() => validateDispatch('strata_project', {X: {length: 8}, Y: {length: 4}, tokens: 1, rows: 4, cols: 8,
        outputStride: 4, outputOffset: 1}), {message: 'Projection batch exceeds buffer layout'});
    assert.throws(() => validateDispatch('strata_quant_project', {bits: 3, cols: 64, rows: 1, groupSize: 64}),
        {message: 'Canonical code width must be 2, 4 or 8'});
});

test('buffers: words, types, round trips and bounds', async () => {
    const addon = fakeAddon(), b = await HipBackend.create({addon});
    assert.strictEqual(b.kind, 'hip');
    const a = b.alloc(new Float32Array([1, 2, 3, 4])), c = b.alloc(4), i = b.alloc(3, 'i32');
    assert.strictEqual(a.length, 4); assert.strictEqual(a.type, 'f32'); assert.strictEqual(i.type, 'i32');
    assert.deepStrictEqual(Array.from(await b.read(a)), [1, 2, 3, 4]);
    assert.deepStrictEqual(Array.from(await b.read(c)), [0, 0, 0, 0]);
    b.copy(a, c, 2, 1, 2);
    assert.deepStrictEqual(Array.from(await b.read(c)), [0, 0, 2, 3]);
    b.write(c, new Float32Array([9]), 3);
    assert.deepStrictEqual(Array.from(await b.read(c)), [0, 0, 2, 9]);
    assert.deepStrictEqual(Array.from(await b.read(a, 'u32')).slice(0, 1), [0x3f800000]);
    assert.throws(() => b.copy(a, c, 4, 1, 0), /Invalid HIP copy/);
    assert.throws(() => b.write(c, new Float32Array(5)), /Invalid HIP write/);
    assert.throws(() => b.alloc(4, 'f64'), /Unsupported buffer type/);
    b.zero(a);
    assert.deepStrictEqual(Array.from(await b.read(a)), [0, 0, 0, 0]);
    b.free(a); b.free(a);  // a second free is ignored, as in the reference
    await assert.rejects(b.read(a), /Invalid HIP read/);
    const info = b.info();
    assert.strictEqual(info.backend, 'hip'); assert.strictEqual(info.liveBuffers, 2);
    await b.dispose();
    assert.strictEqual(addon.mem.size, 0);
    assert.throws(() => b.alloc(1), /disposed/);
});

test('run packs named arguments in parameter order (f32 as bit patterns)', async () => {
    const addon = fakeAddon(), b = await HipBackend.create({addon});
    const X = b.alloc(8), W = b.alloc(8), Y = b.alloc(4);
    b.run('strata_norm', {scale: 0.5, Y, epsilon: 1e-6, W, mode: 2, X, weightRows: 1, rows: 1, cols: 8}, [1, 1, 1]);
    const call = addon.calls[addon.calls.length - 1];
    assert.strictEqual(call.name, 'strata_norm');
    const f = new Float32Array([1e-6, 0.5]), u = new Uint32Array(f.buffer);
    assert.deepStrictEqual(call.slots, [X.id, W.id, Y.id, 8, 1, 1, 2, u[0], u[1]]);
    assert.throws(() => b.run('strata_norm', {X, W, Y, cols: 8, rows: 1, weightRows: 1, mode: 0, epsilon: 1e-6}, [1, 1, 1]),
        /Missing strata_norm.scale/);
    assert.throws(() => b.run('strata_norm', {X: 3, W, Y, cols: 8, rows: 1, weightRows: 1, mode: 0, epsilon: 0, scale: 1},
        [1, 1, 1]), /must be a buffer/);
    assert.throws(() => b.run('strata_nothing', {}, [1, 1, 1]), /Unknown kernel strata_nothing/);
    const other = await HipBackend.create({addon: fakeAddon()});
    const foreign = other.alloc(8);
    assert.throws(() => b.run('strata_elementwise', {A: foreign, B: X, Y: X, n: 8, mode: 0, scale: 1}, [1, 1, 1]),
        /Invalid HIP buffer/);
    b.run('strata_elementwise', {A: X, B: X, Y: X, n: 8, mode: 1, scale: -2}, [1, 1, 1]);
    assert.strictEqual(addon.calls.length, 2);
});

test('residency: the resident layer layout, all-resident admission and info fields', async () => {
    const addon = fakeAddon(), b = await HipBackend.create({addon});
    const store = new SyntheticStore({width: 128, ff: 64, experts: 16, topK: 4, layers: 2});
    const layout = blobLayout(128, 64);
    assert.deepStrictEqual(layout.offsets, {gate_up_codes: 0, down_codes: 4096, gate_up_scales: 6144, down_scales: 6656});
    assert.strictEqual(layout.blob_bytes, 6912);
    assert.strictEqual(blobLayout(2048, 512).blob_bytes, 884736);
    assert.strictEqual(store.stride, 6912);
    const ops = new Ops(b, store), res = new WeightResidency(ops, [], 1 << 30);
    assert.strictEqual(ops.residency, res);
    const entry = await res.loadLayer(1);
    assert.strictEqual(entry.arena.byteLength, 16 * 6912);
    assert.strictEqual(entry.Wr.length, 16 * 128);
    const synth = addon.calls.filter(c => c.name.indexOf('synth') === 0);
    assert.deepStrictEqual(synth.map(c => c.name), ['synthBlobs', 'synthBlobs', 'synthNormal', 'synthNormal', 'synthUniformPm']);
    assert.strictEqual(synth[0].args[7], 16);  // first blob stream
    assert.strictEqual(synth[1].args[7], 32);  // shared expert: stream 16 + experts
    assert.strictEqual(synth[0].args[6], store.seed(1));
    assert.strictEqual(await res.admit('1:3'), true);
    assert.strictEqual(res.hasExpert('1:3'), true);
    assert.strictEqual(res.hasExpert('0:3'), false);
    assert.strictEqual(expertKey('blk.1.expert.3.gate'), '1:3');
    assert.deepStrictEqual(Object.keys(res.info()), ['budgetBytes', 'densePlannedBytes', 'denseResidentBytes',
        'expertResidentBytes', 'residentExperts', 'hits', 'misses', 'evictions']);
    assert.strictEqual(res.info().expertResidentBytes, 17 * 6912);
    assert.throws(() => new WeightResidency(ops, [], 0), RangeError);
    const small = new WeightResidency(new Ops(b, store), [], 1000);
    await assert.rejects(small.loadLayer(0), /choose a larger GPU budget/);
});

test('ops: packedExpert hands the kernels the blob offsets of expert id in the arena', async () => {
    const addon = fakeAddon(), b = await HipBackend.create({addon});
    const store = new SyntheticStore({width: 128, ff: 64, experts: 16, topK: 4});
    const ops = new Ops(b, store), res = new WeightResidency(ops, [], 1 << 30);
    const entry = await res.loadLayer(0);
    const x = b.alloc(128);
    addon.calls.length = 0;
    await ops.packedExpert(0, 5, x);
    const [gu, dn] = addon.calls;
    assert.strictEqual(gu.name, 'strata_q2_gate_up'); assert.strictEqual(dn.name, 'strata_q2_down');
    assert.deepStrictEqual(gu.groups, [64, 1, 1]); assert.deepStrictEqual(dn.groups, [128, 1, 1]);
    // X, Blob, Scales, Mapping, Hidden, width, ff, tokens, mapped, expanded, codeOffset, scaleOffset
    assert.strictEqual(gu.slots[1], entry.arena.id);
    assert.deepStrictEqual(gu.slots.slice(5), [128, 64, 1, 0, 0, 5 * 6912 / 4, (5 * 6912 + 6144) / 2]);
    assert.deepStrictEqual(dn.slots.slice(5), [128, 64, 1, 0, 0, 0, (5 * 6912 + 4096) / 4, (5 * 6912 + 6656) / 2]);
    await assert.rejects(ops.packedExpert(0, 16, x), RangeError);
    addon.calls.length = 0;
    await ops.packedExpert(0, 'shared', x, 2, {mapping: new Int32Array([0, 1, 0, 2])});
    assert.strictEqual(addon.calls[0].slots[1], entry.shared.id);
    assert.deepStrictEqual(addon.calls[0].slots.slice(7, 9), [2, 1]);
    assert.strictEqual(addon.calls[0].slots[10], 0);
});

test('MoE stage: kind hip runs the fused layer with the resident buffers', async () => {
    const addon = fakeAddon(), b = await HipBackend.create({addon});
    const store = new SyntheticStore({width: 128, ff: 64, experts: 16, topK: 4});
    const ops = new Ops(b, store), res = new WeightResidency(ops, [], 1 << 30);
    const entry = await res.loadLayer(0);
    const stage = new MoeStage(ops), x = b.alloc(3 * 128);
    addon.calls.length = 0;
    const r = await stage.prompt(0, x, 3);
    const call = addon.calls[0];
    assert.strictEqual(call.name, 'moeLayer');
    // X, tokens, Wr, bias, arena, stride, shared, Wsg, width, ff, experts, topk, Y, ids, weights, ws, wsBytes
    assert.deepStrictEqual(call.args.slice(0, 12), [x.id, 3, entry.Wr.id, 0, entry.arena.id, 6912, entry.shared.id,
        entry.Wsg.id, 128, 64, 16, 4]);
    assert.deepStrictEqual(call.args.slice(12, 15), [r.y.id, r.ids.id, r.weights.id]);
    assert.ok(call.args[16] >= real.moeWorkspace(3, 128, 64, 16, 4));
    await assert.rejects(stage.decode(0, x), /MoE input must hold tokens x width values/);
    assert.strictEqual(new MoeStage(ops, {fused: false}).fused, false);
});

test('moeBlock passes the layer gamma and the resident buffers in the C ABI order', async () => {
    const addon = fakeAddon(), b = await HipBackend.create({addon});
    const store = new SyntheticStore({width: 128, ff: 64, experts: 16, topK: 4});
    const ops = new Ops(b, store), res = new WeightResidency(ops, [], 1 << 30);
    const entry = await res.loadLayer(0), h = b.alloc(2 * 128);
    addon.calls.length = 0;
    const r = await ops.moeBlock(0, h, 2);
    const call = addon.calls[0];
    assert.strictEqual(call.name, 'moeBlock');
    // H, tokens, gamma, eps, Wr, bias, arena, stride, shared, Wsg, width, ff, experts, topk, Hout, ids, weights, ws, wsBytes
    assert.deepStrictEqual(call.args.slice(0, 14), [h.id, 2, entry.gamma.id, 1e-6, entry.Wr.id, 0, entry.arena.id, 6912,
        entry.shared.id, entry.Wsg.id, 128, 64, 16, 4]);
    assert.deepStrictEqual(call.args.slice(14, 17), [r.h.id, r.ids.id, r.weights.id]);
    assert.ok(call.args[18] >= real.moeBlockWorkspace(2, 128, 64, 16, 4));
    await assert.rejects(ops.moeBlock(0, h, 3), /MoE input must hold tokens x width values/);
});

test('a fused decode fault fails read() and idle() until resetFusedDecode()', async () => {
    // SM_E_FAULT from the library (a device-side wait that gave up) rejects
    // read and idle, as the reference rejects them after a failed dispatch
    // (src/backend.js:95,118); the backend then fails every call like a lost
    // device until the fault is cleared.
    const addon = fakeAddon();
    let faulted = true, resets = 0;
    const fault = () => { const e = Error('the single-launch decode layer gave up'); e.code = 'SM_E_FAULT'; return e; };
    const read = addon.read;
    addon.read = (...a) => { if (faulted) throw fault(); return read(...a); };
    addon.sync = () => { if (faulted) throw fault(); };
    addon.fusedReset = () => { resets++; faulted = false; };
    const b = await HipBackend.create({addon});
    const y = b.alloc(new Float32Array([1, 2]));
    await assert.rejects(b.read(y), {code: 'SM_E_FAULT'});
    assert.throws(() => b.alloc(4), {code: 'SM_E_FAULT'});
    b.resetFusedDecode();
    assert.strictEqual(resets, 1);
    assert.deepStrictEqual(Array.from(await b.read(y)), [1, 2]);
    await b.idle();
});

test('prefetchRouter passes an owned buffer, rejects foreign ones and clears with null', async () => {
    const addon = fakeAddon();
    const calls = [];
    addon.prefetchRouter = (...a) => calls.push(a.slice(1));
    const b = await HipBackend.create({addon});
    const wr = b.alloc(512 * 64);
    b.prefetchRouter(wr, 512, 64);
    b.prefetchRouter(null);
    assert.deepStrictEqual(calls, [[wr.id, 512, 64], [0, 0, 0]]);
    assert.throws(() => b.prefetchRouter({id: 1, byteLength: 4}, 1, 64), /Invalid HIP prefetch/);
    await b.idle();
});

run();
