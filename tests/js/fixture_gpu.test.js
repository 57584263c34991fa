// The whole fixture decode on the GPU through the JavaScript host
// (StrataEngine over HipBackend and the Node-API addon): the reference's own
// known answers, the session API, and a trace of a seeded token sequence
// (tokens, logits bits, routes per step) written to argv[2]/trace.json for
// tests/test_js_fixture.py to compare with the CPU oracle.
import assert from 'assert';
import fs from 'fs';
import path from 'path';
import {test, run} from './harness.js';
import {HipBackend} from '../../stratacuda_amd/src/backend.js';
import {StrataEngine} from '../../stratacuda_amd/src/engine.js';
import {createFixture} from '../../stratacuda_amd/src/fixture.js';

const dir = process.argv[2];
const request = JSON.parse(fs.readFileSync(path.join(dir, 'request.json'), 'utf8'));
let backend = null, store = null;
async function engine() {
    if (!backend) { backend = await HipBackend.create({device: 0}); store = createFixture(1234); }
    return StrataEngine.create(store, backend);
}
const bits = a => Array.from(new Uint32Array(a.buffer, a.byteOffset, a.length));

test('decode 2,7,4,7,4 gives the reference tokens 29,2,15,9,15', async () => {
    const e = await engine();
    try {
        const tokens = [];
        for (const t of [2, 7, 4, 7, 4]) tokens.push((await e.step(t)).token);
        assert.deepStrictEqual(tokens, [29, 2, 15, 9, 15]);
    } finally { await e.dispose(); }
});

test('the step of 8 after 2,7,4,8,7,4 routes like the reference', async () => {
    const e = await engine();
    try {
        for (const t of [2, 7, 4, 8, 7, 4]) await e.step(t, {predict: false});
        await e.step(8);
        assert.deepStrictEqual(e.stats.routes.map(r => r.ids), [[0, 5], [5, 3], [4, 1], [4, 5]]);
    } finally { await e.dispose(); }
});

test('prompt 2,7,4 then greedy generation gives 15,18,3,15', async () => {
    const e = await engine();
    try {
        let next;
        for (const t of [2, 7, 4]) next = (await e.step(t)).token;
        const out = [];
        for (let i = 0; i < 4; i++) { out.push(next); next = (await e.step(next)).token; }
        assert.deepStrictEqual(out, [15, 18, 3, 15]);
    } finally { await e.dispose(); }
});

test('checkpoint / restore replays logits exactly; reset equals a fresh session', async () => {
    const e = await engine();
    try {
        for (const t of [2, 7, 4]) await e.step(t);
        const snap = await e.checkpoint(), first = await e.step(8, {logits: true});
        await e.restore(snap);
        const replay = await e.step(8, {logits: true});
        assert.deepStrictEqual(bits(replay.logits), bits(first.logits));
        await e.reset();
        const again = await e.step(2, {logits: true});
        const fresh = await engine();
        try { assert.deepStrictEqual(bits(again.logits), bits((await fresh.step(2, {logits: true})).logits)); }
        finally { await fresh.dispose(); }
    } finally { await e.dispose(); }
});

test('session errors follow the reference', async () => {
    const e = await engine();
    try {
        await assert.rejects(e.step(40), RangeError);
        await assert.rejects(e.step(1, {logits: true, predict: false}), /Logits require prediction/);
        for (let i = 0; i < 32; i++) await e.step(i % 40, {predict: false});
        await assert.rejects(e.step(1), /Context capacity reached/);
        await assert.rejects(e.restore({owner: 'other'}), /Checkpoint does not match/);
    } finally { await e.dispose(); }
});

test('seeded token trace for the oracle comparison', async () => {
    const e = await engine();
    try {
        const steps = [];
        for (const t of request.tokens) {
            const r = await e.step(t, {logits: true});
            steps.push({token: r.token, logits: bits(r.logits), routes: e.stats.routes.map(x => x.ids)});
        }
        fs.writeFileSync(path.join(dir, 'trace.json'), JSON.stringify({steps, residency: e.residencyInfo()}));
    } finally { await e.dispose(); }
});

// tests/conformance.js:84-92: prompt chunks of 1, 2 and 5 at a nonzero start,
// then the next decode step; logits bits go to prompt.json for the oracle.
test('prompt chunks 1, 2, 5 after a decode step, then decode 8', async () => {
    const e = await engine(), out = [];
    try {
        for (const chunkSize of [1, 2, 5]) {
            await e.reset();
            await e.step(2, {predict: false});
            const prompt = await e.prefill([7, 4, 8, 7, 4], {chunkSize, logits: true});
            const routes = e.stats.routes.map(r => [r.position, r.layer, r.ids]);
            assert.strictEqual(prompt.position, 5);
            assert.strictEqual(e.position, 6);
            const next = await e.step(8, {logits: true});
            out.push({chunkSize, token: prompt.token, logits: bits(prompt.logits), routes,
                nextToken: next.token, next: bits(next.logits)});
        }
        await assert.rejects(e.prefill([]), /Prompt is empty/);
        await assert.rejects(e.prefill([1, 2], {chunkSize: 0}), RangeError);
        await assert.rejects(e.prefill([1, 40]), RangeError);
        fs.writeFileSync(path.join(dir, 'prompt.json'), JSON.stringify(out));
    } finally { await e.dispose(); }
});

run().then(async () => { if (backend) await backend.dispose(); });
