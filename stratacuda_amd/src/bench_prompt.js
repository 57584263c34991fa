// Prompt throughput of StrataEngine on the fixture model (createFixture(1234)):
// the same prompt through prefill() in layer-major chunks and through step()
// token by token (predict: false), so the two differ only in the prompt
// orchestration. Prints one JSON line. Usage: node bench_prompt.js [tokens] [reps]
import {performance} from 'perf_hooks';
import {HipBackend} from './backend.js';
import {StrataEngine} from './engine.js';
import {createFixture} from './fixture.js';

async function main() {
    const n = Number(process.argv[2] || 24), reps = Number(process.argv[3] || 5);
    const backend = await HipBackend.create({device: 0}), store = createFixture(1234);
    const engine = await StrataEngine.create(store, backend);
    const prompt = Array.from({length: n}, (_, i) => (i * 7 + 3) % store.config.vocab);
    const time = async fn => {
        await engine.reset(); await fn(); // warm
        let best = Infinity;
        for (let r = 0; r < reps; r++) {
            await engine.reset();
            const t0 = performance.now();
            await fn();
            await backend.idle();
            best = Math.min(best, performance.now() - t0);
        }
        return best;
    };
    const out = {tokens: n, reps, model: 'createFixture(1234): 4 layers, width ' + store.config.width};
    out.step_ms = await time(async () => { for (const t of prompt) await engine.step(t, {predict: false}); });
    for (const chunk of [4, 16]) {
        const ms = await time(() => engine.prefill(prompt, {chunkSize: chunk, predict: false}));
        out['prefill_chunk' + chunk + '_ms'] = ms;
    }
    out.step_tokens_per_s = n / (out.step_ms / 1e3);
    out.prefill_chunk16_tokens_per_s = n / (out.prefill_chunk16_ms / 1e3);
    console.log(JSON.stringify(out));
    await engine.dispose(); await backend.dispose();
}
main().catch(error => { console.error(error && error.stack || error); process.exitCode = 1; });
