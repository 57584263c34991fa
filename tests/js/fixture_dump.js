// Writes the fixture createFixture(seed) builds (stratacuda_amd/src/fixture.js)
// to argv[2]: index.json (names and shapes in creation order) and values.bin
// (every tensor's f32 values, concatenated in the same order), so the Python
// test can compare it with the oracle's restatement bit for bit.
import fs from 'fs';
import path from 'path';
import {createFixture} from '../../stratacuda_amd/src/fixture.js';
import {ngramRows} from '../../stratacuda_amd/src/model.js';

const dir = process.argv[2], seed = Number(process.argv[3] || 1234);
const store = createFixture(seed), index = [], chunks = [];
for (const [name, t] of store.tensors) {
    index.push({name, shape: t.shape});
    chunks.push(Buffer.from(t.data.buffer, t.data.byteOffset, t.data.byteLength));
}
const rows = [];
for (const prev of [[], [3], [5, 9], [39, 9], [9, 39]])
    for (let token = 0; token < store.config.vocab; token++)
        rows.push(Array.from(ngramRows(token, prev, store.constants, store.config.eos)));
fs.writeFileSync(path.join(dir, 'index.json'), JSON.stringify({config: store.config, tensors: index, ngram: rows}));
fs.writeFileSync(path.join(dir, 'values.bin'), Buffer.concat(chunks));
console.log('ok   fixture dump ' + index.length + ' tensors');
