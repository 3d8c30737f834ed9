'use strict';
// node/loader.js over a checkpoint written in the reference's layout (the
// directory in argv[2], made by tests/ckpt_writer.py): prints, per tensor,
// its kind, length, group and exact sums, for the Python side to compare
// with what was written; and checks the loader's refusals.
const assert = require('assert');
const loader = require('../../chattorrent_amd/node/loader');

const dir = process.argv[2];
const m = loader.loadManifest(dir);
const d = loader.dimsFromManifest(m);
assert.deepStrictEqual(loader.checkManifest(m, d), []);
const bad = Object.assign({}, m, { weight_layout: 'in_out', dtype: 'f16' });
const probs = loader.checkManifest(bad);
assert(probs.some((p) => p.startsWith('weight_layout in_out')));
assert(probs.some((p) => p.startsWith('dtype f16')));
assert.throws(() => loader.dimsFromManifest(Object.assign({}, m, { vocab: undefined })), /manifest is missing vocab/);

const sumI8 = (a) => { let s = 0; for (let i = 0; i < a.length; i++) s += a[i]; return s; };
const sumF = (a) => { let s = 0; for (let i = 0; i < a.length; i++) s += a[i]; return s; };
const summary = (t) => (t.codes
    ? { kind: 'q8', n: t.codes.length, ns: t.scales.length, group: t.group, codes: sumI8(t.codes), scales: sumF(t.scales) }
    : { kind: 'f32', n: t.length, sum: sumF(t) });

const out = { dims: d, files: {} };
for (let i = 0; i < d.n_layer; i++) {
    const b = loader.loadBlock(dir, m, d, i);
    const f = {};
    for (const k of Object.keys(b)) f[k] = summary(b[k]);
    out.files[loader.blockFile(i)] = f;
}
const c = loader.loadClient(dir, m, d);
out.files.client = {};
for (const k of Object.keys(c)) out.files.client[k] = summary(c[k]);

// uploadTensors' refusals, with its messages
const fn = loader.blockFile(0);
const fs = require('fs'), path = require('path');
const buf = fs.readFileSync(path.join(dir, fn));
const shapes = loader.blockShapes(d);
assert.throws(() => loader.readTensors(buf, m.files[fn].filter((e) => e.name !== 'q_proj'), fn, shapes),
    /block_00.bin: no tensor named q_proj/);
assert.throws(() => loader.readTensors(buf, m.files[fn], fn, Object.assign({}, shapes, { q_proj: [1, 2] })),
    /q_proj shape \[.*\], expected \[1,2\]/);
assert.throws(() => loader.readTensors(buf, m.files[fn].concat([Object.assign({}, m.files[fn][0], { name: 'x' })]),
    fn, shapes), /unexpected tensor x/);
console.log(JSON.stringify(out));
