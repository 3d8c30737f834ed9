'use strict';
// The JS Runner's host policy against the reference's expectations
// (tools/stage.test.mjs, web/dev/batch.test.js), on the CPU stub backend.
// Run: node tests/node/runner.test.js (exit status 0 when every case passes).

const assert = require('assert');
const { Runner, MAX_QUEUE, MAX_SESSION_QUEUE } = require('../../chattorrent_amd/node/runner');
const { StubBackend } = require('./stub_backend');
const { toF16, fromF16 } = require('../../chattorrent_amd/node/f16');
const S = require('../../chattorrent_amd/node/sampling');

const D = { hidden: 8, n_layer: 2, n_heads: 2, n_kv_heads: 1, head_dim: 64, ffn: 32, vocab: 101 };
const END = D.n_layer + 2;

function make(o) {
    const opts = Object.assign({ lo: 0, hi: END, nMax: 512, tMax: 16, slots: 2, sessions: 2, idleMs: 50,
                                 waitMs: 200, batchRows: 16 }, o || {});
    const be = new StubBackend(D, { nMax: opts.nMax, slots: opts.slots, frames: opts.sessions + 1, tMax: opts.tMax,
                                    delayMs: opts.delayMs });
    return { r: new Runner(be, D, opts), be };
}
const job = (s, extra) => Object.assign({ k: 'job', s, pos: 0, past: 0, n: 1, ids: [5], opts: { temp: 0 } }, extra);
const sleep = (ms) => new Promise((res) => setTimeout(res, ms));
const rejects = async (p, re) => {
    try { await p; } catch (e) {
        if (re && !re.test(e.message)) throw new Error(`wrong error: ${e.message}`);
        return e;
    }
    throw new Error('expected a rejection');
};

const cases = [];
const test = (name, fn) => cases.push({ name, fn });

test('greedy decode at the head returns the stub model argmax', async () => {
    const { r, be } = make();
    const out = await r.run(job('a', { ids: [3] }));
    assert.strictEqual(out.at, END);
    const want = (0 + END) * 7 + 3;
    assert.strictEqual(out.token, want % D.vocab);
    assert.strictEqual(be.calls.length, 1);
    assert.deepStrictEqual(be.calls[0].jobs[0], { slot: be.calls[0].jobs[0].slot, past: 0, n: 1, sampled: 1 });
});

test('queued jobs with the same cursor share one pass, in order, one per session', async () => {
    const { r, be } = make({ sessions: 4, slots: 4, delayMs: 20 });
    const first = r.run(job('a'));
    await sleep(1);   // a's pass is running: the next jobs queue behind it
    const ps = [r.run(job('b')), r.run(job('c')), r.run(job('b', { past: 1, ids: [6] })), r.run(job('d'))];
    await Promise.all([first].concat(ps));
    assert.strictEqual(be.calls.length, 3);
    assert.strictEqual(be.calls[1].jobs.length, 3);   // b, c, d; b's second job waits
    assert.strictEqual(be.calls[2].jobs.length, 1);
    assert.strictEqual(r.counts.batched, 1);
    assert.strictEqual(r.counts.batchedJobs, 3);
});

test('prefill chunks, replays and other cursors do not join a batch', async () => {
    const { r, be } = make({ sessions: 4, slots: 4, delayMs: 20 });
    const first = r.run(job('a'));
    await sleep(1);
    const ps = [r.run(job('b')), r.run(job('c', { fill: true, n: 2, ids: [1, 2] })),
                r.run(job('d', { pos: 1, ids: undefined }), new Uint16Array(D.hidden))];
    await Promise.all([first].concat(ps));
    assert.deepStrictEqual(be.calls.map((c) => c.jobs.length), [1, 1, 1, 1]);
});

test('batchRows caps the rows of a pass', async () => {
    const { r, be } = make({ sessions: 4, slots: 4, delayMs: 20, batchRows: 3 });
    const first = r.run(job('a'));
    await sleep(1);
    const ps = [r.run(job('b', { n: 2, ids: [1, 2] })), r.run(job('c', { n: 2, ids: [1, 2] })), r.run(job('d'))];
    await Promise.all([first].concat(ps));
    assert.deepStrictEqual(be.calls.map((c) => c.jobs.map((j) => j.n)), [[1], [2, 1], [2]]);
});

test('busy at MAX_SESSION_QUEUE jobs of one session and MAX_QUEUE sessions', async () => {
    const { r } = make({ delayMs: 5, sessions: 2, slots: 2 });
    const ps = [];
    for (let i = 0; i < MAX_SESSION_QUEUE; i++) ps.push(r.run(job('a', { past: i })).catch(() => null));
    const e = await rejects(r.run(job('a', { past: 9 })), /no queue slot free/);
    assert.strictEqual(e.busy, true);
    for (let i = 1; i < MAX_QUEUE; i++) ps.push(r.run(job('s' + i)).catch(() => null));
    const e2 = await rejects(r.run(job('late')), /queue slot/);
    assert.strictEqual(e2.busy, true);
    await Promise.all(ps);
});

test('a job past 0 for a session without a frame is cold; after a refusal it is busy', async () => {
    const { r } = make();
    const e = await rejects(r.run(job('x', { past: 3 })), /session x is no longer cached here/);
    assert.ok(!e.busy);
    r.refused.set('y', Number(process.hrtime.bigint()) / 1e6);
    const e2 = await rejects(r.run(job('y', { past: 3 })), /refused here for capacity/);
    assert.strictEqual(e2.busy, true);
});

test('a rewind is allowed, a skip ahead is cold, and a closed-loop duplicate is stale', async () => {
    const { r } = make();
    await r.run(job('a', { n: 3, ids: [1, 2, 3] }));
    await r.run(job('a', { past: 1, n: 2, ids: [4, 5] }));        // rewind to 1
    await rejects(r.run(job('a', { past: 7 })), /block 0 holds 3 rows, the job continues from 7/);
    const e = await rejects(r.run(job('a', { past: 2, auto: true })), /a duplicate of session a's job at 2/);
    assert.strictEqual(e.stale, true);
});

test('an idle session is evicted for a new one; with none idle and no wait the job is busy', async () => {
    const { r } = make({ sessions: 1, slots: 1, idleMs: 30, waitMs: 0 });
    await r.run(job('a'));
    const e = await rejects(r.run(job('b')), /no session free/);
    assert.strictEqual(e.busy, true);
    await sleep(40);
    await r.run(job('b'));
    assert.strictEqual(r.counts.evicted, 1);
    await rejects(r.run(job('a', { past: 1 })), /session a is no longer cached here/);
});

test('a waiting session is admitted when a frame is released, in arrival order', async () => {
    const { r } = make({ sessions: 1, slots: 1, idleMs: 10000, waitMs: 1000 });
    await r.run(job('a'));
    const pb = r.run(job('b'));
    const pc = r.run(job('c'));
    await sleep(20);
    assert.strictEqual(r.waiting.length, 2);
    await r.release('a');
    const b = await pb;
    assert.strictEqual(b.at, END);
    await r.release('b');
    await pc;
    assert.strictEqual(r.counts.waited, 2);
});

test('waiting past the deadline is a capacity refusal', async () => {
    const { r } = make({ sessions: 1, slots: 1, idleMs: 10000, waitMs: 30 });
    await r.run(job('a'));
    const e = await rejects(r.run(job('b')), /no session free/);
    assert.strictEqual(e.busy, true);
});

test('KV pages: a context larger than a frame is a configuration error', async () => {
    const { r } = make({ nMax: 128, tMax: 16 });
    await r.run(job('a', { n: 16, ids: new Array(16).fill(1) }));
    await rejects(r.run(job('a', { past: 120, n: 16, ids: new Array(16).fill(1) })), /context 136 exceeds 128/);
});

test('KV pages: page pressure evicts an idle session whole', async () => {
    // two frames, pool of one context (2 pages); b needs a page a holds
    const { r, be } = make({ nMax: 128, tMax: 16, slots: 1, sessions: 2, idleMs: 20 });
    for (let past = 0; past < 64; past += 16) await r.run(job('a', { past, n: 16, ids: new Array(16).fill(1) }));
    await r.run(job('a', { past: 64, n: 1 }));
    assert.strictEqual(be.freePages(), 0);
    await sleep(30);
    await r.run(job('b', { n: 16, ids: new Array(16).fill(2) }));
    assert.strictEqual(r.counts.evicted, 1);
    assert.strictEqual(be.slotPages(0) + be.slotPages(1), 1);
});

test('job checks and their messages (stage.js #prepare)', async () => {
    const { r } = make();
    await rejects(r.run(job('a', { n: 0, ids: [] })), /a job of 0 tokens is outside 1–16/);
    await rejects(r.run(job('a', { n: 17, ids: new Array(17).fill(0) })), /outside 1–16/);
    await rejects(r.run(job('a', { past: -1 })), /past -1 is not a position/);
    await rejects(r.run(job('a', { past: 600 })), /context 601 exceeds 512/);
    await rejects(r.run(job('a', { ids: [1, 2] })), /a job at position 0 needs 1 token ids/);
    await rejects(r.run(job('a', { pos: 1, ids: undefined }), new Uint16Array(3)), /payload is 3 floats, expected 8/);
    await rejects(r.run(job('a', { pos: 9 })), /position 9 is not held here/);
    await rejects(r.run(job('a', { n: 2, ids: [1, 2], drafts: [1, 2] })), /a verify job needs 1–7 draft ids/);
    await rejects(r.run(job('a', { fill: true, drafts: [1] })), /a prefill chunk cannot carry drafts/);
});

test('verify: drafts accepted while the sample matches, stop at the first mismatch', async () => {
    const { r } = make();
    const V = D.vocab;
    const best = (pos, x) => (pos * 7 + x) % V;
    // row i sits at position i, input ids[i]; the stub adds the positions crossed
    const ids = [3, 0, 0, 0];
    ids[1] = best(0 + END, ids[0]);
    ids[2] = best(1 + END, ids[1]);
    ids[3] = (best(2 + END, ids[2]) + 1) % V;   // this draft is wrong
    const out = await r.run(job('v', { n: 4, ids, drafts: ids.slice(1) }));
    assert.deepStrictEqual(out.tokens, [ids[1], ids[2], best(2 + END, ids[2])]);
    assert.strictEqual(out.token, best(2 + END, ids[2]));
});

test('a pass that stops before the head hands f16 rows on and keeps the boundary log', async () => {
    const { r } = make();
    const out = await r.run(job('h', { n: 2, ids: [4, 9] }), null, 2);
    assert.strictEqual(out.at, 2);
    assert.ok(out.hidden instanceof Uint16Array);
    assert.deepStrictEqual(Array.from(fromF16(out.hidden.subarray(0, 1))), [6]);
    const log = r.logs.get('h').get(2);
    assert.strictEqual(log.len, 2);
    assert.deepStrictEqual(log.rows.subarray(0, 2 * D.hidden), out.hidden);
});

test('a prefill chunk at the end fills the caches and samples nothing', async () => {
    const { r, be } = make();
    const out = await r.run(job('f', { fill: true, n: 3, ids: [1, 2, 3] }));
    assert.strictEqual(out.filled, true);
    assert.strictEqual(be.calls[0].jobs[0].sampled, 0);
});

test('release is idempotent and rejects the session\'s waiting jobs', async () => {
    const { r } = make({ sessions: 1, slots: 1, idleMs: 10000, waitMs: 1000 });
    await r.run(job('a'));
    const pb = r.run(job('b'));
    await sleep(10);
    await r.release('b');
    await rejects(pb, /session b ended while it waited for a frame/);
    await r.release('zzz');
    await r.release('a');
    assert.strictEqual(r.counts.released, 1);
});

test('temp > 0 without top-k reads whole logits rows', async () => {
    const { r, be } = make();
    const out = await r.run(job('t', { opts: { temp: 0.7 } }));
    assert.strictEqual(be.calls[0].topk, 1);
    assert.ok(Number.isInteger(out.token));
});

test('append loads one position at a time and moves `have`', async () => {
    const { r, be } = make({ have: 0 });
    assert.strictEqual(r.holds(0), false);
    assert.throws(() => r.append({}), /position 0 is the embedding and needs wte/);
    const q8 = (n) => ({ codes: new Int8Array(n), scales: new Uint16Array(n / 32) });
    r.append({ wte: q8(64) });
    assert.strictEqual(r.holds(0), true);
    assert.throws(() => r.append({ wte: q8(64) }), /position 1 is a block and needs its tensors/);
    const block = { q_proj: q8(64), k_proj: q8(64), v_proj: q8(64), o_proj: q8(64), gate_proj: q8(64),
                    up_proj: q8(64), down_proj: q8(64), input_layernorm: new Float32Array(8),
                    post_attention_layernorm: new Float32Array(8) };
    r.append(block);
    r.append(block);
    assert.throws(() => r.append({}), /the last position is the head and needs norm/);
    assert.strictEqual(r.append({ norm: new Float32Array(8) }), END);
    assert.throws(() => r.append({}), /nothing left to append: 0–3 is full/);
    assert.deepStrictEqual(be.uploads.map((u) => [u.layer, u.tensor]),
        [[-1, 9]].concat([0, 1].flatMap((l) => [0, 1, 2, 3, 4, 5, 6, 7, 8].map((t) => [l, t]))).concat([[-1, 10]]));
    const out = await r.run(job('a'));
    assert.strictEqual(out.at, END);
});

test('embed, head and w (engine.js:457, :641-642); growth is refused with a clear error', async () => {
    const whole = make().r;
    assert.strictEqual(whole.embed, true);
    assert.strictEqual(whole.head, true);
    const mid = make({ lo: 1, hi: 3, have: 1 }).r;
    assert.strictEqual(mid.embed, false);
    assert.strictEqual(mid.head, false);
    const q8 = (n) => ({ codes: new Int8Array(n), scales: new Uint16Array(n / 32), group: 32 });
    const block = { q_proj: q8(64), k_proj: q8(64), v_proj: q8(64), o_proj: q8(64), gate_proj: q8(64),
                    up_proj: q8(64), down_proj: q8(64), input_layernorm: new Float32Array(8),
                    post_attention_layernorm: new Float32Array(8) };
    mid.append(block);
    assert.strictEqual(mid.w.layers.length, 1);
    assert.deepStrictEqual(mid.w.layers[0].q_proj, { q8: true, values: 64, group: 32 });
    assert.strictEqual(mid.w.wte, null);
    const ends = make({ have: 0 }).r;
    ends.append({ wte: q8(64) });
    assert.deepStrictEqual(ends.w.wte, { q8: true, values: 64, group: 32 });
    for (const grow of ['prepend', 'growLeft', 'growRight']) {
        assert.throws(() => mid[grow]({}), new RegExp(`${grow}: this Runner's positions 1–2 are fixed`));
    }
});

test('sampler: a row drawn from its GPU candidates equals the whole-row draw', async () => {
    let seed = 12345;
    const rnd = () => ((seed = (seed * 1103515245 + 12345) % 2147483648) / 2147483648);
    const V = 500;
    for (let t = 0; t < 300; t++) {
        const row = new Float32Array(V).map(() => (rnd() * 20) - 10);
        const optsList = [{ temp: 0 }, { temp: 0.8, topK: 40 }, { temp: 1.2, topK: 5, rep: 1.3, pen: [[3, 2], [7, 1]], ban: [11] },
                          { temp: 0, freq: 0.5, pen: [[row.indexOf(Math.max.apply(null, row)), 3]] }];
        for (const opts of optsList) {
            const M = S.candidatesFor(opts, V);
            assert.ok(M !== null);
            const order = Array.from(row.keys()).sort((a, b) => row[b] - row[a] || a - b).slice(0, M);
            const r0 = rnd();
            const whole = S.sampleFromLogitsRow(row, opts, () => r0);
            const cand = S.sampleFromCandidates(order, order.map((i) => row[i]), opts, V, () => r0);
            assert.strictEqual(cand, whole, JSON.stringify(opts));
        }
    }
    assert.strictEqual(S.candidatesFor({ temp: 1 }, V), null);
    // topK clamps to 200; 200 + 60 banned ids is past TOPK_MAX
    assert.strictEqual(S.candidatesFor({ temp: 1, topK: 250, ban: new Array(10).fill(0).map((_, i) => i) }, V), 210);
    assert.strictEqual(S.candidatesFor({ temp: 1, topK: 200, ban: new Array(60).fill(0).map((_, i) => i) }, V), null);
});

test('f16 hand-off: every half round-trips, ties go to even, ±65504 clamps', async () => {
    const all = new Uint16Array(65536).map((_, i) => i);
    const vals = fromF16(all);
    const back = toF16(vals);
    for (let h = 0; h < 65536; h++) {
        const e = (h >>> 10) & 0x1f, m = h & 0x3ff;
        if (e === 0x1f && m) { assert.strictEqual(back[h] & 0x7e00, 0x7e00); continue; }
        if (e === 0x1f) { assert.strictEqual(back[h], (h & 0x8000) | 0x7bff); continue; }
        assert.strictEqual(back[h], h);
    }
    assert.strictEqual(toF16([1 + Math.pow(2, -11)])[0], 0x3c00);            // tie to even (down)
    assert.strictEqual(toF16([1 + 3 * Math.pow(2, -11)])[0], 0x3c02);        // tie to even (up)
    assert.strictEqual(toF16([1e9])[0], 0x7bff);
    assert.strictEqual(toF16([-1e9])[0], 0xfbff);
});

// A hybrid model: block 0 linear_attention, block 1 full_attention, with an
// MTP head (stage.js:1028-1090 rollback, :296-320 drafting).
const DH = Object.assign({}, D, { hybrid: true, layer_types: ['linear_attention', 'full_attention'],
                                  mtp: { draftVocab: 64 } });
function makeHybrid(o) {
    const opts = Object.assign({ lo: 0, hi: END, nMax: 512, tMax: 16, slots: 3, sessions: 3, idleMs: 50,
                                 waitMs: 0, batchRows: 16 }, o || {});
    const be = new StubBackend(DH, { nMax: opts.nMax, slots: opts.slots, frames: opts.sessions + 1, tMax: opts.tMax });
    const r = new Runner(be, DH, opts);
    r.mtp = { draftVocab: 64 };   // as attachMtp leaves it (its uploads are not part of this test)
    return { r, be };
}

test('hybrid: a verify snapshots; the next job inside it rolls back and keeps past - base rows', async () => {
    const { r, be } = makeHybrid();
    await r.run(job('a', { n: 4, ids: [1, 2, 3, 4] }));
    assert.strictEqual(be.spec[0].snap, 0);
    await r.run(job('a', { past: 4, n: 3, ids: [9, 9, 9], drafts: [9, 9] }));   // a verify of 3 rows from 4
    assert.strictEqual(be.spec[0].snap, 1);
    await r.run(job('a', { past: 6, n: 1, ids: [7] }));                         // keeps 2 of the 3
    assert.strictEqual(be.spec[0].keep, 2);
    assert.strictEqual(be.spec[0].snap, 0);
    await r.run(job('a', { past: 7, n: 1, ids: [7] }));                         // a plain continuation
    assert.strictEqual(be.spec[0].keep, undefined);
});

test('hybrid: a recurrent block cannot be rewound (cold), a restart at 0 is fine', async () => {
    const { r } = makeHybrid();
    await r.run(job('a', { n: 5, ids: [1, 2, 3, 4, 5] }));
    await rejects(r.run(job('a', { past: 3, n: 1, ids: [1] })), /no longer cached here/);
    await r.run(job('a', { past: 0, n: 2, ids: [1, 2] }));
});

test('hybrid: after a capacity refusal, a rewound recurrent block is still cold, not busy', async () => {
    const { r } = makeHybrid();
    await r.run(job('a', { n: 5, ids: [1, 2, 3, 4, 5] }));
    r.refused.set('a', Number(process.hrtime.bigint()) / 1e6);
    const cold0 = r.counts.cold;
    const e = await rejects(r.run(job('a', { past: 3, n: 1, ids: [1] })), /session a is no longer cached here/);
    assert.ok(!e.busy);
    assert.strictEqual(r.counts.cold, cold0 + 1);
    // behind the block (rows lost), the refusal still reads as busy
    const e2 = await rejects(r.run(job('a', { past: 9, n: 1, ids: [1] })), /refused here for capacity/);
    assert.strictEqual(e2.busy, true);
});

test('hybrid: replay leases beyond specSlots are refused nospec; an idle session\'s is taken', async () => {
    const { r } = makeHybrid({ specSlots: 1, idleMs: 30 });
    await r.run(job('a', { n: 2, ids: [1, 2] }));
    await r.run(job('b', { n: 2, ids: [1, 2] }));
    await r.run(job('a', { past: 2, n: 2, ids: [3, 4], drafts: [4] }));
    const e = await rejects(r.run(job('b', { past: 2, n: 2, ids: [3, 4], drafts: [4] })), /no speculative replay slot/);
    assert.strictEqual(e.nospec, true);
    assert.strictEqual(r.counts.nospec, 1);
    await sleep(40);                                      // a is idle now: b takes its lease
    await r.run(job('b', { past: 2, n: 2, ids: [3, 4], drafts: [4] }));
    await rejects(r.run(job('a', { past: 3, n: 1, ids: [4] })), /no longer cached here/);   // a lost its rollback
});

test('MTP: an mtp job fills with its ids and, looping with spec on, drafts after the sample', async () => {
    const { r, be } = makeHybrid();
    const out = await r.run(job('a', { n: 3, ids: [1, 2, 3], mtp: true, loop: { spec: true } }));
    assert.strictEqual(be.spec[0].mtp, 1);
    const last = be.drafts[be.drafts.length - 1];
    assert.strictEqual(last.row, 2);
    assert.strictEqual(last.pos, 3);
    assert.strictEqual(last.token, out.token);
    assert.strictEqual(last.k, 7);
    assert.deepStrictEqual(out.mtp, [1, 2, 3, 4, 5, 6, 7].map((i) => (out.token + i) % 64));
    // without spec: the row is kept, no drafts
    const out2 = await r.run(job('a', { past: 3, n: 1, ids: [out.token % 64], mtp: true }));
    assert.strictEqual(be.drafts[be.drafts.length - 1].k, 0);
    assert.strictEqual(out2.mtp, undefined);
});

(async () => {
    let failed = 0;
    for (const c of cases) {
        try {
            await c.fn();
            console.log(`ok   ${c.name}`);
        } catch (e) {
            failed++;
            console.log(`FAIL ${c.name}\n     ${e && e.stack ? e.stack.split('\n').slice(0, 3).join('\n     ') : e}`);
        }
    }
    console.log(`${cases.length - failed}/${cases.length} passed`);
    process.exit(failed ? 1 : 0);
})();
