'use strict';
// GPU check of the Node host: the JS Runner over the N-API addon decodes a few
// chats greedily, once with one Runner holding every position and once split
// at a block boundary into two Runners that hand f16 rows on, as two peers
// do (web/model/stage.js, docs/architecture.md). Prints the tokens as JSON.
// Usage: node tests/node/native_pass.js '<json config>'

const { createRunner, loader } = require('../../chattorrent_amd/node');
const wire = require('../../chattorrent_amd/node/wire');

// The rows leaving one Runner as the link carries them to the next
// (web/net.js framing, fragmented at a small limit so multi-fragment
// messages are exercised).
function overTheLink(h, rows) {
    const st = new wire.Reassembler();
    let msg = null;
    for (const f of wire.fragment(wire.pack({ k: 'job', s: h.s, n: h.n }, rows), 4096, 1)) msg = st.push(f);
    return wire.unpack(msg).payload;
}

async function decode(runners, cfg) {
    const d = cfg.dims;
    const end = d.n_layer + 2;
    // a job enters each runner at its `lo` and leaves at its `hi`
    const through = async (h, ids) => {
        let hidden = null, at = 0, out = null;
        for (const r of runners) {
            out = await r.run(Object.assign({}, h, { pos: at, ids: at === 0 ? ids : undefined }), hidden, r.hi);
            hidden = out.hidden && cfg.wire ? overTheLink(h, out.hidden) : out.hidden;
            at = out.at;
        }
        if (at !== end) throw new Error(`stopped at ${at}`);
        return out;
    };
    const chats = cfg.chats;
    const first = await Promise.all(chats.map((ids, i) =>
        through({ k: 'job', s: 'c' + i, past: 0, n: ids.length, opts: { temp: 0 } }, ids)));
    const hist = first.map((o) => [o.token]);
    const past = chats.map((ids) => ids.length);
    for (let step = 0; step < cfg.steps; step++) {
        const outs = await Promise.all(chats.map((_, i) =>
            through({ k: 'job', s: 'c' + i, past: past[i], n: 1, opts: { temp: 0 } }, [hist[i][hist[i].length - 1]])));
        outs.forEach((o, i) => { hist[i].push(o.token); past[i] += 1; });
    }
    return { hist, batched: runners[0].counts.batched };
}

(async () => {
    const cfg = JSON.parse(process.argv[2]);
    const d = cfg.dims;
    const end = d.n_layer + 2;
    // weights: the shared generator (cfg.seed), or a checkpoint directory
    // (cfg.checkpoint) appended position by position as a peer loads them
    const m = cfg.checkpoint ? loader.loadManifest(cfg.checkpoint) : null;
    const md = m ? loader.dimsFromManifest(m) : null;
    if (m) {
        const problems = loader.checkManifest(m, md);
        if (problems.length) throw new Error(problems.join('; '));
    }
    const client = m ? loader.loadClient(cfg.checkpoint, m, md) : null;
    const mk = (lo, hi) => {
        const r = createRunner(d, { lo, hi, have: m ? lo : hi, nMax: cfg.nMax, tMax: cfg.tMax,
                                    slots: cfg.chats.length, sessions: cfg.chats.length, batchRows: cfg.tMax });
        if (m) {
            for (let p = lo; p < hi; p++) r.append(loader.weightsFor(cfg.checkpoint, m, md, p, client));
        } else {
            r.backend.fillRandom(cfg.seed);
        }
        return r;
    };
    const whole = mk(0, end);
    const a = await decode([whole], cfg);
    whole.backend.destroy();
    const cut = cfg.cut;
    const up = mk(0, cut), down = mk(cut, end);
    const b = await decode([up, down], cfg);
    up.backend.destroy();
    down.backend.destroy();
    console.log(JSON.stringify({ whole: a.hist, split: b.hist, batched: a.batched }));
})().catch((e) => { console.error(e.stack || e); process.exit(1); });
