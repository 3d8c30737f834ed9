'use strict';
// GPU check of speculative decoding through the JS Runner on a hybrid
// checkpoint with an MTP head: greedy decoding with the head's drafts sent as
// verify jobs (rollbacks through the Gated DeltaNet blocks when a draft is
// rejected) must emit the tokens of plain one-token greedy decoding
// (web/model/stage.js:322-335, :1028-1090; model.js:447-470). Prints JSON.
// Usage: node tests/node/spec_pass.js '<json config>'

const { createRunner, loader } = require('../../chattorrent_amd/node');

(async () => {
    const cfg = JSON.parse(process.argv[2]);
    const dir = cfg.checkpoint;
    const m = loader.loadManifest(dir);
    const md = loader.dimsFromManifest(m);
    const problems = loader.checkManifest(m, md);
    if (problems.length) throw new Error(problems.join('; '));
    const d = Object.assign({}, md, { tied: md.tied_lm_head ? 1 : 0 });
    const end = d.n_layer + 2;
    const client = loader.loadClient(dir, m, md);
    const mk = () => {
        const n = cfg.prompts.length;
        const r = createRunner(d, { lo: 0, hi: end, have: 0, nMax: cfg.nMax, tMax: cfg.tMax, slots: n,
                                    sessions: n, batchRows: cfg.tMax });
        for (let p = 0; p < end; p++) r.append(loader.weightsFor(dir, m, md, p, client));
        r.attachMtp(loader.loadMtp(dir, m, md));
        return r;
    };
    const job = (h) => Object.assign({ k: 'job', pos: 0, opts: { temp: 0 } }, h);
    const want = cfg.steps + 1;

    const plain = mk();
    const a = await Promise.all(cfg.prompts.map(async (ids, i) => {
        let out = await plain.run(job({ s: 'p' + i, past: 0, n: ids.length, ids }));
        const toks = [out.token];
        let past = ids.length;
        while (toks.length < want) {
            out = await plain.run(job({ s: 'p' + i, past, n: 1, ids: [toks[toks.length - 1]] }));
            toks.push(out.token);
            past += 1;
        }
        return toks;
    }));
    plain.backend.destroy();

    const spec = mk();
    let verifies = 0, accepted = 0;
    const b = await Promise.all(cfg.prompts.map(async (ids, i) => {
        const loop = { spec: true };
        let out = await spec.run(job({ s: 's' + i, past: 0, n: ids.length, ids, mtp: true, loop }));
        const toks = [out.token];
        let past = ids.length, drafts = out.mtp || [];
        while (toks.length < want) {
            const last = toks[toks.length - 1];
            if (drafts.length) {
                const vids = [last].concat(drafts);
                out = await spec.run(job({ s: 's' + i, past, n: vids.length, ids: vids, drafts, mtp: true, loop }));
                verifies++;
                accepted += out.tokens.length - 1;
                for (const t of out.tokens) toks.push(t);
                past += out.tokens.length;
            } else {
                out = await spec.run(job({ s: 's' + i, past, n: 1, ids: [last], mtp: true, loop }));
                toks.push(out.token);
                past += 1;
            }
            drafts = (out.mtp || []).slice(0, Math.max(0, Math.min(7, cfg.nMax - past - 8)));
        }
        return toks.slice(0, want);
    }));
    const nospec = spec.counts.nospec;
    spec.backend.destroy();

    // Drafts taken from the plain run's own next tokens, 1 to 5 of them, the
    // last one wrong every third verify: rollbacks keep 1..n rows and some
    // verifies accept every draft.
    const known = mk();
    let verifies2 = 0, accepted2 = 0;
    const c = await Promise.all(cfg.prompts.map(async (ids, i) => {
        let out = await known.run(job({ s: 'k' + i, past: 0, n: ids.length, ids }));
        const toks = [out.token];
        let past = ids.length;
        while (toks.length < want) {
            const j = toks.length;
            const drafts = a[i].slice(j, j + 1 + (j % 5));
            if (drafts.length && j % 3 === 0) drafts[drafts.length - 1] = (drafts[drafts.length - 1] + 1) % d.vocab;
            if (!drafts.length) break;
            const vids = [toks[j - 1]].concat(drafts);
            out = await known.run(job({ s: 'k' + i, past, n: vids.length, ids: vids, drafts }));
            verifies2++;
            accepted2 += out.tokens.length - 1;
            for (const t of out.tokens) toks.push(t);
            past += out.tokens.length;
        }
        return toks.slice(0, want);
    }));
    known.backend.destroy();
    console.log(JSON.stringify({ plain: a, spec: b, verifies, accepted, nospec, known: c, verifies2, accepted2 }));
})().catch((e) => { console.error(e.stack || e); process.exit(1); });
