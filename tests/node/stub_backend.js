'use strict';
// A CPU stand-in for the MI355X backend with the C ABI's bookkeeping: a page
// pool taken in job order and returned on release, per-job statuses, one pass
// at a time, top-M candidates at the head or f16 rows before it. Its
// "model" is a fixed function of the row's absolute position and input, so
// tests can predict every token. Test infrastructure only.

const { toF16, fromF16 } = require('../../chattorrent_amd/node/f16');

class StubBackend {
    constructor(d, o) {
        this.d = d;
        this.pageTokens = 64;
        this.maxPages = Math.ceil(o.nMax / 64);
        this.nPages = o.slots * this.maxPages;
        this.freeCount = this.nPages;
        this.owned = new Array(o.frames).fill(0);
        this.tMax = o.tMax;
        this.calls = [];
        this.uploads = [];
        this.busy = false;
        this.lastLogits = null;
        this.delayMs = o.delayMs || 0;
    }

    // Logits of the row at absolute position `pos` whose input token or
    // hidden value is `x`: the best token is (pos * 7 + x) % vocab, ties low.
    logits(pos, x) {
        const V = this.d.vocab;
        const out = new Float32Array(V);
        const best = (pos * 7 + x) % V;
        for (let v = 0; v < V; v++) out[v] = -((v - best + V) % V) / V;
        return out;
    }

    // cc_mtp_draft: drafts t+1, t+2, ... (mod the draft rows), recorded
    mtpDraft(slot, row, token, pos, k) {
        this.drafts = (this.drafts || []).concat([{ slot, row, token, pos, k }]);
        const out = new Uint32Array(k);
        for (let i = 0; i < k; i++) out[i] = (token + 1 + i) % this.d.mtp.draftVocab;
        return out;
    }

    step(jobs, at, to, topk) {
        if (this.busy) return Promise.reject(new Error('a step is already running on this context'));
        this.busy = true;
        this.calls.push({ jobs: jobs.map((j) => ({ slot: j.slot, past: j.past, n: j.n, sampled: j.sampled })), at, to, topk });
        // the speculation and MTP fields of each job, when set
        this.spec = jobs.map((j) => ({ snap: j.snap || 0, keep: j.keep, mtp: j.mtp || 0 }));
        const end = to === this.d.n_layer + 2;
        const status = new Int32Array(jobs.length);
        let need = 0;
        for (const j of jobs) need += Math.max(0, Math.ceil((j.past + j.n) / 64) - this.owned[j.slot]);
        const done = (res) => new Promise((r) => setTimeout(() => { this.busy = false; r(res); }, this.delayMs));
        if (need > this.freeCount) {
            status.fill(1);
            return done({ code: 1, status, error: `no KV page free for the pass (${need} needed, ${this.freeCount} free)` });
        }
        for (const j of jobs) {
            const nw = Math.max(0, Math.ceil((j.past + j.n) / 64) - this.owned[j.slot]);
            this.owned[j.slot] += nw;
            this.freeCount -= nw;
        }
        const H = this.d.hidden;
        const inputs = [];
        for (const j of jobs) {
            for (let i = 0; i < j.n; i++) {
                const x = j.ids ? j.ids[i] : Math.round(fromF16(j.hidden.subarray(i * H, i * H + 1))[0]);
                inputs.push({ pos: j.past + i, x, sampled: i >= j.n - j.sampled });
            }
        }
        if (end) {
            const rows = inputs.filter((r) => r.sampled);
            if (!rows.length) return done({ code: 0, status });
            const V = this.d.vocab;
            const vals = new Float32Array(rows.length * topk), ids = new Uint32Array(rows.length * topk);
            this.lastLogits = new Float32Array(rows.length * V);
            rows.forEach((r, k) => {
                const lg = this.logits(r.pos + to - at, r.x);
                this.lastLogits.set(lg, k * V);
                const order = Array.from(lg.keys()).sort((a, b) => lg[b] - lg[a] || a - b);
                for (let m = 0; m < topk; m++) { vals[k * topk + m] = lg[order[m]]; ids[k * topk + m] = order[m]; }
            });
            return done({ code: 0, status, vals, ids });
        }
        // Before the head: each row's hidden value is its input plus the
        // positions crossed, as f16 bits.
        const hidden = new Float32Array(inputs.length * H);
        inputs.forEach((r, k) => hidden.fill(r.x + (to - at), k * H, (k + 1) * H));
        return done({ code: 0, status, hidden: toF16(hidden) });
    }

    upload(layer, tensor, data, scales) { this.uploads.push({ layer, tensor, n: data.length, ns: scales ? scales.length : 0 }); }

    release(slot) {
        this.freeCount += this.owned[slot];
        this.owned[slot] = 0;
    }
    slotPages(slot) { return this.owned[slot]; }
    freePages() { return this.freeCount; }
    readLogits(rows) { return this.lastLogits.subarray(0, rows * this.d.vocab); }
    stats() { return { vramBytes: 0, passes: this.calls.length }; }
}

module.exports = { StubBackend };
