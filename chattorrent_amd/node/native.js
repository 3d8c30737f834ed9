'use strict';
// The MI355X backend of the JS Runner: the N-API addon over the ccdecode C
// ABI (include/ccdecode.h). Loading fails loudly when the addon or the HIP
// library is missing; there is no fallback.

const path = require('path');

let addon = null;
function load() {
    if (!addon) addon = require(path.join(__dirname, 'ccdecode.node'));
    return addon;
}

const CODES = ['ok', 'busy', 'cold', 'stale', 'nospec', 'earg', 'epool', 'eoom', 'edevice'];

class NativeBackend {
    // d: model dims (loader.js dimsFromManifest names); o: {lo, hi, nMax,
    // tMax, slots, frames, maxJobs, device}. `frames` page tables, one per
    // session the Runner may hold at once (its warm-up frame included).
    constructor(d, o) {
        const a = load();
        this.d = d;
        this.pageTokens = 64;
        this.frames = o.frames;
        this.maxPages = Math.ceil(o.nMax / this.pageTokens);
        this.nPages = o.slots * this.maxPages;
        this.ctx = a.create(d, {
            lo: o.lo, hi: o.hi, nMax: o.nMax, tMax: o.tMax, slots: o.slots, sessions: o.frames,
            maxJobs: o.maxJobs || o.frames, device: o.device || 0,
        });
    }

    // One packed pass (Runner.#pass's GPU half). Resolves with
    // {code, status, vals?, ids?, hidden?, error?}.
    step(jobs, at, to, topk) { return load().step(this.ctx, jobs, at, to, topk); }
    release(slot) { load().release(this.ctx, slot); }
    slotPages(slot) { return load().slotPages(this.ctx, slot); }
    freePages() { return load().freePages(this.ctx); }
    readLogits(rows) { return load().readLogits(this.ctx, rows); }
    // cc_mtp_draft: keep `row` of the last pass, chain k drafts after `token`
    mtpDraft(slot, row, token, pos, k) { return load().mtpDraft(this.ctx, slot, row, token, pos, k); }
    fillRandom(seed) { load().fillRandom(this.ctx, seed); }
    fillRandomKV(slot, tokens, seed, key) { load().fillRandomKV(this.ctx, slot, tokens, seed, key); }
    upload(layer, tensor, data, scales, group) {
        load().upload(this.ctx, layer, tensor, data, scales || null, group || 32);
    }
    stats() { return load().stats(this.ctx); }
    destroy() {
        if (this.ctx) load().destroy(this.ctx);
        this.ctx = null;
    }
}

module.exports = { NativeBackend, CODES };
