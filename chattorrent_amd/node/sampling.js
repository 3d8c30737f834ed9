'use strict';
// Host sampler of the head, restated from the reference's sampling.js
// (web/model/sampling.js:60-215) for the Node 12 runtime: the same limits,
// the same candidate count for a GPU top-M, and the same arithmetic and
// summation order, so a token drawn from the GPU's candidates is the token the
// whole logits row would give.

const PEN_CAP = 1.5;   // sampling.js:57
const LIMITS = { temp: [0, 2], topK: [0, 200], rep: [1, 2], freq: [0, 2], pres: [0, 2], pen: 64, ban: 4096 };
const TOPK_MAX = 256;  // sampling.js:125

function clampNumber(v, range, dflt) {
    if (typeof v !== 'number' || !Number.isFinite(v)) return dflt;
    return Math.min(range[1], Math.max(range[0], v));
}

// clampSampling (sampling.js:74-94): a job's options, clamped; an unusable
// value falls back to the default instead of failing the job.
function clampSampling(opts, vocab) {
    const o = opts || {};
    const V = vocab === undefined ? Infinity : vocab;
    const validId = (v) => Number.isInteger(v) && v >= 0 && v < V;
    const out = {
        temp: clampNumber(o.temp, LIMITS.temp, 0),
        topK: Math.trunc(clampNumber(o.topK, LIMITS.topK, 0)),
        rep: clampNumber(o.rep, LIMITS.rep, 1.0),
        freq: clampNumber(o.freq, LIMITS.freq, 0),
        pres: clampNumber(o.pres, LIMITS.pres, 0),
        pen: null,
        ban: null,
    };
    if (Array.isArray(o.pen)) {
        out.pen = o.pen.slice(0, LIMITS.pen).filter((p) =>
            Array.isArray(p) && validId(p[0]) && Number.isFinite(p[1]) && p[1] >= 0);
    }
    if (Array.isArray(o.ban)) out.ban = o.ban.slice(0, LIMITS.ban).filter(validId);
    return out;
}

function penalised(c) {
    return c.pen && (c.rep !== 1.0 || c.freq !== 0 || c.pres !== 0);
}

// candidatesFor (sampling.js:123-143): raw top logits a row needs, or null
// when only the whole row will do.
function candidatesFor(opts, vocab) {
    const c = clampSampling(opts, vocab);
    let k;
    if (c.temp <= 0) k = 1;
    else if (c.topK > 0 && c.topK < vocab) k = c.topK;
    else return null;
    const hit = new Set(c.ban || []);
    if (penalised(c)) for (const p of c.pen) hit.add(p[0]);
    const m = k + hit.size;
    return m > TOPK_MAX ? null : Math.min(m, vocab);
}

// The sampler over `vals` (every token when ids is null, else the tokens
// `ids` in ascending order) — sampleCore, sampling.js:145-215.
function sampleCore(vals, ids, opts, vocab, random) {
    const c = clampSampling(opts, vocab);
    const adj = Float32Array.from(vals);
    let index = (id) => id;
    if (ids) {
        const where = new Map();
        ids.forEach((id, i) => where.set(id, i));
        index = (id) => where.get(id);
    }
    const tokenAt = (i) => (ids ? ids[i] : i);
    if (c.ban) {
        for (const id of c.ban) {
            const i = index(id);
            if (i !== undefined) adj[i] = -Infinity;
        }
    }
    if (penalised(c)) {
        for (const p of c.pen) {
            const i = index(p[0]);
            if (i === undefined) continue;
            let v = adj[i];
            if (c.rep !== 1.0) v = v > 0 ? v / c.rep : v * c.rep;
            v -= c.pres + Math.min(c.freq * p[1], PEN_CAP);
            adj[i] = v;
        }
    }
    if (c.temp <= 0) {
        let best = 0, bestV = -Infinity;
        for (let i = 0; i < adj.length; i++) if (adj[i] > bestV) { bestV = adj[i]; best = i; }
        return tokenAt(best);
    }
    const scaled = adj.map((v) => v / c.temp);
    if (c.topK > 0 && c.topK < vocab) {
        // k-th largest by an insertion-sorted window of the k best
        const win = new Float32Array(c.topK).fill(-Infinity);
        for (let i = 0; i < scaled.length; i++) {
            const v = scaled[i];
            if (v <= win[c.topK - 1]) continue;
            let j = c.topK - 1;
            while (j > 0 && win[j - 1] < v) { win[j] = win[j - 1]; j--; }
            win[j] = v;
        }
        const cut = win[c.topK - 1];
        for (let i = 0; i < scaled.length; i++) if (scaled[i] < cut) scaled[i] = -Infinity;
    }
    let mx = -Infinity;
    for (const v of scaled) if (v > mx) mx = v;
    let sum = 0;
    for (let i = 0; i < scaled.length; i++) {
        const e = scaled[i] === -Infinity ? 0 : Math.exp(scaled[i] - mx);
        scaled[i] = e;
        sum += e;
    }
    const r = (random || Math.random)() * sum;
    let acc = 0;
    for (let i = 0; i < scaled.length; i++) {
        acc += scaled[i];
        if (r < acc) return tokenAt(i);
    }
    return tokenAt(scaled.length - 1);
}

function sampleFromLogitsRow(row, opts, random) {
    return sampleCore(row, null, opts, row.length, random);
}

// sampleFromCandidates (sampling.js:112-121): the GPU's top-M (any order).
function sampleFromCandidates(ids, vals, opts, vocab, random) {
    const order = Array.from(ids.keys()).sort((a, b) => ids[a] - ids[b]);
    return sampleCore(Float32Array.from(order, (i) => vals[i]), order.map((i) => ids[i]), opts, vocab, random);
}

module.exports = { LIMITS, TOPK_MAX, clampSampling, candidatesFor, sampleFromLogitsRow, sampleFromCandidates };
