'use strict';
// Token sampling at the head, to the contract of the reference's sampler
// (web/model/sampling.js:57-215): the same option limits and defaults, the
// same candidate count for a GPU top-M (candidatesFor), and the same
// arithmetic, so a token drawn from the GPU's candidates is the token the
// whole logits row would give (sampling.js:107-121 requires this).
//
// The draw runs as four stages over a Float32Array of logits: adjust (bans,
// then repetition/frequency/presence penalties in list order), scale by the
// temperature, cut below the k-th largest (found with a min-heap of the k
// best), and draw from the softmax: weights exp(v - max) summed in f64 for
// the total, accumulated from their f32 copies for the walk, tokens in
// ascending order. Greedy (temperature 0) is the first maximum after the
// adjust stage. Node 12 syntax.

const PEN_CAP = 1.5;          // largest frequency penalty one token takes
const TOPK_MAX = 256;         // the most candidates a GPU top-M returns

// option -> [lowest, highest, default]; topK is truncated after clamping
const RANGES = { temp: [0, 2, 0], topK: [0, 200, 0], rep: [1, 2, 1.0], freq: [0, 2, 0], pres: [0, 2, 0] };
const LIST_MAX = { pen: 64, ban: 4096 };
const LIMITS = { temp: [0, 2], topK: [0, 200], rep: [1, 2], freq: [0, 2], pres: [0, 2], pen: 64, ban: 4096 };

// A job's options as the sampler uses them. Unusable numbers take their
// default; penalty entries must be [id, count >= 0] and bans ids, both within
// the vocabulary, and each list keeps only its first LIST_MAX entries.
function clampSampling(opts, vocab) {
    const o = opts || {};
    const V = vocab === undefined ? Infinity : vocab;
    const out = {};
    for (const name of Object.keys(RANGES)) {
        const [lo, hi, dflt] = RANGES[name];
        const v = o[name];
        out[name] = typeof v === 'number' && Number.isFinite(v) ? Math.min(hi, Math.max(lo, v)) : dflt;
    }
    out.topK = Math.trunc(out.topK);
    const isId = (v) => Number.isInteger(v) && v >= 0 && v < V;
    out.pen = Array.isArray(o.pen)
        ? o.pen.slice(0, LIST_MAX.pen).filter((e) => Array.isArray(e) && isId(e[0]) && Number.isFinite(e[1]) && e[1] >= 0)
        : null;
    out.ban = Array.isArray(o.ban) ? o.ban.slice(0, LIST_MAX.ban).filter(isId) : null;
    return out;
}

const penalises = (c) => c.pen !== null && (c.rep !== 1.0 || c.freq !== 0 || c.pres !== 0);

// The raw top logits a row needs for these options (1 for greedy, top-k plus
// every banned or penalised token), or null when only the whole row will do
// (temperature without top-k, or more than TOPK_MAX candidates).
function candidatesFor(opts, vocab) {
    const c = clampSampling(opts, vocab);
    let width = null;
    if (c.temp <= 0) width = 1;
    else if (c.topK > 0 && c.topK < vocab) width = c.topK;
    if (width === null) return null;
    const touched = new Set(c.ban || []);
    if (penalises(c)) c.pen.forEach((e) => touched.add(e[0]));
    const m = width + touched.size;
    return m > TOPK_MAX ? null : Math.min(m, vocab);
}

// Stage 1: bans to -inf, then penalties, on a copy of the logits. `where`
// maps a token to its index in `vals` (undefined: not among them).
function adjust(vals, where, c) {
    const out = Float32Array.from(vals);
    if (c.ban) {
        for (const id of c.ban) {
            const i = where(id);
            if (i !== undefined) out[i] = -Infinity;
        }
    }
    if (penalises(c)) {
        for (const [id, count] of c.pen) {
            const i = where(id);
            if (i === undefined) continue;
            let v = out[i];
            if (c.rep !== 1.0) v = v > 0 ? v / c.rep : v * c.rep;
            out[i] = v - (c.pres + Math.min(c.freq * count, PEN_CAP));
        }
    }
    return out;
}

// The k-th largest value of `a` (-inf when it has fewer than k): a min-heap
// of the k best seen so far, whose root is the answer at the end.
function kthLargest(a, k) {
    if (a.length < k) return -Infinity;
    const heap = new Float32Array(k);
    const down = (i) => {
        for (;;) {
            const l = 2 * i + 1, r = l + 1;
            let m = i;
            if (l < k && heap[l] < heap[m]) m = l;
            if (r < k && heap[r] < heap[m]) m = r;
            if (m === i) return;
            const t = heap[i];
            heap[i] = heap[m];
            heap[m] = t;
            i = m;
        }
    };
    for (let i = 0; i < k; i++) heap[i] = a[i];
    for (let i = (k >> 1) - 1; i >= 0; i--) down(i);
    for (let i = k; i < a.length; i++) {
        if (a[i] > heap[0]) {
            heap[0] = a[i];
            down(0);
        }
    }
    return heap[0];
}

// Stage 4: the index drawn from softmax(w) with u in [0, 1).
function drawIndex(w, u) {
    let top = -Infinity;
    for (let i = 0; i < w.length; i++) if (w[i] > top) top = w[i];
    let total = 0;
    for (let i = 0; i < w.length; i++) {
        const e = w[i] === -Infinity ? 0 : Math.exp(w[i] - top);
        w[i] = e;            // the walk below adds these f32 copies
        total += e;
    }
    const target = u * total;
    let run = 0;
    for (let i = 0; i < w.length; i++) {
        run += w[i];
        if (target < run) return i;
    }
    return w.length - 1;
}

// vals: logits of every token (ids null) or of `ids` in ascending order.
function drawToken(vals, ids, opts, vocab, random) {
    const c = clampSampling(opts, vocab);
    let where = (id) => id;
    if (ids) {
        const pos = new Map();
        for (let i = 0; i < ids.length; i++) pos.set(ids[i], i);
        where = (id) => pos.get(id);
    }
    const tokenAt = (i) => (ids ? ids[i] : i);
    const adj = adjust(vals, where, c);
    if (c.temp <= 0) {
        let best = 0;
        let bestV = -Infinity;
        adj.forEach((v, i) => { if (v > bestV) { bestV = v; best = i; } });
        return tokenAt(best);
    }
    const w = adj.map((v) => v / c.temp);
    if (c.topK > 0 && c.topK < vocab) {
        const cut = kthLargest(w, c.topK);
        for (let i = 0; i < w.length; i++) if (w[i] < cut) w[i] = -Infinity;
    }
    return tokenAt(drawIndex(w, (random || Math.random)()));
}

// A whole logits row (the reference's full-row readback).
function sampleFromLogitsRow(row, opts, random) {
    return drawToken(row, null, opts, row.length, random);
}

// The GPU's top-M candidates (any order): drawn over them in token order.
function sampleFromCandidates(ids, vals, opts, vocab, random) {
    const pairs = Array.from(ids, (id, i) => [id, vals[i]]).sort((a, b) => a[0] - b[0]);
    return drawToken(Float32Array.from(pairs, (p) => p[1]), pairs.map((p) => p[0]), opts, vocab, random);
}

module.exports = { LIMITS, TOPK_MAX, clampSampling, candidatesFor, sampleFromLogitsRow, sampleFromCandidates };
