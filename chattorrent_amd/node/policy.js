'use strict';
// The Runner's host decisions that do not touch the device, as plain
// functions and tables (the contract is the reference's Runner,
// web/model/stage.js): the limits, the checks a job must pass before anything
// changes (:1195-1308), which queued jobs join a pass (:697-728), and whether
// a job continues a session's blocks where they stand (:1023-1091).
// Node 12 syntax.

// positions of a model: 0 the embedding, 1..n_layer the blocks, n_layer + 1 the head
const positions = (nLayer) => nLayer + 2;

const LIMITS = {
    maxQueue: 32,          // sessions with jobs queued or running (stage.js:41)
    maxSessionQueue: 8,    // jobs of one session (stage.js:42)
    refusedMs: 60000,      // a capacity refusal colours a session's next cold miss (stage.js:45)
    activeMs: 5000,        // a session counts as active this long after its last job (stage.js:49)
    pageTokens: 64,        // split.js:75
    idleMs: 2000,          // an idle session may be evicted after this long
    waitMs: 30000,         // a new session waits this long for a frame
    specCols: 8,           // one real row plus up to 7 drafts (split.js:273)
    batchRows: 32,         // the reference's GEMV_ROWS_MAX, the default pass size
    logChunk: 256,         // boundary-log growth step, in rows (stage.js:34)
};
const WARMUP = '\0warmup';

// ------------------------------------------------------------ job checks ---
// Checked in this order; the first that fails names the job's problem. `j`
// carries the job (h, hidden) and what the Runner derived (at, to, gather);
// `r` is the Runner (tMax, nMax, d).
const JOB_RULES = [
    { fails: (j) => !!j.h.fill && j.h.drafts !== undefined && j.h.drafts !== null,
      says: () => 'a prefill chunk cannot carry drafts' },
    { fails: (j, r) => !Number.isInteger(j.h.n) || j.h.n < 1 || j.h.n > r.tMax,
      says: (j, r) => `a job of ${j.h.n} tokens is outside 1–${r.tMax}` },
    { fails: (j) => !Number.isInteger(j.h.past) || j.h.past < 0,
      says: (j) => `past ${j.h.past} is not a position` },
    { fails: (j, r) => j.h.past + j.h.n > r.nMax,
      says: (j, r) => `context ${j.h.past + j.h.n} exceeds ${r.nMax}` },
    { fails: (j) => j.gather && !idsOf(j.h.ids, j.h.n, Infinity),
      says: (j) => `a job at position 0 needs ${j.h.n} token ids` },
    { fails: (j, r) => !j.gather && (j.hidden ? j.hidden.length : 0) !== j.h.n * r.d.hidden,
      says: (j, r) => `payload is ${j.hidden ? j.hidden.length : 0} floats, expected ${j.h.n * r.d.hidden}` },
    { fails: (j) => draftsOf(j.h) !== null && !draftsFit(draftsOf(j.h), j.h.n),
      says: (j) => `a verify job needs 1–${LIMITS.specCols - 1} draft ids, one fewer than its ${j.h.n} tokens` },
    // the WebGPU gather clamps an id past the vocabulary; here it is refused
    { fails: (j, r) => j.gather && !idsOf(j.h.ids, j.h.n, r.d.vocab),
      says: (j) => `a job at position 0 needs ${j.h.n} token ids` },
];

function idsOf(ids, n, vocab) {
    return Array.isArray(ids) && ids.length === n && ids.every((id) => Number.isInteger(id) && id >= 0 && id < vocab);
}
const draftsOf = (h) => (h.drafts === undefined ? null : h.drafts);
function draftsFit(drafts, n) {
    return Array.isArray(drafts) && drafts.length >= 1 && drafts.length === n - 1 && n <= LIMITS.specCols
        && drafts.every((id) => Number.isInteger(id) && id >= 0);
}

// Throws the first failing rule's message (an Error without flags).
function checkJob(j, r) {
    const broken = JOB_RULES.find((rule) => rule.fails(j, r));
    if (broken) throw new Error(broken.says(j, r));
}

// ---------------------------------------------------------------- batching ---
// A job may share a pass with others unless it is a warm-up, a replay, a
// prefill chunk or a profiled job, or it alone exceeds the pass.
function batchable(h, rows) {
    return h.s !== WARMUP && !h.replay && !h.fill && !h.prof && Number.isInteger(h.n) && h.n >= 1 && h.n <= rows;
}

// The queued jobs that join `lead`'s pass, taken out of `queue` (entries
// {s, job}; s null marks a scheduled function, which ends the search). A
// candidate joins when it enters at the lead's position, its session has not
// been seen yet in the queue (so a session's jobs keep their order), and its
// rows still fit under `rows`; every session passed over counts as seen.
function planBatch(lead, queue, rows) {
    if (rows < 2 || !batchable(lead.h, rows)) return [];
    const seen = new Set([lead.h.s]);
    const taken = [];
    let used = lead.h.n;
    let i = 0;
    while (i < queue.length && used < rows) {
        const entry = queue[i];
        if (entry.s === null) break;
        const h = entry.job.h;
        const joins = !seen.has(entry.s) && batchable(h, rows) && h.pos === lead.h.pos && used + h.n <= rows;
        seen.add(entry.s);
        if (joins) {
            taken.push(entry.job);
            used += h.n;
            queue.splice(i, 1);
        } else {
            i++;
        }
    }
    return taken;
}

// --------------------------------------------------------- block counters ---
// Whether a job at `past` continues each of its blocks [first, last) where
// it stands. `fed` and `spec` give a block's rows held and its last verify
// ({base, n}) if that was the block's last job; `recurrent(b)` marks a
// linear_attention block. Per block:
//   * right after a verify of n rows from base, a job at (base, base + n)
//     (or at base for a re-sent refused verify, `rb`) keeps past - base of
//     those rows (a rollback);
//   * a restart at 0 is always fine unless the job must continue exactly;
//   * a full-attention block may be rewound (past <= fed); a recurrent one,
//     or a closed-loop job (`exact`), must continue exactly (past == fed);
//   * otherwise a closed-loop job behind the block is a duplicate (stale),
//     and anything else is a cache the session no longer has (cold).
// Returns {keep} (null: nothing rolled back), {stale: message}, or
// {cold: message, behind}: behind is true only when the block holds fewer
// rows than the job continues from.
function continuation(q) {
    let keep = null;
    for (let p = Math.max(q.at, 1); p < q.last; p++) {
        const b = p - 1;
        const fed = q.fed(b);
        const sp = q.spec(b);
        let k = null;
        const rollback = sp && fed === sp.base + sp.n && q.past < fed && (q.past > sp.base || (q.rb && q.past === sp.base));
        if (rollback) {
            k = q.past - sp.base;
        } else if (q.past === 0 && !q.exact) {
            continue;
        } else if (q.recurrent(b) || q.exact ? q.past === fed : q.past <= fed) {
            continue;
        } else if (q.exact && q.past < fed && !q.specLost) {
            return { stale: `a duplicate of session ${q.session}'s job at ${q.past} (block ${b} is already at ${fed})` };
        } else {
            // behind: the block lost rows the job needs (an eviction, which a
            // capacity refusal may explain); otherwise the block is ahead of
            // a job that cannot rewind it, which no retry can fix
            return { cold: `session ${q.session} is no longer cached here (block ${b} holds ${fed} rows, the job ` +
                           `continues from ${q.past})`, behind: q.past > fed };
        }
        if (keep !== null && keep !== k) {
            return { cold: `session ${q.session}'s blocks disagree on a rollback (${keep} and ${k} rows)` };
        }
        keep = k;
    }
    return { keep };
}

// The cut of a pass entering at `at` for a caller that wants to stop at
// `want` (default: as far as held), clamped to [at + 1, have].
function cutFor(at, want, have) {
    const w = want === undefined || want === null ? have : want;
    return Math.min(Math.max(w, at + 1), have);
}

module.exports = { LIMITS, WARMUP, checkJob, batchable, planBatch, continuation, cutFor, positions };
