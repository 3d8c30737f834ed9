'use strict';
// The Runner of a peer's position range (web/model/stage.js:98-1578), with its
// GPU half on the MI355X backend (native.js, or any object with the same
// methods). The host policy is the reference's, restated for Node 12:
// arrival-order queue with batching of same-cursor jobs (:586-728), frame
// admission with LRU eviction of idle sessions and a waiting list (:730-1021),
// per-block row counters (:1023-1091), KV pages with eviction (:1093-1120),
// boundary logs (:1122-1150), job validation (:1195-1308), one packed pass
// (:1314-1481) and sampling / verify acceptance at the head (:1483-1561).
//
// Out of scope here (as in the MI355X library): linear-attention blocks and
// their replay slots, the MTP draft head, keep-warm kernels and GPU profiles.

const { candidatesFor, sampleFromCandidates, sampleFromLogitsRow } = require('./sampling');
const { toF16 } = require('./f16');

const MAX_QUEUE = 32;            // stage.js:41
const MAX_SESSION_QUEUE = 8;     // stage.js:42
const REFUSED_MS = 60000;        // stage.js:45
const ACTIVE_MS = 5000;          // stage.js:49
const PAGE_TOKENS = 64;          // split.js:75
const IDLE_MS = 2000;            // split.js
const WAIT_MS = 30000;           // split.js
const SPEC_COLS = 8;             // split.js:273
const BATCH_ROWS = 32;           // kernels.js GEMV_ROWS_MAX, the reference's default
const LOG_CHUNK = 256;           // stage.js:34
const WARMUP = '\0warmup';       // stage.js:31

// cc_upload tensor ids (include/ccdecode.h) by HF tensor name.
const TENSOR = { q_proj: 0, k_proj: 1, v_proj: 2, o_proj: 3, gate_proj: 4, up_proj: 5, down_proj: 6,
                 input_layernorm: 7, post_attention_layernorm: 8, wte: 9, norm: 10, lm_head: 11,
                 attn_gate: 12, q_norm: 13, k_norm: 14, in_proj_q: 15, in_proj_k: 16, in_proj_v: 17,
                 in_proj_z: 18, in_proj_b: 19, in_proj_a: 20, conv1d_q: 21, conv1d_k: 22, conv1d_v: 23,
                 gate_params: 24, gated_norm: 25, out_proj: 26, enorm: 27, hnorm: 28, fc_e: 29, fc_h: 30,
                 mtp_norm: 31, embed_draft: 32, head_draft: 33 };
const LAYER_MTP = -2;
const BLOCK_TENSORS = ['q_proj', 'k_proj', 'v_proj', 'o_proj', 'gate_proj', 'up_proj', 'down_proj',
                       'input_layernorm', 'post_attention_layernorm'];
// a hybrid checkpoint's full-attention extras, and its linear_attention
// blocks' tensors (loader.js:543-590)
const HYBRID_FULL = ['attn_gate', 'q_norm', 'k_norm'];
const LINEAR_TENSORS = ['in_proj_q', 'in_proj_k', 'in_proj_v', 'in_proj_z', 'in_proj_b', 'in_proj_a', 'conv1d_q',
                        'conv1d_k', 'conv1d_v', 'gate_params', 'gated_norm', 'out_proj', 'gate_proj', 'up_proj',
                        'down_proj', 'input_layernorm', 'post_attention_layernorm'];
const MTP_TENSORS = ['enorm', 'hnorm', 'fc_e', 'fc_h', 'mtp_norm', 'embed_draft', 'head_draft'];

// Thrown by _cacheFor for a job that must wait for a frame; never escapes.
const WAIT = new Error('waiting for a session frame');

const now = () => Number(process.hrtime.bigint()) / 1e6;
const positions = (nLayer) => nLayer + 2;
function blockRange(lo, hi, nLayer) {
    return [Math.max(lo, 1) - 1, Math.min(hi, nLayer + 1) - 1];
}

// A backend error (status code from the C ABI) as the reference's Error
// classes: busy and stale carry their flag; cold and others are plain.
function backendError(res) {
    const err = new Error(res.error || `the pass failed (status ${res.code})`);
    if (res.code === 1) err.busy = true;
    if (res.code === 3) err.stale = true;
    err.status = res.code;
    return err;
}

class Runner {
    // backend: native.js NativeBackend (created with `sessions + 1` frames:
    // frame `sessions` is the warm-up's). Options as stage.js:107-110, except
    // that batchRows may go up to tMax (the MI355X pass keeps every row's bits
    // at any batch size).
    constructor(backend, d, opts) {
        const o = opts || {};
        this.backend = backend;
        this.d = d;
        this.lo = o.lo;
        this.hi = o.hi;
        this.have = o.have === undefined ? o.hi : o.have;
        this.nMax = o.nMax;
        this.tMax = o.tMax;
        this.slots = o.slots === undefined ? 5 : o.slots;
        this.sessions = o.sessions === undefined ? this.slots : o.sessions;
        this.pageTokens = o.pageTokens === undefined ? PAGE_TOKENS : o.pageTokens;
        this.idleMs = o.idleMs === undefined ? IDLE_MS : o.idleMs;
        this.waitMs = o.waitMs === undefined ? WAIT_MS : o.waitMs;
        const br = o.batchRows === undefined ? BATCH_ROWS : o.batchRows;
        this.batchRows = Math.max(1, Math.min(br, this.tMax));
        this.blockLo = blockRange(this.lo, this.hi, d.n_layer)[0];
        this.maxPages = Math.ceil(this.nMax / this.pageTokens);
        this.nPages = this.slots * this.maxPages;

        this.free = [];
        for (let i = this.sessions - 1; i >= 0; i--) this.free.push({ slot: i });
        this.warm = { slot: this.sessions, fed: new Map() };
        this.live = new Map();       // session -> frame, least recently used first
        this.pending = new Map();    // session -> jobs queued or running
        this.tasks = [];
        this.draining = false;
        this.waiting = [];
        this.waitTimer = undefined;
        this.turn = null;
        this.refused = new Map();
        this.cuts = new Map();
        this.logs = new Map();
        this.onIdle = [];
        this.reserved = 0;           // pages promised to the jobs of the pass being prepared
        this.backlog = 0;
        this.activeAt = 0;
        this.lastJobAt = 0;
        this.queueAvgMs = 0;
        this.msPerPos = null;
        this.overheadMs = null;
        this.decoded = false;
        this.warmups = 0;
        this.counts = { admitted: 0, evicted: 0, released: 0, refused: 0, cold: 0, waited: 0,
                        batched: 0, batchedJobs: 0, nospec: 0 };
        // speculative decoding's replay slots (stage.js:222-228): the device
        // keeps every session's replay data, so a slot here is the lease that
        // bounds how many sessions speculate through linear_attention blocks
        this.specSlots = o.specSlots === undefined ? this.slots : o.specSlots;
        this.specLive = new Set();
        this.mtp = null;
    }

    _kind(b) {
        const lt = this.d.layer_types;
        return lt && lt[b] ? lt[b] : 'full_attention';
    }

    holds(pos) { return pos >= this.lo && pos < this.have; }

    // append(weights) — stage.js:446-468: load position `have`. `weights`
    // holds host tensors by their HF names: q8 ones as {codes: Int8Array
    // [N*K], scales: Uint16Array (f16 bits) or Float32Array
    // [N*ceil(K/group)], group (default 32)}, norms as Float32Array (what
    // node/loader.js's loadBlock / loadClient return). Position 0 needs wte;
    // the last, norm (and lm_head when untied); a block, its seven
    // projections and two norms.
    append(weights) {
        const p = this.have;
        const w = weights || {};
        if (p >= this.hi) throw new Error(`nothing left to append: ${this.lo}–${this.hi - 1} is full`);
        const up = (layer, id, t) => this.backend.upload(layer, id, t.codes || t, t.codes ? t.scales : null,
                                                         t.codes ? t.group : undefined);
        if (p === 0) {
            if (!w.wte) throw new Error('position 0 is the embedding and needs wte');
            up(-1, TENSOR.wte, w.wte);
        } else if (p === positions(this.d.n_layer) - 1) {
            if (!w.norm) throw new Error('the last position is the head and needs norm');
            up(-1, TENSOR.norm, w.norm);
            if (w.lm_head) up(-1, TENSOR.lm_head, w.lm_head);
            else if (w.wte) up(-1, TENSOR.wte, w.wte);
        } else {
            const linear = this._kind(p - 1) === 'linear_attention';
            const names = linear ? LINEAR_TENSORS : this.d.hybrid ? BLOCK_TENSORS.concat(HYBRID_FULL) : BLOCK_TENSORS;
            if (!w[linear ? 'in_proj_q' : 'q_proj']) throw new Error(`position ${p} is a block and needs its tensors`);
            for (const name of names) {
                if (!w[name]) throw new Error(`position ${p} is a block and needs ${name}`);
                up(p - 1, TENSOR[name], w[name]);
            }
        }
        this.have = p + 1;
        return this.have;
    }

    // attachMtp(m) — stage.js:273-289: the MTP head (loader.js loadMtp's
    // tensors: its full-attention block's, enorm, hnorm, fc_e, fc_h,
    // mtp_norm, embed_draft, head_draft), held with the LM head. The
    // backend was created with d.mtp set, which sizes its KV and scratch.
    attachMtp(m) {
        if (this.hi !== positions(this.d.n_layer)) throw new Error('the MTP head is held with the LM head');
        if (!this.d.mtp) throw new Error('the model dims carry no mtp head');
        const up = (layer, id, t) => this.backend.upload(layer, id, t.codes || t, t.codes ? t.scales : null,
                                                         t.codes ? t.group : undefined);
        const names = this.d.hybrid ? BLOCK_TENSORS.concat(HYBRID_FULL) : BLOCK_TENSORS;
        for (const name of names) {
            if (!m[name]) throw new Error(`the MTP head needs ${name}`);
            up(LAYER_MTP, TENSOR[name], m[name]);
        }
        for (const name of MTP_TENSORS) {
            if (!m[name]) throw new Error(`the MTP head needs ${name}`);
            up(-1, TENSOR[name], m[name]);
        }
        this.mtp = { draftVocab: this.d.mtp.draftVocab };
    }

    // #specSlot — stage.js:336-372: the session's lease, taken on its first
    // verify through a linear_attention block here and held until its frame
    // goes. With every lease taken, an idle session's is taken from it (it
    // loses its rollback, #specSteal :374-386) or the job is refused nospec.
    _specSlot(session) {
        if (this.specLive.has(session)) return;
        if (this.specLive.size >= this.specSlots) {
            let stolen = false;
            const t = now();
            for (const [id, frame] of this.live) {
                if (!this.specLive.has(id) || this.pending.has(id) || t - (frame.lastUse || 0) < this.idleMs) continue;
                this.specLive.delete(id);
                if (frame.specAt) frame.specAt.clear();
                frame.specLost = true;
                stolen = true;
                break;
            }
            if (!stolen) {
                this.counts.nospec++;
                const err = new Error(`no speculative replay slot here (${this.specSlots} in use)`);
                err.nospec = true;
                throw err;
            }
        }
        this.specLive.add(session);
    }

    get vramBytes() { return this.backend.stats().vramBytes; }

    // run(h, hidden, want) — stage.js:600-621.
    run(h, hidden, want) {
        const s = h.s;
        const mine = this.pending.get(s) || 0;
        if (mine >= MAX_SESSION_QUEUE || (!mine && this.pending.size >= MAX_QUEUE)) {
            return Promise.reject(this._atCapacity('queue slot', s));
        }
        this.backlog++;
        this.pending.set(s, mine + 1);
        this.activeAt = now();
        const settle = () => {
            this.activeAt = now();
            this.backlog--;
            const n = this.pending.get(s) - 1;
            if (n > 0) this.pending.set(s, n);
            else this.pending.delete(s);
            const frame = this.live.get(s);
            if (frame) frame.lastUse = now();
        };
        return new Promise((resolve, reject) => {
            this._submit({ h, hidden, want, queuedAt: now(), resolve, reject });
        }).then((v) => { settle(); return v; }, (e) => { settle(); throw e; });
    }

    _submit(job) { this._enqueue({ s: job.h.s, fill: !!job.h.fill, job }); }

    schedule(fn) {
        return new Promise((resolve, reject) => {
            this._enqueue({ s: null, fill: false,
                            run: () => Promise.resolve().then(fn).then(resolve, reject) });
        });
    }

    _enqueue(task) {
        this.tasks.push(task);
        if (this.draining) return;
        this.draining = true;
        queueMicrotask(() => this._drain());
    }

    async _drain() {
        while (this.tasks.length) {
            const task = this.tasks.splice(0, 1)[0];
            const run = task.job ? this._runJobs([task.job].concat(this._batchWith(task.job))) : task.run();
            try { await run; } catch (e) { /* a task reports its own failure */ }
        }
        this.draining = false;
        for (const wake of this.onIdle.splice(0)) wake();
    }

    // #batchWith / #batchable — stage.js:697-728.
    _batchWith(lead) {
        if (this.batchRows < 2 || !this._batchable(lead.h)) return [];
        const seen = new Set([lead.h.s]);
        const jobs = [];
        let rows = lead.h.n;
        for (let i = 0; i < this.tasks.length && rows < this.batchRows; i++) {
            const task = this.tasks[i];
            if (task.s === null) break;
            const fits = !seen.has(task.s) && this._batchable(task.job.h)
                && task.job.h.pos === lead.h.pos && rows + task.job.h.n <= this.batchRows;
            seen.add(task.s);
            if (!fits) continue;
            jobs.push(task.job);
            rows += task.job.h.n;
            this.tasks.splice(i--, 1);
        }
        return jobs;
    }

    _batchable(h) {
        return h.s !== WARMUP && !h.replay && !h.fill && !h.prof
            && Number.isInteger(h.n) && h.n >= 1 && h.n <= this.batchRows;
    }

    // #park / #pump — stage.js:730-775.
    _park(job) {
        if (job.deadline === undefined) {
            job.deadline = now() + this.waitMs;
            this.counts.waited++;
            this.waiting.push(job);
        } else {
            let i = 0;
            while (i < this.waiting.length && this.waiting[i].h.s === job.h.s) i++;
            this.waiting.splice(i, 0, job);
        }
        if (this.waitTimer === undefined) {
            this.waitTimer = setInterval(() => this._pump(), Math.max(5, Math.min(250, this.idleMs / 4)));
        }
    }

    _pump() {
        const t = now();
        const late = this.waiting.filter((j) => t >= j.deadline);
        if (late.length) {
            this.waiting = this.waiting.filter((j) => t < j.deadline);
            for (const j of late) j.reject(this._atCapacity('session', j.h.s));
        }
        if (!this.waiting.length) {
            clearInterval(this.waitTimer);
            this.waitTimer = undefined;
            return;
        }
        if (this.turn !== null) return;
        if (!this.free.length && this._evictable() === null) return;
        const s = this.waiting[0].h.s;
        const jobs = this.waiting.filter((j) => j.h.s === s);
        this.waiting = this.waiting.filter((j) => j.h.s !== s);
        this.turn = s;
        for (const job of jobs) this._submit(job);
        this.schedule(() => { this.turn = null; });
    }

    // warmup(from, want) — stage.js:783-821: one row through the held
    // positions in the warm-up frame; non-finite output fails.
    async warmup(from, want) {
        const lo = from === undefined ? this.lo : from;
        const hidden = lo === 0 ? null : new Uint16Array(this.d.hidden);
        const t0 = now();
        try {
            const r = await this.run({ k: 'job', s: WARMUP, pos: lo, past: 0, n: 1, ids: [0],
                                       opts: { temp: 0, topK: 0 } }, hidden, want);
            const out = r.at === positions(this.d.n_layer) ? this.backend.readLogits(1) : r.f32;
            for (let i = 0; i < out.length; i++) {
                if (!Number.isFinite(out[i])) {
                    throw new Error(`a warm-up pass through positions ${lo}–${r.at - 1} produced ` +
                        'non-finite output. This GPU cannot run them');
                }
            }
            const ms = now() - t0;
            const blocks = r.at - lo;
            if (this.warmups++ > 0 && !this.decoded && blocks > 0) {
                const per = ms / blocks;
                this.msPerPos = this.msPerPos === null ? per : 0.8 * this.msPerPos + 0.2 * per;
            }
            return { blocks, ms, blocksPerSec: ms > 0 ? (blocks * 1000) / ms : 0 };
        } finally {
            this.cuts.delete(WARMUP);
            this.backend.release(this.warm.slot);
            this.warm.fed = new Map();
        }
    }

    // #exit — stage.js:832-842: the session's cut, pinned at first entry.
    _exit(session, at, want) {
        let cuts = this.cuts.get(session);
        if (!cuts) this.cuts.set(session, cuts = new Map());
        const pinned = cuts.get(at);
        if (pinned !== undefined) return pinned;
        const to = Math.min(Math.max(want === undefined || want === null ? this.have : want, at + 1), this.have);
        cuts.set(at, to);
        return to;
    }

    release(session) { return this.schedule(() => this._release(session)); }

    // #release — stage.js:857-880 (idempotent).
    _release(session) {
        const frame = this.live.get(session);
        if (frame) {
            this.live.delete(session);
            this.backend.release(frame.slot);
            this.free.push(frame);
            this.counts.released++;
        }
        this.specLive.delete(session);
        this.cuts.delete(session);
        this.logs.delete(session);
        this.refused.delete(session);
        const mine = this.waiting.filter((j) => j.h.s === session);
        if (mine.length) {
            this.waiting = this.waiting.filter((j) => j.h.s !== session);
            for (const j of mine) j.reject(new Error(`session ${session} ended while it waited for a frame`));
        }
        if (this.waiting.length) this._pump();
    }

    get load() { return this._activity().w; }
    get active() { return this._activity().n; }
    get queueMs() { return now() - this.lastJobAt < ACTIVE_MS ? this.queueAvgMs : 0; }

    groups(pos) {
        const t = now();
        const out = new Map();
        for (const [s, frame] of this.live) {
            if (!this.pending.has(s) && t - (frame.lastUse || 0) >= ACTIVE_MS) continue;
            const cuts = this.cuts.get(s);
            const to = cuts ? cuts.get(pos) : undefined;
            if (to !== undefined) out.set(to, (out.get(to) || 0) + 1);
        }
        return out;
    }

    _activity() {
        const t = now();
        let n = 0, w = 0;
        for (const [s, frame] of this.live) {
            if (!this.pending.has(s) && t - (frame.lastUse || 0) >= ACTIVE_MS) continue;
            n++;
            for (const [at, to] of this.cuts.get(s) || []) w += to - at;
        }
        return { n, w };
    }

    // #evictable — stage.js:928-935: least recently used idle session.
    _evictable() {
        const t = now();
        for (const [id, frame] of this.live) {
            if (this.pending.has(id)) continue;
            if (t - (frame.lastUse || 0) >= this.idleMs) return id;
        }
        return null;
    }

    _atCapacity(what, session) {
        const err = new Error(`this peer is serving ${this.live.size} chats and has no ` +
            `${what} free for another right now; try again in a moment`);
        err.busy = true;
        this.counts.refused++;
        if (session !== undefined && session !== null) {
            const t = now();
            for (const [s, at] of this.refused) if (t - at >= REFUSED_MS) this.refused.delete(s);
            this.refused.set(session, t);
        }
        return err;
    }

    _cold(session, msg) {
        const at = this.refused.get(session);
        if (at !== undefined && now() - at < REFUSED_MS) {
            const err = new Error('an earlier job of this chat was refused here for capacity; try again in a moment');
            err.busy = true;
            return err;
        }
        this.counts.cold++;
        return new Error(msg);
    }

    _evict(id) {
        const victim = this.live.get(id);
        this.live.delete(id);
        this.backend.release(victim.slot);
        this.cuts.delete(id);
        this.logs.delete(id);
        this.specLive.delete(id);
        this.counts.evicted++;
        return victim;
    }

    // #cacheFor — stage.js:960-1021.
    _cacheFor(session, past) {
        if (session === WARMUP) return this.warm;
        const live = this.live.get(session);
        if (live) {
            this.live.delete(session);
            this.live.set(session, live);
            live.lastUse = now();
            return live;
        }
        if (this.waiting.some((j) => j.h.s === session)) throw WAIT;
        if (past > 0) throw this._cold(session, `session ${session} is no longer cached here`);
        if (this.waiting.length && this.turn !== session) throw WAIT;
        let frame = this.free.pop();
        if (!frame) {
            const oldest = this._evictable();
            if (oldest === null) throw this.waitMs > 0 ? WAIT : this._atCapacity('session', session);
            frame = this._evict(oldest);
        }
        frame.fed = new Map();
        frame.specAt = new Map();
        frame.specLost = false;
        frame.lastUse = now();
        this.live.set(session, frame);
        this.counts.admitted++;
        return frame;
    }

    // #checkFed — stage.js:1028-1091. A job continues where the block's last
    // one ended: a full-attention block may be rewound (past <= fed), a
    // recurrent (linear_attention) one only restarted (past 0). After a
    // verify of n rows from `base`, the next job may start inside it, at
    // (base, base + n] (or at base for a re-sent refused verify, `rb`): it
    // keeps past - base of those rows. A closed-loop job (`auto`) must
    // continue exactly; one behind is a duplicate (stale). Returns keep (null:
    // nothing rolled back).
    _checkFed(session, frame, at, last, past, exact, rb) {
        let keep = null;
        for (let p = Math.max(at, 1); p < last; p++) {
            const b = p - 1;
            const fed = frame.fed.get(b) || 0;
            const rc = this._kind(b) === 'linear_attention';
            const sp = frame.specAt ? frame.specAt.get(b) : undefined;
            let k = null;
            if (sp && fed === sp.base + sp.n && past < fed && (past > sp.base || (rb && past === sp.base))) {
                k = past - sp.base;
            } else if (past === 0 && !exact) {
                continue;
            } else if (rc || exact ? past === fed : past <= fed) {
                continue;
            } else if (exact && past < fed && !frame.specLost) {
                const err = new Error(`a duplicate of session ${session}'s job at ${past} ` +
                    `(block ${b} is already at ${fed})`);
                err.stale = true;
                throw err;
            } else {
                throw this._cold(session, `session ${session} is no longer cached here ` +
                    `(block ${b} holds ${fed} rows, the job continues from ${past})`);
            }
            if (keep !== null && keep !== k) {
                throw this._cold(session, `session ${session}'s blocks disagree on a rollback ` +
                    `(${keep} and ${k} rows)`);
            }
            keep = k;
        }
        return keep;
    }

    // #pagesFor — stage.js:1096-1120: pages for `tokens` positions, evicting
    // idle sessions whole; the pages themselves are taken by the pass.
    _pagesFor(session, frame, tokens) {
        const want = Math.ceil(tokens / this.pageTokens);
        const need = () => Math.max(0, want - this.backend.slotPages(frame.slot));
        if (want <= this.maxPages && need() <= this.backend.freePages() - this.reserved) {
            this.reserved += need();
            return;
        }
        for (;;) {
            const id = this._evictable();
            if (id === null || id === session) break;
            this.free.push(this._evict(id));
            if (want <= this.maxPages && need() <= this.backend.freePages() - this.reserved) {
                this.reserved += need();
                return;
            }
        }
        if (want > this.maxPages || this.nPages < want) {
            throw new Error(`the KV pool cannot fit ${tokens} tokens for session ` +
                `${session} (${this.nPages} pages of ${this.pageTokens})`);
        }
        throw this._atCapacity('KV page', session);
    }

    // #log — stage.js:1129-1150: rows handed downstream, kept for a replay.
    _log(s, at, past, rows) {
        if (s === WARMUP) return;
        const H = this.d.hidden;
        let boundaries = this.logs.get(s);
        if (!boundaries) this.logs.set(s, boundaries = new Map());
        let log = boundaries.get(at);
        if (!log) {
            const cap = Math.min(LOG_CHUNK, this.nMax);
            boundaries.set(at, log = { rows: new Uint16Array(cap * H), len: 0 });
        }
        const need = past + rows.length / H;
        if (need * H > log.rows.length) {
            let cap = log.rows.length / H;
            while (cap < need) cap = Math.min(this.nMax, cap * 2);
            const grown = new Uint16Array(cap * H);
            grown.set(log.rows);
            log.rows = grown;
        }
        log.rows.set(rows, past * H);
        log.len = need;
    }

    // #runJobs — stage.js:1155-1183.
    async _runJobs(jobs) {
        let t0 = now();
        const groups = new Map();
        this.reserved = 0;
        for (const job of jobs) {
            let plan;
            try { plan = this._prepare(job.h, job.hidden, job.want); } catch (err) {
                this._failed(job, err);
                continue;
            }
            const key = `${plan.to}:${plan.head}:${plan.filling}:${plan.spent}`;
            if (!groups.has(key)) groups.set(key, []);
            groups.get(key).push({ job, plan });
        }
        for (const group of groups.values()) {
            let results;
            try {
                results = await this._pass(group.map((g) => g.plan), group.map((g) => g.job.queuedAt), t0);
            } catch (err) {
                for (const g of group) this._failed(g.job, err);
                continue;
            } finally {
                t0 = now();
            }
            group.forEach((g, i) => {
                if ('err' in results[i]) this._failed(g.job, results[i].err);
                else g.job.resolve(results[i].value);
            });
        }
        this.reserved = 0;
    }

    _failed(job, err) {
        if (err === WAIT) this._park(job);
        else job.reject(err);
    }

    // #prepare — stage.js:1195-1308: checks a job and readies its session;
    // throws before anything changes if it cannot run.
    _prepare(h, hidden, want) {
        const d = this.d;
        const T = h.n, H = d.hidden;
        if (h.s !== WARMUP) this.lastJobAt = now();
        const at = h.pos;
        if (!this.holds(at)) {
            throw new Error(`position ${at} is not held here (this peer has ${this.lo}–${this.have - 1})`);
        }
        const to = this._exit(h.s, at, want);
        const end = to === positions(d.n_layer);
        const filling = end && !h.replay && !!h.fill;
        const head = end && !h.replay && !h.fill;
        const spent = end && !!h.replay;
        if (h.fill && h.drafts !== undefined && h.drafts !== null) throw new Error('a prefill chunk cannot carry drafts');
        if (!Number.isInteger(T) || T < 1 || T > this.tMax) {
            throw new Error(`a job of ${T} tokens is outside 1–${this.tMax}`);
        }
        if (!Number.isInteger(h.past) || h.past < 0) throw new Error(`past ${h.past} is not a position`);
        if (h.past + T > this.nMax) throw new Error(`context ${h.past + T} exceeds ${this.nMax}`);
        const gather = at === 0;
        if (gather && !(Array.isArray(h.ids) && h.ids.length === T &&
                        h.ids.every((id) => Number.isInteger(id) && id >= 0))) {
            throw new Error(`a job at position 0 needs ${T} token ids`);
        }
        const got = hidden ? hidden.length : 0;
        if (!gather && got !== T * H) throw new Error(`payload is ${got} floats, expected ${T * H}`);
        // Rows travel as half bits; f32 rows (always f16 values after a
        // block's round) are converted without loss.
        const bits = gather ? null : hidden instanceof Uint16Array ? hidden : toF16(hidden);
        const drafts = h.drafts === undefined ? null : h.drafts;
        const verify = drafts !== null && h.s !== WARMUP && !h.replay;
        if (drafts !== null && !(Array.isArray(drafts) && drafts.length >= 1
                && drafts.length === T - 1 && T <= SPEC_COLS
                && drafts.every((id) => Number.isInteger(id) && id >= 0))) {
            throw new Error(`a verify job needs 1–${SPEC_COLS - 1} draft ids, one fewer than its ${T} tokens`);
        }
        if (gather && h.ids.some((id) => id >= d.vocab)) {
            // The WebGPU gather clamps its read; here an id past the vocabulary is refused.
            throw new Error(`a job at position 0 needs ${T} token ids`);
        }
        const frame = this._cacheFor(h.s, h.past);
        const first = Math.max(at, 1), last = Math.min(to, d.n_layer + 1);
        const keep = h.s !== WARMUP ? this._checkFed(h.s, frame, at, last, h.past, !!h.auto, !!h.rb) : null;
        // the replay lease, when a linear_attention block here snapshots (a
        // verify) or rolls back (the job after one), taken before anything
        // changes so a nospec refusal leaves the session as it was
        let linear = false;
        for (let q = first; q < last; q++) {
            if (this._kind(q - 1) === 'linear_attention') { linear = true; break; }
        }
        if (linear && keep !== null && !this.specLive.has(h.s)) {
            this.counts.cold++;
            throw new Error(`session ${h.s} has no replay data here to roll back`);
        }
        if (linear && verify) this._specSlot(h.s);
        // the MTP head (stage.js:1287-1293): its KV is filled from a job
        // that carries its ids; the head takes pages for the drafts too
        const mtp = (head || filling) && !!this.mtp && !!h.mtp && h.s !== WARMUP;
        const fill = mtp && Array.isArray(h.ids) && h.ids.length === T;
        this._pagesFor(h.s, frame, mtp && head ? Math.min(this.nMax, h.past + T + SPEC_COLS) : h.past + T);
        const sampled = head && !spent ? (verify ? T : 1) : 0;
        const optsOf = (i) => (i === 0 ? h.opts : ((h.rowOpts && h.rowOpts[i - 1]) || h.opts));
        let M = sampled ? 0 : null;
        for (let i = 0; i < sampled && M !== null; i++) {
            const m = candidatesFor(optsOf(i), d.vocab);
            M = m === null ? null : Math.max(M, m);
        }
        return { h, bits, T, at, to, first, last, head, filling, spent, gather, verify, drafts,
                 frame, sampled, optsOf, M, keep, linear, mtp, fill };
    }

    // #pass — stage.js:1314-1481: one packed pass on the backend.
    async _pass(plans, queued, t0) {
        const d = this.d;
        const H = d.hidden;
        const p0 = plans[0];
        let T = 0, sampled = 0;
        for (const p of plans) {
            p.rowOff = T;
            p.sampledOff = sampled;
            T += p.T;
            sampled += p.sampled;
        }
        let M = sampled ? 0 : null;
        for (const p of plans) {
            if (!p.sampled) continue;
            M = M === null || p.M === null ? null : Math.max(M, p.M);
        }
        const jobs = plans.map((p) => ({
            slot: p.frame.slot, past: p.h.past, n: p.T, sampled: p.sampled,
            ids: p.gather || p.fill ? Int32Array.from(p.h.ids) : undefined,
            hidden: p.gather ? undefined : p.bits,
            snap: p.linear && p.verify ? 1 : 0,
            keep: p.linear && p.keep !== null ? p.keep : undefined,
            mtp: p.fill ? 1 : 0,
        }));
        const t1 = now();
        const res = await this.backend.step(jobs, p0.at, p0.to, sampled ? (M || 1) : 1);
        const t3 = now();
        this.reserved = 0;
        if (res.code !== 0) throw backendError(res);
        if (plans.length > 1) {
            this.counts.batched++;
            this.counts.batchedJobs += plans.length;
        }
        for (const p of plans) {
            if (p.h.s === WARMUP) {
                for (let q = p.first; q < p.last; q++) this.warm.fed.set(q - 1, p.h.past + p.T);
                continue;
            }
            for (let q = p.first; q < p.last; q++) {
                p.frame.fed.set(q - 1, p.h.past + p.T);
                if (p.verify) p.frame.specAt.set(q - 1, { base: p.h.past, n: p.T });
                else p.frame.specAt.delete(q - 1);
            }
        }
        if (p0.spent) return plans.map(() => ({ value: { at: p0.to } }));
        // A sampler that needs whole rows reads the logits back (the
        // reference's full-row readback, stage.js:1428-1436).
        const rows = sampled && M === null ? this.backend.readLogits(sampled) : null;
        const pass = { res, M, rows, t0, t1, t3, batch: plans.length };
        const results = [];
        for (let i = 0; i < plans.length; i++) {
            try { results.push({ value: this._finish(plans[i], queued[i], pass) }); } catch (err) { results.push({ err }); }
        }
        return results;
    }

    // #finish — stage.js:1485-1561.
    _finish(p, queuedAt, pass) {
        const d = this.d;
        const H = d.hidden;
        const { h, T, at, to, head, filling, verify, drafts, optsOf } = p;
        const tf = now();
        const ms = (a, b) => Math.round((b - a) * 100) / 100;
        const phases = { queue: ms(queuedAt, pass.t0), encode: ms(pass.t0, pass.t1), wait: ms(pass.t1, pass.t3) };
        if (pass.batch > 1) phases.batch = pass.batch;
        const timed = () => this._timed(h, queuedAt, pass.t0, pass.t3, to - at, pass.batch);
        if (filling) {
            timed();
            return { at: to, filled: true, phases };
        }
        const sampleRow = (i) => {
            const r = p.sampledOff + i;
            if (pass.rows) return sampleFromLogitsRow(pass.rows.subarray(r * d.vocab, (r + 1) * d.vocab), optsOf(i));
            const M = pass.M;
            const c = [], v = [];
            for (let m = 0; m < M; m++) { v.push(pass.res.vals[r * M + m]); c.push(pass.res.ids[r * M + m]); }
            return sampleFromCandidates(c, v, optsOf(i), d.vocab);
        };
        // #mtpAfter (stage.js:296-320): after sampling t from row a, keep that
        // row for the session and, for a loop job with speculation on, chain
        // up to SPEC_COLS - 1 drafts after t
        const mtpAfter = (a, t) => {
            if (!p.mtp) return null;
            const pos = h.past + a + 1;
            const K = h.loop && h.loop.spec && t < this.mtp.draftVocab
                ? Math.max(0, Math.min(SPEC_COLS - 1, this.nMax - pos - 1)) : 0;
            const ids = this.backend.mtpDraft(p.frame.slot, p.rowOff + a, t, pos, K);
            return K > 0 ? Array.from(ids) : null;
        };
        if (head && verify) {
            const tokens = [];
            for (let i = 0; i < T; i++) {
                const t = sampleRow(i);
                tokens.push(t);
                if (i === T - 1 || t !== drafts[i]) break;
            }
            phases.sample = ms(tf, now());
            const token = tokens[tokens.length - 1];
            const next = mtpAfter(tokens.length - 1, token);
            if (p.mtp) phases.mtp = ms(tf, now()) - phases.sample;
            timed();
            const out = { at: to, token, tokens, phases };
            if (next) out.mtp = next;
            return out;
        }
        if (head) {
            const token = sampleRow(0);
            phases.sample = ms(tf, now());
            const next = mtpAfter(T - 1, token);
            if (p.mtp) phases.mtp = ms(tf, now()) - phases.sample;
            timed();
            const out = { at: to, token, phases };
            if (next) out.mtp = next;
            return out;
        }
        const bits = pass.res.hidden.subarray(p.rowOff * H, (p.rowOff + T) * H).slice();
        this._log(h.s, to, h.past, bits);
        phases.log = ms(tf, now());
        timed();
        const out = { at: to, hidden: bits, phases };
        if (h.s === WARMUP) out.f32 = require('./f16').fromF16(bits);
        return out;
    }

    _timed(h, queuedAt, t0, t3, npos, batch) {
        if (h.s === WARMUP || h.replay) return;
        this.queueAvgMs = 0.8 * this.queueAvgMs + 0.2 * (t0 - queuedAt);
        if (h.n !== 1 || npos < 1 || batch > 1) return;
        const per = (t3 - t0) / npos;
        const over = now() - t3;
        this.msPerPos = this.decoded ? 0.9 * this.msPerPos + 0.1 * per : per;
        this.overheadMs = this.overheadMs === null ? over : 0.9 * this.overheadMs + 0.1 * over;
        this.decoded = true;
    }
}

module.exports = { Runner, WARMUP, MAX_QUEUE, MAX_SESSION_QUEUE, SPEC_COLS, PAGE_TOKENS, positions, TENSOR, LAYER_MTP };
