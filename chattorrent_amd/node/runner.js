'use strict';
// The Runner of a peer's position range with its GPU half on the MI355X
// library (native.js, or any backend with the same methods): the drop-in for
// the reference's `new Runner(device, d, w, opts)` (web/model/stage.js:98-1578),
// keeping its API, option names, error classes and messages, and decisions.
//
// A job goes: run() -> the queue -> a pass with the queued jobs that may
// share it (policy.planBatch) -> per job, the checks (policy.checkJob), its
// session's frame (frames.js), its blocks' row counters
// (policy.continuation) and its KV pages -> one packed cc_step on the
// backend -> per job, sampling at the head (sampling.js), the verify
// acceptance, or the f16 rows handed on with their boundary log.
//
// Not here (as in the MI355X library): keep-warm kernels and GPU profiling
// hooks. Growing the held range (prepend, growLeft, growRight) is refused:
// the backend's context holds a fixed range. Node 12 syntax.

const { candidatesFor, sampleFromCandidates, sampleFromLogitsRow } = require('./sampling');
const { toF16, fromF16 } = require('./f16');
const P = require('./policy');
const { FrameTable, WAIT, now } = require('./frames');

const { LIMITS, WARMUP, positions } = P;
const MAX_QUEUE = LIMITS.maxQueue;
const MAX_SESSION_QUEUE = LIMITS.maxSessionQueue;
const SPEC_COLS = LIMITS.specCols;
const PAGE_TOKENS = LIMITS.pageTokens;

// cc_upload tensor ids (include/ccdecode.h) by HF tensor name.
const TENSOR = { q_proj: 0, k_proj: 1, v_proj: 2, o_proj: 3, gate_proj: 4, up_proj: 5, down_proj: 6,
                 input_layernorm: 7, post_attention_layernorm: 8, wte: 9, norm: 10, lm_head: 11,
                 attn_gate: 12, q_norm: 13, k_norm: 14, in_proj_q: 15, in_proj_k: 16, in_proj_v: 17,
                 in_proj_z: 18, in_proj_b: 19, in_proj_a: 20, conv1d_q: 21, conv1d_k: 22, conv1d_v: 23,
                 gate_params: 24, gated_norm: 25, out_proj: 26, enorm: 27, hnorm: 28, fc_e: 29, fc_h: 30,
                 mtp_norm: 31, embed_draft: 32, head_draft: 33 };
const LAYER_MTP = -2;
// the tensors a block position takes, by kind
const FULL_BLOCK = ['q_proj', 'k_proj', 'v_proj', 'o_proj', 'gate_proj', 'up_proj', 'down_proj',
                    'input_layernorm', 'post_attention_layernorm'];
const HYBRID_EXTRAS = ['attn_gate', 'q_norm', 'k_norm'];
const LINEAR_BLOCK = ['in_proj_q', 'in_proj_k', 'in_proj_v', 'in_proj_z', 'in_proj_b', 'in_proj_a', 'conv1d_q',
                      'conv1d_k', 'conv1d_v', 'gate_params', 'gated_norm', 'out_proj', 'gate_proj', 'up_proj',
                      'down_proj', 'input_layernorm', 'post_attention_layernorm'];
const MTP_OWN = ['enorm', 'hnorm', 'fc_e', 'fc_h', 'mtp_norm', 'embed_draft', 'head_draft'];

// Options: [name, default]; a function default reads the options seen so far.
const OPTIONS = [['lo', undefined], ['hi', undefined], ['have', (o) => o.hi], ['nMax', undefined],
                 ['tMax', undefined], ['slots', 5], ['sessions', (o) => o.slots], ['pageTokens', PAGE_TOKENS],
                 ['idleMs', LIMITS.idleMs], ['waitMs', LIMITS.waitMs], ['batchRows', LIMITS.batchRows],
                 ['specSlots', (o) => o.slots]];

// A backend status as the reference's Error classes.
function backendError(res) {
    const err = new Error(res.error || `the pass failed (status ${res.code})`);
    if (res.code === 1) err.busy = true;
    if (res.code === 3) err.stale = true;
    err.status = res.code;
    return err;
}

// What a host tensor is, kept in Runner.w instead of its bytes.
function describe(t) {
    return t && t.codes ? { q8: true, values: t.codes.length, group: t.group || 32 } : { values: t.length };
}

class Runner {
    // backend: native.js NativeBackend, created with `sessions + 1` frames
    // (frame `sessions` is the warm-up's). batchRows may go up to tMax: the
    // MI355X pass gives every row the same bits at any batch size.
    constructor(backend, d, opts) {
        const given = opts || {};
        const o = {};
        for (const [name, dflt] of OPTIONS) {
            const v = given[name];
            o[name] = v !== undefined ? v : (typeof dflt === 'function' ? dflt(o) : dflt);
        }
        Object.assign(this, { backend, d, lo: o.lo, hi: o.hi, have: o.have, nMax: o.nMax, tMax: o.tMax,
                              slots: o.slots, sessions: o.sessions, pageTokens: o.pageTokens, idleMs: o.idleMs,
                              waitMs: o.waitMs, specSlots: o.specSlots });
        this.batchRows = Math.max(1, Math.min(o.batchRows, this.tMax));
        this.maxPages = Math.ceil(this.nMax / this.pageTokens);
        this.nPages = this.slots * this.maxPages;
        this.w = { wte: null, norm: null, lm_head: null, layers: [] };
        this.frames = new FrameTable(this, this.sessions);
        this.warm = { slot: this.sessions, fed: new Map() };
        this.pending = new Map();       // session -> its jobs queued or running
        this.queue = [];                // {s, job} or {s: null, run}
        this.draining = false;
        this.refused = new Map();       // session -> when it was last refused for capacity
        this.cuts = new Map();          // session -> Map(entry position -> exit)
        this.logs = new Map();          // session -> Map(exit -> {rows, len})
        this.specLive = new Set();      // sessions holding a replay lease
        this.onIdle = [];
        this.reserved = 0;              // pages promised to the pass being prepared
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
        this.mtp = null;
    }

    // ------------------------------------------------------- what is held ---
    get live() { return this.frames.live; }
    get free() { return this.frames.free; }
    get waiting() { return this.frames.waiting; }
    get embed() { return this.lo === 0; }
    get head() { return this.hi === positions(this.d.n_layer); }
    get vramBytes() { return this.backend.stats().vramBytes; }
    holds(pos) { return pos >= this.lo && pos < this.have; }
    kind(b) { return (this.d.layer_types && this.d.layer_types[b]) || 'full_attention'; }

    _upload(layer, name, t) {
        if (t.codes) this.backend.upload(layer, TENSOR[name], t.codes, t.scales, t.group);
        else this.backend.upload(layer, TENSOR[name], t, null, undefined);
    }

    // append(weights): loads position `have` (stage.js:446-468). Tensors by
    // their HF names: q8 as {codes, scales (f16 bits or f32), group}, f32 as
    // Float32Array (node/loader.js's shapes).
    append(weights) {
        const p = this.have;
        const w = weights || {};
        const last = positions(this.d.n_layer) - 1;
        if (p >= this.hi) throw new Error(`nothing left to append: ${this.lo}–${this.hi - 1} is full`);
        if (p === 0) {
            if (!w.wte) throw new Error('position 0 is the embedding and needs wte');
            this._upload(-1, 'wte', w.wte);
            this.w.wte = describe(w.wte);
        } else if (p === last) {
            if (!w.norm) throw new Error('the last position is the head and needs norm');
            this._upload(-1, 'norm', w.norm);
            const head = w.lm_head || w.wte;
            if (head) this._upload(-1, w.lm_head ? 'lm_head' : 'wte', head);
            this.w.norm = describe(w.norm);
            this.w.lm_head = head ? describe(head) : this.w.wte;
        } else {
            const linear = this.kind(p - 1) === 'linear_attention';
            const names = linear ? LINEAR_BLOCK : this.d.hybrid ? FULL_BLOCK.concat(HYBRID_EXTRAS) : FULL_BLOCK;
            if (!w[names[0]]) throw new Error(`position ${p} is a block and needs its tensors`);
            const gap = names.find((n) => !w[n]);
            if (gap) throw new Error(`position ${p} is a block and needs ${gap}`);
            for (const n of names) this._upload(p - 1, n, w[n]);
            const layer = { kind: this.kind(p - 1) };
            for (const n of names) layer[n] = describe(w[n]);
            this.w.layers.push(layer);
        }
        this.have = p + 1;
        return this.have;
    }

    // The held range is fixed by the backend's context (cc_create's lo/hi):
    // growing it needs a new Runner over a new context.
    _fixed(what) {
        return new Error(`${what}: this Runner's positions ${this.lo}–${this.hi - 1} are fixed by its MI355X ` +
                         'context; make a new Runner for a wider range');
    }
    prepend() { throw this._fixed('prepend'); }
    growLeft() { throw this._fixed('growLeft'); }
    growRight() { throw this._fixed('growRight'); }

    // attachMtp(m) — stage.js:273-289: the MTP draft head (loader.js loadMtp's
    // tensors), held with the LM head; the backend was made with d.mtp set.
    attachMtp(m) {
        if (this.hi !== positions(this.d.n_layer)) throw new Error('the MTP head is held with the LM head');
        if (!this.d.mtp) throw new Error('the model dims carry no mtp head');
        const block = this.d.hybrid ? FULL_BLOCK.concat(HYBRID_EXTRAS) : FULL_BLOCK;
        for (const [layer, names] of [[LAYER_MTP, block], [-1, MTP_OWN]]) {
            for (const n of names) {
                if (!m[n]) throw new Error(`the MTP head needs ${n}`);
                this._upload(layer, n, m[n]);
            }
        }
        this.mtp = { draftVocab: this.d.mtp.draftVocab };
    }

    // ------------------------------------------------------------ the queue ---
    // run(h, hidden, want) — stage.js:600-621: resolves with the job's result.
    run(h, hidden, want) {
        const s = h.s;
        const mine = this.pending.get(s) || 0;
        if (mine >= MAX_SESSION_QUEUE || (!mine && this.pending.size >= MAX_QUEUE)) {
            return Promise.reject(this.refuse('queue slot', s));
        }
        this.backlog++;
        this.pending.set(s, mine + 1);
        this.activeAt = now();
        const done = () => {
            this.activeAt = now();
            this.backlog--;
            const left = this.pending.get(s) - 1;
            if (left > 0) this.pending.set(s, left);
            else this.pending.delete(s);
            this.frames.touch(s);
        };
        return new Promise((resolve, reject) => this.resubmit({ h, hidden, want, queuedAt: now(), resolve, reject }))
            .then((v) => { done(); return v; }, (e) => { done(); throw e; });
    }

    resubmit(job) { this._enqueue({ s: job.h.s, job }); }

    schedule(fn) {
        return new Promise((resolve, reject) => {
            this._enqueue({ s: null, run: () => Promise.resolve().then(fn).then(resolve, reject) });
        });
    }

    _enqueue(entry) {
        this.queue.push(entry);
        if (this.draining) return;
        this.draining = true;
        queueMicrotask(() => this._drain());
    }

    async _drain() {
        while (this.queue.length) {
            const entry = this.queue.shift();
            const work = entry.job
                ? this._runJobs([entry.job].concat(P.planBatch(entry.job, this.queue, this.batchRows)))
                : entry.run();
            try { await work; } catch (e) { /* each task settles its own promise */ }
        }
        this.draining = false;
        this.onIdle.splice(0).forEach((wake) => wake());
    }

    // ---------------------------------------------------------- sessions ---
    release(session) { return this.schedule(() => this._release(session)); }

    _release(session) {
        this.forget(session);
        this.refused.delete(session);
        this.frames.release(session);
    }

    // what a session leaves behind when its frame goes
    forget(session) {
        this.cuts.delete(session);
        this.logs.delete(session);
        this.specLive.delete(session);
    }

    refuse(what, session) {
        const err = new Error(`this peer is serving ${this.live.size} chats and has no ${what} free for another ` +
                              'right now; try again in a moment');
        err.busy = true;
        this.counts.refused++;
        if (session !== undefined && session !== null) {
            const t = now();
            for (const [s, at] of this.refused) if (t - at >= LIMITS.refusedMs) this.refused.delete(s);
            this.refused.set(session, t);
        }
        return err;
    }

    cold(session, msg) {
        const at = this.refused.get(session);
        if (at !== undefined && now() - at < LIMITS.refusedMs) {
            const err = new Error('an earlier job of this chat was refused here for capacity; try again in a moment');
            err.busy = true;
            return err;
        }
        this.counts.cold++;
        return new Error(msg);
    }

    // sessions with a job queued or used within ACTIVE_MS, and the positions
    // they cross here
    _activity() {
        const t = now();
        let n = 0, w = 0;
        const cutsBy = new Map();
        for (const [s, frame] of this.live) {
            if (!this.pending.has(s) && t - (frame.lastUse || 0) >= LIMITS.activeMs) continue;
            n++;
            const cuts = this.cuts.get(s);
            if (cuts) for (const [at, to] of cuts) w += to - at;
            if (cuts) cutsBy.set(s, cuts);
        }
        return { n, w, cutsBy };
    }
    get load() { return this._activity().w; }
    get active() { return this._activity().n; }
    get queueMs() { return now() - this.lastJobAt < LIMITS.activeMs ? this.queueAvgMs : 0; }

    // active sessions entering at `pos`, counted by the position they leave at
    groups(pos) {
        const out = new Map();
        for (const cuts of this._activity().cutsBy.values()) {
            const to = cuts.get(pos);
            if (to !== undefined) out.set(to, (out.get(to) || 0) + 1);
        }
        return out;
    }

    // the exit of `session`'s passes entering at `at`, fixed by its first one
    _exit(session, at, want) {
        if (!this.cuts.has(session)) this.cuts.set(session, new Map());
        const cuts = this.cuts.get(session);
        if (!cuts.has(at)) cuts.set(at, P.cutFor(at, want, this.have));
        return cuts.get(at);
    }

    // The session's replay lease, taken on its first verify through a
    // linear_attention block here (stage.js:336-386): with every lease held,
    // an idle session's is taken (it loses its rollback) or the job is
    // refused nospec.
    _lease(session) {
        if (this.specLive.has(session)) return;
        if (this.specLive.size >= this.specSlots) {
            const t = now();
            const donor = Array.from(this.live).find(([id, frame]) => this.specLive.has(id) && !this.pending.has(id)
                && t - (frame.lastUse || 0) >= this.idleMs);
            if (!donor) {
                this.counts.nospec++;
                const err = new Error(`no speculative replay slot here (${this.specSlots} in use)`);
                err.nospec = true;
                throw err;
            }
            this.specLive.delete(donor[0]);
            if (donor[1].specAt) donor[1].specAt.clear();
            donor[1].specLost = true;
        }
        this.specLive.add(session);
    }

    // KV pages for `tokens` positions (stage.js:1093-1120): promised to this
    // pass now and taken on the device by it; idle sessions are evicted whole
    // to make room.
    _pages(session, frame, tokens) {
        const want = Math.ceil(tokens / this.pageTokens);
        const fits = () => {
            const need = Math.max(0, want - this.backend.slotPages(frame.slot));
            if (want > this.maxPages || need > this.backend.freePages() - this.reserved) return false;
            this.reserved += need;
            return true;
        };
        if (fits()) return;
        for (let victim = this.frames.evictable(); victim !== null && victim !== session;
             victim = this.frames.evictable()) {
            this.free.push(this.frames.evict(victim));
            if (fits()) return;
        }
        if (want > this.maxPages || this.nPages < want) {
            throw new Error(`the KV pool cannot fit ${tokens} tokens for session ${session} ` +
                            `(${this.nPages} pages of ${this.pageTokens})`);
        }
        throw this.refuse('KV page', session);
    }

    // Rows handed downstream at `at`, kept per session for a replay
    // (stage.js:1122-1150): one growing buffer per exit, doubling up to nMax.
    _log(s, at, past, rows) {
        if (s === WARMUP) return;
        const H = this.d.hidden;
        if (!this.logs.has(s)) this.logs.set(s, new Map());
        const bySession = this.logs.get(s);
        if (!bySession.has(at)) {
            bySession.set(at, { rows: new Uint16Array(Math.min(LIMITS.logChunk, this.nMax) * H), len: 0 });
        }
        const log = bySession.get(at);
        const len = past + rows.length / H;
        let cap = log.rows.length / H;
        if (len > cap) {
            while (cap < len) cap = Math.min(this.nMax, cap * 2);
            const grown = new Uint16Array(cap * H);
            grown.set(log.rows);
            log.rows = grown;
        }
        log.rows.set(rows, past * H);
        log.len = len;
    }

    // ------------------------------------------------------------ warm-up ---
    // warmup(from, want) — stage.js:783-821: one row through the held
    // positions in the warm-up frame; non-finite output fails.
    async warmup(from, want) {
        const lo = from === undefined ? this.lo : from;
        const t0 = now();
        try {
            const r = await this.run({ k: 'job', s: WARMUP, pos: lo, past: 0, n: 1, ids: [0], opts: { temp: 0, topK: 0 } },
                                     lo === 0 ? null : new Uint16Array(this.d.hidden), want);
            const out = r.at === positions(this.d.n_layer) ? this.backend.readLogits(1) : r.f32;
            if (!out.every((v) => Number.isFinite(v))) {
                throw new Error(`a warm-up pass through positions ${lo}–${r.at - 1} produced non-finite output. ` +
                                'This GPU cannot run them');
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

    // --------------------------------------------------------------- a pass ---
    // The jobs of one dequeued batch (stage.js:1155-1183): each is prepared
    // (a failure settles only that job); jobs that agree on where the pass
    // ends and what it does there run as one backend step.
    async _runJobs(jobs) {
        let t0 = now();
        this.reserved = 0;
        const passes = new Map();
        for (const job of jobs) {
            let plan;
            try {
                plan = this._prepare(job.h, job.hidden, job.want);
            } catch (err) {
                this._settleFailure(job, err);
                continue;
            }
            const key = [plan.to, plan.head, plan.filling, plan.spent].join(':');
            if (!passes.has(key)) passes.set(key, []);
            passes.get(key).push({ job, plan });
        }
        for (const members of passes.values()) {
            let results = null;
            try {
                results = await this._pass(members.map((m) => m.plan), members.map((m) => m.job.queuedAt), t0);
            } catch (err) {
                members.forEach((m) => this._settleFailure(m.job, err));
            }
            t0 = now();
            if (results) {
                members.forEach((m, i) => ('err' in results[i] ? this._settleFailure(m.job, results[i].err)
                                                               : m.job.resolve(results[i].value)));
            }
        }
        this.reserved = 0;
    }

    _settleFailure(job, err) {
        if (err === WAIT) this.frames.park(job);
        else job.reject(err);
    }

    // A job's plan for the pass (stage.js:1195-1308); throws before anything
    // changes if the job cannot run.
    _prepare(h, hidden, want) {
        const d = this.d;
        if (h.s !== WARMUP) this.lastJobAt = now();
        const at = h.pos;
        if (!this.holds(at)) {
            throw new Error(`position ${at} is not held here (this peer has ${this.lo}–${this.have - 1})`);
        }
        const to = this._exit(h.s, at, want);
        const end = to === positions(d.n_layer);
        const gather = at === 0;
        P.checkJob({ h, hidden, gather }, this);
        const T = h.n;
        const drafts = h.drafts === undefined ? null : h.drafts;
        const verify = drafts !== null && h.s !== WARMUP && !h.replay;
        const frame = h.s === WARMUP ? this.warm : this.frames.admit(h.s, h.past);
        const first = Math.max(at, 1), last = Math.min(to, d.n_layer + 1);
        let keep = null;
        if (h.s !== WARMUP) {
            const c = P.continuation({
                session: h.s, at, last, past: h.past, exact: !!h.auto, rb: !!h.rb, specLost: frame.specLost,
                fed: (b) => frame.fed.get(b) || 0, spec: (b) => (frame.specAt ? frame.specAt.get(b) : undefined),
                recurrent: (b) => this.kind(b) === 'linear_attention',
            });
            if (c.stale) {
                const err = new Error(c.stale);
                err.stale = true;
                throw err;
            }
            if (c.cold && c.behind) throw this.cold(h.s, c.cold);
            if (c.cold) {
                this.counts.cold++;
                throw new Error(c.cold);
            }
            keep = c.keep;
        }
        let linear = false;
        for (let q = first; q < last && !linear; q++) linear = this.kind(q - 1) === 'linear_attention';
        if (linear && keep !== null && !this.specLive.has(h.s)) {
            this.counts.cold++;
            throw new Error(`session ${h.s} has no replay data here to roll back`);
        }
        if (linear && verify) this._lease(h.s);
        const head = end && !h.replay && !h.fill;
        const filling = end && !h.replay && !!h.fill;
        const spent = end && !!h.replay;
        // the MTP head fills its KV from a job that carries its ids, and takes
        // pages for the drafts too (stage.js:1287-1293)
        const mtp = (head || filling) && !!this.mtp && !!h.mtp && h.s !== WARMUP;
        const fill = mtp && Array.isArray(h.ids) && h.ids.length === T;
        this._pages(h.s, frame, mtp && head ? Math.min(this.nMax, h.past + T + SPEC_COLS) : h.past + T);
        const sampled = head && !spent ? (verify ? T : 1) : 0;
        const optsOf = (i) => (i > 0 && h.rowOpts && h.rowOpts[i - 1]) || h.opts;
        let M = sampled ? 0 : null;
        for (let i = 0; i < sampled && M !== null; i++) {
            const m = candidatesFor(optsOf(i), d.vocab);
            M = m === null ? null : Math.max(M, m);
        }
        const bits = gather ? null : hidden instanceof Uint16Array ? hidden : toF16(hidden);
        return { h, bits, T, at, to, first, last, head, filling, spent, gather, verify, drafts, frame, sampled,
                 optsOf, M, keep, linear, mtp, fill };
    }

    // One packed pass on the backend (stage.js:1314-1481): rows in job order,
    // the sampled rows' candidates (or whole logits rows when a sampler needs
    // them), then each job finished on its own.
    async _pass(plans, queued, t0) {
        const p0 = plans[0];
        let rows = 0, sampled = 0, M = 0;
        for (const p of plans) {
            Object.assign(p, { rowOff: rows, sampledOff: sampled });
            rows += p.T;
            sampled += p.sampled;
            if (p.sampled) M = M === null || p.M === null ? null : Math.max(M, p.M);
        }
        if (!sampled) M = null;
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
            const fed = p.h.s === WARMUP ? this.warm.fed : p.frame.fed;
            for (let q = p.first; q < p.last; q++) {
                fed.set(q - 1, p.h.past + p.T);
                if (p.h.s === WARMUP) continue;
                if (p.verify) p.frame.specAt.set(q - 1, { base: p.h.past, n: p.T });
                else p.frame.specAt.delete(q - 1);
            }
        }
        if (p0.spent) return plans.map(() => ({ value: { at: p0.to } }));
        const pass = { res, M, rows: sampled && M === null ? this.backend.readLogits(sampled) : null,
                       t0, t1, t3, batch: plans.length };
        return plans.map((p, i) => {
            try {
                return { value: this._finish(p, queued[i], pass) };
            } catch (err) {
                return { err };
            }
        });
    }

    // the token drawn for sampled row `i` of plan `p`
    _sample(p, i, pass) {
        const r = p.sampledOff + i;
        const V = this.d.vocab;
        if (pass.rows) return sampleFromLogitsRow(pass.rows.subarray(r * V, (r + 1) * V), p.optsOf(i));
        const ids = Array.from(pass.res.ids.slice(r * pass.M, (r + 1) * pass.M));
        const vals = Array.from(pass.res.vals.slice(r * pass.M, (r + 1) * pass.M));
        return sampleFromCandidates(ids, vals, p.optsOf(i), V);
    }

    // After sampling `token` from row `a`, the MTP head keeps that row and,
    // for a loop job with speculation on, chains drafts (stage.js:296-320).
    _draftAfter(p, a, token) {
        if (!p.mtp) return null;
        const pos = p.h.past + a + 1;
        const k = p.h.loop && p.h.loop.spec && token < this.mtp.draftVocab
            ? Math.max(0, Math.min(SPEC_COLS - 1, this.nMax - pos - 1)) : 0;
        const ids = this.backend.mtpDraft(p.frame.slot, p.rowOff + a, token, pos, k);
        return k > 0 ? Array.from(ids) : null;
    }

    // One job's result (stage.js:1485-1561).
    _finish(p, queuedAt, pass) {
        const round2 = (a, b) => Math.round((b - a) * 100) / 100;
        const phases = { queue: round2(queuedAt, pass.t0), encode: round2(pass.t0, pass.t1),
                         wait: round2(pass.t1, pass.t3) };
        if (pass.batch > 1) phases.batch = pass.batch;
        const timed = () => this._timed(p.h, queuedAt, pass.t0, pass.t3, p.to - p.at, pass.batch);
        const tf = now();
        if (p.filling) {
            timed();
            return { at: p.to, filled: true, phases };
        }
        if (p.head) {
            // a verify takes rows while each sample equals the next draft
            const tokens = [];
            for (let i = 0; i < (p.verify ? p.T : 1); i++) {
                tokens.push(this._sample(p, i, pass));
                if (!p.verify || i === p.T - 1 || tokens[i] !== p.drafts[i]) break;
            }
            phases.sample = round2(tf, now());
            const token = tokens[tokens.length - 1];
            const drafts = this._draftAfter(p, p.verify ? tokens.length - 1 : p.T - 1, token);
            if (p.mtp) phases.mtp = round2(tf, now()) - phases.sample;
            timed();
            const out = p.verify ? { at: p.to, token, tokens, phases } : { at: p.to, token, phases };
            if (drafts) out.mtp = drafts;
            return out;
        }
        const H = this.d.hidden;
        const bits = pass.res.hidden.subarray(p.rowOff * H, (p.rowOff + p.T) * H).slice();
        this._log(p.h.s, p.to, p.h.past, bits);
        phases.log = round2(tf, now());
        timed();
        const out = { at: p.to, hidden: bits, phases };
        if (p.h.s === WARMUP) out.f32 = fromF16(bits);
        return out;
    }

    // averages the router reads: queue wait, and ms per position and host
    // overhead from single-row unbatched decode passes
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
