'use strict';
// Session frames of a Runner: which sessions hold one of the backend's page
// tables, in least-recently-used order, and the sessions waiting for one.
// The admission rules are the reference's (web/model/stage.js:730-775 wait
// and wake, :915-1021 eviction and admission): a session keeps its frame
// while it has jobs or has been used within idleMs; a new session takes a
// free frame, or the least recently used idle one, or waits (up to waitMs)
// in arrival order, and the waiting sessions are let in one at a time.
// Node 12 syntax.

const now = () => Number(process.hrtime.bigint()) / 1e6;

// Thrown by FrameTable.admit for a job that must wait; the Runner parks it.
const WAIT = new Error('waiting for a session frame');

class FrameTable {
    // owner: {backend, pending (Map session -> jobs), counts, idleMs, waitMs,
    // refuse(what, session) -> Error, cold(session, msg) -> Error,
    // forget(session) (drops its cuts, logs and replay lease),
    // resubmit(job), schedule(fn)}; frames: how many sessions fit at once.
    constructor(owner, frames) {
        this.owner = owner;
        this.free = [];
        for (let slot = frames - 1; slot >= 0; slot--) this.free.push({ slot });
        this.live = new Map();        // session -> frame, least recently used first
        this.waiting = [];            // parked jobs, in arrival order
        this.turn = null;             // the waiting session being let in
        this.timer = undefined;
    }

    touch(session) {
        const frame = this.live.get(session);
        if (frame) frame.lastUse = now();
    }

    idleFor(session, frame, t) {
        return !this.owner.pending.has(session) && t - (frame.lastUse || 0) >= this.owner.idleMs;
    }

    // the least recently used session that may be evicted, or null
    evictable() {
        const t = now();
        for (const [session, frame] of this.live) if (this.idleFor(session, frame, t)) return session;
        return null;
    }

    // takes `session`'s frame away (its pages go back to the pool)
    evict(session) {
        const frame = this.live.get(session);
        this.live.delete(session);
        this.owner.backend.release(frame.slot);
        this.owner.forget(session);
        this.owner.counts.evicted++;
        return frame;
    }

    // The frame a job of `session` at `past` runs in. Throws WAIT when the
    // job must wait for one, or the Runner's capacity / cold errors.
    admit(session, past) {
        const held = this.live.get(session);
        if (held) {
            this.live.delete(session);      // now the most recently used
            this.live.set(session, held);
            held.lastUse = now();
            return held;
        }
        if (this.waiting.some((j) => j.h.s === session)) throw WAIT;
        if (past > 0) throw this.owner.cold(session, `session ${session} is no longer cached here`);
        if (this.waiting.length && this.turn !== session) throw WAIT;
        let frame = this.free.pop();
        if (!frame) {
            const victim = this.evictable();
            if (victim === null) throw this.owner.waitMs > 0 ? WAIT : this.owner.refuse('session', session);
            frame = this.evict(victim);
        }
        Object.assign(frame, { fed: new Map(), specAt: new Map(), specLost: false, lastUse: now() });
        this.live.set(session, frame);
        this.owner.counts.admitted++;
        return frame;
    }

    // ends `session`'s frame, if it has one; its waiting jobs are refused
    release(session) {
        const frame = this.live.get(session);
        if (frame) {
            this.live.delete(session);
            this.owner.backend.release(frame.slot);
            this.free.push(frame);
            this.owner.counts.released++;
        }
        const mine = this.waiting.filter((j) => j.h.s === session);
        if (mine.length) {
            this.waiting = this.waiting.filter((j) => j.h.s !== session);
            for (const j of mine) j.reject(new Error(`session ${session} ended while it waited for a frame`));
        }
        if (this.waiting.length) this.wake();
    }

    // A job that must wait: first time, it joins the back of the line with a
    // deadline; a job let in that had to wait again goes back behind its
    // session's other jobs at the front.
    park(job) {
        if (job.deadline === undefined) {
            job.deadline = now() + this.owner.waitMs;
            this.owner.counts.waited++;
            this.waiting.push(job);
        } else {
            let at = 0;
            while (at < this.waiting.length && this.waiting[at].h.s === job.h.s) at++;
            this.waiting.splice(at, 0, job);
        }
        if (this.timer === undefined) {
            this.timer = setInterval(() => this.wake(), Math.max(5, Math.min(250, this.owner.idleMs / 4)));
        }
    }

    // Refuses the jobs past their deadline, then, when no session is being
    // let in and a frame can be had, lets the first waiting session's jobs
    // run; its turn ends once they have been queued.
    wake() {
        const t = now();
        const late = this.waiting.filter((j) => t >= j.deadline);
        this.waiting = this.waiting.filter((j) => t < j.deadline);
        for (const j of late) j.reject(this.owner.refuse('session', j.h.s));
        if (!this.waiting.length) {
            clearInterval(this.timer);
            this.timer = undefined;
            return;
        }
        if (this.turn !== null || (!this.free.length && this.evictable() === null)) return;
        const session = this.waiting[0].h.s;
        const mine = this.waiting.filter((j) => j.h.s === session);
        this.waiting = this.waiting.filter((j) => j.h.s !== session);
        this.turn = session;
        for (const j of mine) this.owner.resubmit(j);
        this.owner.schedule(() => { this.turn = null; });
    }
}

module.exports = { FrameTable, WAIT, now };
