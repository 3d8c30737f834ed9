'use strict';
// Entry point of the Node host: new Runner(...) over the MI355X backend, the
// drop-in for the reference's `new Runner(device, d, w, opts)`
// (web/model/stage.js:107-110; engine.js:377-382 builds it).

const { Runner } = require('./runner');
const { NativeBackend } = require('./native');

// d: model dims; opts: the Runner's options plus `maxJobs` and `device`.
// The backend holds one page table per session and one for warm-up passes.
function createRunner(d, opts) {
    const o = Object.assign({ slots: 5 }, opts);
    if (o.sessions === undefined) o.sessions = o.slots;
    if (o.batchRows === undefined) o.batchRows = 32;
    const backend = new NativeBackend(d, {
        lo: o.lo, hi: o.hi, nMax: o.nMax, tMax: o.tMax, slots: o.slots, frames: o.sessions + 1,
        maxJobs: o.maxJobs || o.sessions + 1, device: o.device || 0,
    });
    return new Runner(backend, d, o);
}

// loader: the reference's on-disk checkpoint, for Runner.append (node/loader.js)
const loader = require('./loader');

module.exports = { createRunner, Runner, NativeBackend, loader };
