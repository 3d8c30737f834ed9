'use strict';
// The message format peers exchange around a pass (web/net.js:73-207), so a
// Runner on this backend can hand its f16 rows to, and take them from, the
// reference's peers. Networking itself (signalling, WebRTC, routing) is not
// part of this build; this is the byte format on the link.
//
// A message: u32 (little-endian) length n of a UTF-8 JSON header, the header,
// zero padding to a multiple of 4, then the payload, the hidden rows as f16
// bits (f16.js rounding). A message longer than the link's limit travels as
// fragments: u32 0xFFFFFFFF, u32 message id, u32 fragment index, u32 fragment
// count, then a slice of whole 4-byte words. The receiver checks the id and
// the order and refuses a message over 32 MiB.
//
// Node 12 syntax: no ?? / ?. / #private.

const { TextEncoder, TextDecoder } = require('util');
const { toF16 } = require('./f16');

const FRAG_MARK = 0xFFFFFFFF;
const FRAG_HEAD = 16;
const WIRE_DEFAULT = 262144;              // Chrome's advertised SCTP message size
const MAX_MESSAGE = 32 * 1024 * 1024;

const padTo4 = (n) => (4 - (n % 4)) % 4;

// header: a JSON-able object; payload: Uint16Array (f16 bits, sent as they
// are), Float32Array (rounded to f16 here) or null. Returns an ArrayBuffer.
function pack(header, payload) {
    const json = new TextEncoder().encode(JSON.stringify(header));
    const start = 4 + json.length + padTo4(json.length);
    let bits = null;
    if (payload) bits = payload instanceof Uint16Array ? payload : toF16(payload);
    const buf = new ArrayBuffer(start + (bits ? bits.byteLength : 0));
    new DataView(buf).setUint32(0, json.length, true);
    new Uint8Array(buf, 4, json.length).set(json);
    if (bits) new Uint16Array(buf, start, bits.length).set(bits);
    return buf;
}

// -> {header, payload: Uint16Array of f16 bits, or null}
function unpack(buf) {
    const n = new DataView(buf).getUint32(0, true);
    const header = JSON.parse(new TextDecoder().decode(new Uint8Array(buf, 4, n)));
    const start = 4 + n + padTo4(n);
    const payload = buf.byteLength > start ? new Uint16Array(buf, start) : null;
    return { header, payload };
}

// The per-send limit of a connection (its SCTP maxMessageSize, capped at the
// default), or the default when it reports none.
function wireLimit(pc) {
    const n = pc && pc.sctp ? pc.sctp.maxMessageSize : undefined;
    return Number.isFinite(n) && n > FRAG_HEAD ? Math.min(n, WIRE_DEFAULT) : WIRE_DEFAULT;
}

// A packed message as wire-sized pieces; one that fits comes back unchanged
// in a one-element array.
function fragment(buf, limit, id) {
    if (limit === undefined) limit = WIRE_DEFAULT;
    if (buf.byteLength <= limit) return [buf];
    const body = Math.max(4, (limit - FRAG_HEAD) & ~3);
    const count = Math.ceil(buf.byteLength / body);
    const src = new Uint8Array(buf);
    const frames = new Array(count);
    for (let i = 0; i < count; i++) {
        const part = src.subarray(i * body, Math.min(src.length, (i + 1) * body));
        const frame = new ArrayBuffer(FRAG_HEAD + part.length);
        const dv = new DataView(frame);
        dv.setUint32(0, FRAG_MARK, true);
        dv.setUint32(4, (id || 0) >>> 0, true);
        dv.setUint32(8, i, true);
        dv.setUint32(12, count, true);
        new Uint8Array(frame, FRAG_HEAD).set(part);
        frames[i] = frame;
    }
    return frames;
}

// Receiving half, one `state` object per link: the whole message once its
// last fragment arrives, null before that; an unfragmented buffer unchanged.
function reassemble(state, buf) {
    if (buf.byteLength < FRAG_HEAD) return buf;
    const dv = new DataView(buf);
    if (dv.getUint32(0, true) !== FRAG_MARK) return buf;
    const id = dv.getUint32(4, true), i = dv.getUint32(8, true), count = dv.getUint32(12, true);
    if (i === 0) {
        state.id = id;
        state.count = count;
        state.parts = [];
        state.bytes = 0;
    } else if (!state.parts || state.id !== id || state.parts.length !== i) {
        state.parts = null;
        throw new Error(`fragment ${i} of message ${id} arrived out of order`);
    }
    state.bytes += buf.byteLength - FRAG_HEAD;
    if (state.bytes > MAX_MESSAGE) {
        state.parts = null;
        throw new Error(`message ${id} is over ${MAX_MESSAGE / 1048576} MiB`);
    }
    state.parts.push(new Uint8Array(buf, FRAG_HEAD));
    if (state.parts.length < state.count) return null;
    const whole = new Uint8Array(state.bytes);
    let at = 0;
    for (const p of state.parts) {
        whole.set(p, at);
        at += p.length;
    }
    state.parts = null;
    return whole.buffer;
}

module.exports = { pack, unpack, fragment, reassemble, wireLimit, FRAG_MARK, FRAG_HEAD, WIRE_DEFAULT, MAX_MESSAGE };
