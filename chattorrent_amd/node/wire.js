'use strict';
// The byte format peers exchange around a pass, so a Runner on this backend
// can hand its f16 rows to the reference's peers and take theirs
// (web/net.js:73-207 defines it; networking itself is not part of this build).
//
// Message:   u32le n | n bytes of UTF-8 JSON header | zeros to a 4-byte
//            boundary | payload: the hidden rows as f16 bits
// Fragment:  u32le 0xFFFFFFFF | u32le message id | u32le index | u32le count |
//            a slice of the message, a whole number of 4-byte words except
//            for the last
// A message larger than the link's per-send limit travels as fragments; a
// receiver rebuilds it, refusing fragments out of order and any message
// over 32 MiB. Node 12 syntax.

const { TextEncoder, TextDecoder } = require('util');
const { toF16 } = require('./f16');

const FRAG_MARK = 0xFFFFFFFF;
const FRAG_HEAD = 16;
const WIRE_DEFAULT = 262144;              // the per-send limit browsers advertise for a data channel
const MAX_MESSAGE = 32 * 1024 * 1024;

const utf8 = new TextEncoder();
const fromUtf8 = new TextDecoder();
const aligned = (n) => (n + 3) & ~3;

// Message <-> {header, payload}. The payload goes out as half bits: a
// Uint16Array as it is, a Float32Array (or any numbers) rounded by f16.js.
const codec = {
    encode(header, payload) {
        const text = utf8.encode(JSON.stringify(header));
        const bodyAt = 4 + aligned(text.length);
        const half = payload ? (payload instanceof Uint16Array ? payload : toF16(payload)) : null;
        const out = new Uint8Array(bodyAt + (half ? half.byteLength : 0));
        new DataView(out.buffer).setUint32(0, text.length, true);
        out.set(text, 4);
        if (half) out.set(new Uint8Array(half.buffer, half.byteOffset, half.byteLength), bodyAt);
        return out.buffer;
    },
    // -> {header, payload: Uint16Array view of the half bits, or null}
    decode(buf) {
        const n = new DataView(buf).getUint32(0, true);
        const header = JSON.parse(fromUtf8.decode(new Uint8Array(buf, 4, n)));
        const bodyAt = 4 + aligned(n);
        return { header, payload: buf.byteLength > bodyAt ? new Uint16Array(buf, bodyAt) : null };
    },
};

// A link's per-send limit: its SCTP maxMessageSize, at most WIRE_DEFAULT,
// or WIRE_DEFAULT when it reports none usable.
function wireLimit(pc) {
    const reported = pc && pc.sctp ? pc.sctp.maxMessageSize : undefined;
    if (!Number.isFinite(reported) || reported <= FRAG_HEAD) return WIRE_DEFAULT;
    return Math.min(reported, WIRE_DEFAULT);
}

// Sending half: the pieces of one message for a link of limit `limit`; a
// message that fits is the only piece, unchanged.
function fragment(buf, limit, id) {
    const cap = limit === undefined ? WIRE_DEFAULT : limit;
    if (buf.byteLength <= cap) return [buf];
    const step = Math.max(4, (cap - FRAG_HEAD) & ~3);
    const src = new Uint8Array(buf);
    const count = Math.ceil(src.length / step);
    const pieces = [];
    for (let at = 0, index = 0; at < src.length; at += step, index++) {
        const slice = src.subarray(at, Math.min(src.length, at + step));
        const piece = new Uint8Array(FRAG_HEAD + slice.length);
        const head = new DataView(piece.buffer);
        [FRAG_MARK, (id || 0) >>> 0, index, count].forEach((v, k) => head.setUint32(4 * k, v, true));
        piece.set(slice, FRAG_HEAD);
        pieces.push(piece.buffer);
    }
    return pieces;
}

// Receiving half, one per link: push() each buffer as it arrives; it returns
// the whole message when one is complete (an unfragmented buffer at once)
// and null while fragments are still due.
class Reassembler {
    constructor() {
        this.id = 0;
        this.count = 0;
        this.parts = null;
        this.bytes = 0;
    }

    push(buf) {
        if (buf.byteLength < FRAG_HEAD) return buf;
        const head = new DataView(buf);
        if (head.getUint32(0, true) !== FRAG_MARK) return buf;
        const id = head.getUint32(4, true), index = head.getUint32(8, true), count = head.getUint32(12, true);
        if (index === 0) {
            this.id = id;
            this.count = count;
            this.parts = [];
            this.bytes = 0;
        } else if (this.parts === null || this.id !== id || this.parts.length !== index) {
            this.parts = null;
            throw new Error(`fragment ${index} of message ${id} arrived out of order`);
        }
        this.bytes += buf.byteLength - FRAG_HEAD;
        if (this.bytes > MAX_MESSAGE) {
            this.parts = null;
            throw new Error(`message ${id} is over ${MAX_MESSAGE / 1048576} MiB`);
        }
        this.parts.push(new Uint8Array(buf, FRAG_HEAD));
        if (this.parts.length < this.count) return null;
        const whole = new Uint8Array(this.bytes);
        this.parts.reduce((at, p) => { whole.set(p, at); return at + p.length; }, 0);
        this.parts = null;
        return whole.buffer;
    }
}

const pack = (header, payload) => codec.encode(header, payload);
const unpack = (buf) => codec.decode(buf);

module.exports = { pack, unpack, fragment, Reassembler, wireLimit, FRAG_MARK, FRAG_HEAD, WIRE_DEFAULT, MAX_MESSAGE };
