'use strict';
// node/wire.js: the peers' message format (web/net.js:73-207): pack/unpack
// round trips, f32 payloads rounded like f16.js, fragmentation of a prefill
// chunk's rows at the SCTP limit and their reassembly, and the refusals.
const assert = require('assert');
const wire = require('../../chattorrent_amd/node/wire');
const { toF16 } = require('../../chattorrent_amd/node/f16');

let n = 0;
const test = (name, fn) => { fn(); n++; };

test('the bytes of a small message and its fragments, written out by hand', () => {
    // header {"k":1} is 7 bytes: length 7, the text, one zero byte of
    // padding, then the payload's half bits little-endian (1.0 = 0x3c00,
    // -2.0 = 0xc000)
    const buf = wire.pack({ k: 1 }, new Float32Array([1, -2]));
    const want = [7, 0, 0, 0, 0x7b, 0x22, 0x6b, 0x22, 0x3a, 0x31, 0x7d, 0, 0x00, 0x3c, 0x00, 0xc0];
    assert.deepStrictEqual(Array.from(new Uint8Array(buf)), want);
    // the 16-byte message at a 15-byte limit: slices of max(4, (15 - 16) & ~3) = 4 bytes
    const frames = wire.fragment(buf, 15, 0x01020304);
    assert.strictEqual(frames.length, 4);
    const mark = [0xff, 0xff, 0xff, 0xff, 4, 3, 2, 1];
    frames.forEach((f, i) => assert.deepStrictEqual(Array.from(new Uint8Array(f)),
        mark.concat([i, 0, 0, 0, 4, 0, 0, 0], want.slice(4 * i, 4 * i + 4))));
    const st = new wire.Reassembler();
    const back = frames.map((f) => st.push(f));
    assert.deepStrictEqual(back.slice(0, 3), [null, null, null]);
    assert.deepStrictEqual(Array.from(new Uint8Array(back[3])), want);
});

test('header only', () => {
    const buf = wire.pack({ k: 'tok', s: 'c1', token: 42 });
    const { header, payload } = wire.unpack(buf);
    assert.deepStrictEqual(header, { k: 'tok', s: 'c1', token: 42 });
    assert.strictEqual(payload, null);
    assert.strictEqual(new DataView(buf).getUint32(0, true), JSON.stringify(header).length);
});

test('f16 bits pass unchanged, aligned after the header', () => {
    for (const extra of ['', 'x', 'xy', 'xyz']) {
        const bits = new Uint16Array(576 * 3).map((_, i) => (i * 7919) & 0x7bff);
        const buf = wire.pack({ k: 'job', pad: extra }, bits);
        const { header, payload } = wire.unpack(buf);
        assert.strictEqual(header.pad, extra);
        assert.strictEqual(payload.byteOffset % 4, 0);
        assert.deepStrictEqual(Array.from(payload), Array.from(bits));
    }
});

test('f32 payload is rounded as f16.js rounds', () => {
    const x = new Float32Array(1000).map((_, i) => Math.sin(i) * 1000 + i / 7);
    const { payload } = wire.unpack(wire.pack({ k: 'job' }, x));
    assert.deepStrictEqual(Array.from(payload), Array.from(toF16(x)));
});

test('a message that fits is not fragmented', () => {
    const buf = wire.pack({ k: 'job' }, new Uint16Array(5120));
    const frames = wire.fragment(buf);
    assert.strictEqual(frames.length, 1);
    assert.strictEqual(frames[0], buf);
    assert.strictEqual(new wire.Reassembler().push(buf), buf);
});

test('a prefill chunk fragments at the limit and reassembles', () => {
    const rows = 64, H = 5120;
    const bits = new Uint16Array(rows * H).map((_, i) => (i * 2654435761) >>> 17);
    const buf = wire.pack({ k: 'job', n: rows }, bits);
    const frames = wire.fragment(buf, wire.WIRE_DEFAULT, 77);
    assert(frames.length > 1);
    for (const f of frames) {
        assert(f.byteLength <= wire.WIRE_DEFAULT);
        assert.strictEqual(new DataView(f).getUint32(0, true), wire.FRAG_MARK);
        assert.strictEqual((f.byteLength - wire.FRAG_HEAD) % 4 === 0 || f === frames[frames.length - 1], true);
    }
    const st = new wire.Reassembler();
    let out = null;
    frames.forEach((f, i) => {
        out = st.push(f);
        if (i < frames.length - 1) assert.strictEqual(out, null);
    });
    assert.deepStrictEqual(new Uint8Array(out), new Uint8Array(buf));
    const { header, payload } = wire.unpack(out);
    assert.strictEqual(header.n, rows);
    assert.deepStrictEqual(Array.from(payload.subarray(0, 100)), Array.from(bits.subarray(0, 100)));
});

test('out-of-order and oversize fragments are refused', () => {
    const buf = wire.pack({ k: 'job' }, new Uint16Array(300000));
    const frames = wire.fragment(buf, 65536, 5);
    const st = new wire.Reassembler();
    st.push(frames[0]);
    assert.throws(() => st.push(frames[2]), /fragment 2 of message 5 arrived out of order/);
    const huge = new ArrayBuffer(wire.FRAG_HEAD + 8);
    const dv = new DataView(huge);
    dv.setUint32(0, wire.FRAG_MARK, true);
    dv.setUint32(12, 1 << 30, true);
    const st2 = new wire.Reassembler();
    st2.push(huge);
    st2.bytes = wire.MAX_MESSAGE;   // as if 32 MiB had arrived
    const next = huge.slice(0);
    new DataView(next).setUint32(8, 1, true);
    assert.throws(() => st2.push(next), /is over 32 MiB/);
});

test('wireLimit', () => {
    assert.strictEqual(wire.wireLimit(null), wire.WIRE_DEFAULT);
    assert.strictEqual(wire.wireLimit({ sctp: { maxMessageSize: 65536 } }), 65536);
    assert.strictEqual(wire.wireLimit({ sctp: { maxMessageSize: 1 << 30 } }), wire.WIRE_DEFAULT);
});

console.log(`${n} passed`);
