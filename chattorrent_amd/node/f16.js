'use strict';
// f16 row hand-off format of the reference (web/f16.js:15-65): half bits,
// nearest-even, ±65504 clamp (infinities clamp too), NaN kept as a quiet NaN.
// The device produces the same bits (common.h half_bits); this is the host's
// copy for rows a caller hands in as f32.

const scratch = new DataView(new ArrayBuffer(4));
const MAXH = 0x7bff;

function halfOf(x) {
    scratch.setFloat32(0, x);
    const b = scratch.getUint32(0);
    const sign = (b >>> 16) & 0x8000;
    const ex = (b >>> 23) & 0xff;
    const man = b & 0x7fffff;
    if (ex === 0xff) return sign | (man ? 0x7e00 : MAXH);
    const e = ex - 112;   // rebias 127 -> 15
    if (e >= 0x1f) return sign | MAXH;
    if (e <= 0) {
        if (e < -10) return sign;
        const full = man | 0x800000, sh = 14 - e;
        let h = full >>> sh;
        const rest = full & ((1 << sh) - 1), half = 1 << (sh - 1);
        if (rest > half || (rest === half && (h & 1))) h++;
        return sign | h;
    }
    let h = (e << 10) | (man >>> 13);
    const rest = man & 0x1fff;
    if (rest > 0x1000 || (rest === 0x1000 && (h & 1))) h++;
    return sign | Math.min(h, MAXH);
}

function toF16(src) {
    const out = new Uint16Array(src.length);
    for (let i = 0; i < src.length; i++) out[i] = halfOf(src[i]);
    return out;
}

let values = null;
function fromF16(bits) {
    if (!values) {
        values = new Float32Array(65536);
        for (let h = 0; h < 65536; h++) {
            const s = h & 0x8000 ? -1 : 1, e = (h >>> 10) & 0x1f, m = h & 0x3ff;
            if (e === 0) values[h] = s * m * Math.pow(2, -24);
            else if (e === 0x1f) values[h] = m ? NaN : s * Infinity;
            else values[h] = s * (1 + m / 1024) * Math.pow(2, e - 15);
        }
    }
    const out = new Float32Array(bits.length);
    for (let i = 0; i < bits.length; i++) out[i] = values[bits[i]];
    return out;
}

module.exports = { toF16, fromF16 };
