'use strict';
// IEEE-754 binary16 for the row hand-off between peers: the format the
// reference's web/f16.js defines (toF16 rounds to nearest, ties to even,
// clamps finite overflow and infinities to +-65504, keeps NaN as a quiet NaN;
// fromF16 is exact). The device writes the same bits (common.h half_bits).
//
// Encoding works on the binary32 fields. A binary32 value is
// (-1)^s * 1.m * 2^(E-127) with a 23-bit m. Its binary16 neighbour keeps 10
// fraction bits at exponent E-127 >= -14 (normal) and fewer below, where the
// binary16 grid is fixed at 2^-24 (subnormal). Either way the result is the
// 24-bit significand shifted right by some amount with one round-to-nearest-
// even step; adding the rounded significand to the exponent field lets a
// carry out of the fraction move the exponent up, as IEEE rounding does.
// Node 12 syntax.

const F32 = new Float32Array(1);
const U32 = new Uint32Array(F32.buffer);

const HALF_MAX = 0x7bff;       // 65504
const HALF_QNAN = 0x7e00;

// value >> shift, rounded to nearest with ties to even (shift 1..31)
function shiftRound(value, shift) {
    const kept = value >>> shift;
    const lost = value - (kept << shift) >>> 0;
    const halfway = 2 ** (shift - 1);
    if (lost > halfway || (lost === halfway && (kept & 1) === 1)) return kept + 1;
    return kept;
}

function encodeHalf(x) {
    F32[0] = x;
    const bits = U32[0];
    const sign = (bits >>> 31) << 15;
    const field = (bits >>> 23) & 0xff;
    const frac = bits & 0x7fffff;
    if (field === 0xff) return frac === 0 ? sign | HALF_MAX : sign | HALF_QNAN;
    if (field === 0) return sign;                           // binary32 subnormals are far below 2^-25
    const exp = field - 127;                                // unbiased
    if (exp > 15) return sign | HALF_MAX;
    const sig = frac | 0x800000;                            // 24-bit significand, 1.m * 2^23
    if (exp >= -14) {
        // normal: keep 10 fraction bits; the rounded significand carries
        // into the exponent field when it reaches 2^11
        const h = ((exp + 14) << 10) + shiftRound(sig, 13);
        return sign | Math.min(h, HALF_MAX);
    }
    // subnormal grid 2^-24: value / 2^-24 = sig * 2^(exp - 23 + 24)
    const shift = 13 + (-14 - exp);
    if (shift > 24) return sign;                            // below half of 2^-24
    return sign | shiftRound(sig, shift);
}

function decodeHalf(h) {
    const sign = (h & 0x8000) << 16;
    const field = (h >>> 10) & 0x1f;
    const frac = h & 0x3ff;
    if (field === 0) {
        F32[0] = frac * 5.9604644775390625e-8;              // frac * 2^-24, exact in binary32
        U32[0] |= sign;
        return F32[0];
    }
    U32[0] = field === 0x1f ? (sign | 0x7f800000 | (frac << 13)) >>> 0
                            : (sign | ((field + 112) << 23) | (frac << 13)) >>> 0;
    return F32[0];
}

// f32 values (any array-like) -> Uint16Array of half bits
function toF16(src) {
    const out = new Uint16Array(src.length);
    for (let i = 0; i < out.length; i++) out[i] = encodeHalf(src[i]);
    return out;
}

// half bits -> Float32Array of their exact values
function fromF16(bits) {
    const out = new Float32Array(bits.length);
    for (let i = 0; i < out.length; i++) out[i] = decodeHalf(bits[i]);
    return out;
}

module.exports = { toF16, fromF16, encodeHalf, decodeHalf };
