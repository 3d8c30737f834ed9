'use strict';
// Test infrastructure: a single-threaded JavaScript restatement of the decode
// pass, the CPU "JS path" baseline beside the C oracle. Only tests/ and
// bench.py's cpu_baseline run it (through oracle/jsdecode.py), never the
// product. It follows oracle/ccoracle.c function by function:
//   embedding gather + f16 round      web/model/kernels.js:905-928, 1896-1909
//   rmsnorm                           web/model/kernels.js:930-976
//   q8 matmul, per-32 group scales    web/model/kernels.js:449-804
//   store_kv (RoPE, amax, int8 codes) web/model/kernels.js:1024-1073
//   RoPE on Q                         web/model/kernels.js:1093-1129
//   scores, exact softmax, P.V        web/model/kernels.js:1140-1310
//   SwiGLU, residual adds, f16 round  web/model/model.js:307-316, 368-409
//   LM head, greedy pick              web/model/stage.js:1404-1440
// Sums run in f64 (JavaScript numbers) and are stored as f32, so results
// agree with the f32 oracle to rounding, not bit for bit.
//
//   node oracle/js/decode.js <dir> <steps>
// <dir> holds model.json and the tensors oracle/jsdecode.py writes. Prints
// one JSON line: {ms_per_step, steps, ids [step][row], top [step][row]}.
// Node 12 syntax.

const fs = require('fs');
const path = require('path');

function readBytes(file) {
    const b = fs.readFileSync(file);
    const ab = new ArrayBuffer(b.length);   // aligned copy: a pooled Buffer may sit at any offset
    new Uint8Array(ab).set(b);
    return ab;
}
const f32 = (file) => new Float32Array(readBytes(file));
const i8 = (file) => new Int8Array(readBytes(file));

// f32 -> nearest-even f16 -> f32, |x| above 65504 clamped, NaN kept
const cvt = new Float32Array(1);
const cvtBits = new Uint32Array(cvt.buffer);
function rint(v) {
    const r = Math.round(v);
    return Math.abs(v - Math.trunc(v)) === 0.5 && r % 2 !== 0 ? r - 1 : r;
}
function roundF16(v) {
    if (v !== v) return v;
    const a = Math.abs(v);
    if (a > 65504) return v > 0 ? 65504 : -65504;
    if (a < 6.103515625e-5) {                       // f16 subnormals: multiples of 2^-24
        const r = rint(a / 5.960464477539063e-8) * 5.960464477539063e-8;
        return v < 0 ? -r : r;
    }
    cvt[0] = v;
    const u = cvtBits[0];
    const lsb = (u >>> 13) & 1;
    cvtBits[0] = ((u + 0x0fff + lsb) & 0xffffe000) >>> 0;
    return cvt[0];
}

// Y[m][n] = sum over 32-groups g of S[n][g] * (X[m][g] . W[n][g])
function matmul(X, M, K, W, S, N, Y) {
    const ng = K / 32;
    for (let n = 0; n < N; n++) {
        const wo = n * K, so = n * ng;
        for (let m = 0; m < M; m++) {
            const xo = m * K;
            let acc = 0;
            for (let g = 0; g < ng; g++) {
                const k0 = g * 32;
                let s = 0;
                for (let k = 0; k < 32; k++) s += X[xo + k0 + k] * W[wo + k0 + k];
                acc += s * S[so + g];
            }
            Y[m * N + n] = acc;
        }
    }
}

function rmsnorm(x, M, H, w, eps, y) {
    for (let m = 0; m < M; m++) {
        let ss = 0;
        for (let h = 0; h < H; h++) ss += x[m * H + h] * x[m * H + h];
        const sc = 1 / Math.sqrt(ss / H + eps);
        for (let h = 0; h < H; h++) y[m * H + h] = x[m * H + h] * sc * w[h];
    }
}

// split-half RoPE of one head's D values at `off`, position pos, in place
function rope(buf, off, D, pos, tbl) {
    const half = D / 2;
    for (let i = 0; i < half; i++) {
        const c = tbl[(pos * half + i) * 2], s = tbl[(pos * half + i) * 2 + 1];
        const a = buf[off + i], b = buf[off + i + half];
        buf[off + i] = a * c - b * s;
        buf[off + i + half] = b * c + a * s;
    }
}

// A session's K or V rows of one layer: [tokens][nKV] rows of D codes, then
// D/32 f32 scales (the reference row layout, RW = D/4 + D/32 words).
function KvRows(cap, nKV, D, init) {
    const rw = D / 4 + D / 32;
    const ab = new ArrayBuffer(cap * nKV * rw * 4);
    if (init) new Uint8Array(ab).set(new Uint8Array(init));
    return { rw, codes: new Int8Array(ab), scales: new Float32Array(ab) };
}

// store_kv of one row (nKV heads of D f32 values at src[off..]) at token t
function storeRow(rows, t, nKV, D, src, off) {
    const rw = rows.rw;
    const tmp = new Float32Array(32);
    for (let n = 0; n < nKV; n++) {
        const base = (t * nKV + n) * rw;
        for (let b = 0; b < D / 32; b++) {
            let amax = 0;
            for (let j = 0; j < 32; j++) {
                tmp[j] = src[off + n * D + b * 32 + j];
                amax = Math.max(amax, Math.abs(tmp[j]));
            }
            const scale = Math.fround(amax / 127);
            const inv = scale > 0 ? Math.fround(1 / scale) : 0;
            for (let j = 0; j < 32; j++) {
                const q = rint(Math.fround(tmp[j] * inv));
                rows.codes[base * 4 + b * 32 + j] = Math.max(-127, Math.min(127, q));
            }
            rows.scales[base + D / 4 + b] = scale;
        }
    }
}

// one head's attention for one query row: scores over tokens 0..T-1, exact
// softmax, then P . V into out[oo..]
function attendHead(q, qo, K, V, T, kvh, nKV, D, out, oo, p) {
    const rw = K.rw, inv = 1 / Math.sqrt(D);
    let mx = -Infinity;
    for (let t = 0; t < T; t++) {
        const base = (t * nKV + kvh) * rw;
        let sum = 0;
        for (let b = 0; b < D / 32; b++) {
            let s = 0;
            for (let j = 0; j < 32; j++) s += q[qo + b * 32 + j] * K.codes[base * 4 + b * 32 + j];
            sum += s * K.scales[base + D / 4 + b];
        }
        p[t] = sum * inv;
        if (p[t] > mx) mx = p[t];
    }
    let tot = 0;
    for (let t = 0; t < T; t++) {
        p[t] = Math.exp(p[t] - mx);
        tot += p[t];
    }
    for (let d = 0; d < D; d++) out[oo + d] = 0;
    const acc = new Float64Array(D);
    for (let t = 0; t < T; t++) {
        const w = p[t] / tot, base = (t * nKV + kvh) * rw;
        for (let d = 0; d < D; d++) acc[d] += w * (V.codes[base * 4 + d] * V.scales[base + D / 4 + (d >> 5)]);
    }
    for (let d = 0; d < D; d++) out[oo + d] = acc[d];
}

function main() {
    const dir = process.argv[2];
    const steps = parseInt(process.argv[3] || '1', 10);
    const m = JSON.parse(fs.readFileSync(path.join(dir, 'model.json'), 'utf8'));
    const d = m.dims;
    const H = d.hidden, D = d.head_dim, nH = d.n_heads, nKV = d.n_kv_heads, F = d.ffn, Vc = d.vocab;
    const group = nH / nKV, L = d.n_layer, S = m.contexts.length;
    const t = (name) => path.join(dir, name);
    const q8 = (name) => ({ codes: i8(t(name + '.i8')), scales: f32(t(name + '.f32')) });
    const wte = q8('wte');
    const head = m.tied ? wte : q8('lm_head');
    const norm = f32(t('norm.f32'));
    const tbl = f32(t('rope.f32'));
    const layers = [];
    for (let l = 0; l < L; l++) {
        const w = {};
        for (const n of ['q', 'k', 'v', 'o', 'gate', 'up', 'down']) w[n] = q8('L' + l + '_' + n);
        w.ln1 = f32(t('L' + l + '_ln1.f32'));
        w.ln2 = f32(t('L' + l + '_ln2.f32'));
        w.K = [];
        w.V = [];
        for (let s = 0; s < S; s++) {
            const cap = m.contexts[s] + steps;
            w.K.push(KvRows(cap, nKV, D, readBytes(t('L' + l + '_K' + s + '.u32'))));
            w.V.push(KvRows(cap, nKV, D, readBytes(t('L' + l + '_V' + s + '.u32'))));
        }
        layers.push(w);
    }
    const x = new Float32Array(S * H), h = new Float32Array(S * H);
    const qb = new Float32Array(S * nH * D), kb = new Float32Array(S * nKV * D), vb = new Float32Array(S * nKV * D);
    const att = new Float32Array(S * nH * D), ob = new Float32Array(S * H);
    const gb = new Float32Array(S * F), ub = new Float32Array(S * F), dn = new Float32Array(S * H);
    const logits = new Float32Array(S * Vc);
    const pbuf = new Float64Array(Math.max.apply(null, m.contexts) + steps + 1);
    let ids = m.first_ids.slice();
    const out = { ids: [], top: [] };
    const t0 = process.hrtime.bigint();
    for (let step = 0; step < steps; step++) {
        // embedding rows, rounded to f16
        for (let s = 0; s < S; s++) {
            const v = ids[s];
            for (let c = 0; c < H; c++) {
                x[s * H + c] = roundF16(Math.fround(wte.codes[v * H + c] * wte.scales[v * (H / 32) + (c >> 5)]));
            }
        }
        for (let l = 0; l < L; l++) {
            const w = layers[l];
            rmsnorm(x, S, H, w.ln1, d.rms_eps, h);
            matmul(h, S, H, w.q.codes, w.q.scales, nH * D, qb);
            matmul(h, S, H, w.k.codes, w.k.scales, nKV * D, kb);
            matmul(h, S, H, w.v.codes, w.v.scales, nKV * D, vb);
            for (let s = 0; s < S; s++) {
                const pos = m.contexts[s] + step;
                for (let n = 0; n < nKV; n++) rope(kb, (s * nKV + n) * D, D, pos, tbl);
                storeRow(w.K[s], pos, nKV, D, kb, s * nKV * D);
                storeRow(w.V[s], pos, nKV, D, vb, s * nKV * D);
                for (let hh = 0; hh < nH; hh++) {
                    rope(qb, (s * nH + hh) * D, D, pos, tbl);
                    attendHead(qb, (s * nH + hh) * D, w.K[s], w.V[s], pos + 1, (hh / group) | 0, nKV, D, att,
                               (s * nH + hh) * D, pbuf);
                }
            }
            matmul(att, S, nH * D, w.o.codes, w.o.scales, H, ob);
            for (let i = 0; i < S * H; i++) x[i] = x[i] + ob[i];
            rmsnorm(x, S, H, w.ln2, d.rms_eps, h);
            matmul(h, S, H, w.gate.codes, w.gate.scales, F, gb);
            matmul(h, S, H, w.up.codes, w.up.scales, F, ub);
            for (let i = 0; i < S * F; i++) gb[i] = (gb[i] / (1 + Math.exp(-gb[i]))) * ub[i];
            matmul(gb, S, F, w.down.codes, w.down.scales, H, dn);
            for (let i = 0; i < S * H; i++) x[i] = roundF16(Math.fround(x[i] + dn[i]));
        }
        rmsnorm(x, S, H, norm, d.rms_eps, h);
        matmul(h, S, H, head.codes, head.scales, Vc, logits);
        const next = [], top = [];
        for (let s = 0; s < S; s++) {
            let best = 0;
            for (let v = 1; v < Vc; v++) if (logits[s * Vc + v] > logits[s * Vc + best]) best = v;
            next.push(best);
            top.push(logits[s * Vc + best]);
        }
        out.ids.push(next);
        out.top.push(top);
        if (step === 0 && m.logits_out) fs.writeFileSync(path.join(dir, m.logits_out), Buffer.from(logits.buffer));
        ids = next;
    }
    const ms = Number(process.hrtime.bigint() - t0) / 1e6;
    out.ms_per_step = ms / steps;
    out.steps = steps;
    process.stdout.write(JSON.stringify(out) + '\n');
}

main();
