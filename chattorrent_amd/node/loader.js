'use strict';
// The reference's on-disk checkpoint, read from a directory for Runner.append
// (web/model/loader.js's loaders, over the filesystem instead of fetch, and
// handing host tensors to the C ABI instead of creating GPU buffers).
//
// A checkpoint is `manifest.json` plus concatenated-tensor files:
// block_NN.bin per block, client.bin (wte, norm) and, when the head is
// untied, lm_head.bin; a hybrid checkpoint's MTP head in its own file. A q8
// entry is an int8 block [N, K] followed by f32 scales [N, ceil(K/group)]
// (tools/convert_hf.py:594-649 pack_file); norms, conv weights and gate
// parameters are f32. Only q8 checkpoints load (this build's matmuls read q8). cc_upload repeats a group-64 scale over both 32-wide
// groups, which is exact, and keeps scales as f16.
//
// Node 12 syntax: no ?? / ?. / #private.

const fs = require('fs');
const path = require('path');

function loadManifest(dir) {
    return JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
}

const def = (v, d) => (v === undefined || v === null ? d : v);

// loader.js:146-201 dimsFromManifest (the fields this build reads).
function dimsFromManifest(m) {
    const need = ['hidden', 'n_layer', 'n_head', 'n_kv_head', 'head_dim', 'ffn', 'vocab'];
    const missing = need.filter((k) => typeof m[k] !== 'number');
    if (missing.length) throw new Error(`manifest is missing ${missing.join(', ')}`);
    const layerTypes = def(m.layer_types, undefined);
    return {
        hidden: m.hidden,
        n_layer: m.n_layer,
        n_heads: m.n_head,
        n_kv_heads: m.n_kv_head,
        head_dim: m.head_dim,
        ffn: m.ffn,
        vocab: m.vocab,
        n_pos: def(m.n_pos, 2048),
        group: def(m.group, m.n_head / m.n_kv_head),
        rms_eps: def(m.rms_eps, 1e-5),
        rope_theta: def(m.rope_theta, 10000.0),
        rope_scaling: def(m.rope_scaling, undefined),
        tied_lm_head: m.tied_lm_head !== false,
        model: def(m.model, 'unknown'),
        dtype: def(m.dtype, 'f32'),
        layer_types: layerTypes,
        hybrid: !!layerTypes && new Set(layerTypes).size > 1,
        rot_dim: def(m.rot_dim, m.head_dim),
        // the MTP draft head's file and draft rows (loader.js:181-184)
        mtp: m.mtp ? { file: m.mtp.file, draftVocab: m.mtp.draft_vocab } : undefined,
        // Gated DeltaNet's head config (loader.js:185-195)
        linear: layerTypes && new Set(layerTypes).size > 1 ? {
            nK: m.linear_num_key_heads,
            nV: m.linear_num_value_heads,
            Dk: m.linear_key_head_dim,
            Dv: m.linear_value_head_dim,
            K4: m.linear_conv_kernel_dim,
            keyDim: m.linear_num_key_heads * m.linear_key_head_dim,
            valueDim: m.linear_num_value_heads * m.linear_value_head_dim,
            group: m.linear_num_value_heads / m.linear_num_key_heads,
        } : undefined,
    };
}

// loader.js:206-240 checkManifest, plus what this build runs.
function checkManifest(m, d) {
    d = d || dimsFromManifest(m);
    const problems = [];
    if (m.weight_layout !== 'out_in')
        problems.push(`weight_layout ${m.weight_layout}, expected out_in ` +
            `(matmul_nobias computes X @ W^T and consumes [out, in] directly)`);
    if (m.norm && m.norm !== 'rmsnorm') problems.push(`norm ${m.norm}, but only rmsnorm is implemented`);
    if (m.act && m.act !== 'silu') problems.push(`act ${m.act}, but only silu/SwiGLU is implemented`);
    if (d.dtype !== 'q8') problems.push(`dtype ${d.dtype}, but this build's matmuls read q8 weights`);
    if (d.hybrid && d.linear.nV % d.linear.nK !== 0)
        problems.push(`linear_num_value_heads (${d.linear.nV}) not divisible by ` +
            `linear_num_key_heads (${d.linear.nK}): l2NormalizeHeads' integer group factor needs this`);
    if (!d.hybrid && d.n_heads * d.head_dim !== d.hidden)
        problems.push(`n_head*head_dim (${d.n_heads * d.head_dim}) != hidden (${d.hidden})`);
    if (d.n_heads % d.n_kv_heads !== 0)
        problems.push(`n_head (${d.n_heads}) not divisible by n_kv_head (${d.n_kv_heads})`);
    if (d.head_dim % 2 !== 0)
        problems.push(`head_dim (${d.head_dim}) must be even for RoPE's split-half pairing`);
    if (m.rope_scaling) {
        const need = ['factor', 'low_freq_factor', 'high_freq_factor', 'original_max_position_embeddings'];
        const missing = need.filter((k) => typeof m.rope_scaling[k] !== 'number');
        if (missing.length) problems.push(`rope_scaling is missing ${missing.join(', ')}`);
    }
    return problems;
}

// loader.js:543-590: fullAttnBlockShapes (a hybrid checkpoint's full blocks
// also carry attn_gate, q_norm, k_norm) and linearAttnBlockShapes.
function blockShapes(d, kind) {
    const H = d.hidden, kvDim = d.n_kv_heads * d.head_dim, qDim = d.n_heads * d.head_dim;
    if (kind === 'linear_attention') {
        const { keyDim, valueDim, nV, Dv, K4 } = d.linear;
        return {
            input_layernorm: [H], post_attention_layernorm: [H],
            in_proj_q: [keyDim, H], in_proj_k: [keyDim, H], in_proj_v: [valueDim, H], in_proj_z: [valueDim, H],
            in_proj_b: [nV, H], in_proj_a: [nV, H],
            conv1d_q: [keyDim, K4], conv1d_k: [keyDim, K4], conv1d_v: [valueDim, K4],
            gate_params: [2 * nV], gated_norm: [Dv], out_proj: [H, valueDim],
            gate_proj: [d.ffn, H], up_proj: [d.ffn, H], down_proj: [H, d.ffn],
        };
    }
    const shapes = {
        input_layernorm: [H],
        q_proj: [qDim, H],
        k_proj: [kvDim, H],
        v_proj: [kvDim, H],
        o_proj: [H, qDim],
        post_attention_layernorm: [H],
        gate_proj: [d.ffn, H],
        up_proj: [d.ffn, H],
        down_proj: [H, d.ffn],
    };
    if (d.hybrid) {
        shapes.attn_gate = [qDim, H];
        shapes.q_norm = [d.head_dim];
        shapes.k_norm = [d.head_dim];
    }
    return shapes;
}

const kindOf = (d, index) => (d.layer_types && d.layer_types[index]) || 'full_attention';

// uploadTensors (loader.js:455-525) without the device: the expected tensors
// of one file as host views, with its shape, alignment and size checks and
// messages. q8 → {codes: Int8Array, scales: Float32Array, group}; f32 →
// Float32Array. `strict: false` takes a subset of the file's tensors.
function readTensors(buf, entries, filename, expected, opts) {
    const strict = !opts || opts.strict !== false;
    const byName = new Map(entries.map((e) => [e.name, e]));
    const ab = buf.buffer, base = buf.byteOffset;
    const out = {};
    for (const name of Object.keys(expected)) {
        const shape = expected[name];
        const e = byName.get(name);
        if (!e) throw new Error(`${filename}: no tensor named ${name}`);
        if (e.shape.length !== shape.length || e.shape.some((v, i) => v !== shape[i]))
            throw new Error(`${filename}:${name} shape [${e.shape}], expected [${shape}]`);
        const per = def(e.dtype, 'f32');
        if (per === 'q8') {
            if (e.scales_offset === undefined || !e.group)
                throw new Error(`${filename}:${name} is q8 but carries no scales/group`);
            if (e.offset % 4 || e.scales_offset % 4)
                throw new Error(`${filename}:${name} q8 offsets ${e.offset}/${e.scales_offset} are not 4-byte aligned`);
            const ngroup = Math.ceil(shape[1] / e.group);
            if (e.scales_size !== shape[0] * ngroup * 4)
                throw new Error(`${filename}:${name} scales are ${e.scales_size} bytes, expected ` +
                    `${shape[0] * ngroup * 4} for [${shape}] at group ${e.group}`);
            out[name] = {
                codes: new Int8Array(ab, base + e.offset, e.size),
                scales: new Float32Array(ab, base + e.scales_offset, e.scales_size / 4),
                group: e.group,
            };
            continue;
        }
        if (per !== 'f32') throw new Error(`${filename}:${name} is ${per}; this build reads q8 projections and f32 norms`);
        if (e.offset % 4 || e.size % 4)
            throw new Error(`${filename}:${name} offset ${e.offset}/size ${e.size} not aligned to f32`);
        out[name] = new Float32Array(ab, base + e.offset, e.size / 4);
    }
    if (strict) {
        for (const e of entries) {
            if (!(e.name in expected)) throw new Error(`${filename}: unexpected tensor ${e.name}`);
        }
    }
    return out;
}

// A file's bytes, in an ArrayBuffer whose start is 4-byte aligned (the typed
// array views above need it).
function readFile(dir, filename) {
    const b = fs.readFileSync(path.join(dir, filename));
    if (b.byteOffset % 4 === 0) return b;
    const copy = new Uint8Array(new ArrayBuffer(b.length));
    copy.set(b);
    return copy;
}

const blockFile = (index) => `block_${String(index).padStart(2, '0')}.bin`;

// loader.js:610-626 loadBlock: block `index` (model numbering).
function loadBlock(dir, m, d, index) {
    const fn = blockFile(index);
    return readTensors(readFile(dir, fn), m.files[fn], fn, blockShapes(d, kindOf(d, index)));
}

// loader.js:628-638 loadMtp: the MTP head's block and its own tensors, for
// Runner.attachMtp.
function loadMtp(dir, m, d) {
    if (!d.mtp) throw new Error('the checkpoint has no MTP head');
    const fn = d.mtp.file, H = d.hidden, V = d.mtp.draftVocab;
    const shapes = Object.assign({}, blockShapes(d), { enorm: [H], hnorm: [H], fc_e: [H, H], fc_h: [H, H],
                                                       mtp_norm: [H], embed_draft: [V, H], head_draft: [V, H] });
    return readTensors(readFile(dir, fn), m.files[fn], fn, shapes);
}

// loader.js:644-671 loadClient: wte and norm, and lm_head when untied.
function loadClient(dir, m, d) {
    const out = readTensors(readFile(dir, 'client.bin'), m.files['client.bin'], 'client.bin',
        { wte: [d.vocab, d.hidden], norm: [d.hidden] });
    if (!d.tied_lm_head) {
        const head = readTensors(readFile(dir, 'lm_head.bin'), m.files['lm_head.bin'], 'lm_head.bin',
            { lm_head: [d.vocab, d.hidden] });
        out.lm_head = head.lm_head;
    }
    return out;
}

// The weights Runner.append takes at position p (0 the embedding, 1..n_layer
// the blocks, n_layer + 1 the head).
function weightsFor(dir, m, d, p, client) {
    if (p === 0 || p === d.n_layer + 1) return client || loadClient(dir, m, d);
    return loadBlock(dir, m, d, p - 1);
}

module.exports = { loadManifest, dimsFromManifest, checkManifest, blockShapes, readTensors, loadBlock, loadClient,
                   loadMtp, weightsFor, blockFile };
