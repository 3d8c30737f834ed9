'use strict';
// The reference's on-disk checkpoint, read from a directory for
// Runner.append: `manifest.json` plus concatenated-tensor files (block_NN.bin
// per block, client.bin with wte and norm, lm_head.bin when the head is
// untied, a hybrid checkpoint's MTP head in its own file). A q8 entry is an
// int8 block [N, K] followed by f32 scales [N, ceil(K/group)]; norms, conv
// weights and gate parameters are f32. The format and the refusals' messages
// are the reference's (web/model/loader.js:146-240 dims and checks, :455-525
// tensor reads, :543-671 the per-file tensor sets; tools/convert_hf.py:594-649
// writes the files). Tensors come back as host views for cc_upload: q8 as
// {codes: Int8Array, scales: Float32Array, group}, f32 as Float32Array. Only
// q8 checkpoints load: this build's matmuls read q8. Node 12 syntax.

const fs = require('fs');
const path = require('path');

// ----------------------------------------------------------------- dims ---
// [dims field, manifest key]: required numbers
const REQUIRED = [['hidden', 'hidden'], ['n_layer', 'n_layer'], ['n_heads', 'n_head'], ['n_kv_heads', 'n_kv_head'],
                  ['head_dim', 'head_dim'], ['ffn', 'ffn'], ['vocab', 'vocab']];
// [dims field, manifest key, default (a function of the manifest when it depends on it)]
const OPTIONAL = [['n_pos', 'n_pos', 2048], ['group', 'group', (m) => m.n_head / m.n_kv_head],
                  ['rms_eps', 'rms_eps', 1e-5], ['rope_theta', 'rope_theta', 10000.0],
                  ['rope_scaling', 'rope_scaling', undefined], ['model', 'model', 'unknown'], ['dtype', 'dtype', 'f32'],
                  ['rot_dim', 'rot_dim', (m) => m.head_dim]];
// Gated DeltaNet's head configuration: [linear field, manifest key]
const LINEAR = [['nK', 'linear_num_key_heads'], ['nV', 'linear_num_value_heads'], ['Dk', 'linear_key_head_dim'],
                ['Dv', 'linear_value_head_dim'], ['K4', 'linear_conv_kernel_dim']];

const present = (v) => v !== undefined && v !== null;

function dimsFromManifest(m) {
    const missing = REQUIRED.filter(([, key]) => typeof m[key] !== 'number').map(([, key]) => key);
    if (missing.length) throw new Error(`manifest is missing ${missing.join(', ')}`);
    const d = {};
    for (const [field, key] of REQUIRED) d[field] = m[key];
    for (const [field, key, dflt] of OPTIONAL) {
        d[field] = present(m[key]) ? m[key] : (typeof dflt === 'function' ? dflt(m) : dflt);
    }
    d.tied_lm_head = m.tied_lm_head !== false;
    d.layer_types = present(m.layer_types) ? m.layer_types : undefined;
    d.hybrid = !!d.layer_types && new Set(d.layer_types).size > 1;
    d.mtp = m.mtp ? { file: m.mtp.file, draftVocab: m.mtp.draft_vocab } : undefined;
    d.linear = undefined;
    if (d.hybrid) {
        const lin = {};
        for (const [field, key] of LINEAR) lin[field] = m[key];
        lin.keyDim = lin.nK * lin.Dk;
        lin.valueDim = lin.nV * lin.Dv;
        lin.group = lin.nV / lin.nK;
        d.linear = lin;
    }
    // field order as the reference's dims object lists them
    const order = ['hidden', 'n_layer', 'n_heads', 'n_kv_heads', 'head_dim', 'ffn', 'vocab', 'n_pos', 'group', 'rms_eps',
                   'rope_theta', 'rope_scaling', 'tied_lm_head', 'model', 'dtype', 'layer_types', 'hybrid', 'rot_dim',
                   'mtp', 'linear'];
    const out = {};
    for (const k of order) out[k] = d[k];
    return out;
}

// --------------------------------------------------------------- checks ---
// Each rule: when it applies and what it says (the reference's wording).
const RULES = [
    { bad: (m) => m.weight_layout !== 'out_in',
      say: (m) => `weight_layout ${m.weight_layout}, expected out_in ` +
                  '(matmul_nobias computes X @ W^T and consumes [out, in] directly)' },
    { bad: (m) => m.norm && m.norm !== 'rmsnorm', say: (m) => `norm ${m.norm}, but only rmsnorm is implemented` },
    { bad: (m) => m.act && m.act !== 'silu', say: (m) => `act ${m.act}, but only silu/SwiGLU is implemented` },
    { bad: (m, d) => d.dtype !== 'q8', say: (m, d) => `dtype ${d.dtype}, but this build's matmuls read q8 weights` },
    { bad: (m, d) => d.hybrid && d.linear.nV % d.linear.nK !== 0,
      say: (m, d) => `linear_num_value_heads (${d.linear.nV}) not divisible by linear_num_key_heads ` +
                     `(${d.linear.nK}): l2NormalizeHeads' integer group factor needs this` },
    { bad: (m, d) => !d.hybrid && d.n_heads * d.head_dim !== d.hidden,
      say: (m, d) => `n_head*head_dim (${d.n_heads * d.head_dim}) != hidden (${d.hidden})` },
    { bad: (m, d) => d.n_heads % d.n_kv_heads !== 0,
      say: (m, d) => `n_head (${d.n_heads}) not divisible by n_kv_head (${d.n_kv_heads})` },
    { bad: (m, d) => d.head_dim % 2 !== 0,
      say: (m, d) => `head_dim (${d.head_dim}) must be even for RoPE's split-half pairing` },
    { bad: (m) => !!m.rope_scaling && ropeScalingMissing(m).length > 0,
      say: (m) => `rope_scaling is missing ${ropeScalingMissing(m).join(', ')}` },
];

function ropeScalingMissing(m) {
    return ['factor', 'low_freq_factor', 'high_freq_factor', 'original_max_position_embeddings']
        .filter((k) => typeof m.rope_scaling[k] !== 'number');
}

// The manifest's problems (empty when this build can run it).
function checkManifest(m, d) {
    const dims = d || dimsFromManifest(m);
    return RULES.filter((r) => r.bad(m, dims)).map((r) => r.say(m, dims));
}

// --------------------------------------------------------- tensor shapes ---
function blockShapes(d, kind) {
    const H = d.hidden, F = d.ffn, kv = d.n_kv_heads * d.head_dim, q = d.n_heads * d.head_dim;
    const mlp = { gate_proj: [F, H], up_proj: [F, H], down_proj: [H, F] };
    const norms = { input_layernorm: [H], post_attention_layernorm: [H] };
    if (kind === 'linear_attention') {
        const L = d.linear;
        return Object.assign({}, norms, {
            in_proj_q: [L.keyDim, H], in_proj_k: [L.keyDim, H], in_proj_v: [L.valueDim, H], in_proj_z: [L.valueDim, H],
            in_proj_b: [L.nV, H], in_proj_a: [L.nV, H],
            conv1d_q: [L.keyDim, L.K4], conv1d_k: [L.keyDim, L.K4], conv1d_v: [L.valueDim, L.K4],
            gate_params: [2 * L.nV], gated_norm: [L.Dv], out_proj: [H, L.valueDim],
        }, mlp);
    }
    const shapes = Object.assign({}, norms, { q_proj: [q, H], k_proj: [kv, H], v_proj: [kv, H], o_proj: [H, q] }, mlp);
    if (d.hybrid) Object.assign(shapes, { attn_gate: [q, H], q_norm: [d.head_dim], k_norm: [d.head_dim] });
    return shapes;
}

const kindOf = (d, index) => (d.layer_types && d.layer_types[index]) || 'full_attention';
const sameShape = (a, b) => a.length === b.length && a.every((v, i) => v === b[i]);

// ---------------------------------------------------------- tensor reads ---
// One entry's host view, after the checks its kind needs.
const READERS = {
    q8(ab, base, e, shape, where) {
        if (e.scales_offset === undefined || !e.group) throw new Error(`${where} is q8 but carries no scales/group`);
        if (e.offset % 4 || e.scales_offset % 4) {
            throw new Error(`${where} q8 offsets ${e.offset}/${e.scales_offset} are not 4-byte aligned`);
        }
        const want = shape[0] * Math.ceil(shape[1] / e.group) * 4;
        if (e.scales_size !== want) {
            throw new Error(`${where} scales are ${e.scales_size} bytes, expected ${want} for [${shape}] at group ${e.group}`);
        }
        return { codes: new Int8Array(ab, base + e.offset, e.size),
                 scales: new Float32Array(ab, base + e.scales_offset, e.scales_size / 4), group: e.group };
    },
    f32(ab, base, e, shape, where) {
        if (e.offset % 4 || e.size % 4) throw new Error(`${where} offset ${e.offset}/size ${e.size} not aligned to f32`);
        return new Float32Array(ab, base + e.offset, e.size / 4);
    },
};

// The tensors `expected` names (name -> shape) from one file's bytes and its
// manifest entries. strict (the default): the file holds nothing else.
function readTensors(buf, entries, filename, expected, opts) {
    const strict = !opts || opts.strict !== false;
    const index = {};
    for (const e of entries) index[e.name] = e;
    const out = {};
    for (const [name, shape] of Object.entries(expected)) {
        const e = index[name];
        if (!e) throw new Error(`${filename}: no tensor named ${name}`);
        const where = `${filename}:${name}`;
        if (!sameShape(e.shape, shape)) throw new Error(`${where} shape [${e.shape}], expected [${shape}]`);
        const dtype = present(e.dtype) ? e.dtype : 'f32';
        const read = READERS[dtype];
        if (!read) throw new Error(`${where} is ${dtype}; this build reads q8 projections and f32 norms`);
        out[name] = read(buf.buffer, buf.byteOffset, e, shape, where);
    }
    const extra = strict ? entries.find((e) => !(e.name in expected)) : undefined;
    if (extra) throw new Error(`${filename}: unexpected tensor ${extra.name}`);
    return out;
}

// ------------------------------------------------------------ the files ---
const blockFile = (index) => `block_${String(index).padStart(2, '0')}.bin`;

class Checkpoint {
    constructor(dir, manifest) {
        this.dir = dir;
        this.manifest = manifest || JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
        this.dims = dimsFromManifest(this.manifest);
    }

    // a file's bytes with a 4-byte-aligned start (the typed views need it)
    bytes(filename) {
        const b = fs.readFileSync(path.join(this.dir, filename));
        if (b.byteOffset % 4 === 0) return b;
        const copy = new Uint8Array(b.length);
        copy.set(b);
        return copy;
    }

    read(filename, expected) {
        return readTensors(this.bytes(filename), this.manifest.files[filename], filename, expected);
    }

    // block `index` (model numbering)
    block(index) {
        return this.read(blockFile(index), blockShapes(this.dims, kindOf(this.dims, index)));
    }

    // wte and norm, and lm_head when untied
    client() {
        const d = this.dims;
        const out = this.read('client.bin', { wte: [d.vocab, d.hidden], norm: [d.hidden] });
        if (!d.tied_lm_head) out.lm_head = this.read('lm_head.bin', { lm_head: [d.vocab, d.hidden] }).lm_head;
        return out;
    }

    // the MTP head: its full-attention block's tensors and its own
    mtp() {
        const d = this.dims;
        if (!d.mtp) throw new Error('the checkpoint has no MTP head');
        const H = d.hidden, V = d.mtp.draftVocab;
        return this.read(d.mtp.file, Object.assign(blockShapes(d), {
            enorm: [H], hnorm: [H], fc_e: [H, H], fc_h: [H, H], mtp_norm: [H], embed_draft: [V, H], head_draft: [V, H],
        }));
    }

    // what Runner.append takes at position p (0 the embedding, 1..n_layer
    // the blocks, n_layer + 1 the head); `client` reuses a client() result
    weightsFor(p, client) {
        if (p === 0 || p === this.dims.n_layer + 1) return client || this.client();
        return this.block(p - 1);
    }
}

// The module's function form, over a Checkpoint for each call.
const open = (dir, m) => new Checkpoint(dir, m);
const loadManifest = (dir) => open(dir).manifest;
const loadBlock = (dir, m, d, index) => open(dir, m).block(index);
const loadClient = (dir, m) => open(dir, m).client();
const loadMtp = (dir, m) => open(dir, m).mtp();
const weightsFor = (dir, m, d, p, client) => open(dir, m).weightsFor(p, client);

module.exports = { Checkpoint, loadManifest, dimsFromManifest, checkManifest, blockShapes, readTensors, loadBlock,
                   loadClient, loadMtp, weightsFor, blockFile };
