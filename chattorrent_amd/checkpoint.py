"""The reference's on-disk checkpoint, read into a cc_ctx.

A checkpoint is a directory holding `manifest.json` and concatenated-tensor
files (`block_NN.bin` per block, `client.bin` with `wte` and `norm`, and
`lm_head.bin` when the head is untied). The layout is the one the
reference's converter writes and its loader reads:

* manifest fields, as web/model/loader.js:146-201 dimsFromManifest maps them;
* the checks of loader.js:206-240 checkManifest;
* file entries {name, shape, offset, size, dtype} and, for q8, an int8 block
  [N, K] followed by f32 scales [N, ceil(K/group)] at scales_offset
  (tools/convert_hf.py:594-649 pack_file; loader.js:455-525 uploadTensors,
  with its shape, alignment and size checks and its error messages);
* block tensor names and shapes of loader.js:543-590 (fullAttnBlockShapes,
  with a hybrid checkpoint's attn_gate / q_norm / k_norm, and
  linearAttnBlockShapes for its Gated DeltaNet blocks), and the MTP head's
  file (loader.js:628-638 loadMtp).

Only q8 checkpoints load here (this build's matmuls read q8 weights); norms,
conv weights and gate parameters are f32 as the converter writes them. The reference's converter writes group 64 with f32 scales
(convert_hf.py:493); cc_upload repeats each scale over its 32-wide groups,
which is exact, and rounds the scale to f16, the device's scale format.
"""
import json
import mmap
import os

import numpy as np

# cc_upload tensor ids (include/ccdecode.h), by the checkpoint's names.
TENSOR = {"q_proj": 0, "k_proj": 1, "v_proj": 2, "o_proj": 3, "gate_proj": 4, "up_proj": 5, "down_proj": 6,
          "input_layernorm": 7, "post_attention_layernorm": 8, "wte": 9, "norm": 10, "lm_head": 11,
          "attn_gate": 12, "q_norm": 13, "k_norm": 14, "in_proj_q": 15, "in_proj_k": 16, "in_proj_v": 17,
          "in_proj_z": 18, "in_proj_b": 19, "in_proj_a": 20, "conv1d_q": 21, "conv1d_k": 22, "conv1d_v": 23,
          "gate_params": 24, "gated_norm": 25, "out_proj": 26, "enorm": 27, "hnorm": 28, "fc_e": 29, "fc_h": 30,
          "mtp_norm": 31, "embed_draft": 32, "head_draft": 33}
LAYER_MTP = -2


def load_manifest(path):
    with open(os.path.join(path, "manifest.json")) as f:
        return json.load(f)


def dims_from_manifest(m):
    """loader.js:146-201 dimsFromManifest, in the key names of this build's
    dims (chattorrent_amd/configs.py)."""
    need = ["hidden", "n_layer", "n_head", "n_kv_head", "head_dim", "ffn", "vocab"]
    missing = [k for k in need if not isinstance(m.get(k), (int, float)) or isinstance(m.get(k), bool)]
    if missing:
        raise ValueError(f"manifest is missing {', '.join(missing)}")
    layer_types = m.get("layer_types")
    d = dict(hidden=m["hidden"], n_layer=m["n_layer"], n_heads=m["n_head"], n_kv_heads=m["n_kv_head"],
             head_dim=m["head_dim"], ffn=m["ffn"], vocab=m["vocab"],
             rms_eps=m.get("rms_eps", 1e-5), rope_theta=m.get("rope_theta", 10000.0),
             tied=m.get("tied_lm_head") is not False, group_q8=32, dtype=m.get("dtype", "f32"),
             hybrid=bool(layer_types) and len(set(layer_types)) > 1, rot_dim=m.get("rot_dim", m["head_dim"]))
    if layer_types:
        d["layer_types"] = list(layer_types)
    if d["hybrid"]:
        # Gated DeltaNet's own head config (loader.js:185-195 d.linear)
        d.update(lin_nk=m.get("linear_num_key_heads"), lin_nv=m.get("linear_num_value_heads"),
                 lin_dk=m.get("linear_key_head_dim"), lin_dv=m.get("linear_value_head_dim"),
                 lin_conv=m.get("linear_conv_kernel_dim"))
    if m.get("mtp"):
        d["mtp_vocab"] = m["mtp"]["draft_vocab"]
        d["mtp_file"] = m["mtp"]["file"]
    if m.get("rope_scaling"):
        d["rope_scaling"] = dict(m["rope_scaling"])
    return d


def check_manifest(m, d=None):
    """loader.js:206-240 checkManifest, plus what this build runs: the list
    of problems, empty when the checkpoint loads."""
    d = d or dims_from_manifest(m)
    problems = []
    if m.get("weight_layout") != "out_in":
        problems.append(f"weight_layout {m.get('weight_layout')}, expected out_in "
                        f"(matmul_nobias computes X @ W^T and consumes [out, in] directly)")
    if m.get("norm") and m["norm"] != "rmsnorm":
        problems.append(f"norm {m['norm']}, but only rmsnorm is implemented")
    if m.get("act") and m["act"] != "silu":
        problems.append(f"act {m['act']}, but only silu/SwiGLU is implemented")
    if d["dtype"] != "q8":
        problems.append(f"dtype {d['dtype']}, but this build's matmuls read q8 weights")
    if d["hybrid"] and (not d.get("lin_nk") or not d.get("lin_nv") or d["lin_nv"] % d["lin_nk"]):
        problems.append(f"linear_num_value_heads ({d.get('lin_nv')}) not divisible by linear_num_key_heads "
                        f"({d.get('lin_nk')}): l2NormalizeHeads' integer group factor needs this")
    if not d["hybrid"] and d["n_heads"] * d["head_dim"] != d["hidden"]:
        problems.append(f"n_head*head_dim ({d['n_heads'] * d['head_dim']}) != hidden ({d['hidden']})")
    if d["n_heads"] % d["n_kv_heads"] != 0:
        problems.append(f"n_head ({d['n_heads']}) not divisible by n_kv_head ({d['n_kv_heads']})")
    if d["head_dim"] % 2 != 0:
        problems.append(f"head_dim ({d['head_dim']}) must be even for RoPE's split-half pairing")
    sc = m.get("rope_scaling")
    if sc:
        need = ["factor", "low_freq_factor", "high_freq_factor", "original_max_position_embeddings"]
        missing = [k for k in need if not isinstance(sc.get(k), (int, float))]
        if missing:
            problems.append(f"rope_scaling is missing {', '.join(missing)}")
    return problems


def block_shapes(d, kind="full_attention"):
    """loader.js:543-590 fullAttnBlockShapes (with a hybrid checkpoint's
    attn_gate, q_norm, k_norm) / linearAttnBlockShapes."""
    H, F = d["hidden"], d["ffn"]
    if kind == "linear_attention":
        kd, vd, nV = d["lin_nk"] * d["lin_dk"], d["lin_nv"] * d["lin_dv"], d["lin_nv"]
        K4 = d["lin_conv"]
        return {"input_layernorm": [H], "post_attention_layernorm": [H], "in_proj_q": [kd, H], "in_proj_k": [kd, H],
                "in_proj_v": [vd, H], "in_proj_z": [vd, H], "in_proj_b": [nV, H], "in_proj_a": [nV, H],
                "conv1d_q": [kd, K4], "conv1d_k": [kd, K4], "conv1d_v": [vd, K4], "gate_params": [2 * nV],
                "gated_norm": [d["lin_dv"]], "out_proj": [H, vd], "gate_proj": [F, H], "up_proj": [F, H],
                "down_proj": [H, F]}
    kv, q = d["n_kv_heads"] * d["head_dim"], d["n_heads"] * d["head_dim"]
    out = {"input_layernorm": [H], "q_proj": [q, H], "k_proj": [kv, H], "v_proj": [kv, H], "o_proj": [H, q],
           "post_attention_layernorm": [H], "gate_proj": [F, H], "up_proj": [F, H], "down_proj": [H, F]}
    if d.get("hybrid"):
        out.update(attn_gate=[q, H], q_norm=[d["head_dim"]], k_norm=[d["head_dim"]])
    return out


def kind_of(d, index):
    lt = d.get("layer_types")
    return lt[index] if lt else "full_attention"


def read_tensors(path, filename, entries, expected, strict=True):
    """uploadTensors (loader.js:455-525) without the device: each expected
    tensor as an f32 array, or for q8 as (codes int8 [N, K], scales f32
    [N, ceil(K/group)], group). Views over a read-only map of the file."""
    by_name = {e["name"]: e for e in entries}
    with open(os.path.join(path, filename), "rb") as f:
        blob = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    out = {}
    for name, shape in expected.items():
        e = by_name.get(name)
        if e is None:
            raise ValueError(f"{filename}: no tensor named {name}")
        if list(e["shape"]) != list(shape):
            raise ValueError(f"{filename}:{name} shape {list(e['shape'])}, expected {list(shape)}")
        per = e.get("dtype", "f32")
        if per == "q8":
            if e.get("scales_offset") is None or not e.get("group"):
                raise ValueError(f"{filename}:{name} is q8 but carries no scales/group")
            if e["offset"] % 4 or e["scales_offset"] % 4:
                raise ValueError(f"{filename}:{name} q8 offsets {e['offset']}/{e['scales_offset']} are not "
                                 f"4-byte aligned")
            ngroup = -(-shape[1] // e["group"])
            if e["scales_size"] != shape[0] * ngroup * 4:
                raise ValueError(f"{filename}:{name} scales are {e['scales_size']} bytes, expected "
                                 f"{shape[0] * ngroup * 4} for {list(shape)} at group {e['group']}")
            codes = np.frombuffer(blob, np.int8, e["size"], e["offset"]).reshape(shape)
            scales = np.frombuffer(blob, np.float32, e["scales_size"] // 4, e["scales_offset"]).reshape(
                shape[0], ngroup)
            out[name] = (codes, scales, int(e["group"]))
            continue
        if per != "f32":
            raise ValueError(f"{filename}:{name} is {per}; this build reads q8 projections and f32 norms")
        if e["offset"] % 4 or e["size"] % 4:
            raise ValueError(f"{filename}:{name} offset {e['offset']}/size {e['size']} not aligned to f32")
        out[name] = np.frombuffer(blob, np.float32, e["size"] // 4, e["offset"]).reshape(shape)
    if strict:
        for e in entries:
            if e["name"] not in expected:
                raise ValueError(f"{filename}: unexpected tensor {e['name']}")
    return out


def block_file(index):
    return f"block_{index:02d}.bin"


def load_block(path, m, d, index):
    """loader.js:610-626 loadBlock: block `index` (model numbering)."""
    fn = block_file(index)
    return read_tensors(path, fn, m["files"][fn], block_shapes(d, kind_of(d, index)))


def load_mtp(path, m, d):
    """loader.js:628-638 loadMtp: the MTP head's full-attention block and its
    enorm, hnorm, fc_e, fc_h, mtp_norm, embed_draft, head_draft."""
    fn, H, V = d["mtp_file"], d["hidden"], d["mtp_vocab"]
    shapes = dict(block_shapes(d), enorm=[H], hnorm=[H], fc_e=[H, H], fc_h=[H, H], mtp_norm=[H],
                  embed_draft=[V, H], head_draft=[V, H])
    return read_tensors(path, fn, m["files"][fn], shapes)


def load_client(path, m, d):
    """loader.js:644-671 loadClient: wte and norm, and lm_head when untied."""
    out = read_tensors(path, "client.bin", m["files"]["client.bin"],
                       {"wte": [d["vocab"], d["hidden"]], "norm": [d["hidden"]]})
    if not d["tied"]:
        out.update(read_tensors(path, "lm_head.bin", m["files"]["lm_head.bin"],
                                {"lm_head": [d["vocab"], d["hidden"]]}))
    return out


def upload(ctx, path, m=None, d=None):
    """Every position the context holds (its [lo, hi) of the n_layer + 2
    positions: 0 the embedding, 1..n_layer the blocks, n_layer + 1 the head)
    from the checkpoint at `path`."""
    m = m or load_manifest(path)
    d = d or dims_from_manifest(m)
    problems = check_manifest(m, d)
    if problems:
        raise ValueError("; ".join(problems))
    lo, hi = ctx.opts.lo, ctx.opts.hi
    last = d["n_layer"] + 1

    def put(layer, name, t):
        if isinstance(t, tuple):
            codes, scales, group = t
            ctx.upload_q8(layer, TENSOR[name], codes, scales, group)
        else:
            ctx.upload_norm(layer, TENSOR[name], t)

    if lo == 0 or hi - 1 == last:
        client = load_client(path, m, d)
        if lo == 0:
            put(-1, "wte", client["wte"])
        if hi - 1 == last:
            put(-1, "norm", client["norm"])
            if not d["tied"]:
                put(-1, "lm_head", client["lm_head"])
            elif lo != 0:
                put(-1, "wte", client["wte"])
    for pos in range(max(lo, 1), min(hi, last)):
        for name, t in load_block(path, m, d, pos - 1).items():
            put(pos - 1, name, t)
    if hi - 1 == last and d.get("mtp_vocab"):
        # the MTP head, held with the LM head (stage.js:273-289)
        head = {"enorm", "hnorm", "fc_e", "fc_h", "mtp_norm", "embed_draft", "head_draft"}
        for name, t in load_mtp(path, m, d).items():
            put(-1 if name in head else LAYER_MTP, name, t)
