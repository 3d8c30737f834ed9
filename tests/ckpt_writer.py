"""Writes a synthetic checkpoint in the reference's on-disk layout (test
infrastructure): tools/convert_hf.py:594-649 pack_file puts a q8 tensor's
int8 block [N, K] and then its f32 scales [N, ceil(K/group)], and a norm
weight as f32, one after another in a .bin; :768-800 writes the manifest.
The codes and scales here are drawn directly (no f32 weights quantised)."""
import json
import os

import numpy as np

BLOCK_NAMES = ["input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "post_attention_layernorm",
               "gate_proj", "up_proj", "down_proj"]


def f16_exact(x):
    """Values representable in f16 (so the device's f16 scales are exact)."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def pack_file(path, filename, tensors):
    entries, offset = [], 0
    with open(os.path.join(path, filename), "wb") as f:
        for name, t in tensors:
            if isinstance(t, tuple):
                codes, scales, group = t
                codes = np.ascontiguousarray(codes, np.int8)
                scales = np.ascontiguousarray(scales, np.float32)
                f.write(codes.tobytes())
                f.write(scales.tobytes())
                entries.append({"name": name, "shape": list(codes.shape), "offset": offset, "size": codes.nbytes,
                                "dtype": "q8", "group": group, "scales_offset": offset + codes.nbytes,
                                "scales_size": scales.nbytes})
                offset += codes.nbytes + scales.nbytes
            else:
                a = np.ascontiguousarray(t, np.float32)
                f.write(a.tobytes())
                entries.append({"name": name, "shape": list(a.shape), "offset": offset, "size": a.nbytes,
                                "dtype": "f32"})
                offset += a.nbytes
    return entries


def q8(rng, N, K, group, f32_scales=False):
    """Codes and scales drawn directly. By default the scales are f16 values;
    with f32_scales they are what the converter writes (amax / 127 in f32,
    tools/convert_hf.py:493), which f16 does not hold exactly."""
    codes = rng.integers(-127, 128, (N, K)).astype(np.int8)
    amax = rng.uniform(127e-4, 508e-4, (N, -(-K // group)))
    scales = (amax.astype(np.float32) / np.float32(127)) if f32_scales else f16_exact(amax / 127)
    return codes, scales, group


def make(path, d, seed=11, group=64, f32_scales=False):
    """A q8 checkpoint of dims `d` (this build's key names) at `path`.
    Returns {filename: {name: tensor}} with what was written."""
    os.makedirs(path, exist_ok=True)
    rng = np.random.default_rng(seed)
    H, D, F, V = d["hidden"], d["head_dim"], d["ffn"], d["vocab"]
    q, kv = d["n_heads"] * D, d["n_kv_heads"] * D
    shapes = {"q_proj": (q, H), "k_proj": (kv, H), "v_proj": (kv, H), "o_proj": (H, q),
              "gate_proj": (F, H), "up_proj": (F, H), "down_proj": (H, F)}
    manifest = {"model": "synthetic", "arch": "llama", "hidden": H, "n_layer": d["n_layer"],
                "n_head": d["n_heads"], "n_kv_head": d["n_kv_heads"], "head_dim": D,
                "group": d["n_heads"] // d["n_kv_heads"], "ffn": F, "vocab": V, "n_pos": 2048,
                "rms_eps": d["rms_eps"], "rope_theta": d["rope_theta"], "rope_scaling": d.get("rope_scaling"),
                "norm": "rmsnorm", "act": "silu", "dtype": "q8", "layout": "row_major",
                "weight_layout": "out_in", "tied_lm_head": d.get("tied", True), "files": {}}
    written = {}
    for i in range(d["n_layer"]):
        ts = []
        for name in BLOCK_NAMES:
            if name.endswith("layernorm"):
                ts.append((name, f16_exact(rng.uniform(0.5, 1.5, H))))
            else:
                ts.append((name, q8(rng, *shapes[name], group, f32_scales)))
        fn = f"block_{i:02d}.bin"
        manifest["files"][fn] = pack_file(path, fn, ts)
        written[fn] = dict(ts)
    client = [("wte", q8(rng, V, H, group, f32_scales)), ("norm", f16_exact(rng.uniform(0.5, 1.5, H)))]
    manifest["files"]["client.bin"] = pack_file(path, "client.bin", client)
    written["client.bin"] = dict(client)
    if not d.get("tied", True):
        head = [("lm_head", q8(rng, V, H, group, f32_scales))]
        manifest["files"]["lm_head.bin"] = pack_file(path, "lm_head.bin", head)
        written["lm_head.bin"] = dict(head)
    with open(os.path.join(path, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=2)
    return written


# tests/hybrid_weights.py names -> the checkpoint's (loader.js:543-590, 628-638)
HYBRID_NAMES = {"ln1": "input_layernorm", "ln2": "post_attention_layernorm", "q": "q_proj", "k": "k_proj",
                "v": "v_proj", "o": "o_proj", "gate": "gate_proj", "up": "up_proj", "down": "down_proj",
                "attn_gate": "attn_gate", "q_norm": "q_norm", "k_norm": "k_norm", "in_q": "in_proj_q",
                "in_k": "in_proj_k", "in_v": "in_proj_v", "in_z": "in_proj_z", "in_b": "in_proj_b", "in_a": "in_proj_a",
                "out": "out_proj", "gate_params": "gate_params", "gated_norm": "gated_norm"}


def _block_tensors(lw, kd):
    out = []
    for k, t in lw.items():
        if k == "kind":
            continue
        if k == "conv":   # the converter splits conv1d into the q, k, v channel ranges
            out += [("conv1d_q", t[:kd]), ("conv1d_k", t[kd:2 * kd]), ("conv1d_v", t[2 * kd:])]
            continue
        out.append((HYBRID_NAMES[k], (t[0], t[1], 32) if isinstance(t, tuple) else t))
    return out


def make_hybrid(path, d, w, wm=None):
    """A hybrid (Qwen3.5-layout) q8 checkpoint of tests/hybrid_weights.py's
    weights `w` (and MTP head `wm`) at group 32: layer_types, the
    linear_num_* keys, rot_dim, and the MTP file in the manifest."""
    os.makedirs(path, exist_ok=True)
    kd = d["lin_nk"] * d["lin_dk"]
    manifest = {"model": "synthetic-hybrid", "arch": "qwen3_5", "hidden": d["hidden"], "n_layer": d["n_layer"],
                "n_head": d["n_heads"], "n_kv_head": d["n_kv_heads"], "head_dim": d["head_dim"],
                "group": d["n_heads"] // d["n_kv_heads"], "ffn": d["ffn"], "vocab": d["vocab"], "n_pos": 2048,
                "rms_eps": d["rms_eps"], "rope_theta": d["rope_theta"], "rot_dim": d["rot_dim"],
                "layer_types": d["layer_types"], "linear_num_key_heads": d["lin_nk"],
                "linear_num_value_heads": d["lin_nv"], "linear_key_head_dim": d["lin_dk"],
                "linear_value_head_dim": d["lin_dv"], "linear_conv_kernel_dim": d["lin_conv"],
                "norm": "rmsnorm", "act": "silu", "dtype": "q8", "weight_layout": "out_in",
                "tied_lm_head": d.get("tied", True), "files": {}}
    for i, lw in enumerate(w["layers"]):
        fn = f"block_{i:02d}.bin"
        manifest["files"][fn] = pack_file(path, fn, _block_tensors(lw, kd))
    manifest["files"]["client.bin"] = pack_file(path, "client.bin",
                                                [("wte", (*w["wte"], 32)), ("norm", w["norm"])])
    if not d.get("tied", True):
        manifest["files"]["lm_head.bin"] = pack_file(path, "lm_head.bin", [("lm_head", (*w["lm_head"], 32))])
    if wm is not None:
        ts = _block_tensors(wm["block"], kd)
        for k in ("enorm", "hnorm", "mtp_norm"):
            ts.append((k, wm[k]))
        for k in ("fc_e", "fc_h", "embed_draft", "head_draft"):
            ts.append((k, (*wm[k], 32)))
        manifest["files"]["mtp.bin"] = pack_file(path, "mtp.bin", ts)
        manifest["mtp"] = {"file": "mtp.bin", "draft_vocab": int(wm["embed_draft"][0].shape[0])}
    with open(os.path.join(path, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=2)
